"""A caller's workspace whose arrival-count header was not zeroed before its
first use: the decode's workgroup schedule and the split Q4L GEMV count
their workgroups in that header, and a count above what one call can reach
is reported by the next lnskv_sync as LNSKV_ERR_WORKSPACE (the results of
that call are wrong, and no kernel faults).  The report clears on reading;
the counts stay as they were, so the next call on the same header is
reported again, and a zeroed header gives correct results once more."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import TOL, dev_f32, dev_i32, fill_pages, host_pages, rel_err, say
from lnskv import DTYPE_Q8A, NO_PAGE
from lnskv._lib import ERR_WORKSPACE, WORKSPACE_HEADER_BYTES as HEADER_BYTES, LnskvError
from lnskv.device import PagedKV, Q4LMatrix, sync

pytestmark = pytest.mark.gpu

POISON = 0x40  # every count word reads 0x40404040, far above any workgroup count


def _expect_reported():
    with pytest.raises(LnskvError) as e:
        sync()
    assert e.value.status == ERR_WORKSPACE
    sync()  # the report is cleared on reading


def _drain_report():
    try:
        sync()
    except LnskvError:
        pass


def test_decode_poisoned_header_is_reported(gpu, monkeypatch):
    monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", "workgroup")
    monkeypatch.delenv("LNSKV_FORCE_VALU", raising=False)  # the matrix-core schedule itself
    say("decode workgroup schedule, poisoned workspace header")
    n_kv, d, rep, L = 8, 128, 4, 4096
    rng = np.random.default_rng(5)
    npg = L // 16
    pk = PagedKV(npg + 8, n_kv, d, DTYPE_Q8A, gpu)
    fill_pages(pk, seed=5)
    tables = np.full((1, npg + 1), NO_PAGE, np.uint32)
    tables[0, :npg] = rng.permutation(npg + 8)[:npg].astype(np.uint32)
    kv_len = np.array([L], np.int32)
    q = rng.standard_normal((1, n_kv * rep, d)).astype(np.float32)
    hp, _ = host_pages(pk)
    ref = O.decode_f64(hp, q, tables, kv_len, None, 0.0883883)
    nbytes = pk.workspace_size(1, n_kv * rep, L, 0)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    args = (dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu))
    kw = dict(n_heads=n_kv * rep, max_kv_len=L, scale=0.0883883, split=0, workspace=ws)
    try:
        out = pk.decode(*args, **kw)
        sync()
        assert rel_err(out, ref).max() < TOL[DTYPE_Q8A]
        ws[:HEADER_BYTES].fill_(POISON)
        for _ in range(2):  # the counts stay poisoned: reported on every call
            pk.decode(*args, **kw)
            _expect_reported()
        ws[:HEADER_BYTES].zero_()
        out = pk.decode(*args, **kw)
        sync()
        assert rel_err(out, ref).max() < TOL[DTYPE_Q8A]
        assert int(ws[:HEADER_BYTES].count_nonzero()) == 0
    finally:
        _drain_report()


def test_q4l_poisoned_header_is_reported(gpu):
    say("q4l split launch, poisoned workspace header")
    rows, cols, n_vec = 4096, 4096, 32
    rng = np.random.default_rng(9)
    n = rows * (cols // 256)
    disk = rng.integers(0, 256, (n, O.Q4L_DISK_BYTES), dtype=np.uint8)
    disk[:, 0:2] = np.exp2(rng.uniform(-12, -2, n)).astype(np.float16).view(np.uint8).reshape(n, 2)
    W = Q4LMatrix(disk.reshape(-1), rows, cols, gpu)
    ws = torch.zeros(W.workspace_size(n_vec), dtype=torch.uint8, device=gpu)
    x = torch.from_numpy(rng.standard_normal((n_vec, cols)).astype(np.float32)).to(gpu)
    y0 = torch.from_numpy(rng.standard_normal((n_vec, rows)).astype(np.float32)).to(gpu)
    try:
        good = y0.clone()
        W.gemv_accumulate(x, good, ws)
        sync()
        ws[:HEADER_BYTES].fill_(POISON)
        y = y0.clone()
        W.gemv_accumulate(x, y, ws)
        _expect_reported()
        ws[:HEADER_BYTES].zero_()
        y = y0.clone()
        W.gemv_accumulate(x, y, ws)
        sync()
        assert torch.equal(y, good)
    finally:
        _drain_report()


def test_q4l_unsplit_call_needs_no_workspace(gpu):
    """8192 rows with up to 16 vectors fill the GPU without splitting a row's
    blocks: such a call reads no workspace, so a NULL workspace works under
    graph capture without growing the library buffer."""
    say("q4l unsplit call under capture, NULL workspace")
    rows, cols, n_vec = 8192, 2048, 8
    rng = np.random.default_rng(13)
    n = rows * (cols // 256)
    disk = rng.integers(0, 256, (n, O.Q4L_DISK_BYTES), dtype=np.uint8)
    disk[:, 0:2] = np.exp2(rng.uniform(-12, -2, n)).astype(np.float16).view(np.uint8).reshape(n, 2)
    W = Q4LMatrix(disk.reshape(-1), rows, cols, gpu)
    x = torch.from_numpy(rng.standard_normal((n_vec, cols)).astype(np.float32)).to(gpu)
    y0 = torch.from_numpy(rng.standard_normal((n_vec, rows)).astype(np.float32)).to(gpu)
    eager = y0.clone()
    W.gemv_accumulate(x, eager)
    sync()
    from lnskv import lib
    from lnskv._lib import check
    check(lib().lnskv_workspace_release())
    y = y0.clone()
    s = torch.cuda.Stream(device=gpu)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            W.gemv_accumulate(x, y)
    for _ in range(3):
        y.copy_(y0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
