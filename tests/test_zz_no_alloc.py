"""lnskv_append_decode_noalloc (the entry point that allocates nothing) against
lnskv_append_decode on the same inputs, through the C ABI.

Both run the same kernels, so the bar is bit-for-bit: identical output rows and
identical pages (and Q8A scales) after the fused append.  Two calls in a row on
the static scratch, the second with a smaller batch, so that the second call
runs over what the first left in the scratch.  A call whose schedule needs more
than the scratch holds is refused before anything is launched."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import TOL, dev_f32, dev_i32, fill_pages, host_pages, rel_err, say
from lnskv import DTYPE_F16, DTYPE_F32, DTYPE_NAMES, DTYPE_Q8A, NO_PAGE
from lnskv._lib import ERR_WORKSPACE, lib
from lnskv.device import PagedKV, sync

pytestmark = pytest.mark.gpu


def _stream(dev):
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _batch(gpu, dtype, lens, seed, n_kv=8, rep=4, d=128):
    rng = np.random.default_rng(seed)
    pages_per = [(L + 1 + 15) // 16 for L in lens]  # room for the appended token
    num_pages = sum(pages_per) + 16
    pk = PagedKV(num_pages, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=seed, scale=0.5)
    perm = rng.permutation(num_pages).astype(np.uint32)
    stride = max(pages_per) + 1
    tables = np.full((len(lens), stride), NO_PAGE, np.uint32)
    k = 0
    for s, n in enumerate(pages_per):
        tables[s, :n] = perm[k:k + n]
        k += n
    n_seq = len(lens)
    q = rng.standard_normal((n_seq, n_kv * rep, d)).astype(np.float32)
    k_new = rng.standard_normal((n_seq, n_kv, d)).astype(np.float32)
    v_new = rng.standard_normal((n_seq, n_kv, d)).astype(np.float32)
    kv_len = np.array(lens, np.int32) + 1  # includes the appended token
    return pk, tables, kv_len, q, k_new, v_new


def _clone(pk: PagedKV) -> PagedKV:
    twin = PagedKV(pk.num_pages, pk.n_kv, pk.head_dim, pk.dtype, pk.device)
    twin.k.copy_(pk.k)
    twin.v.copy_(pk.v)
    if pk.ks is not None:
        twin.ks.copy_(pk.ks)
        twin.vs.copy_(pk.vs)
    return twin


def _pools_equal(a: PagedKV, b: PagedKV) -> bool:
    same = torch.equal(a.k.view(torch.uint8), b.k.view(torch.uint8)) and \
        torch.equal(a.v.view(torch.uint8), b.v.view(torch.uint8))
    if a.ks is not None:
        same = same and torch.equal(a.ks.view(torch.int32), b.ks.view(torch.int32)) and \
            torch.equal(a.vs.view(torch.int32), b.vs.view(torch.int32))
    return same


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_Q8A])
def test_noalloc_matches_append_decode_twice(gpu, dtype):
    rng = np.random.default_rng(11 + dtype)
    cases = [
        ("large", [int(x) for x in rng.integers(512, 4097, 32)]),
        ("smaller", [int(x) for x in rng.integers(20, 900, 5)]),
    ]
    for what, lens in cases:
        say("noalloc", DTYPE_NAMES[dtype], what, "n_seq", len(lens), "max len", max(lens))
        pk, tables, kv_len, q, k_new, v_new = _batch(gpu, dtype, lens, seed=len(lens) * 7 + dtype)
        twin = _clone(pk)
        hp_before, _ = host_pages(pk) if what == "smaller" else (None, None)
        n_seq, n_heads = len(lens), 32
        dq, dk, dv = dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu)
        dt, dl = dev_i32(tables, gpu), dev_i32(kv_len, gpu)
        max_len = int(kv_len.max())
        scale = float(1.0 / np.sqrt(128))
        ws = torch.zeros(max(pk.workspace_size(n_seq, n_heads, max_len, 0), 16), dtype=torch.uint8, device=gpu)
        ref_out = pk.append_decode(dq, dk, dv, dt, dl, n_heads=n_heads, max_kv_len=max_len, scale=scale,
                                   workspace=ws)
        out = torch.full((n_seq, n_heads, 128), float("nan"), dtype=torch.float32, device=gpu)
        rc = lib().lnskv_append_decode_noalloc(C.byref(twin.desc), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                               out.data_ptr(), dt.data_ptr(), int(tables.shape[1]), dl.data_ptr(),
                                               None, n_seq, n_heads, max_len, scale, 0, _stream(gpu))
        assert rc == 0, lib().lnskv_last_error()
        sync()
        assert torch.equal(out.view(torch.int32), ref_out.view(torch.int32)), what
        assert _pools_equal(pk, twin), what
        if hp_before is not None:
            # the smaller case also against the oracle: append, then the f64 scan
            O.append(hp_before, k_new, v_new, np.arange(n_seq, dtype=np.int32), kv_len - 1, tables)
            ref = O.decode_f64(hp_before, q, tables, kv_len, None, scale)
            assert rel_err(out, ref).max() < TOL[dtype]


def test_noalloc_refuses_a_schedule_larger_than_the_scratch(gpu):
    say("noalloc refusal (f32 pages, split-K partials over the scratch size)")
    n_seq, n_kv, rep, d, L = 64, 8, 4, 128, 500
    pk, tables, kv_len, q, k_new, v_new = _batch(gpu, DTYPE_F32, [L] * n_seq, seed=3, n_kv=n_kv, rep=rep, d=d)
    n_heads = n_kv * rep
    need = pk.workspace_size(n_seq, n_heads, int(kv_len.max()), 16)
    assert need > (24 << 20)
    twin = _clone(pk)
    dq, dk, dv = dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu)
    dt, dl = dev_i32(tables, gpu), dev_i32(kv_len, gpu)
    out = torch.full((n_seq, n_heads, d), 7.0, dtype=torch.float32, device=gpu)
    rc = lib().lnskv_append_decode_noalloc(C.byref(pk.desc), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                           out.data_ptr(), dt.data_ptr(), int(tables.shape[1]), dl.data_ptr(),
                                           None, n_seq, n_heads, int(kv_len.max()), 0.08, 16, _stream(gpu))
    assert rc == ERR_WORKSPACE, (rc, lib().lnskv_last_error())
    sync()
    assert bool((out == 7.0).all())          # nothing ran
    assert _pools_equal(pk, twin)


def test_noalloc_allocates_nothing_and_replays_under_capture(gpu):
    """After one warm-up call (the scratch address lookup and the schedule
    caches), the library's own buffers are released: an eager call then takes
    no device memory, and the call captured into a HIP graph replays with the
    eager call's bits (the append rewrites the same slot with the same values)."""
    say("noalloc: no device memory taken, graph capture and replay")
    lens = [700, 1500, 3000, 64]
    pk, tables, kv_len, q, k_new, v_new = _batch(gpu, DTYPE_Q8A, lens, seed=21)
    n_seq, n_heads = len(lens), 32
    dq, dk, dv = dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu)
    dt, dl = dev_i32(tables, gpu), dev_i32(kv_len, gpu)
    max_len = int(kv_len.max())
    scale = float(1.0 / np.sqrt(128))
    out = torch.zeros((n_seq, n_heads, 128), dtype=torch.float32, device=gpu)

    def call():
        rc = lib().lnskv_append_decode_noalloc(C.byref(pk.desc), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                               out.data_ptr(), dt.data_ptr(), int(tables.shape[1]), dl.data_ptr(),
                                               None, n_seq, n_heads, max_len, scale, 0, _stream(gpu))
        assert rc == 0, lib().lnskv_last_error()

    call()
    sync()
    assert lib().lnskv_workspace_release() == 0
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(gpu)[0]
    call()
    sync()
    assert torch.cuda.mem_get_info(gpu)[0] == free0
    eager = out.clone()
    s = torch.cuda.Stream(device=gpu)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call()
    for i in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), eager.view(torch.int32)), i
