"""GPU o_proj over Q4_L weights (lnskv_q4l_gemv_accumulate) against the
float64 oracle: y_in + W x for every vector, within 2e-6 of
sum_c |W[r][c] x[c]| + |y_in| (f32 sums of exact f16 x f16 products: ~cols/32
f32 roundings of the sub-block partial sums, x split into two f16 parts
rounded toward zero, to 2^-20; measured at most 1.8e-7 at 4096 columns.
Dropping the lo part of x would give ~2^-11).  Shapes cover one vector, odd counts, row counts that
are not multiples of 16, padded strides, more than 64 vectors (two passes),
the Llama-3-8B o_proj shape at batch 32 and wider rows whose waves take two
blocks each (the next block's weights arriving during the products); every
call gives the same bits, and the padding of y is not written."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import say
from lnskv.device import Q4LMatrix, sync

pytestmark = pytest.mark.gpu


def _disk(rng, rows, cols):
    n = rows * (cols // 256)
    d = rng.integers(0, 256, (n, O.Q4L_DISK_BYTES), dtype=np.uint8)
    g = np.exp2(rng.uniform(-12, -2, n)).astype(np.float16)  # scale_global ~ max |w| of a block
    g[::13] = np.float16(3.0e-5)                             # f16 subnormal global scales
    d[:, 0:2] = g.view(np.uint8).reshape(n, 2)
    return d.reshape(-1)


@pytest.mark.parametrize("rows,cols,n_vec,xpad,ypad", [
    (16, 256, 1, 0, 0),
    (37, 512, 3, 4, 3),
    (64, 1024, 8, 0, 0),
    (100, 2048, 13, 8, 5),
    (48, 512, 70, 0, 0),
    (4096, 4096, 32, 0, 0),
    (2048, 8192, 3, 0, 0),    # split launch, two blocks per wave (one vector tile)
    (4096, 8192, 24, 4, 0),   # split launch, two blocks per wave (two vector tiles)
    (512, 4096, 70, 0, 3),    # two split launches (4 tiles, then 1) sharing the arrival counts
])
def test_q4l_gemv_accumulate(gpu, rows, cols, n_vec, xpad, ypad):
    say("q4l gemv", rows, cols, n_vec, xpad, ypad)
    rng = np.random.default_rng(rows + cols + n_vec)
    disk = _disk(rng, rows, cols)
    W = Q4LMatrix(disk, rows, cols, gpu)
    x = rng.standard_normal((n_vec, cols + xpad)).astype(np.float32)
    y0 = rng.standard_normal((n_vec, rows + ypad)).astype(np.float32)
    xd = torch.from_numpy(x).to(gpu)[:, :cols] if xpad == 0 else torch.from_numpy(x).to(gpu)
    yd = torch.from_numpy(y0).to(gpu)
    W.gemv_accumulate(xd, yd)
    sync()
    got = yd.cpu().numpy()
    dev = W.blocks.cpu().numpy()
    assert np.array_equal(dev, O.q4l_prepare(disk))
    ref = O.q4l_gemv_f64(dev, x[:, :cols], y0[:, :rows], rows, cols)
    wabs = np.abs(O.q4l_decode_matrix(dev, rows, cols).astype(np.float64))
    bound = 2e-6 * (np.abs(x[:, :cols]).astype(np.float64) @ wabs.T + np.abs(y0[:, :rows])) + 1e-30
    err = np.abs(got[:, :rows] - ref)
    say("max err / bound", float((err / bound).max()))
    assert np.all(err <= bound)
    assert np.array_equal(got[:, rows:], y0[:, rows:])  # padding untouched
    # the same bits on a second call
    yd2 = torch.from_numpy(y0).to(gpu)
    W.gemv_accumulate(xd, yd2)
    sync()
    assert torch.equal(yd2, yd)


def test_q4l_caller_workspace(gpu):
    """A caller's workspace (arrival counts zeroed once) gives the bits of the
    library's buffer, call after call and across shapes that share it (every
    call leaves the counts zero); one too small is refused before any
    launch, leaving y untouched."""
    from lnskv import _lib
    say("q4l caller workspace")
    rng = np.random.default_rng(11)
    shapes = [(4096, 4096, 32), (1000, 2048, 5), (4096, 4096, 64)]
    mats = {}
    need = 0
    for rows, cols, n_vec in shapes:
        mats[(rows, cols)] = Q4LMatrix(_disk(rng, rows, cols), rows, cols, gpu)
        need = max(need, mats[(rows, cols)].workspace_size(n_vec))
    assert need > _lib.WORKSPACE_HEADER_BYTES
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    for rep in range(2):
        for rows, cols, n_vec in shapes:
            W = mats[(rows, cols)]
            x = torch.from_numpy(rng.standard_normal((n_vec, cols)).astype(np.float32)).to(gpu)
            y0 = torch.from_numpy(rng.standard_normal((n_vec, rows)).astype(np.float32)).to(gpu)
            ya, yb = y0.clone(), y0.clone()
            W.gemv_accumulate(x, ya, ws)
            W.gemv_accumulate(x, yb)
            sync()
            assert torch.equal(ya, yb), (rep, rows, cols, n_vec)
    assert int(ws[:_lib.WORKSPACE_HEADER_BYTES].count_nonzero()) == 0
    W = mats[(4096, 4096)]
    # the call's own need (its launch plan) is at most the query's bound; the
    # count header alone holds none of its partial sums
    small = torch.zeros(_lib.WORKSPACE_HEADER_BYTES + 16, dtype=torch.uint8, device=gpu)
    x = torch.ones((32, 4096), device=gpu)
    y = torch.zeros((32, 4096), device=gpu)
    with pytest.raises(RuntimeError, match="workspace"):
        W.gemv_accumulate(x, y, small)
    sync()
    assert int(y.count_nonzero()) == 0


def test_q4l_graph_replay_library_buffer(gpu):
    """lnskv_workspace_reserve grows the library's Q4L buffer (its arrival
    counts zeroed) before a capture; the captured y = y0; y += W x (a split
    launch, 4096 x 4096 with 32 vectors) then replays with unrelated eager
    work between the replays, each replay equal to the eager call bit for
    bit, so the counts are back at zero after every replay."""
    from lnskv._lib import check, lib
    say("q4l graph replay")
    rng = np.random.default_rng(21)
    rows, cols, n_vec = 4096, 4096, 32
    W = Q4LMatrix(_disk(rng, rows, cols), rows, cols, gpu)
    check(lib().lnskv_workspace_reserve(0, 0, W.workspace_size(n_vec)))
    x = torch.from_numpy(rng.standard_normal((n_vec, cols)).astype(np.float32)).to(gpu)
    y0 = torch.from_numpy(rng.standard_normal((n_vec, rows)).astype(np.float32)).to(gpu)
    want = y0.clone()
    W.gemv_accumulate(x, want)
    y = torch.empty_like(y0)
    sync()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y.copy_(y0)
        W.gemv_accumulate(x, y)
    torch.cuda.synchronize()
    scratch = torch.randn(1 << 20, device=gpu)
    for rep in range(4):
        y.zero_()
        g.replay()
        got = y.clone()
        scratch.mul_(1.0001)  # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(got, want), rep
