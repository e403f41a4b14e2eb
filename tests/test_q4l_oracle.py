"""Q4_L (o_proj weights) without a GPU: pins of the oracle's repack, decode
and float64 GEMV, and the library's host repack (lnskv_q4l_prepare) against
the oracle's, bit for bit.

Pins: a hand-built block whose weights are known in closed form (sign,
magnitude grid 2^(m-5), zero code, nibble order, one scale per 32 weights);
the repacked scales against numpy's round-to-nearest-even float16 of the f32
products; the GEMV against numpy's matmul of the decoded weights."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from lnskv import _lib


def _disk_block(g_f16: float, sl, nibbles) -> np.ndarray:
    b = np.zeros(O.Q4L_DISK_BYTES, np.uint8)
    b[0:2] = np.frombuffer(np.float16(g_f16).tobytes(), np.uint8)
    for i in range(8):
        b[2 + i // 2] |= (sl[i] & 0xF) << (4 * (i % 2))
    for i in range(256):
        b[6 + i // 2] |= (nibbles[i] & 0xF) << (4 * (i % 2))
    return b


def _random_disk(rng, n_blocks):
    d = rng.integers(0, 256, (n_blocks, O.Q4L_DISK_BYTES), dtype=np.uint8)
    # global scales: f16 values over many octaves, some subnormal and some huge
    g = np.exp2(rng.uniform(-20, 12, n_blocks)).astype(np.float16)
    g[::17] = np.float16(6.0e-8)   # smallest subnormal
    g[5::29] = np.float16(65504.0)  # with local scales above 7 the product overflows f16
    d[:, 0:2] = g.view(np.uint8).reshape(n_blocks, 2)
    return d.reshape(-1)


def test_decode_closed_forms():
    # scale_global 1, local scales 7 + (0, 1, ..., ) -> effective 2^(sl-7)
    sl = [7, 8, 6, 7, 0, 15, 7, 7]
    nib = [0] * 256
    nib[0], nib[1] = 0x5, 0xD            # +1, -1 (low nibble = even weight)
    nib[2], nib[3] = 0x1, 0x7            # 2^-4, 2^2
    nib[4], nib[5] = 0x0, 0x8            # zero, negative zero code
    nib[32], nib[33] = 0x5, 0xE          # sub-block 1: scale 2: +2, -4
    nib[64] = 0x5                        # sub-block 2: scale 1/2
    nib[128], nib[160] = 0x5, 0x7        # sub-block 4: scale 2^-7; sub-block 5: 2^8 * 4
    dev = O.q4l_prepare(_disk_block(1.0, sl, nib))
    scales = dev[:16].view(np.float16).astype(np.float64)
    assert np.array_equal(scales, np.exp2(np.array(sl, np.float64) - 7))
    assert np.array_equal(dev[16:], _disk_block(1.0, sl, nib)[6:])
    w = O.q4l_decode_block(dev)
    assert w[0] == 1.0 and w[1] == -1.0 and w[2] == 0.0625 and w[3] == 4.0
    assert w[4] == 0.0 and w[5] == 0.0
    assert w[32] == 2.0 and w[33] == -4.0 and w[64] == 0.5
    assert w[128] == 2.0 ** -7 and w[160] == 2.0 ** 8 * 4
    assert np.count_nonzero(w) == 9


def test_prepare_scales_are_rne_float16():
    rng = np.random.default_rng(1)
    n = 300
    disk = _random_disk(rng, n)
    dev = O.q4l_prepare(disk).reshape(n, O.Q4L_DEV_BYTES)
    d = disk.reshape(n, O.Q4L_DISK_BYTES)
    g = d[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(n)
    for i in range(8):
        sl = (d[:, 2 + i // 2] >> (4 * (i % 2))) & 0xF
        prod = g * np.exp2(sl.astype(np.float32) - 7).astype(np.float32)  # exact in f32
        with np.errstate(over="ignore"):
            exp = prod.astype(np.float16)  # round to nearest even, overflow to inf
        got = dev[:, 2 * i:2 * i + 2].copy().view(np.float16).reshape(n)
        assert np.array_equal(got.view(np.uint16), exp.view(np.uint16)), i
    assert np.array_equal(dev[:, 16:], d[:, 6:])


def test_gemv_f64_against_numpy():
    rng = np.random.default_rng(2)
    rows, cols, n_vec = 19, 768, 3
    disk = _random_disk(rng, rows * cols // 256)
    # keep the values finite: no overflowing scales here
    dd = disk.reshape(-1, O.Q4L_DISK_BYTES)
    dd[:, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    dev = O.q4l_prepare(dd.reshape(-1))
    x = rng.standard_normal((n_vec, cols)).astype(np.float32)
    y0 = rng.standard_normal((n_vec, rows)).astype(np.float32)
    got = O.q4l_gemv_f64(dev, x, y0, rows, cols)
    W = O.q4l_decode_matrix(dev, rows, cols).astype(np.float64)
    ref = y0.astype(np.float64) + x.astype(np.float64) @ W.T
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    # the whole-matrix decode agrees with the per-block one
    assert np.array_equal(W[3, 256:512], O.q4l_decode_block(dev[(3 * 3 + 1) * 144:(3 * 3 + 2) * 144]))


def test_library_prepare_matches_oracle():
    lib = _lib.lib()
    rng = np.random.default_rng(3)
    rows, cols = 7, 1000  # 4 blocks per row, the last one partly padding
    n = rows * ((cols + 255) // 256)
    disk = _random_disk(rng, n)
    out = np.zeros(n * O.Q4L_DEV_BYTES, np.uint8)
    rc = lib.lnskv_q4l_prepare(disk.ctypes.data_as(C.c_void_p), disk.nbytes, rows, cols,
                               out.ctypes.data_as(C.c_void_p))
    assert rc == 0, _lib.last_error()
    assert np.array_equal(out, O.q4l_prepare(disk))
    # too few bytes is refused
    rc = lib.lnskv_q4l_prepare(disk.ctypes.data_as(C.c_void_p), disk.nbytes - 1, rows, cols,
                               out.ctypes.data_as(C.c_void_p))
    assert rc == _lib.ERR_INVALID


@pytest.mark.parametrize("bad", ["cols", "null", "x_stride", "y_stride", "x_align", "ws_small", "ws_align"])
def test_gemv_rejects_bad_arguments(bad):
    """Every check runs before anything touches the GPU (the pointers here
    are never dereferenced): the call returns the status and leaves nothing
    queued."""
    lib = _lib.lib()
    f = lib.lnskv_q4l_gemv_accumulate
    # blocks, x, y, rows, cols, n_vec, x_stride, y_stride, ws, ws_bytes, stream
    if bad == "cols":
        assert f(16, 16, 16, 4, 300, 1, 300, 4, None, 0, None) == _lib.ERR_UNSUPPORTED
        assert "256" in _lib.last_error()
    elif bad == "null":
        assert f(None, 16, 16, 4, 256, 1, 256, 4, None, 0, None) == _lib.ERR_INVALID
    elif bad == "x_stride":
        assert f(16, 16, 16, 4, 512, 1, 256, 4, None, 0, None) == _lib.ERR_INVALID
    elif bad == "y_stride":
        assert f(16, 16, 16, 64, 256, 1, 256, 32, None, 0, None) == _lib.ERR_INVALID
    elif bad == "x_align":
        assert f(16, 20, 16, 4, 256, 1, 256, 4, None, 0, None) == _lib.ERR_INVALID
    else:
        # 4096 columns split a row's blocks over workgroups: a workspace is read
        need = C.c_size_t()
        assert lib.lnskv_q4l_workspace_size(4096, 32, C.byref(need)) == 0 and need.value > 0
        if bad == "ws_small":
            # the call's own need (its launch plan) is at most the query's bound;
            # a workspace of the count header alone holds no partial sums
            assert f(16, 16, 16, 64, 4096, 32, 4096, 64, 32, _lib.WORKSPACE_HEADER_BYTES, None) == \
                _lib.ERR_WORKSPACE
        else:
            assert f(16, 16, 16, 64, 4096, 32, 4096, 64, 24, need.value, None) == _lib.ERR_WORKSPACE
        assert "workspace" in _lib.last_error()
