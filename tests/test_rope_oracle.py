"""The oracle's RoPE (engine.rs:137-229) pinned by closed forms on the CPU.

Inverse frequencies: the Default and Linear modes against theta^(-2i/d) in
float64; the Llama-3 and YaRN modes against the piecewise rule evaluated in
float64 on the published Llama-3.1 and YaRN settings, plus the regime each
frequency falls in.  Rotation: position 0 is the identity, each pair turns as
the complex product (x0 + i x1) e^{i pos f}, the pair norms are kept, the
dimensions past rotary_dim are untouched, and scores depend only on the
position difference (<R(m)q, R(n)k> = <R(m-n)q, k>)."""
import numpy as np
import pytest

import oracle as O


def _f64_base(d, theta):
    i = np.arange(d // 2, dtype=np.float64)
    return theta ** (-2.0 * i / d)


@pytest.mark.parametrize("d,theta,s", [(128, 10000.0, 1.0), (128, 500000.0, 1.0), (64, 10000.0, 4.0), (96, 1e6, 0.5)])
def test_default_and_linear_inv_freqs(d, theta, s):
    ref = _f64_base(d, theta) / max(s, 1.0)
    for mode in (O.ROPE_DEFAULT, O.ROPE_LINEAR):
        got = O.rope_inv_freqs(d, theta, mode, (s,)).astype(np.float64)
        np.testing.assert_allclose(got, ref, rtol=2e-6)


def _piecewise_f64(d, theta, factor, omp, lo, hi):
    base = _f64_base(d, theta)
    wavelen = 2 * np.pi / base
    low_w, high_w = omp / lo, omp / hi
    smooth = (omp / wavelen - lo) / (hi - lo)
    out = np.where(wavelen < high_w, base, np.where(wavelen > low_w, base / factor,
                                                    base * ((1 - smooth) / factor + smooth)))
    regime = np.where(wavelen < high_w, 0, np.where(wavelen > low_w, 2, 1))
    return out, regime


def test_llama3_inv_freqs():
    # Llama 3.1: theta 500000, factor 8, original context 8192, low 1, high 4
    got = O.rope_inv_freqs(128, 500000.0, O.ROPE_LLAMA3, (8.0, 8192.0, 1.0, 4.0)).astype(np.float64)
    ref, regime = _piecewise_f64(128, 500000.0, 8.0, 8192.0, 1.0, 4.0)
    assert set(regime.tolist()) == {0, 1, 2}  # all three regimes occur
    np.testing.assert_allclose(got, ref, rtol=1e-5)
    base = _f64_base(128, 500000.0)
    np.testing.assert_allclose(got[regime == 0], base[regime == 0], rtol=2e-6)      # high frequencies kept
    np.testing.assert_allclose(got[regime == 2], base[regime == 2] / 8, rtol=2e-6)  # low frequencies / factor
    assert np.all(np.diff(got) < 0)  # still strictly decreasing


def test_yarn_inv_freqs():
    # YaRN as the reference applies it: factor 4, original 4096, beta_fast 32, beta_slow 1
    got = O.rope_inv_freqs(128, 10000.0, O.ROPE_YARN, (4.0, 4096.0, 32.0, 1.0)).astype(np.float64)
    ref, regime = _piecewise_f64(128, 10000.0, 4.0, 4096.0, 1.0, 32.0)
    assert set(regime.tolist()) == {0, 1, 2}
    np.testing.assert_allclose(got, ref, rtol=1e-5)


def _complex_rotation(x, rd, inv, pos):
    half = rd // 2
    x = x.astype(np.float64)
    ang = np.outer(np.asarray(pos, np.float64), inv.astype(np.float64))  # [rows][half]
    ang = np.float32(ang).astype(np.float64)  # the angle is an f32 product
    z = (x[..., :half] + 1j * x[..., half:rd]) * np.exp(1j * ang)[:, None, :]
    out = x.copy()
    out[..., :half] = z.real
    out[..., half:rd] = z.imag
    return out


@pytest.mark.parametrize("d,rd", [(128, 128), (128, 64), (64, 64), (256, 96)])
def test_rotation_closed_forms(d, rd):
    rng = np.random.default_rng(d + rd)
    x = rng.standard_normal((5, 3, d)).astype(np.float32)
    inv = O.rope_inv_freqs(rd, 10000.0)
    pos = np.array([0, 1, 17, 4095, 131071], np.int32)
    y = O.rope_apply(x, rd, inv, pos)
    assert np.array_equal(y[0], x[0])                   # position 0: identity
    assert np.array_equal(y[:, :, rd:], x[:, :, rd:])   # past rotary_dim: untouched
    ref = _complex_rotation(x, rd, inv, pos)
    np.testing.assert_allclose(y, ref, rtol=0, atol=2e-5 * np.abs(x).max())
    half = rd // 2
    n_in = x[..., :half].astype(np.float64) ** 2 + x[..., half:rd].astype(np.float64) ** 2
    n_out = y[..., :half].astype(np.float64) ** 2 + y[..., half:rd].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=1e-5, atol=1e-6)


def test_rope_sincos_is_libm_double_rounded_once():
    """orc_rope_sincos (the rotation's sin/cos, evaluated in f64 and rounded
    once) against libm's double sin/cos of the same f32 angle rounded to f32:
    equal wherever libm's double value is not within 1e-13 (relative) of an
    f32 rounding boundary, over small, RoPE-sized and large angles up to
    2^26 rad, zero (a RoPE angle is pos * inv_freq >= 0: never -0) and quadrant
    edges; a dropped reduction term, a wrong
    quadrant or sign, or a polynomial coefficient off by one term would each
    fail this.  Also sin^2 + cos^2 = 1 to f32 rounding."""
    rng = np.random.default_rng(11)
    th = np.concatenate([
        rng.uniform(-4.0, 4.0, 4000), rng.uniform(0.0, 8192.0, 4000), rng.uniform(0.0, 2.0 ** 20, 2000),
        rng.uniform(0.0, 2.0 ** 26, 500), np.arange(0, 64) * (np.pi / 4), [0.0, 1e-30, 1e-8, 65504.0],
    ]).astype(np.float32)
    sn, cs = O.rope_sincos(th)
    t64 = th.astype(np.float64)
    for got, ref in ((sn, np.sin(t64)), (cs, np.cos(t64))):
        r32 = ref.astype(np.float32)
        # distance of libm's value from the nearest f32 midpoint, in units of the value
        lo = np.nextafter(r32, np.float32(-np.inf)).astype(np.float64)
        hi = np.nextafter(r32, np.float32(np.inf)).astype(np.float64)
        mid = np.minimum(np.abs(ref - (r32.astype(np.float64) + lo) / 2), np.abs(ref - (r32.astype(np.float64) + hi) / 2))
        safe = mid > 1e-13 * np.maximum(np.abs(ref), 1e-300)
        assert safe.mean() > 0.99
        assert np.array_equal(got[safe].view(np.uint32), r32[safe].view(np.uint32))
    n = sn.astype(np.float64) ** 2 + cs.astype(np.float64) ** 2
    np.testing.assert_allclose(n, 1.0, rtol=0, atol=3e-7)
    assert sn[np.flatnonzero(th == 0.0)[0]] == 0.0 and cs[np.flatnonzero(th == 0.0)[0]] == 1.0


def test_rotation_uses_rope_sincos_and_two_roundings():
    """orc_rope_apply turns each pair with orc_rope_sincos's values and rounds
    each product and each sum once: recomputed here from rope_sincos with
    float32 numpy arithmetic (which rounds every operation), bit for bit."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 2, 128)).astype(np.float32)
    inv = O.rope_inv_freqs(64, 1.0e7)
    pos = np.array([5, 4095, 100000], np.int32)
    y = O.rope_apply(x, 64, inv, pos)
    for r in range(3):
        ang = (np.float32(pos[r]) * inv).astype(np.float32)
        sn, cs = O.rope_sincos(ang)
        x0, x1 = x[r, :, :32], x[r, :, 32:64]
        y0 = (x0 * cs).astype(np.float32) - (x1 * sn).astype(np.float32)
        y1 = (x0 * sn).astype(np.float32) + (x1 * cs).astype(np.float32)
        assert np.array_equal(y[r, :, :32], y0) and np.array_equal(y[r, :, 32:64], y1)
        assert np.array_equal(y[r, :, 64:], x[r, :, 64:])


def test_scores_depend_on_position_difference():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 1, 128)).astype(np.float32)
    inv = O.rope_inv_freqs(128, 10000.0)
    for m, n in ((10, 3), (200, 150), (1000, 999)):
        lhs = float(np.dot(O.rope_apply(q, 128, inv, [m])[0, 0], O.rope_apply(k, 128, inv, [n])[0, 0]))
        rhs = float(np.dot(O.rope_apply(q, 128, inv, [m - n])[0, 0], k[0, 0]))
        assert abs(lhs - rhs) <= 1e-3 * (np.linalg.norm(q) * np.linalg.norm(k)), (m, n)


def test_library_inv_freqs_match_oracle():
    """The product's host helper (lnskv_rope_inv_freqs) and the oracle agree
    to the last bit or one ulp on every mode (both are f32 restatements)."""
    import ctypes as C
    from lnskv import _lib
    L = _lib.lib()
    cases = [(128, 10000.0, O.ROPE_DEFAULT, (1.0,)), (64, 1e6, O.ROPE_LINEAR, (4.0,)),
             (128, 500000.0, O.ROPE_LLAMA3, (8.0, 8192.0, 1.0, 4.0)), (96, 10000.0, O.ROPE_YARN, (4.0, 4096.0, 32.0, 1.0))]
    for d, theta, mode, params in cases:
        p = np.zeros(4, np.float32)
        p[:len(params)] = params
        got = np.zeros(d // 2, np.float32)
        assert L.lnskv_rope_inv_freqs(d, theta, mode, p.ctypes.data_as(C.c_void_p), got.ctypes.data_as(C.c_void_p)) == 0
        ref = O.rope_inv_freqs(d, theta, mode, params)
        ulps = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert ulps.max() <= 1, (mode, ulps.max())
    out = np.zeros(2, np.float32)
    assert L.lnskv_rope_inv_freqs(3, 1e4, 0, p.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p)) == _lib.ERR_INVALID
    assert L.lnskv_rope_inv_freqs(4, 1e4, 9, p.ctypes.data_as(C.c_void_p), out.ctypes.data_as(C.c_void_p)) == _lib.ERR_INVALID


def test_rope_dim_rule():
    """engine.rs:826-833: round(head_dim * factor) when in [2, head_dim)."""
    from lnskv import _lib
    L = _lib.lib()
    assert L.lnskv_rope_dim(128, 1.0) == 128
    assert L.lnskv_rope_dim(128, 0.5) == 64
    assert L.lnskv_rope_dim(128, 0.25) == 32
    assert L.lnskv_rope_dim(64, 0.0) == 64   # below 2: the whole head
    assert L.lnskv_rope_dim(80, 0.4) == 32
