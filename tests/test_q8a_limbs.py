"""The int8-limb split of q that the Q8A matrix-core decode uses for q.k
(lnskv_decode_mfma.hip, init_wave_state_q8), restated in float32 and checked
for the two facts the kernel relies on: every limb is an int8 in [-127, 127]
(so 128 products of two int8 values sum below 2^31, exactly), and
limb0 + limb1/254 + limb2/254^2 reproduces y = q*127/amax to within
0.5/254^2 plus float32 rounding -- over random heads and the edges: values at
+-amax, at the rounding midpoints of each limb, zeros and a 10^6 range."""
import numpy as np
import pytest

F = np.float32


def limbs(x):
    """float32 steps in the kernel's order: amax over the head, y = x * (127 / amax)."""
    x = x.astype(F)
    amax = F(np.max(np.abs(x)))
    inv = F(127.0) / amax if amax >= F(2.0 ** -100) else F(0.0)
    y = (x * inv).astype(F)
    l0 = np.rint(y).astype(F)
    r1 = ((y - l0) * F(254.0)).astype(F)
    l1 = np.rint(r1).astype(F)
    l2 = np.rint(((r1 - l1) * F(254.0)).astype(F)).astype(F)
    return y, l0, l1, l2, amax


def check(x):
    y, l0, l1, l2, amax = limbs(x)
    for l in (l0, l1, l2):
        assert np.all(np.abs(l) <= 127), l
        assert np.all(l == np.round(l))
    rec = l0.astype(np.float64) + l1 / 254.0 + l2 / 254.0 ** 2
    # the split is of the float32 y; its own rounding error is 2^-24 |y|
    assert np.all(np.abs(rec - y.astype(np.float64)) <= 0.5 / 254.0 ** 2 + 127 * 2.0 ** -24), np.abs(rec - y).max()
    # and y is x * 127 / amax to float32 rounding
    if amax > 0:
        assert np.allclose(y, x.astype(np.float64) * 127.0 / amax, rtol=2 ** -22, atol=0)


@pytest.mark.parametrize("seed", range(20))
def test_random_heads(seed):
    rng = np.random.default_rng(seed)
    for scale in (1e-30, 1e-3, 1.0, 37.0, 1e5):
        check(rng.standard_normal(128).astype(F) * F(scale))


def test_edges():
    base = np.linspace(-1, 1, 128).astype(F)
    check(base)                                   # +-amax exactly
    check(np.zeros(128, F))                       # zero head: limbs 0
    # values at the rounding midpoints of limb 0 and limb 1 (y = k + 0.5,
    # y = k + 0.5/254) and just around them
    y = np.array([0.5, -0.5, 126.5, -126.5, 0.5 / 254, 1 + 0.5 / 254, 127.0], np.float64)
    for eps in (0.0, 1e-7, -1e-7):
        x = np.concatenate([(y + eps) / 127.0, np.zeros(121)]).astype(F)
        x[-1] = 1.0  # amax = 1: y = 127 x
        check(x)
    # a 10^6 range inside one head
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(128) * 3e-5).astype(F)
    x[17] = 30.0
    check(x)


def test_tiny_head_scores_zero():
    y, l0, l1, l2, amax = limbs(np.full(128, 1e-35, F))
    assert amax < 2.0 ** -100 and not l0.any() and not l1.any() and not l2.any()


def test_sums_stay_exact_in_int32():
    # the largest |sum of 128 products| of int8 limbs and int8 codes
    assert 128 * 127 * 127 < 2 ** 31
    # and below 2^24, so its conversion to float is exact as well
    assert 128 * 127 * 127 < 2 ** 24
