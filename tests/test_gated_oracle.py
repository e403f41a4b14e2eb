"""Pins of the oracle's gated-query split (orc_split_gated_query, a
restatement of split_gated_query_interleaved, engine.rs:287-307): the
interleaved layout on a hand-built case, and the f32 logistic function
against closed forms and a float64 evaluation."""
import numpy as np

import oracle as O


def _ulps(a, b):
    """Distance in f32 units in the last place (same-sign finite values)."""
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


def test_layout_hand_built():
    # 2 rows x 3 heads x head_dim 4: head (r, h) holds q = 100r + 10h + [0..3],
    # then gate logits = -(100r + 10h + [0..3]) / 50
    rows, heads, d = 2, 3, 4
    x = np.zeros((rows, heads, 2 * d), np.float32)
    for r in range(rows):
        for h in range(heads):
            base = 100 * r + 10 * h + np.arange(d)
            x[r, h, :d] = base
            x[r, h, d:] = -base / 50.0
    q, g = O.split_gated_query(x, heads, d)
    assert q.shape == (rows, heads, d) and g.shape == (rows, heads, d)
    for r in range(rows):
        for h in range(heads):
            base = 100 * r + 10 * h + np.arange(d)
            assert np.array_equal(q[r, h], base.astype(np.float32))
            ref = 1.0 / (1.0 + np.exp(base / 50.0))  # logistic of -base/50, in f64
            assert np.all(_ulps(g[r, h], ref.astype(np.float32)) <= 2)
    # the flat form (one row of all heads) reads the same
    q2, g2 = O.split_gated_query(x.reshape(-1), heads, d)
    assert np.array_equal(q2, q) and np.array_equal(g2, g)


def test_logistic_closed_forms():
    heads, d = 1, 8
    logits = np.array([0.0, -0.0, 17.0, 30.0, 88.0, 1e30, -1e30, -200.0], np.float32)
    x = np.concatenate([np.zeros(d, np.float32), logits])[None, None, :]
    _, g = O.split_gated_query(x, heads, d)
    g = g.reshape(-1)
    assert g[0] == 0.5 and g[1] == 0.5            # exp(0) = 1
    assert np.all(g[2:6] == 1.0)                  # 1 + exp(-x) rounds to 1 for x >= 17
    assert g[6] == 0.0 and g[7] == 0.0            # exp(+big) overflows to inf: 1 / inf


def test_logistic_against_float64_and_symmetry():
    rng = np.random.default_rng(3)
    d = 64
    z = np.concatenate([rng.standard_normal(d * 20) * 6, np.linspace(-12, 12, d * 4)]).astype(np.float32)
    n = len(z) // d
    x = np.zeros((n, 1, 2 * d), np.float32)
    x[:, 0, d:] = z.reshape(n, d)
    _, g = O.split_gated_query(x, 1, d)
    g = g.reshape(-1)
    ref = (1.0 / (1.0 + np.exp(-z.astype(np.float64)))).astype(np.float32)
    assert np.all(_ulps(g, ref) <= 2)
    # sigma(-z) = 1 - sigma(z): a sign slip (exp(+z)) fails this and the
    # float64 comparison at once
    xm = x.copy()
    xm[:, 0, d:] = -z.reshape(n, d)
    _, gm = O.split_gated_query(xm, 1, d)
    assert np.all(np.abs(gm.reshape(-1).astype(np.float64) + g - 1.0) <= 2.5e-7)
    # monotone on the sorted grid
    lin = g[d * 20:]
    assert np.all(np.diff(lin) >= 0) and lin[0] < 1e-5 and lin[-1] > 1 - 1e-5
