"""The committed c1 fixture (tests/golden/c1_golden.npz, oracle-generated)
against the oracle and its input generator, on the CPU: a change to the
generator, to configs.make_c1's table or to the oracle's append and scans
fails here.  Closed forms on the fixture itself: the appended slot holds the
new token's values exactly (an f32 copy) and the rest of that page is zero;
the f32 reference-order scan agrees with the f64 scan to 1e-5."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as G  # noqa: E402

FIX = os.path.join(HERE, "golden", "c1_golden.npz")


def load():
    return np.load(FIX, allow_pickle=False)


def test_inputs_and_table_are_reproduced():
    f = load()
    assert G.digest(G.gen_inputs(0)) == str(f["inputs_sha256"])
    assert np.array_equal(G.c1_table(), f["table"])


def test_generator_draws_standard_normals():
    x = G.normals(0, 9, 200000).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01


def test_oracle_reproduces_the_fixture():
    f = load()
    e = G.expected(G.gen_inputs(0), f["table"])
    assert np.array_equal(e["k_page"].view(np.uint32), f["k_page"].view(np.uint32))
    assert np.array_equal(e["v_page"].view(np.uint32), f["v_page"].view(np.uint32))
    assert np.array_equal(e["out_refscan"].view(np.uint32), f["out_refscan"].view(np.uint32))
    assert np.array_equal(e["out_f64"], f["out_f64"])


def test_fixture_closed_forms():
    f = load()
    x = G.gen_inputs(0)
    assert np.array_equal(f["k_page"][0], x["k_new"]) and np.array_equal(f["v_page"][0], x["v_new"])
    assert not f["k_page"][1:].any() and not f["v_page"][1:].any()
    ref = f["out_f64"]
    err = np.abs(f["out_refscan"] - ref).max(axis=1) / np.abs(ref).max(axis=1)
    assert err.max() < 1e-5
