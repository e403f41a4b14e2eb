"""The five benchmark configurations at full size, one step each, vs the oracle.

Per config: the step (page copies, chunk appends, fused append + decode) runs
on the GPU; the oracle replays it on a host copy of every page the step can
touch.  Pages must match bit for bit; attention outputs must be within the
row-normwise tolerance (1e-3 f16, 1e-5 f32 and Q8A) of the f64 oracle over the exact
stored values, and within the same tolerance of the reference-order f32 scan
(the reference CPU path); the element-wise relative error (floor 1e-6) is
reported.  Every page outside the step's footprint is compared with its
contents before the step.  c2-rope / c2-q8a-rope run the same c2 step
through the fused RoPE entry point (Llama-3.1 inverse frequencies, rotary =
head_dim): the oracle rotates q and the new K at position kv_len - 1 before
its append and scan, and the rotated pages must still match bit for bit."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import TOL, host_pages, rel_err, remap_tables, say
from lnskv import DTYPE_Q8A, NO_PAGE
from lnskv.configs import make, used_pages
from lnskv.device import RopeTable, sync
from lnskv.step import StepRunner

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5", "c2-q8a", "c2-rope", "c2-q8a-rope"])
def test_config_step(gpu, name):
    """c2-q8a: the c2 draw with the reference's own page type (int8 codes
    and scales; the matrix-core Q8A decode with its in-kernel quantizer)."""
    say("config", name, "build")
    w = make("c2", dtype=DTYPE_Q8A) if name.startswith("c2-q8a") else make(name.split("-")[0])
    rope = None
    if name.endswith("-rope"):
        rope = RopeTable(w.head_dim, 500000.0, O.ROPE_LLAMA3, (8.0, 8192.0, 1.0, 4.0), device=gpu)
    r = StepRunner(w, gpu, n_layers=1, seed=17, rope=rope)
    pk = r.layers[0]
    pages = used_pages(w.tables)
    if w.copies:
        pages = np.union1d(pages, np.array(w.copies, np.uint32).ravel())
    hp, remap = host_pages(pk, pages)
    tables = remap_tables(w.tables, remap)

    # oracle replay of the step on the host copy
    if w.copies:
        src = remap[np.array([c[0] for c in w.copies], np.uint32)]
        dst = remap[np.array([c[1] for c in w.copies], np.uint32)]
        O.page_copy(hp, src, dst)
    cs, cp = w.chunk_tokens()
    turn = (lambda x, pos: O.rope_apply(x, rope.rotary_dim, rope.inv_freqs_host, pos)) if rope else \
        (lambda x, pos: x)
    if len(cs):
        assert O.append(hp, turn(r.chunk_k.cpu().numpy(), cp), r.chunk_v.cpu().numpy(), cs, cp, tables) == 0
    rows = r.dec_rows
    dec_tables = tables[rows]
    kv_len = w.kv_len[rows]
    assert O.append(hp, turn(r.k_new.cpu().numpy(), kv_len - 1), r.v_new.cpu().numpy(),
                    np.arange(len(rows), dtype=np.int32), kv_len - 1, dec_tables) == 0

    # the whole pools before the step: pages outside its footprint must come
    # out untouched
    before = {t: getattr(pk, t).clone() for t in ("k", "v", "ks", "vs") if getattr(pk, t) is not None}
    say("config", name, "step on gpu")
    out = r.run(0)
    sync()
    outside = np.setdiff1d(np.arange(w.num_pages, dtype=np.int64), pages.astype(np.int64))
    if len(outside):
        idx = torch.from_numpy(outside).to(gpu)
        sidx = (idx[:, None] * 16 + torch.arange(16, device=gpu)[None, :]).reshape(-1)
        for t, b in before.items():
            i = sidx if t in ("ks", "vs") else idx
            assert torch.equal(getattr(pk, t).index_select(0, i), b.index_select(0, i)), f"{t} outside the footprint"
    del before
    got, _ = host_pages(pk, pages)
    assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8)), "K pages differ"
    assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8)), "V pages differ"
    if w.dtype == DTYPE_Q8A:
        assert np.array_equal(got.ks, hp.ks) and np.array_equal(got.vs, hp.vs), "scales differ"

    q = turn(r.q.cpu().numpy(), kv_len - 1)
    o = out.cpu().numpy()
    assert np.isfinite(o).all()
    ref = O.decode_f64(hp, q, dec_tables, kv_len, None, w.scale)
    err = rel_err(o, ref)
    ele = O.rel_err_elements(o, ref)
    say("config", name, "max rel err vs f64: row-normwise", float(err.max()), "element-wise (floor 1e-6)",
        float(ele.max()), "median element", float(np.median(ele)))
    assert err.max() < TOL[w.dtype]
    assert np.isfinite(ele).all()
    if name in ("c1", "c2", "c2-q8a", "c2-q8a-rope"):
        scan = O.decode_refscan(hp, q, dec_tables, kv_len, None, w.scale)
        assert rel_err(o, scan.astype(np.float64)).max() < TOL[w.dtype]
    # pages outside the step's footprint are untouched: a second step is
    # idempotent (same token rewritten to the same slot, same output)
    out2 = r.run(0).cpu().numpy()
    assert np.array_equal(out2, o)



def test_c5_churn_steps(gpu):
    """c5's churn continued step by step (a smaller batch): every step frees
    the previous children and a quarter of the batch, refills those rows with
    new sequences on the freed pages, forks children (tail pages copied) and
    uploads the changed tables inside the step.  After each step the pages
    the step touched are bit-exact with the oracle's replay and every output
    row is within tolerance of the f64 oracle."""
    from lnskv.configs import churn_plan, make_c5
    from lnskv.step import ChurnRunner

    w = make_c5(n_seq=24, lo=40, hi=700, n_free=6, n_fork=3, spare=256)
    r = StepRunner(w, gpu, n_layers=1, seed=5)
    plan = churn_plan(w, 3, seed=2, n_free=6, lo=40, hi=700)
    cr = ChurnRunner(r, plan, max_kv_len=700 + 8)
    pk = r.layers[0]
    for i, st in enumerate(plan):
        say("c5 churn step", i, "copies", len(st["copies"]), "freed", st["freed"])
        hp, _ = host_pages(pk)
        tables = st["tables"]
        if st["copies"]:
            cps = np.array(st["copies"], np.uint32)
            O.page_copy(hp, cps[:, 0], cps[:, 1])
        kv_len = st["kv_len"]
        assert O.append(hp, r.k_new.cpu().numpy(), r.v_new.cpu().numpy(), np.arange(len(kv_len), dtype=np.int32),
                        kv_len - 1, tables) == 0
        out = cr.run(i).cpu().numpy()
        sync()
        got, _ = host_pages(pk)
        assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8)), i
        assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8)), i
        ref = O.decode_f64(hp, r.q.cpu().numpy(), tables, kv_len, None, w.scale)
        assert rel_err(out, ref).max() < TOL[w.dtype], i
