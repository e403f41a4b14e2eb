"""GPU paged decode attention vs the oracle.

Outputs are compared with the f64 oracle over the exact stored page values,
row-normwise: max_i |o_i - r_i| / max_i |r_i| per (sequence, query head), with
the tolerance 1e-3 for f16 pages and 1e-5 for f32 and Q8A pages (TOL).  Pages
written by the fused append are compared bit for bit."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import TOL, dev_f32, dev_i32, fill_pages, host_pages, rel_err, say
from lnskv import DTYPE_F16, DTYPE_F32, DTYPE_Q8A, DTYPE_NAMES, NO_PAGE
from lnskv._lib import ERR_WORKSPACE, WORKSPACE_HEADER_BYTES as HEADER_BYTES, LnskvError
from lnskv.device import PagedKV, sync

pytestmark = pytest.mark.gpu


def _case(gpu, dtype, d, rep, n_kv, lens, seed, num_pages=None, scale_vals=1.0):
    rng = np.random.default_rng(seed)
    pages_per = [(L + 15) // 16 for L in lens]
    num_pages = num_pages or sum(pages_per) + 8
    pk = PagedKV(num_pages, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=seed, scale=scale_vals)
    perm = rng.permutation(num_pages).astype(np.uint32)
    stride = max(pages_per) + 1
    tables = np.full((len(lens), stride), NO_PAGE, np.uint32)
    k = 0
    for s, n in enumerate(pages_per):
        tables[s, :n] = perm[k:k + n]
        k += n
    q = rng.standard_normal((len(lens), n_kv * rep, d)).astype(np.float32)
    return pk, tables, np.array(lens, np.int32), q


LENS = (1, 15, 16, 17, 100, 513, 1000)


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_Q8A])
@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("rep", [1, 2, 4, 8])
def test_decode_matrix(gpu, dtype, d, rep):
    say("decode", DTYPE_NAMES[dtype], "d", d, "rep", rep)
    n_kv = 2
    pk, tables, kv_len, q = _case(gpu, dtype, d, rep, n_kv, LENS, seed=d * 10 + rep)
    hp, _ = host_pages(pk)
    scale = 1.0 / np.sqrt(d)
    ref = O.decode_f64(hp, q, tables, kv_len, None, scale)
    for split in (0, 64):
        out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                        max_kv_len=int(kv_len.max()), scale=float(scale), split=split)
        sync()
        err = rel_err(out, ref)
        assert err.max() < TOL[dtype], (split, err.max())


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_Q8A])
def test_windows_empty_and_missing_pages(gpu, dtype):
    say("windows", DTYPE_NAMES[dtype])
    d, rep, n_kv = 128, 4, 2
    lens = (0, 1, 40, 300, 300, 700, 64)
    pk, tables, kv_len, q = _case(gpu, dtype, d, rep, n_kv, lens, seed=3)
    p_start = np.array([0, 1, 5, 33, 300, 650, 17], np.int32)  # empty, empty, ..., empty(300=L)
    tables[5, 3] = NO_PAGE            # a missing page inside a window: skipped
    tables[6, 2] = 1 << 30            # an entry past the pool: skipped
    hp, _ = host_pages(pk)
    scale = 0.09
    ref = O.decode_f64(hp, q, tables, kv_len, p_start, scale)
    for split in (0, 16, 48):
        out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=8,
                        max_kv_len=700, scale=scale, p_start=dev_i32(p_start, gpu), split=split)
        sync()
        o = out.cpu().numpy()
        assert not np.isnan(o).any()
        assert (o[0] == 0).all() and (o[1] == 0).all() and (o[4] == 0).all()
        assert rel_err(o[2:4], ref[2:4]).max() < TOL[dtype]
        assert rel_err(o[5:], ref[5:]).max() < TOL[dtype]


def test_single_token_returns_stored_v_exactly(gpu):
    for dtype in (DTYPE_F32, DTYPE_F16):
        say("single token", DTYPE_NAMES[dtype])
        pk, tables, kv_len, q = _case(gpu, dtype, 128, 4, 2, (1, 1, 1), seed=4)
        out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=8,
                        max_kv_len=1, scale=0.1)
        sync()
        hp, _ = host_pages(pk)
        V = O.stored_values(hp, True).astype(np.float32)
        o = out.cpu().numpy()
        for s in range(3):
            for h in range(8):
                assert np.array_equal(o[s, h], V[tables[s, 0] * 16, h // 4])


def test_split_invariance_and_page_permutation(gpu):
    say("split invariance / permutation")
    d, rep, n_kv = 128, 4, 8
    lens = (3000, 1, 777, 4096, 16)
    pk, tables, kv_len, q = _case(gpu, DTYPE_F16, d, rep, n_kv, lens, seed=5, scale_vals=0.5)
    hp, _ = host_pages(pk)
    ref = O.decode_f64(hp, q, tables, kv_len, None, 0.0883883)
    outs = {}
    for split in (16, 32, 256, 512, 1024, 4096):
        outs[split] = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=32,
                                max_kv_len=4096, scale=0.0883883, split=split).cpu().numpy()
        assert rel_err(outs[split], ref).max() < TOL[DTYPE_F16]
    # physically permuting pages together with the table: bit-identical output
    perm = torch.randperm(pk.num_pages, generator=torch.Generator().manual_seed(9)).to(gpu)
    inv = torch.argsort(perm).cpu().numpy().astype(np.uint32)
    pk2 = PagedKV(pk.num_pages, n_kv, d, DTYPE_F16, gpu)
    pk2.k.copy_(pk.k[perm])
    pk2.v.copy_(pk.v[perm])
    t2 = tables.copy()
    m = t2 != NO_PAGE
    t2[m] = inv[t2[m]]
    o2 = pk2.decode(dev_f32(q, gpu), dev_i32(t2, gpu), dev_i32(kv_len, gpu), n_heads=32, max_kv_len=4096,
                    scale=0.0883883, split=256).cpu().numpy()
    assert np.array_equal(o2, outs[256])


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_Q8A])
@pytest.mark.parametrize("d,rep", [(64, 8), (128, 4), (256, 2)])
def test_fused_append_decode(gpu, dtype, d, rep):
    """append_decode == append then decode: pages bit-exact, output in tolerance."""
    say("append_decode", DTYPE_NAMES[dtype], "d", d, "rep", rep)
    n_kv = 4
    ctx = (0, 15, 16, 31, 200, 511, 1200)
    lens = tuple(c + 1 for c in ctx)
    pk, tables, kv_len, q = _case(gpu, dtype, d, rep, n_kv, lens, seed=d + rep + dtype)
    rng = np.random.default_rng(11)
    k_new = (rng.standard_normal((len(lens), n_kv, d)) * 2).astype(np.float32)
    v_new = (rng.standard_normal((len(lens), n_kv, d)) * 2).astype(np.float32)
    p_start = np.array([0, 3, 0, 31, 100, 0, 1100], np.int32)
    hp, _ = host_pages(pk)
    O.append(hp, k_new, v_new, np.arange(len(lens), dtype=np.int32), kv_len - 1, tables)
    scale = 1.0 / np.sqrt(d)
    ref = O.decode_f64(hp, q, tables, kv_len, p_start, scale)
    for split in (0, 32):
        out = pk.append_decode(dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tables, gpu),
                               dev_i32(kv_len, gpu), n_heads=n_kv * rep, max_kv_len=int(kv_len.max()),
                               scale=float(scale), p_start=dev_i32(p_start, gpu), split=split)
        sync()
        got, _ = host_pages(pk)
        assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8))
        assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8))
        if dtype == DTYPE_Q8A:
            assert np.array_equal(got.ks, hp.ks) and np.array_equal(got.vs, hp.vs)
        assert rel_err(out, ref).max() < TOL[dtype], split


@pytest.mark.parametrize("force_valu", ["0", "1"])
def test_f16_d128_both_kernels(gpu, monkeypatch, force_valu):
    """f16 / head_dim 128 runs the MFMA kernel; LNSKV_FORCE_VALU=1 the generic
    one.  Both against the f64 oracle, fused and unfused, rep 1/2/4/8."""
    monkeypatch.setenv("LNSKV_FORCE_VALU", force_valu)
    for rep in (1, 2, 4, 8):
        say("f16 d128 force_valu", force_valu, "rep", rep)
        n_kv = 2
        lens = (1, 2, 16, 17, 33, 255, 256, 257, 700, 2049)
        pk, tables, kv_len, q = _case(gpu, DTYPE_F16, 128, rep, n_kv, lens, seed=40 + rep)
        rng = np.random.default_rng(rep)
        k_new = rng.standard_normal((len(lens), n_kv, 128)).astype(np.float32)
        v_new = rng.standard_normal((len(lens), n_kv, 128)).astype(np.float32)
        hp, _ = host_pages(pk)
        ref0 = O.decode_f64(hp, q, tables, kv_len, None, 0.0883883)
        out0 = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                         max_kv_len=2049, scale=0.0883883, split=64)
        sync()
        assert rel_err(out0, ref0).max() < TOL[DTYPE_F16]
        O.append(hp, k_new, v_new, np.arange(len(lens), dtype=np.int32), kv_len - 1, tables)
        ref1 = O.decode_f64(hp, q, tables, kv_len, None, 0.0883883)
        for split in (0, 256):
            out1 = pk.append_decode(dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu),
                                    dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                                    max_kv_len=2049, scale=0.0883883, split=split)
            sync()
            got, _ = host_pages(pk)
            assert np.array_equal(got.k, hp.k) and np.array_equal(got.v, hp.v)
            assert rel_err(out1, ref1).max() < TOL[DTYPE_F16], (rep, split)


def test_large_query_values_keep_precision(gpu):
    """q entries far outside f16 range: the MFMA path rescales each head by a
    power of two before splitting it into f16 hi/lo parts."""
    say("large q")
    pk, tables, kv_len, q = _case(gpu, DTYPE_F16, 128, 4, 2, (40, 300), seed=77)
    q = (q * 1e6).astype(np.float32)
    q[1] *= 1e-12
    hp, _ = host_pages(pk)
    scale = 1e-6
    ref = O.decode_f64(hp, q, tables, kv_len, None, scale)
    out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=8, max_kv_len=300,
                    scale=scale)
    sync()
    assert rel_err(out, ref).max() < TOL[DTYPE_F16]


def test_reference_single_sequence_call_c1_shape(gpu):
    """lnskv_attention_paged: the reference's encode_attention_paged_q8a call
    (append token `pos`, attend [p_start, pos], scale rsqrt(d)), here on the
    C1 shape (Hq32/Hkv4/d64, f32, 512 context tokens) and on Q8A with a window."""
    for dtype, p_start in ((DTYPE_F32, 0), (DTYPE_Q8A, 300), (DTYPE_F16, 7)):
        say("attention_paged", DTYPE_NAMES[dtype], "p_start", p_start)
        rng = np.random.default_rng(0)
        pk = PagedKV(64, 4, 64, dtype, gpu)
        fill_pages(pk, seed=0)
        perm = rng.permutation(64).astype(np.uint32)
        bt = np.full(512, NO_PAGE, np.uint32)   # the reference's MAX_LOGICAL_PAGES table
        bt[:33] = perm[:33]
        q = rng.standard_normal((32, 64)).astype(np.float32)
        k_in = rng.standard_normal(4 * 64).astype(np.float32)
        v_in = rng.standard_normal(4 * 64).astype(np.float32)
        hp, _ = host_pages(pk)
        O.append(hp, k_in[None], v_in[None], np.zeros(1, np.int32), np.array([512], np.int32), bt[None])
        ref = O.decode_f64(hp, q[None], bt[None], np.array([513], np.int32), np.array([p_start], np.int32),
                           1.0 / np.sqrt(64.0))[0]
        out = pk.attention_paged(dev_f32(q, gpu), dev_f32(k_in, gpu), dev_f32(v_in, gpu), dev_i32(bt, gpu),
                                 pos=512, n_heads=32, p_start=p_start, dispatch=True)
        got, _ = host_pages(pk)
        assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8))
        assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8))
        assert rel_err(out, ref).max() < TOL[dtype]


def test_reference_single_sequence_call_q8a_d128(gpu):
    """lnskv_attention_paged with the reference's own page type at head_dim
    128 (the matrix-core Q8A path: the new token quantized and stored by the
    decode kernel itself): Hq32/Hkv8, 700 context tokens, windows 0 and 650;
    codes and scales bit-exact, output within 1e-5."""
    for p_start in (0, 650):
        say("attention_paged q8a d128 p_start", p_start)
        rng = np.random.default_rng(p_start + 1)
        pk = PagedKV(64, 8, 128, DTYPE_Q8A, gpu)
        fill_pages(pk, seed=2)
        perm = rng.permutation(64).astype(np.uint32)
        bt = np.full(512, NO_PAGE, np.uint32)
        bt[:44] = perm[:44]
        q = rng.standard_normal((32, 128)).astype(np.float32)
        k_in = (rng.standard_normal(8 * 128) * 2).astype(np.float32)
        v_in = (rng.standard_normal(8 * 128) * 2).astype(np.float32)
        hp, _ = host_pages(pk)
        O.append(hp, k_in[None], v_in[None], np.zeros(1, np.int32), np.array([700], np.int32), bt[None])
        ref = O.decode_f64(hp, q[None], bt[None], np.array([701], np.int32), np.array([p_start], np.int32),
                           1.0 / np.sqrt(128.0))[0]
        out = pk.attention_paged(dev_f32(q, gpu), dev_f32(k_in, gpu), dev_f32(v_in, gpu), dev_i32(bt, gpu),
                                 pos=700, n_heads=32, p_start=p_start, dispatch=True)
        got, _ = host_pages(pk)
        assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8))
        assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8))
        assert np.array_equal(got.ks, hp.ks) and np.array_equal(got.vs, hp.vs)
        assert rel_err(out, ref).max() < TOL[DTYPE_Q8A]


@pytest.mark.parametrize("shape", [(32, 8, 128), (16, 4, 256)])
@pytest.mark.parametrize("dtype", [DTYPE_Q8A, DTYPE_F16])
def test_reference_call_page_counts(gpu, dtype, shape):
    """lnskv_attention_paged at contexts around 4096 tokens (the workgroup
    schedule): page counts per kv head that are and are not a multiple of
    the workgroups' share (253 to 258 pages, and a short context), so that
    segments start inside a workgroup's nominal range and some take fewer
    workgroups than ceil(pages / share); windows 0 and 1000; Llama-3-8B's
    and Qwen3.5's head shapes.  Pages bit-exact, output against the f64
    oracle."""
    hq, n_kv, d = shape
    pk = PagedKV(272, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=4)
    rng = np.random.default_rng(11)
    bt = np.full(512, NO_PAGE, np.uint32)
    bt[:272] = rng.permutation(272).astype(np.uint32)
    for pos, p_start in ((4031, 0), (4063, 0), (4064, 0), (4095, 0), (4096, 0), (4111, 1000), (4127, 0),
                         (130, 0)):
        say("attention_paged page counts", DTYPE_NAMES[dtype], "pos", pos, "p_start", p_start)
        q = rng.standard_normal((hq, d)).astype(np.float32)
        k_in = rng.standard_normal(n_kv * d).astype(np.float32)
        v_in = rng.standard_normal(n_kv * d).astype(np.float32)
        hp, _ = host_pages(pk)
        O.append(hp, k_in[None], v_in[None], np.zeros(1, np.int32), np.array([pos], np.int32), bt[None])
        ref = O.decode_f64(hp, q[None], bt[None], np.array([pos + 1], np.int32), np.array([p_start], np.int32),
                           1.0 / np.sqrt(d))[0]
        out = pk.attention_paged(dev_f32(q, gpu), dev_f32(k_in, gpu), dev_f32(v_in, gpu), dev_i32(bt, gpu),
                                 pos=pos, n_heads=hq, p_start=p_start, dispatch=True)
        got, _ = host_pages(pk)
        assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8))
        assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8))
        if dtype == DTYPE_Q8A:
            assert np.array_equal(got.ks, hp.ks) and np.array_equal(got.vs, hp.vs)
        assert rel_err(out, ref).max() < TOL[dtype], (pos, p_start)


@pytest.mark.parametrize("dtype", [DTYPE_Q8A, DTYPE_F16])
def test_workgroup_schedule_small_batches(gpu, monkeypatch, dtype):
    """The workgroup schedule on batches of 2 to 9 sequences whose segments
    get workgroups of their own (ragged lengths, an empty sequence, one of a
    single token, windows), unfused and fused, against the f64 oracle."""
    monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", "workgroup")
    monkeypatch.delenv("LNSKV_FORCE_VALU", raising=False)
    n_kv, d, rep = 8, 128, 4
    for lens in ((4097, 17), (0, 1, 2049, 333, 4000), (1500,) * 3 + (1501, 1499, 16, 32, 48, 4111)):
        say("workgroup schedule small batch", DTYPE_NAMES[dtype], lens)
        pk, tables, kv_len, q = _case(gpu, dtype, d, rep, n_kv, lens, seed=len(lens))
        p_start = np.zeros(len(lens), np.int32)
        p_start[-1] = min(int(kv_len[-1]), 700)
        hp, _ = host_pages(pk)
        scale = 1.0 / np.sqrt(d)
        ref = O.decode_f64(hp, q, tables, kv_len, p_start, scale)
        out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                        max_kv_len=int(kv_len.max()), scale=float(scale), p_start=dev_i32(p_start, gpu), split=0)
        sync()
        assert rel_err(out, ref).max() < TOL[dtype]
        kv1 = np.minimum(kv_len + 1, tables.shape[1] * 16).astype(np.int32)
        rng = np.random.default_rng(len(lens))
        k_new = rng.standard_normal((len(lens), n_kv, d)).astype(np.float32)
        v_new = rng.standard_normal((len(lens), n_kv, d)).astype(np.float32)
        O.append(hp, k_new, v_new, np.arange(len(lens), dtype=np.int32), kv1 - 1, tables)
        ref1 = O.decode_f64(hp, q, tables, kv1, p_start, scale)
        out1 = pk.append_decode(dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tables, gpu),
                                dev_i32(kv1, gpu), n_heads=n_kv * rep, max_kv_len=int(kv1.max()),
                                scale=float(scale), p_start=dev_i32(p_start, gpu), split=0)
        sync()
        got, _ = host_pages(pk)
        assert np.array_equal(got.k, hp.k) and np.array_equal(got.v, hp.v)
        assert rel_err(out1, ref1).max() < TOL[dtype]


def _sk_lens(n, seed):
    """Lengths for a stream-K batch: empty, sub-page, page-edge and long
    sequences, so that waves hold several pieces and segments span waves."""
    rng = np.random.default_rng(seed)
    base = [0, 1, 15, 16, 17, 31, 33, 3000, 4096, 2047]
    lens = base + list(rng.integers(1, 2500, n - len(base)))
    return tuple(int(x) for x in lens[:n])


SCHEDULES = ["stream-k", "workgroup"]


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_Q8A])
@pytest.mark.parametrize("rep", [1, 2, 4, 8])
@pytest.mark.parametrize("d", [128, 256])
def test_stream_k_schedule(gpu, monkeypatch, rep, dtype, schedule, d):
    """split_tokens = 0 on the MFMA path runs one of two schedules, forced
    here through LNSKV_DECODE_SCHEDULE: stream-K (every wave an equal share
    of all pages; pieces merged by combine_sk_kernel) or the workgroup
    schedule (every workgroup an equal share; pieces merged in LDS and, across
    workgroups, by the last workgroup to finish).  64 sequences (one group)
    with empty, short and long lengths, windows, a missing page; unfused and
    fused, against the f64 oracle and against the split-K schedule; f16 and
    Q8A pages (pages and scales bit-exact); heads of 128 and of 256 dims (two
    halves sharing one softmax)."""
    monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", schedule)
    say(schedule, "rep", rep, DTYPE_NAMES[dtype], "d", d)
    n_kv = 8 if d == 128 else 4
    lens = _sk_lens(64, seed=rep)
    pk, tables, kv_len, q = _case(gpu, dtype, d, rep, n_kv, lens, seed=90 + rep)
    tables[5, 0] = NO_PAGE  # a missing page: its tokens are skipped
    rng = np.random.default_rng(rep + 7)
    p_start = np.zeros(len(lens), np.int32)
    p_start[7:12] = [10, 2900, 0, 17, 1000]
    hp, _ = host_pages(pk)
    scale = 1.0 / np.sqrt(d)
    ref = O.decode_f64(hp, q, tables, kv_len, p_start, scale)
    for split in (0, 128):
        out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                        max_kv_len=int(kv_len.max()), scale=float(scale), p_start=dev_i32(p_start, gpu),
                        split=split)
        sync()
        err = rel_err(out, ref)
        assert err.max() < TOL[dtype], (split, err.max())
        assert np.all(out.cpu().numpy()[0] == 0.0)  # empty sequence
    # fused: every sequence gains one token
    kv1 = np.minimum(kv_len + 1, (tables.shape[1]) * 16).astype(np.int32)
    k_new = rng.standard_normal((len(lens), n_kv, d)).astype(np.float32)
    v_new = rng.standard_normal((len(lens), n_kv, d)).astype(np.float32)
    O.append(hp, k_new, v_new, np.arange(len(lens), dtype=np.int32), kv1 - 1, tables)
    ref1 = O.decode_f64(hp, q, tables, kv1, p_start, scale)
    out1 = pk.append_decode(dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tables, gpu),
                            dev_i32(kv1, gpu), n_heads=n_kv * rep, max_kv_len=int(kv1.max()), scale=float(scale),
                            p_start=dev_i32(p_start, gpu), split=0)
    sync()
    got, _ = host_pages(pk)
    assert np.array_equal(got.k, hp.k) and np.array_equal(got.v, hp.v)
    if dtype == DTYPE_Q8A:
        assert np.array_equal(got.ks.view(np.uint32), hp.ks.view(np.uint32))
        assert np.array_equal(got.vs.view(np.uint32), hp.vs.view(np.uint32))
    assert rel_err(out1, ref1).max() < TOL[dtype]


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_stream_k_caller_workspace_and_fallback(gpu, monkeypatch, schedule):
    """A caller-provided workspace of exactly the queried size serves each
    schedule (its size does not depend on the batch up to 4096 sequences;
    4097 fall back to split-K); 65 sequences take two groups of 64; one short
    sequence leaves most waves idle.  The workspace is zeroed once and
    reused: every call leaves its counter header zero."""
    monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", schedule)
    monkeypatch.delenv("LNSKV_FORCE_VALU", raising=False)  # the matrix-core schedules themselves
    say(schedule, "workspace / fallback")
    n_kv, d, rep = 8, 128, 4
    pk0 = PagedKV(16, n_kv, d, DTYPE_F16, gpu)
    sizes = [pk0.workspace_size(n, n_kv * rep, 4096, 0) for n in (1, 64, 4096, 4097)]
    assert sizes[0] == sizes[1] == sizes[2] != sizes[3], sizes
    for lens in (_sk_lens(64, 3), _sk_lens(65, 4), (5,), (1,) * 64, (3,) * 4097):
        pk, tables, kv_len, q = _case(gpu, DTYPE_F16, d, rep, n_kv, lens, seed=len(lens))
        hp, _ = host_pages(pk)
        ref = O.decode_f64(hp, q, tables, kv_len, None, 0.0883883)
        mkv = int(kv_len.max())
        nbytes = pk.workspace_size(len(lens), n_kv * rep, mkv, 0)
        # the workgroup schedule (up to 4096 sequences) has its counter header
        assert nbytes > HEADER_BYTES or len(lens) > 4096
        ws = torch.zeros(max(nbytes, HEADER_BYTES), dtype=torch.uint8, device=gpu)
        for _ in range(2):
            out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                            max_kv_len=mkv, scale=0.0883883, split=0, workspace=ws)
            sync()
            assert rel_err(out, ref).max() < TOL[DTYPE_F16], len(lens)
            assert int(ws[:HEADER_BYTES].count_nonzero()) == 0, len(lens)
    # a workspace that is large enough but not 16-byte aligned is refused
    pk, tables, kv_len, q = _case(gpu, DTYPE_F16, d, rep, n_kv, _sk_lens(64, 3), seed=64)
    mkv = int(kv_len.max())
    nbytes = pk.workspace_size(64, n_kv * rep, mkv, 0)
    ws = torch.zeros(nbytes + 64, dtype=torch.uint8, device=gpu)[4:]
    with pytest.raises(LnskvError) as e:
        pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                  max_kv_len=mkv, scale=0.0883883, split=0, workspace=ws)
    assert e.value.status == ERR_WORKSPACE


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_Q8A])
@pytest.mark.parametrize("n_seq", [130, 4096, 9000])
def test_stream_k_many_sequences(gpu, monkeypatch, n_seq, dtype, schedule):
    """More than 64 sequences on both schedules (groups of 64, one lane per
    sequence): a whole group of empty sequences, ragged lengths and windows,
    unfused and fused, against the f64 oracle; f16 and Q8A pages (the Q8A
    fused call quantizes each new token in the wave that holds it; pages and
    scales bit-exact).  9000 sequences: Q8A pages run stream-K in three
    launches of at most 4096 sequences, f16 pages split-K."""
    monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", schedule)
    say(schedule, "n_seq", n_seq, DTYPE_NAMES[dtype])
    n_kv, d, rep = 8, 128, 4
    rng = np.random.default_rng(n_seq)
    hi = 700 if n_seq < 1000 else 48
    lens = [int(x) for x in rng.integers(0, hi, n_seq)]
    lens[64:128] = [0] * 64  # group 1 holds no units
    lens[0], lens[-1] = hi, 1
    pk, tables, kv_len, q = _case(gpu, dtype, d, rep, n_kv, tuple(lens), seed=n_seq)
    p_start = np.minimum(rng.integers(0, 40, n_seq), kv_len).astype(np.int32)
    hp, _ = host_pages(pk)
    scale = 1.0 / np.sqrt(d)
    ref = O.decode_f64(hp, q, tables, kv_len, p_start, scale)
    out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                    max_kv_len=int(kv_len.max()), scale=float(scale), p_start=dev_i32(p_start, gpu), split=0)
    sync()
    assert rel_err(out, ref).max() < TOL[dtype]
    assert np.all(out.cpu().numpy()[64:128] == 0.0)
    kv1 = np.minimum(kv_len + 1, tables.shape[1] * 16).astype(np.int32)
    k_new = rng.standard_normal((n_seq, n_kv, d)).astype(np.float32)
    v_new = rng.standard_normal((n_seq, n_kv, d)).astype(np.float32)
    O.append(hp, k_new, v_new, np.arange(n_seq, dtype=np.int32), kv1 - 1, tables)
    ref1 = O.decode_f64(hp, q, tables, kv1, p_start, scale)
    out1 = pk.append_decode(dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tables, gpu),
                            dev_i32(kv1, gpu), n_heads=n_kv * rep, max_kv_len=int(kv1.max()), scale=float(scale),
                            p_start=dev_i32(p_start, gpu), split=0)
    sync()
    got, _ = host_pages(pk)
    assert np.array_equal(got.k, hp.k) and np.array_equal(got.v, hp.v)
    if dtype == DTYPE_Q8A:
        assert np.array_equal(got.ks.view(np.uint32), hp.ks.view(np.uint32))
        assert np.array_equal(got.vs.view(np.uint32), hp.vs.view(np.uint32))
    assert rel_err(out1, ref1).max() < TOL[dtype]


def test_schedule_chosen_by_batch_size(gpu, monkeypatch):
    """Without LNSKV_DECODE_SCHEDULE the library runs the workgroup schedule
    for a batch of at most 16 pages per compute unit (the reference's
    one-sequence call: 4096 tokens, 8 kv heads) and stream-K for a larger one
    (64 such sequences): the workspace sizes match the forced settings'."""
    monkeypatch.delenv("LNSKV_FORCE_VALU", raising=False)  # the matrix-core schedules themselves
    n_kv, d, rep = 8, 128, 4
    pk = PagedKV(16, n_kv, d, DTYPE_Q8A, gpu)

    def size(n, setting):
        if setting is None:
            monkeypatch.delenv("LNSKV_DECODE_SCHEDULE", raising=False)
        else:
            monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", setting)
        return pk.workspace_size(n, n_kv * rep, 4096, 0)

    wg, sk = size(1, "workgroup"), size(1, "stream-k")
    assert wg != sk
    assert size(1, None) == wg
    assert size(64, None) == sk
    assert size(64, "bogus") == sk


@pytest.mark.parametrize("force_valu", ["0", "1"])
def test_q8a_d128_both_kernels(gpu, monkeypatch, force_valu):
    """Q8A pages with head_dim 128 run the MFMA stream-K kernel (q.k as int8
    products of the K codes and three int8 limbs of q, V codes turned into
    f16 exactly, K and V scales applied per token; in the fused call the wave
    that holds the new token quantizes and stores it); LNSKV_FORCE_VALU=1 the
    generic kernel.  Both against the f64 oracle (1e-5), rep 1/2/4/8, with
    windows, an empty window and a missing page; pages and scales bit-exact."""
    monkeypatch.setenv("LNSKV_FORCE_VALU", force_valu)
    for rep in (1, 2, 4, 8):
        say("q8a d128 force_valu", force_valu, "rep", rep)
        n_kv = 2
        lens = (1, 2, 16, 17, 33, 255, 256, 257, 700, 2049)
        pk, tables, kv_len, q = _case(gpu, DTYPE_Q8A, 128, rep, n_kv, lens, seed=60 + rep)
        p_start = np.array([0, 0, 3, 16, 0, 100, 0, 257, 650, 1000], np.int32)  # row 7: empty window
        tables[9, 70] = NO_PAGE  # a missing page inside a window
        rng = np.random.default_rng(rep + 7)
        k_new = rng.standard_normal((len(lens), n_kv, 128)).astype(np.float32)
        v_new = (rng.standard_normal((len(lens), n_kv, 128)) * 3).astype(np.float32)
        hp, _ = host_pages(pk)
        ref0 = O.decode_f64(hp, q, tables, kv_len, p_start, 0.0883883)
        out0 = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                         max_kv_len=2049, scale=0.0883883, p_start=dev_i32(p_start, gpu))
        sync()
        o0 = out0.cpu().numpy()
        assert (o0[7] == 0).all()
        assert rel_err(o0, ref0).max() < TOL[DTYPE_Q8A], rep
        O.append(hp, k_new, v_new, np.arange(len(lens), dtype=np.int32), kv_len - 1, tables)
        ref1 = O.decode_f64(hp, q, tables, kv_len, p_start, 0.0883883)
        out1 = pk.append_decode(dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tables, gpu),
                                dev_i32(kv_len, gpu), n_heads=n_kv * rep, max_kv_len=2049, scale=0.0883883,
                                p_start=dev_i32(p_start, gpu))
        sync()
        got, _ = host_pages(pk)
        assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8))
        assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8))
        assert np.array_equal(got.ks, hp.ks) and np.array_equal(got.vs, hp.vs)
        assert rel_err(out1, ref1).max() < TOL[DTYPE_Q8A], rep


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("rep", [4, 8])
def test_q8a_query_extremes(gpu, monkeypatch, rep, schedule):
    """q rows at the edges of the int8-limb q.k of the Q8A matrix-core path
    (limbs scaled to each head's largest |q*scale|): an all-zero head, a head
    with one element 10^6 times the rest, a head whose largest element is
    below 2^-100 (it scores zero), a head of large values (a sharp softmax)
    and ordinary heads.  Against the f64 oracle (1e-5), both schedules."""
    monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", schedule)
    say("q8a q extremes", schedule, "rep", rep)
    n_kv, d = 2, 128
    lens = (40, 300, 1000, 2049)
    pk, tables, kv_len, q = _case(gpu, DTYPE_Q8A, d, rep, n_kv, lens, seed=200 + rep)
    rng = np.random.default_rng(rep)
    for s_ in range(len(lens)):
        for kvh in range(n_kv):
            h0 = kvh * rep
            q[s_, h0 + 0] = 0.0
            q[s_, h0 + 1] = rng.standard_normal(d).astype(np.float32) * 3e-5
            q[s_, h0 + 1, rng.integers(d)] = 30.0
            q[s_, h0 + 2] = rng.standard_normal(d).astype(np.float32) * 1e-32
            q[s_, h0 + 3] = rng.standard_normal(d).astype(np.float32) * 8.0
    hp, _ = host_pages(pk)
    scale = 1.0 / np.sqrt(d)
    ref = O.decode_f64(hp, q, tables, kv_len, None, scale)
    out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                    max_kv_len=int(kv_len.max()), scale=float(scale), split=0)
    sync()
    err = rel_err(out, ref)
    assert err.max() < TOL[DTYPE_Q8A], err.max()
    assert np.isfinite(out.cpu().numpy()).all()



@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_Q8A])
def test_out_of_range_kv_len_stores_nothing(gpu, dtype):
    # kv_len past max_kv_len, or past 16 * bt_stride: the row is out of range.
    # The fused call stores nothing for it (no existing token is overwritten)
    # and its output row is zero; the other rows are unaffected.
    say("out-of-range kv_len", DTYPE_NAMES[dtype])
    d, rep, n_kv = 128, 4, 2
    lens = (300, 200, 500, 64)
    pk, tables, kv_len, q = _case(gpu, dtype, d, rep, n_kv, lens, seed=21)
    stride = tables.shape[1]
    kv = kv_len.copy()
    kv[1] = 301                  # > max_kv_len (300): out of range
    kv[3] = 16 * stride + 5      # past the table row: out of range
    kv[2] = 300                  # in range
    rng = np.random.default_rng(2)
    k_new = rng.standard_normal((len(lens), n_kv, d)).astype(np.float32)
    v_new = rng.standard_normal((len(lens), n_kv, d)).astype(np.float32)
    hp, _ = host_pages(pk)
    in_range = np.array([True, False, True, False])
    O.append(hp, k_new[in_range], v_new[in_range], np.arange(2, dtype=np.int32), kv[in_range] - 1,
             tables[in_range])
    ref = O.decode_f64(hp, q[in_range], tables[in_range], kv[in_range], None, 0.1)
    for split in (0, 64):
        out = pk.append_decode(dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tables, gpu),
                               dev_i32(kv, gpu), n_heads=n_kv * rep, max_kv_len=300, scale=0.1, split=split)
        sync()
        o = out.cpu().numpy()
        assert (o[1] == 0).all() and (o[3] == 0).all()
        assert rel_err(o[in_range], ref).max() < TOL[dtype]
        # every page byte equals the oracle's after the in-range appends
        hp_now, _ = host_pages(pk)
        assert np.array_equal(hp_now.k, hp.k) and np.array_equal(hp_now.v, hp.v), split
        if hp.ks is not None:
            assert np.array_equal(hp_now.ks, hp.ks) and np.array_equal(hp_now.vs, hp.vs)


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_schedules_random_batches(gpu, monkeypatch, schedule):
    """Seeded random small batches on each schedule against the f64 oracle:
    1-70 sequences of 0-900 tokens, rep 1/2/4/8, f16 or Q8A pages, head_dim
    128 or 256, random
    window starts, a missing page now and then, unfused and fused (pages and
    Q8A scales bit-exact after the fused call)."""
    monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", schedule)
    rng = np.random.default_rng(2024 if schedule == "stream-k" else 2025)
    for case in range(16):
        dtype = DTYPE_F16 if case % 2 == 0 else DTYPE_Q8A
        d = 256 if case % 4 >= 2 else 128
        rep = int(rng.choice([1, 2, 4, 8]))
        n_kv = int(rng.choice([1, 2, 4]))
        n_seq = int(rng.integers(1, 71))
        lens = tuple(int(x) for x in rng.integers(0, 901, n_seq))
        say(schedule, "random case", case, DTYPE_NAMES[dtype], "d", d, "rep", rep, "n_kv", n_kv, "n_seq", n_seq)
        pk, tables, kv_len, q = _case(gpu, dtype, d, rep, n_kv, lens, seed=1000 + case)
        if case % 3 == 0 and kv_len.max() > 40:
            s_miss = int(np.argmax(kv_len))
            tables[s_miss, 1] = NO_PAGE
        p_start = np.array([int(rng.integers(0, L + 1)) if rng.random() < 0.4 else 0 for L in kv_len], np.int32)
        hp, _ = host_pages(pk)
        scale = 1.0 / np.sqrt(d)
        ref = O.decode_f64(hp, q, tables, kv_len, p_start, scale)
        mkv = max(int(kv_len.max()), 1)
        out = pk.decode(dev_f32(q, gpu), dev_i32(tables, gpu), dev_i32(kv_len, gpu), n_heads=n_kv * rep,
                        max_kv_len=mkv, scale=float(scale), p_start=dev_i32(p_start, gpu), split=0)
        sync()
        assert rel_err(out, ref).max() < TOL[dtype], (schedule, case)
        # fused: one more token per sequence (every table row has a spare
        # entry; a new token on a page the row lacks is stored nowhere and
        # skipped, by the oracle as by the library)
        kv1 = (kv_len + 1).astype(np.int32)
        assert (kv1 <= tables.shape[1] * 16).all()
        k_new = rng.standard_normal((n_seq, n_kv, d)).astype(np.float32)
        v_new = rng.standard_normal((n_seq, n_kv, d)).astype(np.float32)
        O.append(hp, k_new, v_new, np.arange(n_seq, dtype=np.int32), kv1 - 1, tables)
        ref1 = O.decode_f64(hp, q, tables, kv1, np.minimum(p_start, kv1), scale)
        out1 = pk.append_decode(dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tables, gpu),
                                dev_i32(kv1, gpu), n_heads=n_kv * rep, max_kv_len=max(int(kv1.max()), 1),
                                scale=float(scale), p_start=dev_i32(np.minimum(p_start, kv1), gpu), split=0)
        sync()
        got, _ = host_pages(pk)
        assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8)), (schedule, case)
        assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8)), (schedule, case)
        if dtype == DTYPE_Q8A:
            assert np.array_equal(got.ks.view(np.uint32), hp.ks.view(np.uint32)), (schedule, case)
            assert np.array_equal(got.vs.view(np.uint32), hp.vs.view(np.uint32)), (schedule, case)
        assert rel_err(out1, ref1).max() < TOL[dtype], (schedule, case)
