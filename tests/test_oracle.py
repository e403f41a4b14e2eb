"""Pins of the CPU oracle (oracle/lnskv_oracle.c) by facts independent of it.

Each test checks the restatement against something that fixes the answer on
its own: the x86 F16C converter and numpy for binary16 rounding, closed forms
of the Q8A quantizer and of softmax attention, a numpy softmax written here in
a different form (two passes over gathered values, not an online scan), brute
force on tiny shapes, and invariants (split-K, page permutation, GQA == MHA
with replicated heads).  Planted mistakes in the oracle (a dropped term, a
wrong head index, a transposed operand, rint instead of round) fail at least one.
"""
import numpy as np
import pytest

import oracle as O

RNG = np.random.default_rng(12345)


# ---------------------------------------------------------------- f16 ------
def test_f16_exhaustive_matches_f16c():
    # all 2^32 f32 bit patterns (NaN payloads included) vs the x86 F16C converter
    assert O.f16_check_range(0, 1 << 32) == 0


def test_f16_matches_numpy_on_specials_and_random():
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 65520.0, -65520.0, 1e-8, 2.0 ** -24,
                        2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -11),
                        np.inf, -np.inf, 3.14159265, 1.0009765625, 1.00048828125, 1.000732421875],
                       np.float32)
    rnd = RNG.standard_normal(200_000).astype(np.float32) * np.float32(100.0)
    tiny = (RNG.standard_normal(50_000) * 1e-6).astype(np.float32)
    x = np.concatenate([special, rnd, tiny])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16_bits(x), ref)


def test_f16_widening_exact_for_all_patterns():
    lib = O.lib()
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


# ---------------------------------------------------------------- Q8A ------
def _q8a_numpy(x):
    """Q8A written independently: f32 scale, f32 divide, half-away-from-zero in f64."""
    x = x.astype(np.float32)
    amax = np.float32(np.max(np.abs(x))) if x.size else np.float32(0)
    sc = np.float32(1.0) if amax == 0 else np.float32(amax / np.float32(127.0))
    r = (x / sc).astype(np.float64)
    q = np.sign(r) * np.floor(np.abs(r) + 0.5)
    return np.clip(q, -127, 127).astype(np.int8), float(sc)


def test_q8a_zero_head():
    q, sc = O.q8a_quantize(np.zeros(128, np.float32))
    assert sc == 1.0 and not q.any()


def test_q8a_ties_round_half_away_from_zero():
    # amax 127 makes the scale exactly 1, so x/sc == x and ties are exact
    x = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, 0.49999997], np.float32)
    q, sc = O.q8a_quantize(x)
    assert sc == 1.0
    assert q.tolist() == [127, 3, -3, 1, -1, 2, -2, 127, 0]


@pytest.mark.parametrize("d", [64, 128, 256])
def test_q8a_amax_and_brute_force(d):
    for _ in range(200):
        x = (RNG.standard_normal(d) * RNG.uniform(1e-3, 1e3)).astype(np.float32)
        q, sc = O.q8a_quantize(x)
        i = int(np.argmax(np.abs(x)))
        assert abs(int(q[i])) == 127 and np.sign(q[i]) == np.sign(x[i])
        qr, scr = _q8a_numpy(x)
        assert sc == scr
        assert np.array_equal(q, qr)


# ---------------------------------------------------------- PagePool -------
def test_pool_fifo_closed_form():
    p = O.Pool(4)
    assert [p.alloc() for _ in range(5)] == [0, 1, 2, 3, None]
    p.free_page(2)
    p.free_page(0)
    assert p.num_free == 2
    assert [p.alloc(), p.alloc(), p.alloc()] == [2, 0, None]
    p.reset()
    assert p.num_free == 4 and p.alloc() == 0


def test_ensure_evict_pstart_closed_forms():
    import ctypes as C
    lib = O.lib()
    p = lib.orc_pool_new(8)
    bt = np.full(8, O.NO_PAGE, np.uint32)
    n = C.c_int(0)
    for pos in range(40):  # 3 logical pages
        assert lib.orc_ensure_kv_page(p, bt.ctypes.data, C.byref(n), 8, pos) == 0
    assert n.value == 3 and bt[:3].tolist() == [0, 1, 2]
    # window 20 at pos 39: p_start = 20, pages [0, 20//16=1) evicted
    assert lib.orc_kv_p_start(39, 20) == 20
    lib.orc_evict_kv_pages(p, bt.ctypes.data, n.value, 39, 20)
    assert bt[:3].tolist() == [O.NO_PAGE, 1, 2]
    assert lib.orc_pool_num_free(p) == 6
    assert lib.orc_kv_p_start(5, 20) == 0 and lib.orc_kv_p_start(100, 0) == 0
    # freed page 0 goes to the back of the FIFO: next allocations 3,4,...,7,0
    got = []
    for pos in range(48, 48 + 16 * 6, 16):
        lib.orc_ensure_kv_page(p, bt.ctypes.data, C.byref(n), 8, pos)
    got = bt[3:8].tolist()
    assert got == [3, 4, 5, 6, 7]
    lib.orc_pool_delete(p)


# ------------------------------------------------- append/gather/copy ------
def _random_pool(num_pages, n_kv, d, dtype):
    hp = O.HostPages.zeros(num_pages, n_kv, d, dtype)
    if dtype == O.F32:
        hp.k[...] = RNG.standard_normal(hp.k.shape)
        hp.v[...] = RNG.standard_normal(hp.v.shape)
    elif dtype == O.F16:
        hp.k[...] = RNG.standard_normal(hp.k.shape).astype(np.float16).view(np.uint16)
        hp.v[...] = RNG.standard_normal(hp.v.shape).astype(np.float16).view(np.uint16)
    else:
        hp.k[...] = RNG.integers(-127, 128, hp.k.shape)
        hp.v[...] = RNG.integers(-127, 128, hp.v.shape)
        hp.ks[...] = RNG.uniform(0.001, 0.1, hp.ks.shape)
        hp.vs[...] = RNG.uniform(0.001, 0.1, hp.vs.shape)
    return hp


def _expected_stored(x, dtype):
    """What a head row [.., d] f32 becomes in the page, computed independently."""
    if dtype == O.F32:
        return x.astype(np.float32), None
    if dtype == O.F16:
        return x.astype(np.float16).view(np.uint16), None
    qs, scs = [], []
    for row in x.reshape(-1, x.shape[-1]):
        q, sc = _q8a_numpy(row)
        qs.append(q)
        scs.append(sc)
    return np.stack(qs).reshape(x.shape), np.array(scs, np.float32).reshape(x.shape[:-1])


@pytest.mark.parametrize("dtype", [O.F32, O.F16, O.Q8A])
def test_append_then_gather_identity(dtype):
    n_kv, d, num_pages = 4, 64, 24
    hp = _random_pool(num_pages, n_kv, d, dtype)
    before = hp.copy()
    perm = RNG.permutation(num_pages).astype(np.uint32)
    tables = np.full((2, 8), O.NO_PAGE, np.uint32)
    tables[0, :5] = perm[:5]
    tables[1, :4] = perm[5:9]
    # seq 0 appends a 37-token chunk at 35 (straddles pages 2..4); seq 1 one token at 60
    tok_seq = np.array([0] * 37 + [1], np.int32)
    tok_pos = np.array(list(range(35, 72)) + [60], np.int32)
    k_new = RNG.standard_normal((38, n_kv, d)).astype(np.float32)
    v_new = RNG.standard_normal((38, n_kv, d)).astype(np.float32)
    assert O.append(hp, k_new, v_new, tok_seq, tok_pos, tables) == 0
    ko, vo, kso, vso = O.gather(hp, tables[0], 35, 37)
    ek, eks = _expected_stored(k_new[:37], dtype)
    ev, evs = _expected_stored(v_new[:37], dtype)
    assert np.array_equal(ko.view(np.uint8), ek.view(np.uint8))
    assert np.array_equal(vo.view(np.uint8), ev.view(np.uint8))
    if dtype == O.Q8A:
        assert np.array_equal(kso, eks) and np.array_equal(vso, evs)
    # tokens before the chunk and untouched pages are unchanged
    k0, _, _, _ = O.gather(hp, tables[0], 0, 35)
    k0b, _, _, _ = O.gather(before, tables[0], 0, 35)
    assert np.array_equal(k0, k0b)
    untouched = np.setdiff1d(np.arange(num_pages), np.concatenate([tables[0, 2:5], tables[1, 3:4]]))
    assert np.array_equal(hp.k[untouched], before.k[untouched])
    # a chunk equals token-by-token appends
    hp2 = before.copy()
    for t in range(38):
        O.append(hp2, k_new[t:t + 1], v_new[t:t + 1], tok_seq[t:t + 1], tok_pos[t:t + 1], tables)
    assert np.array_equal(hp2.k, hp.k) and np.array_equal(hp2.v, hp.v)


def test_append_skips_missing_pages():
    hp = _random_pool(4, 2, 64, O.F16)
    before = hp.copy()
    tables = np.full((1, 4), O.NO_PAGE, np.uint32)
    tables[0, 1] = 9  # outside the pool
    x = RNG.standard_normal((2, 2, 64)).astype(np.float32)
    assert O.append(hp, x, x, np.zeros(2, np.int32), np.array([3, 17], np.int32), tables) == 2
    assert np.array_equal(hp.k, before.k)
    tables[0, 0] = 1  # a real page, but the rows named below are outside the table
    assert O.append(hp, x, x, np.array([-1, 1], np.int32), np.array([3, 3], np.int32), tables) == 2
    assert np.array_equal(hp.k, before.k)


@pytest.mark.parametrize("dtype", [O.F32, O.F16, O.Q8A])
def test_page_copy_then_gather(dtype):
    hp = _random_pool(16, 2, 128, dtype)
    before = hp.copy()
    src = np.array([3, 7, 1], np.uint32)
    dst = np.array([10, 11, 12], np.uint32)
    O.page_copy(hp, src, dst)
    for s, t in zip(src, dst):
        a = O.gather(hp, np.array([t], np.uint32), 0, 16)
        b = O.gather(before, np.array([s], np.uint32), 0, 16)
        for x, y in zip(a, b):
            if x is not None:
                assert np.array_equal(x, y)
    rest = np.setdiff1d(np.arange(16), dst)
    assert np.array_equal(hp.k[rest], before.k[rest])


# --------------------------------------------------------------- decode ----
def _numpy_attention(hp, q, tables, kv_len, p_start, scale):
    """Two-pass softmax over gathered stored values, written independently."""
    K = O.stored_values(hp, False)
    V = O.stored_values(hp, True)
    n_seq, n_heads, d = q.shape
    rep = n_heads // hp.n_kv
    out = np.zeros(q.shape, np.float64)
    for s in range(n_seq):
        p0 = 0 if p_start is None else p_start[s]
        toks = [p for p in range(p0, kv_len[s])
                if tables[s, p // 16] != O.NO_PAGE and tables[s, p // 16] < hp.num_pages]
        if not toks:
            continue
        slots = np.array([tables[s, p // 16] * 16 + p % 16 for p in toks])
        for h in range(n_heads):
            Kh = K[slots, h // rep]
            Vh = V[slots, h // rep]
            sc = Kh @ q[s, h].astype(np.float64) * scale
            w = np.exp(sc - sc.max())
            out[s, h] = (w / w.sum()) @ Vh
    return out


def _decode_case(dtype, n_kv=2, rep=4, d=64, lens=(1, 17, 40, 64), num_pages=40, seed=0, window=0):
    rng = np.random.default_rng(seed)
    hp = _random_pool(num_pages, n_kv, d, dtype)
    n_seq = len(lens)
    stride = max(lens) // 16 + 1
    perm = rng.permutation(num_pages).astype(np.uint32)
    tables = np.full((n_seq, stride), O.NO_PAGE, np.uint32)
    k = 0
    for s, L in enumerate(lens):
        n = (L + 15) // 16
        tables[s, :n] = perm[k:k + n]
        k += n
    kv_len = np.array(lens, np.int32)
    p_start = None
    if window:
        p_start = np.array([max(0, L - window) for L in lens], np.int32)
    q = rng.standard_normal((n_seq, n_kv * rep, d)).astype(np.float32)
    return hp, q, tables, kv_len, p_start


@pytest.mark.parametrize("dtype", [O.F32, O.F16, O.Q8A])
@pytest.mark.parametrize("window", [0, 20])
def test_f64_matches_numpy_softmax(dtype, window):
    hp, q, tables, kv_len, p_start = _decode_case(dtype, window=window)
    scale = 0.125
    got = O.decode_f64(hp, q, tables, kv_len, p_start, scale)
    ref = _numpy_attention(hp, q, tables, kv_len, p_start, scale)
    assert np.abs(got - ref).max() < 1e-12


def test_f64_matches_numpy_with_missing_page():
    hp, q, tables, kv_len, _ = _decode_case(O.F16)
    tables[3, 1] = O.NO_PAGE
    got = O.decode_f64(hp, q, tables, kv_len, None, 0.125)
    ref = _numpy_attention(hp, q, tables, kv_len, None, 0.125)
    assert np.abs(got - ref).max() < 1e-12


def test_closed_form_single_token_returns_v_exactly():
    hp, q, tables, _, _ = _decode_case(O.F32, lens=(1, 1))
    kv_len = np.array([1, 1], np.int32)
    ref32 = O.decode_refscan(hp, q, tables, kv_len, None, 0.125)
    V = O.stored_values(hp, True)
    for s in range(2):
        slot = tables[s, 0] * 16
        for h in range(q.shape[1]):
            assert np.array_equal(ref32[s, h], V[slot, h // 4].astype(np.float32))


def test_closed_form_equal_keys_and_zero_query_give_mean_v():
    hp, q, tables, kv_len, _ = _decode_case(O.F32, lens=(40,))
    slots = [tables[0, p // 16] * 16 + p % 16 for p in range(40)]
    kk = hp.k.reshape(-1, hp.n_kv, hp.head_dim)
    kk[slots] = kk[slots[0]]
    V = O.stored_values(hp, True)
    out = O.decode_f64(hp, q, tables, kv_len, None, 0.125)
    mean = V[slots].mean(axis=0)
    for h in range(q.shape[1]):
        assert np.abs(out[0, h] - mean[h // 4]).max() < 1e-12
    hp2, _, tables2, kv2, _ = _decode_case(O.F16, lens=(33,))
    q0 = np.zeros((1, 8, 64), np.float32)
    out0 = O.decode_f64(hp2, q0, tables2, kv2, None, 0.125)
    V2 = O.stored_values(hp2, True)
    s2 = [tables2[0, p // 16] * 16 + p % 16 for p in range(33)]
    assert np.abs(out0[0, 5] - V2[s2].mean(axis=0)[5 // 4]).max() < 1e-12


def test_closed_form_dominant_score_selects_v():
    hp, q, tables, kv_len, _ = _decode_case(O.F32, lens=(40,))
    K = hp.k.reshape(-1, hp.n_kv, hp.head_dim)
    slot = tables[0, 1] * 16 + 5  # token 21
    K[slot, 0] = q[0, 0] * 50.0
    out = O.decode_f64(hp, q, tables, kv_len, None, 0.125)
    V = O.stored_values(hp, True)
    assert np.abs(out[0, 0] - V[slot, 0]).max() < 1e-6


@pytest.mark.parametrize("dtype,tol", [(O.F32, 1e-5), (O.F16, 1e-5), (O.Q8A, 1e-5)])
def test_refscan_f32_within_tolerance_of_f64(dtype, tol):
    hp, q, tables, kv_len, p_start = _decode_case(dtype, lens=(1, 100, 256, 300), num_pages=60, window=0)
    a = O.decode_refscan(hp, q, tables, kv_len, p_start, 0.125)
    b = O.decode_f64(hp, q, tables, kv_len, p_start, 0.125)
    assert O.rel_err_rows(a, b).max() < tol


@pytest.mark.parametrize("split", [16, 32, 48, 160, 1024])
def test_split_k_combine_equals_full_softmax(split):
    hp, q, tables, kv_len, p_start = _decode_case(O.F16, lens=(5, 100, 256, 300), num_pages=60, window=70)
    a = O.decode_split_f64(hp, q, tables, kv_len, split, p_start, 0.125)
    b = O.decode_f64(hp, q, tables, kv_len, p_start, 0.125)
    assert np.abs(a - b).max() < 1e-12


def test_gqa_equals_mha_with_replicated_heads():
    hp, q, tables, kv_len, _ = _decode_case(O.F16, n_kv=2, rep=4, lens=(40, 70), num_pages=20)
    rep = 4
    k_rep = np.repeat(hp.k, rep, axis=2)
    v_rep = np.repeat(hp.v, rep, axis=2)
    mha = O.HostPages(k_rep, v_rep, dtype=O.F16)
    a = O.decode_f64(hp, q, tables, kv_len, None, 0.125)
    b = O.decode_f64(mha, q, tables, kv_len, None, 0.125)
    assert np.abs(a - b).max() == 0.0


def test_page_permutation_invariance_bitwise():
    hp, q, tables, kv_len, _ = _decode_case(O.F16, lens=(40, 70, 3), num_pages=20)
    a = O.decode_refscan(hp, q, tables, kv_len, None, 0.125)
    perm = np.random.default_rng(7).permutation(hp.num_pages)
    inv = np.argsort(perm)
    hp2 = O.HostPages(hp.k[perm], hp.v[perm], dtype=O.F16)  # new page i holds old page perm[i]
    t2 = tables.copy()
    mask = t2 != O.NO_PAGE
    t2[mask] = inv[t2[mask]]
    b = O.decode_refscan(hp2, q, t2, kv_len, None, 0.125)
    assert np.array_equal(a, b)


def test_append_decode_refscan_is_append_then_scan():
    hp, q, tables, kv_len, _ = _decode_case(O.F16, lens=(17, 40, 64, 3), num_pages=40)
    k_new = RNG.standard_normal((4, 2, 64)).astype(np.float32)
    v_new = RNG.standard_normal((4, 2, 64)).astype(np.float32)
    a_pages = hp.copy()
    a = O.append_decode_refscan(a_pages, q, k_new, v_new, tables, kv_len, None, 0.125)
    b_pages = hp.copy()
    O.append(b_pages, k_new, v_new, np.arange(4, dtype=np.int32), kv_len - 1, tables)
    b = O.decode_refscan(b_pages, q, tables, kv_len, None, 0.125)
    assert np.array_equal(a_pages.k, b_pages.k) and np.array_equal(a, b)


def test_error_measures_by_hand():
    """The two error measures of the tolerance definition on values worked
    by hand: row-normwise max|o-r| / max|r| (floor 1e-30) and element-wise
    |o-r| / max(|r|, 1e-6)."""
    ref = np.array([[1.5, 1e-7, 0.0, -2.0]])
    out = np.array([[1.0, 0.0, 2e-7, -2.0]])
    assert np.allclose(O.rel_err_rows(out, ref), [0.5 / 2.0])
    assert np.allclose(O.rel_err_elements(out, ref)[0], [0.5 / 1.5, 1e-7 / 1e-6, 2e-7 / 1e-6, 0.0])
    assert O.rel_err_rows(np.zeros((1, 3)), np.zeros((1, 3)))[0] == 0.0
