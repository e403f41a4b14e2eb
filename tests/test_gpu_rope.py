"""RoPE fused into the append and the append+decode (GPU vs the oracle).

The oracle turns q and K with apply_cpu_rope_with_freqs' rotation
(engine.rs:200-229) at the reference's positions (the new token's position
kv_len-1 for a decode, tok_pos for a chunk append), appends and attends; the
GPU entry points take the unrotated values.  Both take each angle's sin and
cos from the same f64 evaluation rounded once to f32 and round each product
and sum of the turn once, so the pages the call writes (rotated K, V, Q8A
codes and scales) are bit-exact with the oracle's, and every other byte of
the pools is unchanged.  Outputs: row-normwise error against the f64 oracle
within TOL.  Cases cover both MFMA schedules with rotary widths 128 and 64
(turned in registers, f16 and Q8A pages, heads of 128 and 256 dims), a width
of 96 and the VALU kernel (turned by the separate pass), f32 pages, and the
chunk append's in-kernel and separate-pass paths."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import TOL, dev_f32, dev_i32, fill_pages, host_pages, rel_err, say
from lnskv import DTYPE_F16, DTYPE_F32, DTYPE_Q8A, DTYPE_NAMES, NO_PAGE
from lnskv.device import PagedKV, RopeTable, sync

pytestmark = pytest.mark.gpu


def _tables(rng, lens, num_pages):
    pages_per = [(L + 15) // 16 for L in lens]
    perm = rng.permutation(num_pages).astype(np.uint32)
    stride = max(pages_per) + 1
    t = np.full((len(lens), stride), NO_PAGE, np.uint32)
    k = 0
    for s, n in enumerate(pages_per):
        t[s, :n] = perm[k:k + n]
        k += n
    return t


def _check_pages(got, exp, before, dtype):
    """Every byte of both pools (and the Q8A scales) equals the oracle's: the
    rows the call wrote (rotated K, V) and, unchanged, all the others."""
    del before  # the oracle's pages started as a copy of the same bytes
    for which in ("k", "v"):
        g, e = getattr(got, which), getattr(exp, which)
        assert np.array_equal(g.view(np.uint8), e.view(np.uint8)), which
    if dtype == DTYPE_Q8A:
        assert np.array_equal(got.ks.view(np.uint32), exp.ks.view(np.uint32))
        assert np.array_equal(got.vs.view(np.uint32), exp.vs.view(np.uint32))


CASES = [  # dtype, head_dim, rep, rotary_dim, split, force_valu
    (DTYPE_F16, 128, 4, 128, 0, "0"),
    (DTYPE_F16, 128, 4, 64, 0, "0"),
    (DTYPE_F16, 128, 2, 128, 128, "0"),
    (DTYPE_F16, 128, 4, 96, 0, "0"),
    (DTYPE_F16, 128, 4, 128, 0, "1"),
    (DTYPE_F32, 64, 2, 64, 0, "0"),
    (DTYPE_Q8A, 128, 4, 128, 0, "0"),   # Q8A: turned in registers before the quantizer
    (DTYPE_Q8A, 128, 4, 64, 0, "0"),
    (DTYPE_Q8A, 256, 4, 64, 0, "0"),    # lns-ml's Qwen3.5 layers: rotary 64 of 256
    (DTYPE_F16, 256, 4, 64, 0, "0"),
    (DTYPE_F16, 256, 2, 128, 128, "0"),  # split-K, 256-wide heads
    (DTYPE_F16, 256, 4, 96, 0, "0"),    # pre-pass (rotary 96)
]


@pytest.mark.parametrize("dtype,d,rep,rd,split,valu", CASES)
def test_rope_append_decode(gpu, monkeypatch, dtype, d, rep, rd, split, valu):
    monkeypatch.setenv("LNSKV_FORCE_VALU", valu)
    say("rope append_decode", DTYPE_NAMES[dtype], "d", d, "rep", rep, "rotary", rd, "split", split, "valu", valu)
    rng = np.random.default_rng(d + rd + rep + split)
    n_kv = 4
    lens = np.array([1, 16, 17, 300, 1000, 2049, 5], np.int32)
    num_pages = int(sum((L + 15) // 16 for L in lens)) + 8
    pk = PagedKV(num_pages, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=rd + d)
    tables = _tables(rng, lens, num_pages)
    rope = RopeTable(rd, 500000.0, O.ROPE_LLAMA3, (8.0, 8192.0, 1.0, 4.0), device=gpu)
    n = len(lens)
    q = rng.standard_normal((n, n_kv * rep, d)).astype(np.float32)
    k_new = rng.standard_normal((n, n_kv, d)).astype(np.float32)
    v_new = rng.standard_normal((n, n_kv, d)).astype(np.float32)
    before, _ = host_pages(pk)
    hp = before.copy()
    pos = lens - 1
    q_r = O.rope_apply(q, rd, rope.inv_freqs_host, pos)
    k_r = O.rope_apply(k_new, rd, rope.inv_freqs_host, pos)
    O.append(hp, k_r, v_new, np.arange(n, dtype=np.int32), pos, tables)
    scale = 1.0 / np.sqrt(d)
    ref = O.decode_f64(hp, q_r, tables, lens, None, scale)
    qd, kd = dev_f32(q, gpu), dev_f32(k_new, gpu)
    out = pk.rope_append_decode(rope, qd, kd, dev_f32(v_new, gpu), dev_i32(tables, gpu), dev_i32(lens, gpu),
                                n_heads=n_kv * rep, max_kv_len=int(lens.max()), scale=float(scale), split=split)
    sync()
    assert torch.equal(qd.cpu(), torch.from_numpy(q)) and torch.equal(kd.cpu(), torch.from_numpy(k_new))
    got, _ = host_pages(pk)
    _check_pages(got, hp, before, dtype)
    assert rel_err(out, ref).max() < TOL[dtype]


APPEND_CASES = [  # dtype, head_dim, rotary_dim
    (DTYPE_F16, 128, 128), (DTYPE_F16, 128, 64), (DTYPE_F16, 128, 96), (DTYPE_F32, 64, 32),
    (DTYPE_F32, 256, 256), (DTYPE_Q8A, 128, 128),
]


@pytest.mark.parametrize("dtype,d,rd", APPEND_CASES)
def test_rope_chunk_append(gpu, dtype, d, rd):
    say("rope append", DTYPE_NAMES[dtype], "d", d, "rotary", rd)
    rng = np.random.default_rng(d * 7 + rd)
    n_kv, num_pages = 4, 48
    pk = PagedKV(num_pages, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=3)
    tables = _tables(rng, [96, 128, 40], num_pages)
    # seq 0: 45 tokens from 37; seq 1: 1 token at 127; seq 2: 9 tokens from 14; one on a missing page
    tok_seq = np.array([0] * 45 + [1] + [2] * 9 + [2], np.int32)
    tok_pos = np.array(list(range(37, 82)) + [127] + list(range(14, 23)) + [100], np.int32)
    k_new = (rng.standard_normal((len(tok_seq), n_kv, d)) * 2).astype(np.float32)
    v_new = (rng.standard_normal((len(tok_seq), n_kv, d)) * 2).astype(np.float32)
    rope = RopeTable(rd, 10000.0, device=gpu)
    before, _ = host_pages(pk)
    hp = before.copy()
    k_r = O.rope_apply(k_new, rd, rope.inv_freqs_host, tok_pos)
    assert O.append(hp, k_r, v_new, tok_seq, tok_pos, tables) == 1
    pk.rope_append(rope, dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tok_seq, gpu), dev_i32(tok_pos, gpu),
                   dev_i32(tables, gpu))
    sync()
    got, _ = host_pages(pk)
    _check_pages(got, hp, before, dtype)
