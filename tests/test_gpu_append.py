"""GPU append: page bytes after the HIP append are bit-exact with the oracle.

Covers f32 / f16 / Q8A at head_dim 64/128/256, multi-sequence chunks that
straddle partially filled pages, missing pages (not written), the exhaustive
f32 -> f16 sweep over all 2^32 bit patterns, and Q8A ties / zero heads /
subnormal heads."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev_f32, dev_i32, fill_pages, host_pages, say
from lnskv import DTYPE_F16, DTYPE_F32, DTYPE_Q8A, DTYPE_NAMES, NO_PAGE
from lnskv.device import PagedKV, sync

pytestmark = pytest.mark.gpu


def _tables(rng, n_seq, stride, num_pages, used):
    perm = rng.permutation(num_pages).astype(np.uint32)
    t = np.full((n_seq, stride), NO_PAGE, np.uint32)
    k = 0
    for s in range(n_seq):
        t[s, :used[s]] = perm[k:k + used[s]]
        k += used[s]
    return t


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_Q8A])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_append_bit_exact(gpu, dtype, d):
    say("append", DTYPE_NAMES[dtype], "d", d)
    rng = np.random.default_rng(d + 10 * dtype)
    n_kv, num_pages, n_seq = 4, 64, 3
    pk = PagedKV(num_pages, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=1)
    tables = _tables(rng, n_seq, 8, num_pages, [6, 8, 3])
    # seq 0: 41-token chunk from 37 (pages 2..4); seq 1: single token at 127;
    # seq 2: 5 tokens from 14 (straddles pages 0/1); plus a token on a missing page
    # and two naming rows outside the table (-1 and n_seq), all skipped
    tok_seq = np.array([0] * 41 + [1] + [2] * 5 + [2, -1, n_seq], np.int32)
    tok_pos = np.array(list(range(37, 78)) + [127] + list(range(14, 19)) + [100, 5, 5], np.int32)
    n = len(tok_seq)
    k_new = (rng.standard_normal((n, n_kv, d)) * 3).astype(np.float32)
    v_new = (rng.standard_normal((n, n_kv, d)) * 3).astype(np.float32)
    hp, _ = host_pages(pk)
    assert O.append(hp, k_new, v_new, tok_seq, tok_pos, tables) == 3
    pk.append(dev_f32(k_new, gpu), dev_f32(v_new, gpu), dev_i32(tok_seq, gpu), dev_i32(tok_pos, gpu),
              dev_i32(tables, gpu))
    sync()
    got, _ = host_pages(pk)
    assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8))
    assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8))
    if dtype == DTYPE_Q8A:
        assert np.array_equal(got.ks, hp.ks) and np.array_equal(got.vs, hp.vs)


@pytest.mark.parametrize("part", range(8))
def test_f16_append_exhaustive_all_f32_patterns(gpu, part):
    """Every f32 bit pattern (in 8 parts of 2^29) through the GPU append;
    every one must give the oracle's bits (RNE for numbers; for NaNs the quiet
    NaN with the input's sign and top 10 payload bits)."""
    n_kv, d = 8, 128
    chunk = 1 << 26
    tok = chunk // (n_kv * d)
    pages = tok // 16
    pk = PagedKV(pages, n_kv, d, DTYPE_F16, gpu)
    tables = dev_i32(np.arange(pages, dtype=np.uint32)[None, :], gpu)
    tok_seq = torch.zeros(tok, dtype=torch.int32, device=gpu)
    tok_pos = torch.arange(tok, dtype=torch.int32, device=gpu)
    per_part = (1 << 29) // chunk
    say("f16 sweep part", part)
    for c in range(part * per_part, (part + 1) * per_part):
        lo = c * chunk
        bits = torch.arange(lo, lo + chunk, dtype=torch.int64, device=gpu)
        bits = torch.where(bits >= (1 << 31), bits - (1 << 32), bits).to(torch.int32)
        x = bits.view(torch.float32)
        pk.append(x, x, tok_seq, tok_pos, tables)
        got = pk.k.view(torch.int16).reshape(-1).cpu().numpy().view(np.uint16)
        exp = O.f16_of_patterns(lo, chunk)
        assert np.array_equal(got, exp), f"chunk {c}"


@pytest.mark.parametrize("d", [64, 128, 256])
def test_q8a_append_edge_cases(gpu, d):
    say("q8a edge cases d", d)
    n_kv = 2
    rows = []
    rows.append(np.zeros(d))                                     # zero head: scale 1, q 0
    t = np.zeros(d)
    t[:7] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 126.5]             # exact ties (scale 1)
    rows.append(t)
    rows.append(np.full(d, -3.0))                                 # constant head
    rows.append(np.random.default_rng(3).standard_normal(d) * 1e-40)  # f32 subnormals
    rows.append(np.random.default_rng(4).standard_normal(d) * 1e30)
    rng = np.random.default_rng(5)
    for _ in range(27):
        rows.append(rng.standard_normal(d) * rng.uniform(1e-3, 1e3))
    x = np.array(rows, np.float32).reshape(-1, n_kv, d)
    n = x.shape[0]
    pk = PagedKV(8, n_kv, d, DTYPE_Q8A, gpu)
    tables = np.arange(8, dtype=np.uint32)[None, :]
    tok_seq = np.zeros(n, np.int32)
    tok_pos = np.arange(n, dtype=np.int32)
    hp, _ = host_pages(pk)
    O.append(hp, x, x[::-1].copy(), tok_seq, tok_pos, tables)
    pk.append(dev_f32(x, gpu), dev_f32(x[::-1].copy(), gpu), dev_i32(tok_seq, gpu), dev_i32(tok_pos, gpu),
              dev_i32(tables, gpu))
    sync()
    got, _ = host_pages(pk)
    assert np.array_equal(got.k, hp.k) and np.array_equal(got.v, hp.v)
    assert np.array_equal(got.ks.view(np.uint32), hp.ks.view(np.uint32))
    assert np.array_equal(got.vs.view(np.uint32), hp.vs.view(np.uint32))
