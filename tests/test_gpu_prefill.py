"""GPU chunked-prefill attention (lnskv_prefill_attention) against the
float64 oracle run token by token: query t of a chunk must equal the decode
of that token alone with kv_len = pos(t) + 1 (what the reference's
token-at-a-time forward computes), within the page type's tolerance (1e-3
relative per row for f16 pages, 1e-5 for Q8A pages).  f16 and Q8A pages,
head_dim 128 and 256.  Covers head ratios 1/2/4/8, a chunk with no earlier context, a
single-token chunk, a chunk whose row start lies past all its queries (whole
tiles with nothing to attend), ragged tile ends, a sliding window, a missing page, a
chunk naming a table row outside the tables (skipped: its rows untouched),
chunks out of sequence order, and two 128-token chunks over ~1500-token
contexts (full pages)."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import TOL, dev_f32, dev_i32, fill_pages, host_pages, rel_err, say
from lnskv import DTYPE_F16, DTYPE_NAMES, DTYPE_Q8A, NO_PAGE
from lnskv.device import PagedKV, sync

pytestmark = pytest.mark.gpu


def _run(gpu, rep, chunks, ctx_pages, p_start=None, missing=(), n_kv=2, seed=0, extra_rows=0, window=0,
         dtype=DTYPE_F16, d=128):
    """chunks: list of (table row, first position, length); tokens laid out in list order.
    window > 0: every token's reference start is max(p_start, kv_p_start(pos, window))."""
    rng = np.random.default_rng(seed)
    n_rows = len(ctx_pages)
    num_pages = sum(ctx_pages) + 8
    pk = PagedKV(num_pages, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=seed + 1)
    perm = rng.permutation(num_pages).astype(np.uint32)
    stride = max(ctx_pages) + 1
    tables = np.full((n_rows, stride), NO_PAGE, np.uint32)
    k = 0
    for s, npg in enumerate(ctx_pages):
        tables[s, :npg] = perm[k:k + npg]
        k += npg
    for s, pg in missing:
        tables[s, pg] = NO_PAGE
    desc, tok = [], 0
    for row, pos0, ln in chunks:
        desc.append((row, pos0, ln, tok))
        tok += ln
    n_tok = tok + extra_rows
    n_heads = n_kv * rep
    q = rng.standard_normal((n_tok, n_heads, d)).astype(np.float32)
    scale = float(1.0 / np.sqrt(d))
    ps = None if p_start is None else np.array(p_start, np.int32)
    out = torch.full((n_tok, n_heads, d), 7.0, device=gpu)
    pk.prefill_attention(dev_f32(q, gpu), torch.tensor(desc, dtype=torch.int32, device=gpu), dev_i32(tables, gpu),
                         n_heads=n_heads, scale=scale, p_start=None if ps is None else dev_i32(ps, gpu),
                         window=window, out=out)
    sync()
    hp, _ = host_pages(pk)
    rows, kvl, pst, idx = [], [], [], []
    for row, pos0, ln, t0 in desc:
        if not (0 <= row < n_rows):
            continue
        for i in range(ln):
            rows.append(tables[row])
            kvl.append(pos0 + i + 1)
            p0 = 0 if ps is None else int(ps[row])
            if window > 0:
                p0 = max(p0, max(0, pos0 + i - window + 1))  # kv_p_start(pos, window), engine.rs:3007-3013
            pst.append(p0)
            idx.append(t0 + i)
    idx = np.array(idx)
    ref = O.decode_f64(hp, q[idx], np.array(rows, np.uint32), np.array(kvl, np.int32), np.array(pst, np.int32),
                       scale)
    got = out.cpu().numpy()
    err = rel_err(got[idx], ref)
    say("prefill", DTYPE_NAMES[dtype], "d", d, "rep", rep, "tokens", len(idx), "max rel err", float(err.max()))
    assert err.max() < TOL[dtype]
    untouched = np.setdiff1d(np.arange(n_tok), idx)
    assert np.all(got[untouched] == 7.0)


DTYPES = [DTYPE_F16, DTYPE_Q8A]


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rep", [1, 2, 4, 8])
def test_prefill_small_cases(gpu, rep, dtype, d):
    chunks = [(1, 1000, 16),   # a whole tile at a long context, with a missing page in its window
              (0, 0, 37),      # no earlier context; 3 tiles, the last ragged
              (2, 15, 1),      # a single token at the end of page 0
              (3, 300, 100),   # windowed: attends [200, pos]
              (4, 100, 80),    # row start 400, past every query: nothing attended (zero rows)
              (9, 5, 4)]       # table row outside the tables: skipped
    ctx_pages = [3, 64, 1, 26, 12]
    _run(gpu, rep, chunks, ctx_pages, p_start=[0, 0, 0, 200, 400], missing=[(1, 20)], seed=rep, extra_rows=4,
         dtype=dtype, d=d)


@pytest.mark.parametrize("dtype", DTYPES)
def test_prefill_long_chunks(gpu, dtype):
    chunks = [(0, 1400, 128), (1, 1600, 128)]
    _run(gpu, 4, chunks, [(1400 + 128 + 15) // 16, (1600 + 128 + 15) // 16], n_kv=8, seed=11, dtype=dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_prefill_long_chunks_d256(gpu, dtype):
    """lns-ml's Qwen3.5 full-attention shape (16 query heads over 4 kv heads of
    256): two 128-token chunks over ~1500-token contexts."""
    chunks = [(0, 1400, 128), (1, 1600, 128)]
    _run(gpu, 4, chunks, [(1400 + 128 + 15) // 16, (1600 + 128 + 15) // 16], n_kv=4, seed=12, dtype=dtype,
         d=256)


@pytest.mark.parametrize("dtype", DTYPES)
def test_prefill_many_chunks(gpu, dtype):
    """70 chunks (past one 64-chunk scan group), lengths 1..40, some sharing a
    table row at different offsets, one outside the tables (skipped)."""
    rng = np.random.default_rng(5)
    n_rows = 24
    ctx_pages = [int(x) for x in rng.integers(2, 12, n_rows)]
    chunks = []
    for i in range(70):
        row = i % n_rows
        cap = ctx_pages[row] * 16
        ln = int(rng.integers(1, min(41, cap + 1)))
        pos0 = int(rng.integers(0, cap - ln + 1))
        chunks.append((row, pos0, ln))
    chunks[33] = (n_rows + 3, 0, 8)
    for rep in (4, 8):
        _run(gpu, rep, chunks, ctx_pages, seed=20 + rep, dtype=dtype)


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rep", [2, 4, 8])
def test_prefill_sliding_window(gpu, rep, dtype, d):
    """A sliding-window layer: each prompt token attends its own window
    [pos - w + 1, pos] (the reference's per-token kv_p_start), checked token by
    token against the oracle.  Chunks that cross the window (longer than it,
    starting before and after it fills), windows of 1 and 16 tokens, unaligned
    windows, a row start past some tokens' windows, and a missing page."""
    chunks = [(0, 0, 200),     # starts empty and runs past a 100-token window
              (1, 700, 130),   # long context: every tile's first pages leave the window
              (2, 37, 64),     # window larger than the context at first
              (3, 500, 40)]    # row p_start 520 inside the chunk: early tokens have empty windows
    ctx_pages = [13, 53, 7, 35]
    for w in (100, 1, 16, 33):
        _run(gpu, rep, chunks, ctx_pages, p_start=[0, 0, 0, 520], missing=[(1, 44)], seed=30 + rep + w,
             window=w, dtype=dtype, d=d)
