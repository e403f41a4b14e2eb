"""Seeded synthetic workloads for the five benchmark configurations.

Integers (lengths, page orders, choices) come from SplitMix64 streams so that
the same seed gives the same tables in every process and on every machine;
floating-point values are drawn on the device by torch (seeded generator) and
are read back when the oracle needs them, so checks always use the exact
stored bits.

Configurations (head counts / head_dim / dtype / batch):
  c1  1 seq, Hq32/Hkv4/d64, f32, context 512, pool of 64 pages in a shuffled
      free list; the new token (pos 512) takes the next free page.
  c2  Llama-3-8B layer: Hq32/Hkv8/d128, f16, B=32, context U{512..4096},
      pool 16384 pages in a shuffled free list, values N(0,1)*0.5.
  c3  long context: Hq32/Hkv8/d128, f16, B=4 x 32768 tokens, split-K 512.
  c4  chunked prefill + decode: 16 sequences append a 256-token chunk at
      length 16k+o (o in 0..15), 48 sequences decode at U{1024..8192}.
  c5  eviction churn: B=128 at U{256..8192}; free 32 sequences, give their
      pages to 32 new sequences, copy-on-write fork 8; 136 sequences then
      append one token and decode.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from ._lib import DTYPE_F16, DTYPE_F32, DTYPE_Q8A, NO_PAGE, PAGE_SIZE
from .host import BlockTables, PagePool

MASK64 = (1 << 64) - 1


class SplitMix64:
    """SplitMix64 stream for (seed, stream id)."""

    def __init__(self, seed: int, stream: int):
        self.state = (seed * 0x9E3779B97F4A7C15 + (stream + 1) * 0xD1B54A32D192ED03) & MASK64

    def next_u64(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & MASK64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
        return z ^ (z >> 31)

    def randint(self, lo: int, hi: int) -> int:
        """Uniform integer in [lo, hi] (modulo bias < 2^-40 for these ranges)."""
        return lo + self.next_u64() % (hi - lo + 1)

    def shuffle(self, items: list) -> list:
        """Fisher-Yates, in place; returns items."""
        for i in range(len(items) - 1, 0, -1):
            j = self.next_u64() % (i + 1)
            items[i], items[j] = items[j], items[i]
        return items


# stream ids
S_LEN, S_PERM, S_CHUNK, S_CHURN, S_FORK, S_NEWLEN = range(6)


@dataclass
class Workload:
    """One step of one layer: which tokens are appended where, and which
    sequences run decode attention, over host-built block tables."""

    name: str
    n_heads: int
    n_kv: int
    head_dim: int
    dtype: int
    num_pages: int
    ctx_len: np.ndarray          # int32 [n_seq] tokens present before the step
    n_new: np.ndarray            # int32 [n_seq] tokens appended this step
    decode: np.ndarray           # bool  [n_seq] runs decode attention
    tables: np.ndarray           # uint32 [n_seq][stride]
    value_scale: float = 1.0
    split: int = 0               # split-K tokens (0 = library choice)
    seed: int = 0
    copies: list = field(default_factory=list)  # (src, dst) page copies of the step
    pool: PagePool | None = None
    bt: BlockTables | None = None
    info: dict = field(default_factory=dict)  # config-specific facts (c5: churn)

    @property
    def n_seq(self) -> int:
        return len(self.ctx_len)

    @property
    def rep(self) -> int:
        return self.n_heads // self.n_kv

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    @property
    def elem_bytes(self) -> int:
        return {0: 4, 1: 2, 2: 1}[self.dtype]

    @property
    def kv_len(self) -> np.ndarray:
        return (self.ctx_len + self.n_new).astype(np.int32)

    def decode_rows(self) -> np.ndarray:
        return np.nonzero(self.decode)[0].astype(np.int32)

    def chunk_tokens(self):
        """(tok_seq, tok_pos) of the multi-token appends (sequences with
        n_new > 1 or that do not decode)."""
        seqs, poss = [], []
        for s in range(self.n_seq):
            if self.decode[s] and self.n_new[s] == 1:
                continue
            for p in range(int(self.ctx_len[s]), int(self.ctx_len[s] + self.n_new[s])):
                seqs.append(s)
                poss.append(p)
        return np.asarray(seqs, np.int32), np.asarray(poss, np.int32)

    def algorithmic_bytes(self) -> dict:
        """Bytes one step must move at minimum (the roofline numerator):
        K+V read over each decode window (new token included), the append's
        f32 read and page write, q read and out write, block-table entries,
        and page copies (read + write of K and V)."""
        d, nkv, hq, e = self.head_dim, self.n_kv, self.n_heads, self.elem_bytes
        per_tok_kv = 2 * nkv * d * e + (2 * nkv * 4 if self.dtype == 2 else 0)
        dec = self.decode
        L = self.kv_len.astype(np.int64)
        kv_read = int((L[dec]).sum()) * per_tok_kv
        n_app = int(self.n_new.sum())
        append = n_app * (2 * nkv * d * 4 + per_tok_kv)
        qo = int(dec.sum()) * hq * d * 8
        table = int(np.ceil(L[dec] / PAGE_SIZE).sum()) * 4
        page_bytes = PAGE_SIZE * nkv * d * e + (PAGE_SIZE * nkv * 4 if self.dtype == 2 else 0)
        copy = len(self.copies) * 2 * 2 * page_bytes
        total = kv_read + append + qo + table + copy
        return {"kv_read": kv_read, "append": append, "q_out": qo, "table": table,
                "copy": copy, "total": total}


def _shuffled_pool(capacity: int, rng: SplitMix64) -> tuple[PagePool, list]:
    """PagePool whose FIFO free list is a seeded permutation of 0..capacity:
    allocate every page, then free them in permuted order (push_back)."""
    order = rng.shuffle(list(range(capacity)))
    pool = PagePool(capacity)
    for _ in range(capacity):
        pool.alloc()
    for p in order:
        pool.free_page(p)
    return pool, order


def _alloc_rows(bt: BlockTables, pool: PagePool, rows, lengths) -> None:
    """ensure_kv_page for every page of tokens [0, length) of each row."""
    for s, L in zip(rows, lengths):
        for lp in range((int(L) + PAGE_SIZE - 1) // PAGE_SIZE):
            bt.ensure_kv_page(pool, int(s), lp * PAGE_SIZE)


def _finish(w: Workload) -> Workload:
    w.tables = w.bt.array()
    return w


def make_c1(seed: int = 0) -> Workload:
    rng = SplitMix64(seed, S_PERM)
    pool, _ = _shuffled_pool(64, rng)
    ctx = np.array([512], np.int32)
    bt = BlockTables(1, 64)
    _alloc_rows(bt, pool, [0], ctx + 1)
    w = Workload("c1", 32, 4, 64, DTYPE_F32, 64, ctx, np.ones(1, np.int32), np.ones(1, bool),
                 None, value_scale=1.0, seed=seed, pool=pool, bt=bt)
    return _finish(w)


def make_c2(seed: int = 0, n_seq: int = 32, lo: int = 512, hi: int = 4096,
            num_pages: int = 16384, dtype: int = DTYPE_F16) -> Workload:
    """dtype: the page type (f16 as the config states; Q8A, the reference's
    own paged type, or f32 to run the same shapes through those paths)."""
    rl = SplitMix64(seed, S_LEN)
    ctx = np.array([rl.randint(lo, hi) for _ in range(n_seq)], np.int32)
    pool, _ = _shuffled_pool(num_pages, SplitMix64(seed, S_PERM))
    stride = (hi + 1 + PAGE_SIZE - 1) // PAGE_SIZE
    bt = BlockTables(n_seq, stride)
    _alloc_rows(bt, pool, range(n_seq), ctx + 1)
    w = Workload("c2", 32, 8, 128, dtype, num_pages, ctx, np.ones(n_seq, np.int32),
                 np.ones(n_seq, bool), None, value_scale=0.5, seed=seed, pool=pool, bt=bt)
    return _finish(w)


def make_c3(seed: int = 0, n_seq: int = 4, length: int = 32768, split: int = 512) -> Workload:
    pages_per = (length + 1 + PAGE_SIZE - 1) // PAGE_SIZE
    num_pages = n_seq * pages_per
    pool, _ = _shuffled_pool(num_pages, SplitMix64(seed, S_PERM))
    ctx = np.full(n_seq, length, np.int32)
    bt = BlockTables(n_seq, pages_per)
    _alloc_rows(bt, pool, range(n_seq), ctx + 1)
    w = Workload("c3", 32, 8, 128, DTYPE_F16, num_pages, ctx, np.ones(n_seq, np.int32),
                 np.ones(n_seq, bool), None, value_scale=1.0, split=split, seed=seed, pool=pool, bt=bt)
    return _finish(w)


def make_c4(seed: int = 0, n_chunk: int = 16, chunk: int = 256, n_dec: int = 48,
            lo: int = 1024, hi: int = 8192) -> Workload:
    rc = SplitMix64(seed, S_CHUNK)
    chunk_ctx = [16 * rc.randint(0, 63) + rc.randint(0, 15) for _ in range(n_chunk)]
    rl = SplitMix64(seed, S_LEN)
    dec_ctx = [rl.randint(lo, hi) for _ in range(n_dec)]
    ctx = np.array(chunk_ctx + dec_ctx, np.int32)
    n_new = np.array([chunk] * n_chunk + [1] * n_dec, np.int32)
    decode = np.array([False] * n_chunk + [True] * n_dec)
    need = int(sum((int(c) + int(n) + PAGE_SIZE - 1) // PAGE_SIZE for c, n in zip(ctx, n_new)))
    num_pages = 1 << max(10, math.ceil(math.log2(need + 1)))
    pool, _ = _shuffled_pool(num_pages, SplitMix64(seed, S_PERM))
    stride = (max(hi + 1, 16 * 63 + 15 + chunk) + PAGE_SIZE - 1) // PAGE_SIZE
    bt = BlockTables(len(ctx), stride)
    _alloc_rows(bt, pool, range(len(ctx)), ctx + n_new)
    w = Workload("c4", 32, 8, 128, DTYPE_F16, num_pages, ctx, n_new, decode, None,
                 value_scale=1.0, seed=seed, pool=pool, bt=bt)
    return _finish(w)


def make_c5(seed: int = 0, n_seq: int = 128, lo: int = 256, hi: int = 8192, n_free: int = 32,
            n_fork: int = 8, spare: int = 64, extra_pages: int = 0) -> Workload:
    """State after one churn step.  Rows 0..n_seq-1 hold the original batch; the
    n_free freed rows are refilled by new sequences (seeded lengths); rows
    n_seq..n_seq+n_fork-1 are copy-on-write children of n_fork surviving
    sequences.  The step's page copies are the children's tail pages."""
    rl = SplitMix64(seed, S_LEN)
    ctx0 = [rl.randint(lo, hi) for _ in range(n_seq)]
    total = n_seq + n_fork
    stride = (hi + 1 + PAGE_SIZE - 1) // PAGE_SIZE + extra_pages  # extra: room for later churn steps
    # Draw every choice first so the pool can be sized tightly: the new
    # sequences then take the freed pages once the few spare ones run out.
    freed = sorted(SplitMix64(seed, S_CHURN).shuffle(list(range(n_seq)))[:n_free])
    rn = SplitMix64(seed, S_NEWLEN)
    new_len = {s: rn.randint(lo, hi) for s in freed}
    survivors = [s for s in range(n_seq) if s not in set(freed)]
    parents = SplitMix64(seed, S_FORK).shuffle(list(survivors))[:n_fork]
    pages = lambda n: (n + PAGE_SIZE - 1) // PAGE_SIZE  # noqa: E731
    need0 = sum(pages(c) for c in ctx0)
    final = [new_len.get(s, ctx0[s]) for s in range(n_seq)] + [ctx0[p] for p in parents]
    need1 = sum(pages(c + 1) for c in final)
    num_pages = max(need0, need1) + spare
    pool, _ = _shuffled_pool(num_pages, SplitMix64(seed, S_PERM))
    bt = BlockTables(total, stride)
    _alloc_rows(bt, pool, range(n_seq), ctx0)
    before = bt.array()
    freed_pages = before[freed][before[freed] != NO_PAGE]
    for s in freed:
        bt.free_sequence(pool, s)
    ctx = list(ctx0)
    for s in freed:
        ctx[s] = new_len[s]
    _alloc_rows(bt, pool, freed, [ctx[s] for s in freed])
    copies = []
    for i, p in enumerate(parents):
        child = n_seq + i
        cp = bt.fork_sequence(pool, p, child, ctx[p])
        if cp is not None:
            copies.append(cp)
        ctx.append(ctx[p])
    ctx = np.array(ctx, np.int32)
    # The appended token of a sequence whose last page is shared needs a page
    # of its own: a parent's tail page is still shared only when its length is
    # a multiple of 16, in which case the new token opens a fresh page anyway.
    _alloc_rows(bt, pool, range(total), ctx + 1)
    w = Workload("c5", 32, 8, 128, DTYPE_F16, num_pages, ctx, np.ones(total, np.int32),
                 np.ones(total, bool), None, value_scale=1.0, seed=seed, copies=copies,
                 pool=pool, bt=bt, info={"freed_rows": freed, "freed_pages": freed_pages,
                                         "parents": parents})
    return _finish(w)


def churn_plan(w: Workload, n_steps: int, seed: int = 1, n_free: int = 32, lo: int = 256,
               hi: int = 8192) -> list[dict]:
    """c5's churn continued for n_steps more steps from the state of make_c5,
    on its PagePool and BlockTables.  Step i: the previous step's copy-on-write
    children are freed; n_free seeded sequences of the base batch are freed
    and their rows refilled by new sequences of seeded lengths (ensure_kv_page
    over their pages, which come from the FIFO free list, the freed pages
    among them); as many children are forked from seeded survivors (full
    pages shared by refcount, the tail page copied); every live sequence gets
    the page of its appended token.  Each step records what its device step
    needs: the block tables, kv_len (the appended token included) and the
    (src, dst) page copies.  Lengths grow by one per step."""
    n_fork = len(w.info["parents"])
    n_seq = w.n_seq - n_fork
    pool, bt = w.pool, w.bt
    L = [int(x) for x in w.kv_len]  # after make_c5's step
    if max(L) + n_steps > bt.max_pages * PAGE_SIZE:
        raise ValueError(f"{n_steps} churn steps need rows of {max(L) + n_steps} positions; the table holds "
                         f"{bt.max_pages * PAGE_SIZE} (make_c5 extra_pages)")
    plan = []
    for i in range(n_steps):
        rs = SplitMix64(seed + 97 * i, S_CHURN)
        for c in range(n_seq, n_seq + n_fork):
            bt.free_sequence(pool, c)
        freed = sorted(rs.shuffle(list(range(n_seq)))[:n_free])
        rn = SplitMix64(seed + 97 * i, S_NEWLEN)
        for s in freed:
            bt.free_sequence(pool, s)
        for s in freed:
            L[s] = rn.randint(lo, hi)
        _alloc_rows(bt, pool, freed, [L[s] for s in freed])
        keep = set(freed)
        survivors = [s for s in range(n_seq) if s not in keep]
        parents = SplitMix64(seed + 97 * i, S_FORK).shuffle(survivors)[:n_fork]
        copies = []
        for j, par in enumerate(parents):
            child = n_seq + j
            cp = bt.fork_sequence(pool, par, child, L[par])
            if cp is not None:
                copies.append(cp)
            L[child] = L[par]
        _alloc_rows(bt, pool, range(n_seq + n_fork), [x + 1 for x in L])
        plan.append({"tables": bt.array(), "kv_len": np.array([x + 1 for x in L], np.int32),
                     "copies": copies, "freed": freed, "parents": parents})
        L = [x + 1 for x in L]
    return plan


def make_qwen35(seed: int = 0, n_seq: int = 32, lo: int = 512, hi: int = 4096, num_pages: int = 16384,
                dtype: int = DTYPE_Q8A) -> Workload:
    """lns-ml's own full-attention layer (Qwen3.5, model_config.rs:563-593):
    16 query heads, 4 kv heads, head_dim 256, on the engine's Q8A pages
    (engine.rs:731-734), with c2's batch: n_seq sequences at seeded contexts
    U[lo, hi], pages from a shuffled free list.  The step it is measured with
    turns q and k by RoPE (rotary 64 of 256, theta 1e7) and multiplies the
    output by the query gate (engine.rs:1700-1720, 3424-3431)."""
    rl = SplitMix64(seed, S_LEN)
    ctx = np.array([rl.randint(lo, hi) for _ in range(n_seq)], np.int32)
    pool, _ = _shuffled_pool(num_pages, SplitMix64(seed, S_PERM))
    stride = (hi + 1 + PAGE_SIZE - 1) // PAGE_SIZE
    bt = BlockTables(n_seq, stride)
    _alloc_rows(bt, pool, range(n_seq), ctx + 1)
    w = Workload("qwen35", 16, 4, 256, dtype, num_pages, ctx, np.ones(n_seq, np.int32),
                 np.ones(n_seq, bool), None, value_scale=0.5, seed=seed, pool=pool, bt=bt)
    return _finish(w)


MAKERS = {"c1": make_c1, "c2": make_c2, "c3": make_c3, "c4": make_c4, "c5": make_c5, "qwen35": make_qwen35}


def make(name: str, **kw) -> Workload:
    return MAKERS[name](**kw)


def used_pages(tables: np.ndarray) -> np.ndarray:
    t = tables.ravel()
    return np.unique(t[t != NO_PAGE])
