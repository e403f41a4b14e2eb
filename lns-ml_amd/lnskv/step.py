"""One step of one layer on the device, in the reference's call order.

lns-inference/src/engine.rs:3218-3237 allocates pages, evicts and uploads the
block tables on the host, then (engine.rs:3401-3422) appends the new token and
attends in one kernel.  A Workload carries the host side already done (pages
allocated by ensure_kv_page, CoW forks planned); StepRunner uploads its tables
once and then runs, per step:
  1. page_copy of the planned copy-on-write tail pages (if any),
  2. lnskv_append of multi-token chunks (if any),
  3. lnskv_append_decode for the decoding sequences (append 1 token + attend).
`n_layers` pools of identical geometry let a benchmark cycle through layers so
consecutive steps do not find the previous step's pages in the 256 MB
last-level cache.  capture() records one layer's step in a HIP graph, as a
serving loop would replay it, so that replays cost no host-side launch work.
"""
from __future__ import annotations

import numpy as np
import torch

from ._lib import DTYPE_Q8A
from .configs import Workload
from .device import PagedKV


def _i32(a: np.ndarray, dev) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a.astype(np.int32, copy=False)).to(dev)


class StepRunner:
    def __init__(self, w: Workload, device="cuda", n_layers: int = 1, seed: int = 0,
                 fill: bool = True, rope=None, gated: bool = False):
        """rope: a RopeTable to run the step through the fused RoPE entry
        points (q and the new K/chunk K are then taken before the rotation).
        gated: multiply the output by a per-element query gate in the same
        call (lnskv_gated_append_decode, the gated attention's last step)."""
        self.w = w
        self.rope = rope
        self.dev = torch.device(device)
        if self.dev.type == "cuda" and self.dev.index is None:
            self.dev = torch.device("cuda", torch.cuda.current_device())
        self.layers = [PagedKV(w.num_pages, w.n_kv, w.head_dim, w.dtype, self.dev) for _ in range(n_layers)]
        if fill:
            for i, pk in enumerate(self.layers):
                self.fill(pk, seed + 1000 * i)
        g = torch.Generator(device=self.dev)
        g.manual_seed(seed + 7)
        d, nkv, hq = w.head_dim, w.n_kv, w.n_heads
        self.tables = _i32(w.tables, self.dev)
        # decoding sequences get their own compact table / length rows
        self.dec_rows = w.decode_rows()
        self.n_dec = len(self.dec_rows)
        self.dec_tables = _i32(w.tables[self.dec_rows], self.dev)
        self.dec_kv_len = _i32(w.kv_len[self.dec_rows], self.dev)
        self.max_kv_len = int(w.kv_len[self.dec_rows].max()) if self.n_dec else 0
        self.q = torch.randn((self.n_dec, hq, d), generator=g, device=self.dev)
        self.k_new = torch.randn((self.n_dec, nkv, d), generator=g, device=self.dev) * w.value_scale
        self.v_new = torch.randn((self.n_dec, nkv, d), generator=g, device=self.dev) * w.value_scale
        self.out = torch.empty((self.n_dec, hq, d), device=self.dev)
        self.gate = torch.rand((self.n_dec, hq, d), generator=g, device=self.dev) if gated else None
        cs, cp = w.chunk_tokens()
        self.n_chunk_tok = len(cs)
        self.chunk_seq = _i32(cs, self.dev)
        self.chunk_pos = _i32(cp, self.dev)
        self.chunk_k = torch.randn((len(cs), nkv, d), generator=g, device=self.dev) * w.value_scale
        self.chunk_v = torch.randn((len(cs), nkv, d), generator=g, device=self.dev) * w.value_scale
        self.copy_src = _i32(np.array([c[0] for c in w.copies], np.uint32), self.dev)
        self.copy_dst = _i32(np.array([c[1] for c in w.copies], np.uint32), self.dev)
        if self.rope is not None:
            ws = self.layers[0].rope_decode_workspace_size(self.rope, max(self.n_dec, 1), hq, self.max_kv_len,
                                                           w.split)
            ws_chunk = self.layers[0].rope_append_workspace_size(self.rope, len(cs))
            self.chunk_workspace = torch.empty(max(ws_chunk, 16), dtype=torch.uint8, device=self.dev)
        else:
            ws = self.layers[0].workspace_size(max(self.n_dec, 1), hq, self.max_kv_len, w.split)
            self.chunk_workspace = None
        self.workspace = torch.zeros(max(ws, 16), dtype=torch.uint8, device=self.dev)

    def fill(self, pk: PagedKV, seed: int) -> None:
        g = torch.Generator(device=self.dev)
        g.manual_seed(seed)
        if pk.dtype == DTYPE_Q8A:
            for t in (pk.k, pk.v):
                t.copy_(torch.randint(-127, 128, t.shape, generator=g, device=self.dev, dtype=torch.int8))
            for t in (pk.ks, pk.vs):
                t.copy_(torch.rand(t.shape, generator=g, device=self.dev) * 0.02 + 0.001)
            return
        for t in (pk.k, pk.v):
            t.copy_((torch.randn(t.shape, generator=g, device=self.dev) * self.w.value_scale).to(t.dtype))

    def run(self, layer: int = 0) -> torch.Tensor:
        pk = self.layers[layer]
        w = self.w
        if len(w.copies):
            pk.page_copy(self.copy_src, self.copy_dst)
        if self.n_chunk_tok:
            if self.rope is not None:
                pk.rope_append(self.rope, self.chunk_k, self.chunk_v, self.chunk_seq, self.chunk_pos, self.tables,
                               workspace=self.chunk_workspace)
            else:
                pk.append(self.chunk_k, self.chunk_v, self.chunk_seq, self.chunk_pos, self.tables)
        if self.n_dec:
            if self.gate is not None:
                pk.gated_append_decode(self.gate, self.q, self.k_new, self.v_new, self.dec_tables, self.dec_kv_len,
                                       n_heads=w.n_heads, max_kv_len=self.max_kv_len, scale=w.scale,
                                       rope=self.rope, split=w.split, workspace=self.workspace, out=self.out)
            elif self.rope is not None:
                pk.rope_append_decode(self.rope, self.q, self.k_new, self.v_new, self.dec_tables, self.dec_kv_len,
                                      n_heads=w.n_heads, max_kv_len=self.max_kv_len, scale=w.scale,
                                      split=w.split, workspace=self.workspace, out=self.out)
            else:
                pk.append_decode(self.q, self.k_new, self.v_new, self.dec_tables, self.dec_kv_len,
                                 n_heads=w.n_heads, max_kv_len=self.max_kv_len, scale=w.scale, split=w.split,
                                 workspace=self.workspace, out=self.out)
        return self.out

    def capture(self, layer: int = 0) -> "torch.cuda.CUDAGraph":
        """One layer's step recorded in a HIP graph (run it eagerly first, so
        the library's per-device caches are filled before the capture; every
        call of the step passes its own workspace, so nothing is allocated
        while capturing)."""
        self.run(layer)
        torch.cuda.synchronize(self.dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.run(layer)
        torch.cuda.synchronize(self.dev)
        return g


class ChurnRunner:
    """c5's eviction churn step by step (configs.churn_plan): each step's
    block tables, kv_len and copy-on-write page copies differ, so every step
    uploads them (one packed host-to-device copy from pinned memory: tables,
    kv_len, copy sources, copy destinations), then runs the tail-page copies
    and the fused append + decode of every live sequence.  The pools,
    q/k_new/v_new and the layers come from a StepRunner of the c5 workload."""

    def __init__(self, runner: StepRunner, plan: list[dict], max_kv_len: int):
        self.r = runner
        self.plan = plan
        w = runner.w
        self.n, self.stride = w.tables.shape
        self.max_copies = max(1, max(len(st["copies"]) for st in plan))
        self.max_kv_len = max_kv_len
        n, sd, mc = self.n, self.stride, self.max_copies
        words = n * sd + n + 2 * mc
        self.host = torch.empty((len(plan), words), dtype=torch.int32, pin_memory=True)
        for i, st in enumerate(plan):
            row = np.zeros(words, np.int32)
            row[:n * sd] = st["tables"].astype(np.uint32).view(np.int32).ravel()
            row[n * sd:n * sd + n] = st["kv_len"]
            cps = np.array(st["copies"], np.uint32).reshape(-1, 2)
            row[n * sd + n:n * sd + n + len(cps)] = cps[:, 0].view(np.int32)
            row[n * sd + n + mc:n * sd + n + mc + len(cps)] = cps[:, 1].view(np.int32)
            self.host[i].copy_(torch.from_numpy(row))
        self.dev_buf = torch.empty(words, dtype=torch.int32, device=runner.dev)
        self.tables = self.dev_buf[:n * sd].view(n, sd)
        self.kv_len = self.dev_buf[n * sd:n * sd + n]
        self.src = self.dev_buf[n * sd + n:n * sd + n + mc]
        self.dst = self.dev_buf[n * sd + n + mc:]
        ws = runner.layers[0].workspace_size(n, w.n_heads, max_kv_len, w.split)
        self.workspace = torch.zeros(max(ws, 16), dtype=torch.uint8, device=runner.dev)

    def run(self, i: int, layer: int = 0) -> torch.Tensor:
        r, w = self.r, self.r.w
        st = self.plan[i % len(self.plan)]
        pk = r.layers[layer]
        self.dev_buf.copy_(self.host[i % len(self.plan)], non_blocking=True)
        nc = len(st["copies"])
        if nc:
            pk.page_copy(self.src[:nc], self.dst[:nc])
        return pk.append_decode(r.q, r.k_new, r.v_new, self.tables, self.kv_len, n_heads=w.n_heads,
                                max_kv_len=self.max_kv_len, scale=w.scale, split=w.split,
                                workspace=self.workspace, out=r.out)

    def step_bytes(self, i: int) -> int:
        """Algorithmic HBM bytes of churn step i (as Workload.algorithmic_bytes:
        K+V windows, append, q/out, table entries, page copies)."""
        w = self.r.w
        st = self.plan[i % len(self.plan)]
        d, nkv, hq, e = w.head_dim, w.n_kv, w.n_heads, w.elem_bytes
        L = st["kv_len"].astype(np.int64)
        per_tok = 2 * nkv * d * e
        page = 16 * nkv * d * e
        return int(L.sum() * per_tok + len(L) * (2 * nkv * d * 4 + per_tok) + len(L) * hq * d * 8 +
                   np.ceil(L / 16).sum() * 4 + len(st["copies"]) * 2 * 2 * page)
