#!/usr/bin/env python3
"""Benchmark: paged decode attention + append on one MI355X.

One step = one layer's work for the whole batch of the chosen configuration
(default c2, the Llama-3-8B-shaped B=32 ragged batch): page copies and chunk
appends where the config has them, then the fused 1-token append + paged
decode attention (one lnskv_append_decode call: the stream-K decode kernel and
its combine kernel for c2).  Inputs are resident in HBM before timing starts.
Steps cycle through --layers independent pools (4 by default, 4 GB for c2) so
that no step finds the previous step's pages in the 256 MB last-level cache,
as in a real multi-layer decode.

Prints ONE JSON line.  `value` is achieved GB/s = algorithmic bytes per step
(K+V of every attended token, append read+write, q/out, block-table entries,
page copies) / wall time per step; `roofline` divides the same bytes by the
HIP-event duration of the step's kernels, measured live on their stream;
`cpu_baseline` times the oracle's reference-order CPU scan (append + online
softmax per query head, OpenMP over sequence x kv head) on this host.
`roofline.traffic` is the HBM bytes per step that rocprofv3's FETCH_SIZE and
WRITE_SIZE counters gave for the same workload, scaled by what they read for
a plain copy of known size; it is read from profiles/<config>_traffic.json
(profiles/<config>_q8a_traffic.json for Q8A pages; written from those counter
runs, with the commit whose build they measured) and is null when that file is
absent.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "lns-ml_amd"))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "paged decode-attn+append µs/step and achieved HBM GB/s (% of peak), 8B-shape b=32"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    p.add_argument("--layers", type=int, default=4, help="pools cycled across steps (defeats the LLC)")
    p.add_argument("--split", type=int, default=-1, help="split-K tokens (-1 = the config's choice)")
    p.add_argument("--kv-dtype", default="config", choices=["config", "f32", "f16", "q8a"],
                   help="page type of c2 (config: f16 as the config states; q8a is the reference's own paged "
                        "type, f32 the wide one)")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline sample budget (0 = skip)")
    p.add_argument("--cpu-threads", type=int, default=0, help="0 = all cores the process may use")
    p.add_argument("--copy-mb", type=int, default=1024,
                   help="size of the device-to-device copy that measures the copy ceiling (0 = skip)")
    p.add_argument("--graph", type=int, default=0,
                   help="1: replay each layer's step from a captured HIP graph (no per-step host launch work); "
                        "0: launch eagerly from Python")
    p.add_argument("--rope", type=int, default=0,
                   help="1: the step goes through the fused RoPE entry points (Llama-3.1 table, rotary = head_dim)")
    p.add_argument("--pattern-reps", type=int, default=40,
                   help="launches of the load probe over the step's decode pages (0 = skip)")
    p.add_argument("--oproj-reps", type=int, default=100,
                   help="launches of the o_proj Q4L GEMV-accumulate at the config's shape (0 = skip)")
    p.add_argument("--prefill-reps", type=int, default=20,
                   help="launches of chunked-prefill attention over the config's pages (0 = skip)")
    p.add_argument("--extras", type=int, default=1,
                   help="c2 only: also measure c1/c3/c4/c5, c2 on Q8A pages, the reference's one-sequence call and "
                        "the block-table upload (0 = skip)")
    p.add_argument("--copy-only", action="store_true",
                   help="run only the plain copy (the calibration kernel for HBM byte counters)")
    p.add_argument("--reference-call-only", action="store_true",
                   help="run only the reference's one-sequence call (lnskv_attention_paged, Q8A, pos 4095)")
    p.add_argument("--qwen35-only", action="store_true",
                   help="run only lns-ml's Qwen3.5 attention shape (Hq16/Hkv4/d256, Q8A, RoPE 64, gated), with "
                        "--prefill-reps chunked-prefill launches")
    return p.parse_args()


def copy_ceiling(dev, mb: int, reps: int = 20) -> dict:
    """Same-run HBM ceiling: a plain device-to-device copy of `mb` MiB (reads
    and writes mb MiB each), timed with HIP events; bytes moved = 2 * size."""
    import torch

    n = mb * (1 << 20) // 4
    a = torch.empty(n, dtype=torch.float32, device=dev).uniform_()
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        b.copy_(a)
    e.record()
    torch.cuda.synchronize()
    dt = s.elapsed_time(e) / 1e3 / reps
    return {"bytes_per_copy": 2 * n * 4, "gb_per_s": round(2 * n * 4 / dt / 1e9, 1)}


def read_ceiling(dev, mib: int = 1024, reps: int = 10) -> dict:
    """Same-run plain read ceiling: lnskv_read_stream over one buffer of `mib`
    MiB (1 GiB by default, four times the 256 MB last-level cache, so every
    launch reads from HBM), front to back with 16-byte loads; the best of a
    sweep of loads in flight per thread (4, 8, 16) and workgroups per CU
    (2, 4, 8), each timed with HIP events over `reps` launches."""
    import ctypes as C

    import torch

    from lnskv._lib import check, lib

    nbytes = mib << 20
    buf = torch.empty(nbytes // 4, dtype=torch.int32, device=dev).random_()
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    sweep = {}
    for u in (4, 8, 16):
        for bpc in (2, 4, 8):
            def launch():
                check(lib().lnskv_read_stream(buf.data_ptr(), nbytes, u, bpc, sink.data_ptr(), stream))
            for _ in range(2):
                launch()
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(reps):
                launch()
            e.record()
            torch.cuda.synchronize()
            dt = s.elapsed_time(e) / 1e3 / reps
            sweep[f"{u}x{bpc}"] = round(nbytes / dt / 1e9, 1)
    best = max(sweep, key=sweep.get)
    return {"bytes_per_launch": nbytes, "gb_per_s": sweep[best], "best": best,
            "sweep_gbs": sweep, "note": "loads in flight per thread x workgroups of 256 threads per CU"}


def sk_waves(w, runner) -> int:
    """The stream-K decode's wave count for this workload, read back from the
    library's workspace size (header + per wave 2 * rep partial rows of
    (acc[d], m, l) and a 16-byte descriptor)."""
    ws = runner.layers[0].workspace_size(runner.n_dec, w.n_heads, runner.max_kv_len, 0)
    per_wave = 2 * w.rep * (w.head_dim + 2) * 4 + 16
    return (ws - 4096) // per_wave


def pattern_ceiling(w, runner, dev, reps: int) -> dict | None:
    """Load ceiling of the step's decode page pattern, timed live with HIP
    events: lnskv_read_units over the same (page, kv head) units as the
    decode, in its order ((sequence, kv head, page)) and its stream-K wave
    split (CUs x 4 waves), cycling the same layers' pools (no cache reuse
    between launches).  Bytes per launch: units x 2 pools x 16 rows x 256 B
    (f16 d128 / f32 d64), or x (128 B + a 4-byte scale) for Q8A d128 pages,
    whose decode runs 8 waves per CU.  None for shapes the probe does not
    read."""
    import ctypes as C

    import numpy as np
    import torch

    from lnskv._lib import check, lib

    row_bytes = w.head_dim * {0: 4, 1: 2, 2: 1}[w.dtype]
    q8 = w.dtype == 2
    if reps <= 0 or runner.n_dec == 0 or not (row_bytes in (256, 512) and not q8 or row_bytes in (128, 256) and q8):
        return None
    pages, kvhs = [], []
    for s in runner.dec_rows:
        npg = (int(w.kv_len[s]) + 15) // 16  # window from position 0, including the appended token
        row = np.asarray(w.tables[s][:npg], dtype=np.uint32)
        for k in range(w.n_kv):
            pages.append(row)
            kvhs.append(np.full(npg, k, dtype=np.int32))
    unit_page = np.concatenate(pages)
    unit_kvh = np.concatenate(kvhs)
    n_units = len(unit_page)
    waves = sk_waves(w, runner)
    chunk = max(4, -(-n_units // waves))
    start = np.minimum(np.arange(waves + 1, dtype=np.int64) * chunk, n_units).astype(np.int32)
    d_page = torch.from_numpy(unit_page.view(np.int32)).to(dev)
    d_kvh = torch.from_numpy(unit_kvh).to(dev)
    d_start = torch.from_numpy(start).to(dev)
    sink = torch.empty(waves * 64, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)

    def launch(i):
        pk = runner.layers[i % len(runner.layers)]
        check(lib().lnskv_read_units(C.byref(pk.desc), d_page.data_ptr(), d_kvh.data_ptr(), d_start.data_ptr(),
                                     waves, sink.data_ptr(), C.c_void_p(stream.cuda_stream)))

    for i in range(2 * len(runner.layers)):
        launch(i)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for i in range(reps):
        launch(i)
    e.record(stream)
    torch.cuda.synchronize()
    dt = s.elapsed_time(e) / 1e3 / reps
    nbytes = n_units * 2 * 16 * (row_bytes + (4 if q8 else 0))
    return {"bytes_per_launch": int(nbytes), "us_per_launch": round(dt * 1e6, 2),
            "gb_per_s": round(nbytes / dt / 1e9, 1), "waves": int(waves), "units": int(n_units)}


def oproj_measure(w, runner, dev, reps: int) -> dict | None:
    """The step after the path: o_proj, y += W_o attn_out over Q4_L weights
    (lnskv_q4l_gemv_accumulate), at the config's shape: W_o is
    (n_heads*head_dim) x (n_heads*head_dim) (Llama-3-8B: 4096 x 4096), one
    vector per decoding sequence.  Random Q4L blocks; 32 weight copies are
    cycled (300 MB for c2, more than the 256 MB MALL).  HIP events around
    `reps` launches; bytes per launch: the weight blocks + x + y read and
    written.  Beside it, the reference's order of work (q4l_gemv_accumulate
    once per sequence, engine.rs:3433-3446): the same vectors one call each."""
    import numpy as np
    import torch

    from lnskv.device import Q4LMatrix

    dim = w.n_heads * w.head_dim
    if reps <= 0 or runner.n_dec == 0 or dim % 256 != 0:
        return None
    rng = np.random.default_rng(5)
    nb = dim * dim // 256
    disk = rng.integers(0, 256, (nb, 134), dtype=np.uint8)
    g = np.exp2(rng.uniform(-12, -2, nb)).astype(np.float16)
    disk[:, 0:2] = g.view(np.uint8).reshape(nb, 2)
    mats = [Q4LMatrix(disk.reshape(-1), dim, dim, dev) for _ in range(32)]
    n_vec = runner.n_dec
    x = torch.randn(n_vec, dim, device=dev)
    y = torch.zeros(n_vec, dim, device=dev)
    ws = torch.zeros(max(mats[0].workspace_size(n_vec), 16), dtype=torch.uint8, device=dev)  # counts start at zero
    for i in range(len(mats)):
        mats[i].gemv_accumulate(x, y, ws)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(reps):
        mats[i % len(mats)].gemv_accumulate(x, y, ws)
    e.record()
    torch.cuda.synchronize()
    dt = s.elapsed_time(e) / 1e3 / reps
    # the reference's order: one call per sequence (one vector each)
    per_seq_reps = max(reps // 10, 4)
    s.record()
    for i in range(per_seq_reps):
        for v in range(n_vec):
            mats[(i * n_vec + v) % len(mats)].gemv_accumulate(x[v:v + 1], y[v:v + 1], ws)
    e.record()
    torch.cuda.synchronize()
    dt_seq = s.elapsed_time(e) / 1e3 / per_seq_reps
    nbytes = nb * 144 + n_vec * dim * 4 * 3
    del mats
    return {"shape": f"{dim} x {dim} Q4L, {n_vec} vectors", "us_per_launch": round(dt * 1e6, 2),
            "bytes_per_launch": int(nbytes), "gb_per_s": round(nbytes / dt / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / dt / 1e9 / HBM_PEAK_GBS, 4),
            "us_one_call_per_sequence": round(dt_seq * 1e6, 2),
            "note": "us_one_call_per_sequence: the same vectors in the reference's order, "
                    f"{n_vec} calls of one vector (weights cycled as above)"}


def prefill_measure(w, runner, dev, reps: int, chunk: int = 256) -> dict | None:
    """Chunked-prefill attention (lnskv_prefill_attention) over the config's
    pages.  Configs with prompt chunks (c4) use those chunks (every step
    appends their K/V); the others take the last `chunk` tokens of every
    decoding sequence as its prompt chunk (their K/V are in the pages).  Each
    query attends [0, its position].  Algorithmic work: 4 * head_dim flops
    per (query, head, attended token) (q.k and p.v); the kernel runs q and p
    as f16 hi and lo parts, twice that on the matrix cores.  Layers cycled,
    HIP events around `reps` launches.  Up to 8192 queries, the same queries
    also go through lnskv_decode as one row each (kv_len = position + 1: the
    reference's token-at-a-time order of work, batched into one launch), and
    the two results are compared."""
    import numpy as np
    import torch

    if reps <= 0 or w.dtype not in (1, 2) or w.head_dim not in (128, 256):
        return None
    cs, cp = w.chunk_tokens()
    desc, tok = [], 0
    if len(cs):
        i = 0
        while i < len(cs):
            j = i
            while j + 1 < len(cs) and cs[j + 1] == cs[i] and cp[j + 1] == cp[j] + 1:
                j += 1
            desc.append((int(cs[i]), int(cp[i]), j - i + 1, i))
            i = j + 1
        tok = len(cs)
        what = f"the config's {len(desc)} prompt chunks ({tok} queries)"
    else:
        if runner.n_dec == 0:
            return None
        for s in runner.dec_rows:
            L = int(w.kv_len[s])
            ln = min(chunk, L)
            desc.append((int(s), L - ln, ln, tok))
            tok += ln
        what = f"last {chunk} tokens of each of {len(desc)} sequences ({tok} queries)"
    chunks = torch.tensor(desc, dtype=torch.int32, device=dev)
    q = torch.randn(tok, w.n_heads, w.head_dim, device=dev)
    out = torch.empty_like(q)
    flops = sum(4 * w.head_dim * w.n_heads * (p0 + i + 1) for (_, p0, ln, _) in desc for i in range(ln))

    def launch(i):
        runner.layers[i % len(runner.layers)].prefill_attention(q, chunks, runner.tables, n_heads=w.n_heads,
                                                               scale=w.scale, out=out)

    def timed(fn):
        for i in range(2 * len(runner.layers)):
            fn(i)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(reps):
            fn(i)
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / 1e3 / reps

    dt = timed(launch)
    res = {"shape": f"{what}, Hq{w.n_heads}/Hkv{w.n_kv}/d{w.head_dim} {('f32', 'f16', 'Q8A')[w.dtype]} pages",
           "us_per_launch": round(dt * 1e6, 1), "gflop": round(flops / 1e9, 2),
           "tflop_per_s": round(flops / dt / 1e12, 1),
           "frac_of_f16_mfma_peak": round(flops / dt / 1e12 / 2500.0, 4),
           "mfma_tflop_per_s_with_hi_lo": round(2 * flops / dt / 1e12, 1)}
    if not len(cs):  # the queries' rows and positions, from the chunks
        cs = np.concatenate([np.full(ln, r, np.int64) for (r, _, ln, _) in desc])
        cp = np.concatenate([np.arange(p0, p0 + ln) for (_, p0, ln, _) in desc])
    if tok <= 8192:
        # the same queries as single-token decode rows of one lnskv_decode call
        tables = runner.tables[torch.from_numpy(cs.astype(np.int64)).to(dev)].contiguous()
        kv_len = torch.from_numpy((cp + 1).astype(np.int32)).to(dev)
        pk0 = runner.layers[0]
        ws = torch.zeros(max(pk0.workspace_size(tok, w.n_heads, int(cp.max()) + 1, 0), 4), dtype=torch.uint8,
                         device=dev)
        out_d = torch.empty_like(q)

        def launch_d(i):
            runner.layers[i % len(runner.layers)].decode(q, tables, kv_len, n_heads=w.n_heads,
                                                         max_kv_len=int(cp.max()) + 1, scale=w.scale,
                                                         workspace=ws, out=out_d)

        dt_d = timed(launch_d)
        launch(0)
        launch_d(0)
        torch.cuda.synchronize()
        diff = float((out - out_d).abs().max() / out_d.abs().max())
        res.update({"decode_rows_us_per_launch": round(dt_d * 1e6, 1),
                    "prefill_speedup_vs_decode_rows": round(dt_d / dt, 2),
                    "max_abs_diff_vs_decode_rows_rel": diff})
    return res


def step_distribution(step, stream, n: int) -> dict:
    """Per-step HIP-event durations of n more steps (an event pair around
    each step, on the kernels' stream): median and spread, in µs."""
    import numpy as np
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        step(i)
        b.record(stream)
    torch.cuda.synchronize()
    t = np.array([a.elapsed_time(b) * 1e3 for a, b in evs])
    return {"steps": n, "median": round(float(np.median(t)), 2), "p10": round(float(np.percentile(t, 10)), 2),
            "p90": round(float(np.percentile(t, 90)), 2), "min": round(float(t.min()), 2)}


def timed_steps(step, stream, steps: int, warmup: int) -> tuple[float, float]:
    """(event mean, wall mean) seconds per step over exactly `steps` steps
    after `warmup`, one event pair around all of them."""
    import torch

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        step(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps, (time.perf_counter() - t0) / steps


def config_measure(name: str, dev, steps: int, layers: int = 2, kv_dtype: int | None = None,
                   pattern_reps: int = 0, prefill_reps: int = 0, rope: bool = False) -> dict:
    """One configuration's step (its own workload and pools, `layers` of them
    cycled): event mean over `steps` steps, median of per-step events,
    algorithmic GB/s and fraction of 8 TB/s; optionally the load ceiling of
    its page pattern and chunked prefill over its pages.  rope: the step
    through the fused RoPE entry point (the --rope table).  c5 adds the
    full-copy fork variant."""
    import torch

    from lnskv.configs import make
    from lnskv.step import StepRunner

    w = make(name) if kv_dtype is None else make(name, dtype=kv_dtype)
    table = None
    if rope:
        from lnskv.device import RopeTable

        table = RopeTable(w.head_dim, 500000.0, 2, (8.0, 8192.0, 1.0, 4.0), device=dev)
    runner = StepRunner(w, dev, n_layers=layers, seed=1, rope=table)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    step = lambda i: runner.run(i % layers)  # noqa: E731
    ev, wall = timed_steps(step, stream, steps, 10)
    dist = step_distribution(step, stream, min(steps, 200))
    nb = w.algorithmic_bytes()["total"]
    res = {"us_per_step_events": round(ev * 1e6, 2), "us_per_step_wall": round(wall * 1e6, 2),
           "us_per_step_median": dist["median"], "algorithmic_bytes": int(nb),
           "gb_per_s": round(nb / ev / 1e9, 1), "frac_of_hbm_peak": round(nb / ev / 1e9 / HBM_PEAK_GBS, 4)}
    if pattern_reps > 0:
        pc = pattern_ceiling(w, runner, dev, pattern_reps)
        if pc:
            res["pattern_ceiling_us"] = pc["us_per_launch"]
            res["frac_of_pattern_ceiling"] = round(pc["us_per_launch"] / (ev * 1e6), 4)
    traffic = measured_traffic(name, w.dtype, rope)
    if traffic:
        res["traffic_bytes"] = traffic["bytes"]
        res["traffic_over_algorithmic"] = traffic["over_algorithmic"]
        res["traffic_measured_at_commit"] = traffic["measured_at_commit"]
    if prefill_reps > 0:
        res["chunked_prefill_attention"] = prefill_measure(w, runner, dev, prefill_reps)
    if name == "c5" and w.info.get("parents"):
        res["full_copy_fork"] = full_copy_fork(w, runner, dev)
    del runner
    torch.cuda.empty_cache()
    return res


def c5_churn_measure(dev, steps: int, n_plan: int = 20, layers: int = 2) -> dict:
    """c5 with churn in every timed step: each step frees the previous step's
    forks and 32 sequences, refills their rows with new sequences on the freed
    pages, forks 8 survivors (copy-on-write: tail pages copied) and appends +
    attends over all 136 live sequences.  The host bookkeeping (PagePool and
    BlockTables through the C ABI) is done for n_plan steps ahead of the timed
    loop (its time per step is reported); inside each timed step the changed
    tables, kv_len and copy lists go to the device (one host-to-device copy
    from pinned memory), then the page copies and the fused append + decode
    run.  Event mean over `steps` steps cycling the plan and the layers."""
    import time

    import torch

    from lnskv.configs import churn_plan, make_c5
    from lnskv.step import ChurnRunner, StepRunner

    w = make_c5(spare=4096, extra_pages=2)
    runner = StepRunner(w, dev, n_layers=layers, seed=1)
    t0 = time.perf_counter()
    plan = churn_plan(w, n_plan)
    host_s = (time.perf_counter() - t0) / n_plan
    cr = ChurnRunner(runner, plan, max_kv_len=w.tables.shape[1] * 16)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    step = lambda i: cr.run(i, i % layers)  # noqa: E731
    ev, wall = timed_steps(step, stream, steps, 10)
    nb = sum(cr.step_bytes(i) for i in range(steps)) / steps
    res = {"us_per_step_events": round(ev * 1e6, 2), "us_per_step_wall": round(wall * 1e6, 2),
           "algorithmic_bytes_mean": int(nb), "gb_per_s": round(nb / ev / 1e9, 1),
           "frac_of_hbm_peak": round(nb / ev / 1e9 / HBM_PEAK_GBS, 4),
           "upload_bytes_per_step": int(cr.host.shape[1] * 4),
           "page_copies_per_step_mean": round(sum(len(p["copies"]) for p in plan) / n_plan, 2),
           "host_bookkeeping_ms_per_step": round(host_s * 1e3, 2),
           "note": "timed step = upload of the step's tables/kv_len/copy lists + tail-page copies + fused "
                   "append/decode of 136 sequences; host bookkeeping (free 40, allocate 32, fork 8) done "
                   "ahead, from Python through the C ABI, one call per page"}
    del cr, runner
    torch.cuda.empty_cache()
    return res


def full_copy_fork(w, runner, dev, reps: int = 20) -> dict:
    """c5's fork with every page of the 8 children copied (no sharing): one
    lnskv_page_copy of all their pages, K and V, read and written."""
    import numpy as np
    import torch

    n_seq = w.n_seq - len(w.info["parents"])
    src_pages = []
    for i, parent in enumerate(w.info["parents"]):
        npg = (int(w.ctx_len[n_seq + i]) + 15) // 16
        src_pages += [int(p) for p in w.tables[parent][:npg] if p != 0xFFFFFFFF]
    # destinations: other pages of the pool (this runner is not stepped again)
    dst_pages = np.setdiff1d(np.arange(w.num_pages), np.array(src_pages))[:len(src_pages)]
    src_pages = src_pages[:len(dst_pages)]
    src = torch.tensor(np.array(src_pages, np.uint32).view(np.int32), device=dev)
    dst = torch.tensor(dst_pages.astype(np.uint32).view(np.int32), device=dev)
    pk = runner.layers[0]
    pk.page_copy(src, dst)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        pk.page_copy(src, dst)
    b.record()
    torch.cuda.synchronize()
    dt = a.elapsed_time(b) / 1e3 / reps
    nbytes = len(src_pages) * 2 * 2 * 16 * w.n_kv * w.head_dim * w.elem_bytes
    return {"pages": len(src_pages), "bytes": int(nbytes), "us": round(dt * 1e6, 1),
            "gb_per_s": round(nbytes / dt / 1e9, 1),
            "note": "every page of the 8 forked children copied (the page-sharing fork copies only tail pages)"}


def qwen35_measure(dev, steps: int, layers: int = 4, pattern_reps: int = 40, prefill_reps: int = 0) -> dict:
    """lns-ml's own full-attention layer (Qwen3.5: Hq16/Hkv4/d256) on the
    engine's Q8A pages, the engine's per-layer order in one call
    (lnskv_gated_append_decode: RoPE rotary 64 of 256 with theta 1e7 turned
    in registers, the quantizing append, the decode, the query gate): a batch
    of 32 at c2's contexts U[512, 4096] (stream-K), with its page pattern's
    load ceiling; and the reference's one-sequence call at pos 4095 (one
    kernel, the workgroup schedule), per call from HIP graph replay over 32
    layers.  Bytes: the K/V codes and scales of every attended token, the
    append, q/out, the gate read, table entries.  prefill_reps > 0: also the
    chunked prefill of the batch's last 256 tokens per sequence over its
    pages (the 256-wide heads' prompt path)."""
    import torch

    from lnskv import DTYPE_Q8A
    from lnskv.configs import make
    from lnskv.device import RopeTable
    from lnskv.step import StepRunner

    def gated_bytes(w):
        return w.algorithmic_bytes()["total"] + int(w.decode.sum()) * w.n_heads * w.head_dim * 4

    rope = RopeTable(64, 1.0e7, device=dev)
    w = make("qwen35", dtype=DTYPE_Q8A)
    runner = StepRunner(w, dev, n_layers=layers, seed=1, rope=rope, gated=True)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    step = lambda i: runner.run(i % layers)  # noqa: E731
    ev, wall = timed_steps(step, stream, steps, 10)
    nb = gated_bytes(w)
    res = {"shape": "32 sequences at U[512,4096], Hq16/Hkv4/d256, Q8A pages, RoPE rotary 64 (theta 1e7), gated",
           "us_per_step_events": round(ev * 1e6, 2), "us_per_step_wall": round(wall * 1e6, 2),
           "algorithmic_bytes": int(nb), "gb_per_s": round(nb / ev / 1e9, 1),
           "frac_of_hbm_peak": round(nb / ev / 1e9 / HBM_PEAK_GBS, 4)}
    pc = pattern_ceiling(w, runner, dev, pattern_reps)
    if pc:
        res["pattern_ceiling_us"] = pc["us_per_launch"]
        res["frac_of_pattern_ceiling"] = round(pc["us_per_launch"] / (ev * 1e6), 4)
    if prefill_reps > 0:
        res["chunked_prefill_attention"] = prefill_measure(w, runner, dev, prefill_reps)
    del runner
    torch.cuda.empty_cache()
    # the one-sequence call, 32 layers' pools cycled
    w1 = make("qwen35", n_seq=1, lo=4095, hi=4095, num_pages=256 + 8, dtype=DTYPE_Q8A)
    r1 = StepRunner(w1, dev, n_layers=32, seed=2, rope=rope, gated=True)
    for i in range(64):
        r1.run(i % 32)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(32):
            r1.run(i)
    torch.cuda.synchronize()
    ev_g, _ = timed_steps(lambda i: graph.replay(), stream, 20, 3)
    nb1 = gated_bytes(w1)
    res["b1_pos4095"] = {"us_per_call_graph_replay": round(ev_g / 32 * 1e6, 2), "bytes_per_call": int(nb1),
                         "gb_per_s": round(nb1 / (ev_g / 32) / 1e9, 1)}
    del graph, r1
    torch.cuda.empty_cache()
    return res


def reference_call_measure(dev, calls: int = 400, n_layers: int = 32) -> dict:
    """The reference's own call: lnskv_attention_paged (encode_attention_paged_q8a's
    arguments) for ONE sequence, Hq32/Hkv8/d128 on Q8A pages, appending the
    token at pos 4095 and attending [0, 4095]: 256 pages x 8 kv heads.  A
    32-layer model's worth of pools is cycled (8.6 MB per call, 276 MB over
    the layers, more than the 256 MB last-level cache).  Wall time per call is
    the host launch loop's rate (asynchronous calls back to back); event time
    per call is the GPU's."""
    import ctypes as C

    import numpy as np
    import torch

    from lnskv import DTYPE_Q8A
    from lnskv.device import PagedKV

    pos, hq, hkv, d = 4095, 32, 8, 128
    npg = pos // 16 + 1
    layers = []
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    for _ in range(n_layers):
        pk = PagedKV(npg + 8, hkv, d, DTYPE_Q8A, dev)
        for t in (pk.k, pk.v):
            t.copy_(torch.randint(-127, 128, t.shape, generator=g, device=dev, dtype=torch.int8))
        for t in (pk.ks, pk.vs):
            t.copy_(torch.rand(t.shape, generator=g, device=dev) * 0.02 + 0.001)
        layers.append(pk)
    table = torch.from_numpy(np.random.default_rng(1).permutation(npg + 8)[:npg].astype(np.int32)).to(dev)
    q = torch.randn(hq * d, device=dev)
    k_in = torch.randn(hkv * d, device=dev)
    v_in = torch.randn(hkv * d, device=dev)
    out = torch.empty(hq * d, device=dev)
    call = lambda i: layers[i % n_layers].attention_paged(q, k_in, v_in, table, pos, hq, out=out)  # noqa: E731
    stream = torch.cuda.current_stream(dev)
    ev, wall = timed_steps(call, stream, calls, 2 * n_layers)
    dist = step_distribution(call, stream, 200)
    # The GPU's time per call without the host's launch work: the calls of
    # all layers captured once in a HIP graph and the graph replayed (the
    # eager calls above grew the library's workspace, so nothing allocates
    # under capture).
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for i in range(n_layers):
            call(i)
    torch.cuda.synchronize()
    replays = max(calls // n_layers, 10)
    ev_graph, _ = timed_steps(lambda i: graph.replay(), stream, replays, 3)
    per_call_graph = ev_graph / n_layers
    # the same call at contexts whose page count per kv head (254, 257, 258)
    # is not a multiple of the workgroups' share of pages
    table_all = torch.from_numpy(np.random.default_rng(1).permutation(npg + 8).astype(np.int32)).to(dev)
    by_pos = {}
    for p in (4063, 4096, 4127):
        ev_p, _ = timed_steps(lambda i, p=p: layers[i % n_layers].attention_paged(q, k_in, v_in, table_all, p, hq,
                                                                                  out=out),
                              stream, calls, 2 * n_layers)
        by_pos[str(p)] = round(ev_p * 1e6, 2)
    nbytes = (pos + 1) * 2 * hkv * (d + 4) + 2 * hkv * d * 4 + 2 * hq * d * 4 + npg * 4
    del graph, layers
    torch.cuda.empty_cache()
    return {"shape": "1 sequence, Hq32/Hkv8/d128, Q8A pages, pos 4095 (append + attend 4096 tokens)",
            "us_per_call_events": round(ev * 1e6, 2), "us_per_call_median": dist["median"],
            "us_per_call_wall": round(wall * 1e6, 2),
            "us_per_call_graph_replay": round(per_call_graph * 1e6, 2),
            "us_per_call_events_at_pos": by_pos,
            "host_launch_share": round(max(0.0, 1.0 - per_call_graph / wall), 3),
            "bytes_per_call": int(nbytes),
            "gb_per_s": round(nbytes / ev / 1e9, 1),
            "gb_per_s_graph_replay": round(nbytes / per_call_graph / 1e9, 1),
            "layers_cycled": n_layers,
            "note": "eager: one Python/ctypes call per layer, the host's launch rate bounds it; graph replay: the "
                    "same calls replayed from one captured graph, the GPU's own time per call"}


def token_loop_measure(dev, tokens: int = 64, reps: int = 12) -> dict:
    """The reference engine's per-token work for one full-attention layer
    (engine.rs:1600-1604 then the attention at :3405): lnskv_step_pages, the
    block table to the device, lnskv_attention_paged -- one sequence,
    Hq32/Hkv8/d128 Q8A pages, positions 4064 .. 4064 + tokens - 1 (a new page
    every 16).  Two ways to move the table: the whole row every token
    (lnskv_block_tables_upload, upload_block_table's copy) and only the changed
    entries (lnskv_block_tables_sync: nothing on 15 of 16 tokens, a by-value
    patch when a page is mapped).  Per token: wall time of the host loop and
    HIP-event time on the stream."""
    import ctypes as C

    import torch

    from lnskv import DTYPE_Q8A
    from lnskv._lib import lib
    from lnskv.device import PagedKV
    from lnskv.host import BlockTables, PagePool

    pos0, hq, hkv, d, max_pages = 4064, 32, 8, 128, 512
    n_pages = (pos0 + tokens) // 16 + 8
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    pk = PagedKV(n_pages, hkv, d, DTYPE_Q8A, dev)
    for t in (pk.k, pk.v):
        t.copy_(torch.randint(-127, 128, t.shape, generator=g, device=dev, dtype=torch.int8))
    for t in (pk.ks, pk.vs):
        t.copy_(torch.rand(t.shape, generator=g, device=dev) * 0.02 + 0.001)
    q, k_in, v_in = (torch.randn(n, device=dev) for n in (hq * d, hkv * d, hkv * d))
    out = torch.empty(hq * d, device=dev)
    table_dev = torch.empty(max_pages, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    pool, bt = PagePool(n_pages), BlockTables(1, max_pages)
    # the C ABI called directly with its arguments prepared once, as a native
    # engine would (the Python wrappers' argument checks cost more host time
    # than the GPU work being measured)
    L = lib()
    st = C.c_void_p(stream.cuda_stream)
    args = [C.c_void_p(t.data_ptr()) for t in (q, k_in, v_in)]
    tdev, odev, desc = C.c_void_p(table_dev.data_ptr()), C.c_void_p(out.data_ptr()), C.byref(pk.desc)
    move = {"upload": L.lnskv_block_tables_upload, "sync": L.lnskv_block_tables_sync}
    res = {}
    for mode in ("upload", "sync"):
        ev_sum, wall_sum, moved = 0.0, 0.0, 0
        fn = move[mode]
        for r in range(reps + 1):
            bt.reset()
            pool.reset()
            for p in range(0, pos0, 16):
                bt.ensure_kv_page(pool, 0, p)
            bt.sync(table_dev.data_ptr(), stream.cuda_stream)
            torch.cuda.synchronize()
            moved += sum(1 for pos in range(pos0, pos0 + tokens) if pos % 16 == 0)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            a.record(stream)
            for pos in range(pos0, pos0 + tokens):
                if L.lnskv_step_pages(bt.handle, pool.handle, 0, 0, pos, 0) or fn(bt.handle, tdev, st) or \
                        L.lnskv_attention_paged(*args, desc, tdev, odev, pos, d, hq, hkv, 0, st):
                    raise RuntimeError(f"token loop failed at pos {pos}")
            b.record(stream)
            torch.cuda.synchronize()
            if r > 0:  # the first round warms up
                wall_sum += time.perf_counter() - t0
                ev_sum += a.elapsed_time(b) / 1e3
        res[mode] = {"us_per_token_wall": round(wall_sum / reps / tokens * 1e6, 2),
                     "us_per_token_events": round(ev_sum / reps / tokens * 1e6, 2)}
        if mode == "sync":
            res[mode]["pages_mapped_per_token"] = round(moved / (reps + 1) / tokens, 3)
    del pk
    torch.cuda.empty_cache()
    return {"shape": f"1 sequence, Hq32/Hkv8/d128, Q8A pages, positions {pos0}..{pos0 + tokens - 1}, one layer",
            "table_upload_every_token": res["upload"], "table_sync_changed_entries": res["sync"],
            "note": "per token: lnskv_step_pages (host) + the table to the device + lnskv_attention_paged, "
                    "the C ABI called from a Python loop with prepared arguments"}


def table_upload_measure(w, dev, reps: int = 200) -> dict:
    """upload_block_table's replacement timed on its own: lnskv_block_tables_upload
    of the configuration's [n_seq][stride] table from host memory (the
    library's C++ tables) to the device, HIP events around `reps` uploads."""
    import torch

    from lnskv.host import BlockTables, PagePool

    bt = BlockTables(w.n_seq, w.tables.shape[1])
    pool = PagePool(w.num_pages)
    for s in range(w.n_seq):
        for lp in range(int((w.tables[s] != 0xFFFFFFFF).sum())):
            bt.ensure_kv_page(pool, s, lp * 16)
    dst = torch.empty(w.n_seq * w.tables.shape[1], dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    bt.upload(dst.data_ptr(), stream.cuda_stream)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record(stream)
    for _ in range(reps):
        bt.upload(dst.data_ptr(), stream.cuda_stream)
    b.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / reps
    nbytes = int(dst.numel() * 4)
    # decode steps: every sequence appends one token (a page mapped when it
    # crosses a page boundary), then the device table is brought up to date,
    # by the whole upload or by the changed-entries sync; HIP events around
    # that one call per step (the host's page bookkeeping is outside them)
    lens = [int((w.tables[s] != 0xFFFFFFFF).sum()) * 16 for s in range(w.n_seq)]
    stride = w.tables.shape[1] + (2 * reps + 16) // 16 + 2  # room for the appended tokens
    bt = BlockTables(w.n_seq, stride)
    pool = PagePool(w.num_pages)
    for s in range(w.n_seq):
        for p in range(0, lens[s], 16):
            bt.ensure_kv_page(pool, s, p)
    dst = torch.empty(w.n_seq * stride, dtype=torch.int32, device=dev)
    per_step = {}
    for mode in ("upload", "sync"):
        fn = bt.upload if mode == "upload" else bt.sync
        fn(dst.data_ptr(), stream.cuda_stream)
        torch.cuda.synchronize()
        total, moved, warm = 0.0, 0, 8  # the first steps (kernel loading) are not timed
        for step in range(reps + warm):
            for s in range(w.n_seq):
                bt.ensure_kv_page(pool, s, lens[s] + (step if mode == "upload" else reps + warm + step))
            if step >= warm:
                moved += bt.changed() if mode == "sync" else 0
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn(dst.data_ptr(), stream.cuda_stream)
            e1.record(stream)
            e1.synchronize()
            if step >= warm:
                total += e0.elapsed_time(e1) * 1e3
        per_step[mode] = round(total / reps, 2)
        if mode == "sync":
            per_step["entries_per_step"] = round(moved / reps, 2)
    return {"bytes": nbytes, "us_per_upload_events": round(a.elapsed_time(b) * 1e3 / reps, 2),
            "us_per_upload_wall": round(wall * 1e6, 2),
            "decode_steps": {"us_per_step_upload_events": per_step["upload"],
                             "us_per_step_sync_events": per_step["sync"],
                             "changed_entries_per_step": per_step["entries_per_step"],
                             "note": f"{reps} steps of one token per sequence: the whole table "
                                     "(lnskv_block_tables_upload) against the changed entries "
                                     "(lnskv_block_tables_sync), HIP events around the one call"},
            "note": "hipMemcpyAsync from pageable host memory; the step's kernels are not in the timed region"}


def measured_traffic(name: str, dtype: int, rope: bool = False) -> dict | None:
    """HBM bytes per step from the committed counter summary of this workload
    and page type (FETCH_SIZE + WRITE_SIZE, calibrated on a plain copy), with
    the commit whose build it measured; None when there is none."""
    if rope:
        return None
    path = os.path.join(ROOT, "profiles", f"{name}_{'q8a_' if dtype == 2 else ''}traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        t = json.load(f)
    if t.get("kv_dtype", "f16") != {0: "f32", 1: "f16", 2: "q8a"}[dtype]:
        return None
    return {"bytes": int(t["hbm_bytes_per_step"]), "over_algorithmic": t.get("traffic_over_algorithmic"),
            "measured_at_commit": t.get("measured_at_commit")}


def cpu_baseline(w, runner, seconds: float, threads: int):
    """Oracle reference-order scan on a host copy of the step's pages, timed on
    a bounded sample: whole steps until `seconds` of CPU work have run."""
    import numpy as np

    import oracle as O
    from lnskv.configs import used_pages

    pk = runner.layers[0]
    pages = used_pages(w.tables)
    idx = __import__("torch").from_numpy(pages.astype(np.int64)).to(pk.device)
    conv = (lambda t: t.cpu().numpy().view(np.uint16)) if w.dtype == 1 else (lambda t: t.cpu().numpy())
    ks = vs = None
    if pk.ks is not None:
        sidx = (idx[:, None] * 16 + __import__("torch").arange(16, device=pk.device)[None, :]).reshape(-1)
        ks, vs = pk.ks.index_select(0, sidx).cpu().numpy(), pk.vs.index_select(0, sidx).cpu().numpy()
    hp = O.HostPages(conv(pk.k.index_select(0, idx)), conv(pk.v.index_select(0, idx)), ks, vs, dtype=w.dtype)
    remap = np.full(w.num_pages, O.NO_PAGE, np.uint32)
    remap[pages] = np.arange(len(pages), dtype=np.uint32)
    rows = runner.dec_rows
    t = w.tables[rows]
    tables = np.where(t != O.NO_PAGE, remap[np.minimum(t, w.num_pages - 1)], O.NO_PAGE).astype(np.uint32)
    kv_len = w.kv_len[rows]
    q = runner.q.cpu().numpy()
    k_new, v_new = runner.k_new.cpu().numpy(), runner.v_new.cpu().numpy()
    def timed(n_threads: int, budget: float):
        n = 0
        t0 = time.perf_counter()
        while True:
            O.append_decode_refscan(hp, q, k_new, v_new, tables, kv_len, None, w.scale, n_threads=n_threads)
            n += 1
            if time.perf_counter() - t0 >= budget:
                break
        return (time.perf_counter() - t0) / n, n

    dt, n = timed(threads, seconds)
    dt1, n1 = timed(1, 0.0) if threads > 1 else (dt, n)  # one whole step on one thread
    # the checker's use of the oracle: the GPU's output of this step against
    # the f64 oracle over the same stored pages (the step rewrites the same
    # token to the same slot, so the pages the oracle holds are the step's)
    import torch

    o = runner.run(0)
    torch.cuda.synchronize()
    o = o.cpu().numpy()
    ref = O.decode_f64(hp, q, tables, kv_len, None, w.scale)
    row, ele = O.rel_err_rows(o, ref), O.rel_err_elements(o, ref)
    parity = {"vs": "f64 oracle over the step's stored pages (layer 0)",
              "max_row_rel_err": float(row.max()),
              "row_tolerance": {0: 1e-5, 1: 1e-3, 2: 1e-5}[w.dtype],
              "max_elem_rel_err_floor_1e-6": float(ele.max()),
              "median_elem_rel_err_floor_1e-6": float(np.median(ele))}
    return {"value": round(dt * 1e6, 1), "unit": "µs/step", "cores": threads, "kind": "port",
            "parity": parity,
            "sample": f"{n} whole {w.name} steps (append + reference-order f32 scan of all "
                      f"{len(rows)} decoding sequences), {threads} OpenMP threads, "
                      f"{dt * n:.1f} s; nproc={os.cpu_count()}",
            "gb_per_s": round(w.algorithmic_bytes()["total"] / dt / 1e9, 2),
            "value_1_thread": round(dt1 * 1e6, 1),
            "sample_1_thread": f"{n1} whole {w.name} step(s) on 1 thread"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}); the paged KV path shards by sequence "
              f"or kv head, one process per GPU with no exchange between them", file=sys.stderr)
        sys.exit(2)
    import torch

    from lnskv.configs import make
    from lnskv.step import StepRunner

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_only:
        print(json.dumps({"copy_ceiling": copy_ceiling(dev, args.copy_mb or 1024)}), flush=True)
        return
    if args.reference_call_only:
        print(json.dumps({"reference_call_b1_q8a": reference_call_measure(dev),
                          "reference_token_loop_b1_q8a": token_loop_measure(dev)}), flush=True)
        return
    if args.qwen35_only:
        print(json.dumps({"qwen35_shape": qwen35_measure(dev, min(args.steps, 100), pattern_reps=args.pattern_reps,
                                                         prefill_reps=args.prefill_reps)}), flush=True)
        return
    if args.kv_dtype != "config":
        if args.config != "c2":
            print("--kv-dtype applies to c2 only", file=sys.stderr)
            sys.exit(2)
        w = make(args.config, dtype={"f32": 0, "f16": 1, "q8a": 2}[args.kv_dtype])
    else:
        w = make(args.config)
    if args.split >= 0:
        w.split = args.split
    rope = None
    if args.rope:
        from lnskv.device import RopeTable

        rope = RopeTable(w.head_dim, 500000.0, 2, (8.0, 8192.0, 1.0, 4.0), device=dev)
    runner = StepRunner(w, dev, n_layers=args.layers, seed=1, rope=rope)
    torch.cuda.synchronize()
    nb = w.algorithmic_bytes()
    stream = torch.cuda.current_stream(dev)

    if args.graph:
        graphs = [runner.capture(layer) for layer in range(args.layers)]
        step = lambda i: graphs[i % args.layers].replay()  # noqa: E731  (slower than eager on ROCm 7: measured)
    else:
        step = lambda i: runner.run(i % args.layers)  # noqa: E731
    # timed region: exactly K steps, synchronized on both sides; one pair of
    # HIP events on the kernels' stream brackets the K steps (an event pair
    # per step would add its own gaps between the steps); the per-step
    # distribution comes from a second run of steps with an event pair each
    ev_mean, wall = timed_steps(step, stream, args.steps, args.warmup)
    dist = step_distribution(step, stream, max(100, min(args.steps, 400)))

    gbs_wall = nb["total"] / wall / 1e9
    gbs_ev = nb["total"] / ev_mean / 1e9
    copy = copy_ceiling(dev, args.copy_mb) if args.copy_mb > 0 else None
    readc = read_ceiling(dev) if args.copy_mb > 0 else None
    pattern = pattern_ceiling(w, runner, dev, args.pattern_reps)
    oproj = oproj_measure(w, runner, dev, args.oproj_reps)
    prefill = prefill_measure(w, runner, dev, args.prefill_reps)
    extras = None
    if args.extras and w.name == "c2" and args.kv_dtype == "config" and not args.rope:
        extras = {"c2_q8a_pages": config_measure("c2", dev, args.steps, layers=args.layers, kv_dtype=2,
                                                 pattern_reps=args.pattern_reps, prefill_reps=args.prefill_reps),
                  "c2_q8a_pages_rope": config_measure("c2", dev, args.steps, layers=args.layers, kv_dtype=2,
                                                      rope=True),
                  "reference_call_b1_q8a": reference_call_measure(dev),
                  "reference_token_loop_b1_q8a": token_loop_measure(dev),
                  "qwen35_shape": qwen35_measure(dev, min(args.steps, 100), pattern_reps=args.pattern_reps,
                                                 prefill_reps=args.prefill_reps),
                  "block_table_upload": table_upload_measure(w, dev)}
        for name in ("c1", "c3", "c4", "c5"):
            extras[name] = config_measure(name, dev, min(args.steps, 100))
        extras["c5_churn_every_step"] = c5_churn_measure(dev, min(args.steps, 100))
    cpu = None
    if args.cpu_seconds > 0:
        threads = args.cpu_threads or len(os.sched_getaffinity(0))
        threads = min(threads, int(os.environ.get("OMP_NUM_THREADS", threads)))
        cpu = cpu_baseline(w, runner, args.cpu_seconds, threads)

    traffic = measured_traffic(w.name, w.dtype, bool(args.rope))
    line = {
        "metric": METRIC,
        "value": round(gbs_wall, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3, 5),
        "us_per_step": round(wall * 1e6, 2),
        "us_per_step_events": round(ev_mean * 1e6, 2),
        "us_per_step_median": dist["median"],
        "step_event_distribution_us": dist,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1)*scale pages, seeded SplitMix64 lengths and page order)",
        "config": {
            "workload": {"c1": "c1 single sequence Hq32/Hkv4/d64 f32 ctx 512",
                         "c2": f"c2 Llama-3-8B layer Hq32/Hkv8/d128 {('f32', 'f16', 'q8a')[w.dtype]} pages, B=32, "
                               "ctx U[512,4096], 1-token append + decode",
                         "c3": "c3 Hq32/Hkv8/d128 f16, B=4 x 32768, split-K 512",
                         "c4": "c4 16 x 256-token chunk appends + 48 decodes at U[1024,8192]",
                         "c5": "c5 B=128 churn: 32 freed/reallocated, 8 CoW forks, 136 decodes"}[w.name],
            "kv_dtype": {0: "f32", 1: "f16", 2: "q8a"}[w.dtype],
            "n_seq": int(w.n_seq),
            "tokens_attended": int(w.kv_len[w.decode].sum()),
            "split_tokens": int(w.split),
            "layers_cycled": args.layers,
            "launch": "HIP graph replay per step" if args.graph else "eager launches from Python",
            "rope": ("fused RoPE (lnskv_rope_append_decode), Llama-3.1 inverse frequencies, rotary = head_dim"
                     if args.rope else None),
            "algorithmic_bytes_per_step": int(nb["total"]),
            "bytes_breakdown": {k: int(v) for k, v in nb.items() if k != "total"},
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs_ev, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs_ev / HBM_PEAK_GBS, 4),
            "traffic": (traffic or {}).get("bytes"),
            "traffic_over_algorithmic": (traffic or {}).get("over_algorithmic"),
            "traffic_measured_at_commit": (traffic or {}).get("measured_at_commit"),
            "kernel": ("one step's kernels on their stream (c2: decode_sk_kernel + combine_sk_kernel "
                       "of one lnskv_append_decode call), mean HIP-event duration per step"),
            "copy_ceiling_gbs": copy["gb_per_s"] if copy else None,
            "frac_of_copy_ceiling": round(gbs_ev / copy["gb_per_s"], 4) if copy else None,
            "read_ceiling_gbs": readc["gb_per_s"] if readc else None,
            "frac_of_read_ceiling": round(gbs_ev / readc["gb_per_s"], 4) if readc else None,
            "read_ceiling": readc,
            "pattern_ceiling": pattern,
            "frac_of_pattern_ceiling": round(gbs_ev / pattern["gb_per_s"], 4) if pattern else None,
        },
        "cpu_baseline": cpu,
        "more_measurements": extras,
        "after_the_path": {"o_proj_q4l_gemv_accumulate": oproj},
        "prefill": {"chunked_prefill_attention": prefill},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
