"""lns-ml's own full-attention shape on the matrix cores: the Qwen3.5 layers
the engine runs on Q8A pages (model_config.rs:563-593: 16 query heads, 4 kv
heads, head_dim 256, partial rotary factor 0.25 so rotary 64 of 256 with
theta 1e7, gated query attention; pages engine.rs:731-734), one step of the
engine's per-layer order (rotate q and k by the token's position, append,
attend, multiply by the gate: engine.rs:1700-1720, 3401-3431) in one
lnskv_gated_append_decode call.

Cases: the reference's one-sequence call at position 4095 (the workgroup
schedule) and a batch of 32 at contexts U[512, 4096] (stream-K), Q8A and f16
pages, some sequences on a sliding window.  Against the oracle, which
rotates, appends (quantizes) and attends in float64: every byte of the pools
and scales matches the oracle's (the rotated, quantized new token included),
and the output rows are within the tolerance (1e-5 Q8A, 1e-3 f16) of the
float64 attention times the gate."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import TOL, dev_f32, dev_i32, fill_pages, host_pages, rel_err, say
from lnskv import DTYPE_F16, DTYPE_Q8A, DTYPE_NAMES, NO_PAGE
from lnskv.device import PagedKV, RopeTable, sync
from test_gpu_rope import _check_pages

pytestmark = pytest.mark.gpu

N_HEADS, N_KV, D, ROTARY, THETA = 16, 4, 256, 64, 1.0e7


def _batch(rng, lens, num_pages):
    pages_per = [(L + 15) // 16 for L in lens]
    perm = rng.permutation(num_pages).astype(np.uint32)
    t = np.full((len(lens), max(pages_per) + 1), NO_PAGE, np.uint32)
    k = 0
    for s, n in enumerate(pages_per):
        t[s, :n] = perm[k:k + n]
        k += n
    return t


@pytest.mark.parametrize("dtype", [DTYPE_Q8A, DTYPE_F16])
@pytest.mark.parametrize("case", ["b1_pos4095", "b32_ragged"])
def test_qwen35_step(gpu, dtype, case):
    say("qwen3.5 shape", DTYPE_NAMES[dtype], case)
    rng = np.random.default_rng(35 + dtype + (0 if case == "b1_pos4095" else 100))
    if case == "b1_pos4095":
        lens = np.array([4096], np.int32)
    else:
        lens = rng.integers(512, 4097, 32).astype(np.int32)
    num_pages = int(sum((L + 15) // 16 for L in lens)) + 16
    pk = PagedKV(num_pages, N_KV, D, dtype, gpu)
    fill_pages(pk, seed=int(lens.sum()) % 1000, scale=0.5)
    tables = _batch(rng, lens, num_pages)
    n = len(lens)
    p_start = np.zeros(n, np.int32)
    if n > 1:
        p_start[3] = max(0, lens[3] - 1024)  # a 1024-token sliding window
        p_start[9] = lens[9] - 1             # a window of the new token alone
    rope = RopeTable(ROTARY, THETA, device=gpu)
    q = rng.standard_normal((n, N_HEADS, D)).astype(np.float32)
    k_new = rng.standard_normal((n, N_KV, D)).astype(np.float32)
    v_new = rng.standard_normal((n, N_KV, D)).astype(np.float32)
    gate = rng.random((n, N_HEADS, D)).astype(np.float32)
    before, _ = host_pages(pk)
    hp = before.copy()
    pos = lens - 1
    q_r = O.rope_apply(q, ROTARY, rope.inv_freqs_host, pos)
    k_r = O.rope_apply(k_new, ROTARY, rope.inv_freqs_host, pos)
    O.append(hp, k_r, v_new, np.arange(n, dtype=np.int32), pos, tables)
    scale = 1.0 / np.sqrt(D)
    out = pk.gated_append_decode(dev_f32(gate, gpu), dev_f32(q, gpu), dev_f32(k_new, gpu), dev_f32(v_new, gpu),
                                 dev_i32(tables, gpu), dev_i32(lens, gpu), rope=rope, n_heads=N_HEADS,
                                 max_kv_len=int(lens.max()), scale=float(scale), p_start=dev_i32(p_start, gpu))
    sync()
    got, _ = host_pages(pk)
    _check_pages(got, hp, before, dtype)
    ref = O.decode_f64(hp, q_r, tables, lens, p_start, scale) * gate.astype(np.float64)
    err = rel_err(out, ref)
    say("max row error", float(err.max()))
    assert err.max() < TOL[dtype]
