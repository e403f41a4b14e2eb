"""GPU gated attention.

lnskv_split_gated_query against the oracle: q bit-exact, gate within three
f32 ulps of the oracle's logistic.  Both compute 1 / (1 + exp(-x)) in f32;
each exp is within about one ulp of the true value, so the two can differ by
two, and the add and the divide each round once more.  Cases: the 16-byte
path, the scalar path (head_dim not a multiple of 4), an unaligned buffer.

lnskv_gated_append_decode: the stored output equals, bit for bit, the
ungated call's output times the gate (one f32 multiply as the row is
written), on every schedule that writes output rows -- stream-K MFMA with its
combine (f16, and Q8A after its quantizing append), split-K MFMA with
combine_kernel, the generic kernel (f32, Q8A, f16 forced), fused RoPE and the
RoPE pre-pass -- and the appended pages are the
ungated call's; one case is also checked against the f64 oracle times the
gate."""
import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import TOL, dev_f32, dev_i32, fill_pages, host_pages, rel_err, say
from lnskv import DTYPE_F16, DTYPE_F32, DTYPE_Q8A, DTYPE_NAMES, NO_PAGE
from lnskv.device import PagedKV, RopeTable, split_gated_query, sync

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


@pytest.mark.parametrize("d,offset", [(128, 0), (6, 0), (128, 1)])
def test_split_gated_query(gpu, d, offset):
    say("split_gated_query d", d, "offset", offset)
    rows, heads = 3, 5
    rng = np.random.default_rng(d + offset)
    x = (rng.standard_normal((rows, heads, 2 * d)) * 4).astype(np.float32)
    x[0, 0, d:d + 4] = [0.0, 30.0, -30.0, -100.0]
    buf = torch.zeros(x.size + offset, dtype=torch.float32, device=gpu)
    buf[offset:] = torch.from_numpy(x.reshape(-1)).to(gpu)
    src = buf[offset:]
    q, g = split_gated_query(src, heads, d)
    sync()
    qr, gr = O.split_gated_query(x, heads, d)
    assert np.array_equal(q.cpu().numpy(), qr)
    assert np.all(_ulps(g.cpu().numpy(), gr) <= 3)


CASES = [  # dtype, head_dim, rep, split, force_valu, rotary_dim
    (DTYPE_F16, 128, 4, 0, "0", 0),      # stream-K MFMA (+ combine_sk_kernel)
    (DTYPE_F16, 128, 2, 64, "0", 0),     # split-K MFMA (+ combine_kernel)
    (DTYPE_F16, 128, 4, 0, "1", 0),      # generic kernel, f16
    (DTYPE_F32, 64, 2, 0, "0", 0),       # generic kernel, f32
    (DTYPE_Q8A, 128, 4, 32, "0", 0),     # generic kernel, Q8A, split-K
    (DTYPE_Q8A, 128, 4, 0, "0", 0),      # Q8A stream-K MFMA after the quantizing append
    (DTYPE_F16, 128, 4, 0, "0", 128),    # RoPE turned inside the MFMA kernel
    (DTYPE_F16, 128, 8, 0, "0", 96),     # RoPE pre-pass (rotary 96), REP 8
    (DTYPE_Q8A, 128, 4, 0, "0", 128),    # Q8A, RoPE turned inside the MFMA kernel
    (DTYPE_Q8A, 256, 4, 0, "0", 64),     # lns-ml's Qwen3.5 shape: Q8A, 256-wide heads, rotary 64
    (DTYPE_F16, 256, 4, 0, "0", 64),     # f16, 256-wide heads, rotary 64
    (DTYPE_F16, 256, 2, 64, "0", 0),     # split-K MFMA, 256-wide heads
]


@pytest.mark.parametrize("dtype,d,rep,split,force_valu,rotary", CASES)
def test_gated_equals_ungated_times_gate(gpu, monkeypatch, dtype, d, rep, split, force_valu, rotary):
    say("gated append_decode", DTYPE_NAMES[dtype], d, rep, split, force_valu, rotary)
    monkeypatch.setenv("LNSKV_FORCE_VALU", force_valu)
    n_kv = 2
    lens = (1, 17, 200, 700, 1300)
    rng = np.random.default_rng(d + rep + split + rotary)
    pages_per = [(L + 15) // 16 for L in lens]
    num_pages = sum(pages_per) + 8
    pk = PagedKV(num_pages, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=7)
    perm = rng.permutation(num_pages).astype(np.uint32)
    tables = np.full((len(lens), max(pages_per) + 1), NO_PAGE, np.uint32)
    k = 0
    for s, n in enumerate(pages_per):
        tables[s, :n] = perm[k:k + n]
        k += n
    kv_len = np.array(lens, np.int32)
    n_heads = n_kv * rep
    q = dev_f32(rng.standard_normal((len(lens), n_heads, d)).astype(np.float32), gpu)
    k_new = dev_f32(rng.standard_normal((len(lens), n_kv, d)).astype(np.float32), gpu)
    v_new = dev_f32(rng.standard_normal((len(lens), n_kv, d)).astype(np.float32), gpu)
    gate = torch.rand((len(lens), n_heads, d), device=gpu)
    gate[0, 0, :4] = torch.tensor([0.0, 1.0, 0.5, 1e-30], device=gpu)
    t, kl = dev_i32(tables, gpu), dev_i32(kv_len, gpu)
    kw = dict(n_heads=n_heads, max_kv_len=int(kv_len.max()), scale=float(1.0 / np.sqrt(d)), split=split)
    rope = RopeTable(rotary, 10000.0, device=gpu) if rotary else None
    if rope is None:
        plain = pk.append_decode(q, k_new, v_new, t, kl, **kw)
    else:
        plain = pk.rope_append_decode(rope, q, k_new, v_new, t, kl, **kw)
    sync()
    pages_after, _ = host_pages(pk)
    gated = pk.gated_append_decode(gate, q, k_new, v_new, t, kl, rope=rope, **kw)
    sync()
    pages_again, _ = host_pages(pk)
    # the second append stores the same token: pages unchanged
    assert np.array_equal(pages_again.k.view(np.uint8), pages_after.k.view(np.uint8))
    assert np.array_equal(pages_again.v.view(np.uint8), pages_after.v.view(np.uint8))
    assert torch.equal(gated, plain * gate)
    if dtype == DTYPE_F16 and rope is None and split == 0 and force_valu == "0":
        hp, _ = host_pages(pk)
        ref = O.decode_f64(hp, q.cpu().numpy(), tables, kv_len, None, kw["scale"])
        g = gate.cpu().numpy().astype(np.float64)
        assert rel_err(gated, ref * g).max() < TOL[dtype]

