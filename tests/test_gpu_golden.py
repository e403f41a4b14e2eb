"""The product path against the committed c1 fixture (oracle-generated):
lnskv_append writes the 512 context tokens, the reference-style single
sequence call (lnskv_attention_paged) appends token 512 and attends; the new
token's page must equal the fixture bit for bit, and the output must be within
1e-5 (row-normwise, f32 pages) of the fixture's f64 output."""
import os
import sys

import numpy as np
import pytest
import torch

from gpu_util import TOL, dev_f32, dev_i32, rel_err, say
from lnskv import DTYPE_F32
from lnskv.device import PagedKV, sync

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden as G  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dispatch", [False, True])
def test_c1_fixture(gpu, dispatch):
    say("c1 golden, dispatch", dispatch)
    f = np.load(os.path.join(HERE, "golden", "c1_golden.npz"), allow_pickle=False)
    x = G.gen_inputs(0)
    table = f["table"]
    pk = PagedKV(64, G.N_KV, G.D, DTYPE_F32, gpu)
    pk.clear()
    bt = dev_i32(table[None], gpu)
    pk.append(dev_f32(x["k_ctx"], gpu), dev_f32(x["v_ctx"], gpu), dev_i32(np.zeros(G.CTX, np.int32), gpu),
              dev_i32(np.arange(G.CTX, dtype=np.int32), gpu), bt)
    out = pk.attention_paged(dev_f32(x["q"], gpu), dev_f32(x["k_new"], gpu), dev_f32(x["v_new"], gpu),
                             dev_i32(table, gpu), pos=G.CTX, n_heads=G.N_HEADS, dispatch=dispatch)
    sync()
    page = int(table[G.CTX // 16])
    assert np.array_equal(pk.k[page].cpu().numpy().view(np.uint32), f["k_page"].view(np.uint32))
    assert np.array_equal(pk.v[page].cpu().numpy().view(np.uint32), f["v_page"].view(np.uint32))
    assert rel_err(out, f["out_f64"]).max() < TOL[DTYPE_F32]
    assert rel_err(out, f["out_refscan"].astype(np.float64)).max() < TOL[DTYPE_F32]
