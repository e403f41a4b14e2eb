"""HIP graph capture of a whole step (the bench's launch mode).

A captured step is replayed several times, with other eager work on the same
stream between the replays, and every replay's output and pages must equal
the eager step's bit for bit (the kernels are deterministic for fixed inputs
and launch shape)."""
import numpy as np
import pytest
import torch

from gpu_util import say
from lnskv.configs import make
from lnskv.step import StepRunner

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["c1", "c2", "c5", "c2-workgroup"])
def test_graph_replay_matches_eager(gpu, monkeypatch, name):
    """c2-workgroup: c2 forced onto the workgroup schedule, whose
    cross-workgroup counts in the workspace header must be back at zero
    after every replay."""
    say("graph replay", name)
    if name.endswith("-workgroup"):
        monkeypatch.setenv("LNSKV_DECODE_SCHEDULE", "workgroup")
        name = name.split("-")[0]
    w = make(name)
    r = StepRunner(w, gpu, n_layers=2, seed=3)
    eager = [r.run(layer).clone() for layer in (0, 1)]
    pages = [(pk.k.clone(), pk.v.clone()) for pk in r.layers]
    torch.cuda.synchronize()
    graphs = [r.capture(layer) for layer in (0, 1)]
    scratch = torch.randn(1 << 20, device=gpu)
    for rep in range(4):
        for layer in (0, 1):
            r.out.zero_()
            graphs[layer].replay()
            got = r.out.clone()
            scratch.mul_(1.0001)  # unrelated eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(got, eager[layer]), (name, rep, layer)
            assert torch.equal(r.layers[layer].k, pages[layer][0])
            assert torch.equal(r.layers[layer].v, pages[layer][1])
    if r.workspace is not None and r.workspace.numel() >= 4096:
        assert int(r.workspace[:4096].count_nonzero()) == 0


def test_library_workspace_under_capture(gpu):
    """A call with a NULL workspace whose library buffer is too small does not
    allocate while its stream is being captured: it fails with
    LNSKV_ERR_WORKSPACE before enqueuing anything.  After
    lnskv_workspace_reserve the same capture succeeds and every replay
    matches the eager call."""
    from lnskv._lib import ERR_WORKSPACE, LnskvError, check, lib

    say("library workspace under capture")
    w = make("c2", n_seq=6, lo=40, hi=1500, num_pages=1024)
    r = StepRunner(w, gpu, n_layers=1, seed=5)
    pk = r.layers[0]
    kw = dict(n_heads=w.n_heads, max_kv_len=r.max_kv_len, scale=w.scale)
    torch.cuda.synchronize()
    check(lib().lnskv_workspace_release())
    need = pk.workspace_size(r.n_dec, w.n_heads, r.max_kv_len, 0)
    assert need > 0
    g = torch.cuda.CUDAGraph()
    with pytest.raises(LnskvError) as e:
        with torch.cuda.graph(g):
            pk.decode(r.q, r.dec_tables, r.dec_kv_len, out=r.out, **kw)
    assert e.value.status == ERR_WORKSPACE and "lnskv_workspace_reserve" in e.value.message
    torch.cuda.synchronize()
    check(lib().lnskv_workspace_reserve(need, 0, 0))
    eager = pk.decode(r.q, r.dec_tables, r.dec_kv_len, **kw).clone()
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        pk.decode(r.q, r.dec_tables, r.dec_kv_len, out=r.out, **kw)
    for _ in range(3):
        r.out.zero_()
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(r.out, eager)
    del g, g2
    torch.cuda.synchronize()
    check(lib().lnskv_workspace_release())
