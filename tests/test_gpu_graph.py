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


@pytest.mark.parametrize("name", ["c1", "c2", "c5"])
def test_graph_replay_matches_eager(gpu, name):
    say("graph replay", name)
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
