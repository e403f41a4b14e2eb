"""Helpers shared by the GPU tests (not collected: no test_ prefix).

Device pools are filled on the GPU; whenever the oracle checks a result it
reads back the exact stored bits, so the CPU restatement and the HIP kernels
always see identical inputs."""
from __future__ import annotations

import sys

import numpy as np
import torch

import oracle as O
from lnskv import DTYPE_F16, DTYPE_F32, DTYPE_Q8A, NO_PAGE
from lnskv.device import PagedKV

TOL = {DTYPE_F32: 1e-5, DTYPE_F16: 1e-3, DTYPE_Q8A: 1e-5}


def say(*args) -> None:
    """Names the case about to run on the GPU, flushed, so a crash is attributable."""
    print("[gpu]", *args, flush=True)
    sys.stdout.flush()


def dev_i32(a: np.ndarray, dev) -> torch.Tensor:
    """int32 device tensor holding the bits of an int32/uint32 array."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a.astype(np.int32, copy=False)).to(dev)


def dev_f32(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def fill_pages(pk: PagedKV, seed: int, scale: float = 1.0) -> None:
    """Seeded N(0,1)*scale contents (Q8A: random int8 and positive scales)."""
    g = torch.Generator(device=pk.device)
    g.manual_seed(seed)
    if pk.dtype == DTYPE_Q8A:
        pk.k.copy_(torch.randint(-127, 128, pk.k.shape, generator=g, device=pk.device, dtype=torch.int8))
        pk.v.copy_(torch.randint(-127, 128, pk.v.shape, generator=g, device=pk.device, dtype=torch.int8))
        pk.ks.copy_(torch.rand(pk.ks.shape, generator=g, device=pk.device) * 0.02 + 0.001)
        pk.vs.copy_(torch.rand(pk.vs.shape, generator=g, device=pk.device) * 0.02 + 0.001)
        return
    for t in (pk.k, pk.v):
        t.copy_((torch.randn(t.shape, generator=g, device=pk.device) * scale).to(t.dtype))


def host_pages(pk: PagedKV, pages: np.ndarray | None = None) -> tuple[O.HostPages, np.ndarray | None]:
    """Host copy of the pools (all pages, or only `pages`, compacted).  Returns
    (HostPages, remap) where remap[old_page] = new index (None when whole)."""
    if pages is None:
        idx = None
        k, v = pk.k, pk.v
        ks, vs = pk.ks, pk.vs
    else:
        idx = torch.from_numpy(pages.astype(np.int64)).to(pk.device)
        k, v = pk.k.index_select(0, idx), pk.v.index_select(0, idx)
        ks = vs = None
        if pk.ks is not None:
            sidx = (idx[:, None] * 16 + torch.arange(16, device=pk.device)[None, :]).reshape(-1)
            ks, vs = pk.ks.index_select(0, sidx), pk.vs.index_select(0, sidx)
    conv = (lambda t: t.cpu().numpy().view(np.uint16)) if pk.dtype == DTYPE_F16 else (lambda t: t.cpu().numpy())
    hp = O.HostPages(conv(k), conv(v), None if ks is None else ks.cpu().numpy(),
                     None if vs is None else vs.cpu().numpy(), dtype=pk.dtype)
    remap = None
    if pages is not None:
        remap = np.full(pk.num_pages, NO_PAGE, np.uint32)
        remap[pages] = np.arange(len(pages), dtype=np.uint32)
    return hp, remap


def remap_tables(tables: np.ndarray, remap: np.ndarray | None) -> np.ndarray:
    if remap is None:
        return tables
    out = np.full(tables.shape, NO_PAGE, np.uint32)
    m = tables != NO_PAGE
    out[m] = remap[tables[m]]
    return out


def rel_err(out: torch.Tensor | np.ndarray, ref: np.ndarray) -> np.ndarray:
    o = out.cpu().numpy() if isinstance(out, torch.Tensor) else out
    return O.rel_err_rows(o, ref)
