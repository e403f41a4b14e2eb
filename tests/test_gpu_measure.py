"""GPU load probe (lnskv_read_units, measurement only): every lane's XOR word
equals the host XOR of exactly the bytes the header says it loads -- each
unit once, empty waves zero, odd and even unit counts, page ids and kv heads
outside the pools reading page 0 / kv head 0; 256-byte rows (f16 d128, f32
d64), 512-byte rows (f16 d256) and Q8A rows (128 or 256 bytes plus the K and
V scales)."""
import ctypes as C

import numpy as np
import pytest
import torch

from gpu_util import fill_pages, say
from lnskv import DTYPE_F16, DTYPE_F32, DTYPE_Q8A
from lnskv._lib import check, lib
from lnskv.device import PagedKV, _stream, sync

pytestmark = pytest.mark.gpu


def _expected(k32, v32, ks, vs, pages, kvhs, start, num_pages, n_kv, row_bytes):
    """sink[w*64 + lane], lane (r, c) = (lane // L, lane % L) with L = row
    bytes / 16: XOR over the wave's units, K and V, of the four words of
    16-byte chunk c of rows r, r + 64/L, ... of the unit's kv-head row, plus
    (Q8A: ks/vs given) one scale word: the V scale of token lane % 16 for
    lanes with bit 4 set, the K scale otherwise."""
    n_waves = len(start) - 1
    L = row_bytes // 16
    lane = np.arange(64)
    out = np.zeros((n_waves, 64), np.uint32)
    for w in range(n_waves):
        acc = np.zeros(64, np.uint32)
        for u in range(start[w], start[w + 1]):
            p = int(pages[u]) if pages[u] < num_pages else 0
            h = int(kvhs[u]) if 0 <= kvhs[u] < n_kv else 0
            for pool in (k32, v32):
                chunk = np.bitwise_xor.reduce(pool[p, :, h, :].reshape(16, L, 4), axis=2)  # row, chunk
                acc ^= np.bitwise_xor.reduce(chunk.reshape(16 // (64 // L), 64 // L, L), axis=0).reshape(64)
            if ks is not None:
                acc ^= np.where(lane & 16, vs[p * 16 + (lane & 15), h], ks[p * 16 + (lane & 15), h])
        out[w] = acc
    return out.reshape(-1)


@pytest.mark.parametrize("dtype,d", [(DTYPE_F16, 128), (DTYPE_F32, 64), (DTYPE_Q8A, 128), (DTYPE_Q8A, 256),
                                     (DTYPE_F16, 256)])
def test_read_units_checksum(gpu, dtype, d):
    say("read_units", dtype, d)
    n_kv, num_pages = 4, 40
    pk = PagedKV(num_pages, n_kv, d, dtype, gpu)
    fill_pages(pk, seed=5)
    rng = np.random.default_rng(d)
    n_units = 61
    pages = rng.integers(0, num_pages, n_units).astype(np.uint32)
    kvhs = rng.integers(0, n_kv, n_units).astype(np.int32)
    pages[3], pages[10] = num_pages, 0xFFFFFFFF  # outside the pool: page 0
    kvhs[7], kvhs[20] = n_kv, -1                 # outside: kv head 0
    # waves with 0, 1, 2, 3, 5, 7 ... units
    counts = [0, 1, 2, 3, 5, 7, 0, 11, 4, 28]
    assert sum(counts) == n_units
    start = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    n_waves = len(counts)
    sink = torch.full((n_waves * 64,), -1, dtype=torch.int32, device=gpu)
    d_pages = torch.from_numpy(pages.view(np.int32)).to(gpu)
    d_kvhs = torch.from_numpy(kvhs).to(gpu)
    d_start = torch.from_numpy(start).to(gpu)
    check(lib().lnskv_read_units(C.byref(pk.desc), d_pages.data_ptr(), d_kvhs.data_ptr(), d_start.data_ptr(),
                                 n_waves, sink.data_ptr(), _stream(gpu)))
    sync()
    k32 = pk.k.view(torch.int32).cpu().numpy().view(np.uint32).reshape(num_pages, 16, n_kv, -1)
    v32 = pk.v.view(torch.int32).cpu().numpy().view(np.uint32).reshape(num_pages, 16, n_kv, -1)
    ks = vs = None
    if dtype == DTYPE_Q8A:
        ks = pk.ks.view(torch.int32).cpu().numpy().view(np.uint32)
        vs = pk.vs.view(torch.int32).cpu().numpy().view(np.uint32)
    row_bytes = d * {DTYPE_F32: 4, DTYPE_F16: 2, DTYPE_Q8A: 1}[dtype]
    exp = _expected(k32, v32, ks, vs, pages, kvhs, start, num_pages, n_kv, row_bytes)
    got = sink.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("where", ["first", "middle", "last"])
def test_read_stream_reads_every_chunk(gpu, where):
    """lnskv_read_stream (the plain read ceiling) reads every 16-byte chunk: a
    buffer of zeros with one word set to the marker makes the thread that
    reads that chunk store 1; an all-zero buffer stores nothing.  Sizes that
    do and do not fill whole rounds of loads."""
    import ctypes as C

    from lnskv._lib import check, lib

    say("read stream", where)
    stream = C.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    for n16 in (1 << 16, (1 << 16) + 37):
        for u, bpc in ((4, 2), (16, 8), (1, 1)):
            buf = torch.zeros(n16 * 4, dtype=torch.int32, device=gpu)
            sink = torch.zeros(1, dtype=torch.int32, device=gpu)
            check(lib().lnskv_read_stream(buf.data_ptr(), n16 * 16, u, bpc, sink.data_ptr(), stream))
            torch.cuda.synchronize()
            assert int(sink.item()) == 0
            chunk = {"first": 0, "middle": n16 // 2 + 3, "last": n16 - 1}[where]
            buf[4 * chunk + 2] = np.int32(np.uint32(0x9E3779B9).view(np.int32))
            check(lib().lnskv_read_stream(buf.data_ptr(), n16 * 16, u, bpc, sink.data_ptr(), stream))
            torch.cuda.synchronize()
            assert int(sink.item()) == 1, (n16, u, bpc)
