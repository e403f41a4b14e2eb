"""GPU page copy, block-table gather, clear and library-owned pools, bit-exact
against the oracle."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from gpu_util import dev_i32, fill_pages, host_pages, say
from lnskv import DTYPE_F16, DTYPE_F32, DTYPE_Q8A, DTYPE_NAMES, NO_PAGE
from lnskv import _lib
from lnskv.device import PagedKV, sync

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_Q8A])
def test_page_copy_bit_exact(gpu, dtype):
    say("page_copy", DTYPE_NAMES[dtype])
    pk = PagedKV(128, 8, 128, dtype, gpu)
    fill_pages(pk, seed=2)
    rng = np.random.default_rng(2)
    perm = rng.permutation(128).astype(np.uint32)
    src, dst = perm[:40], perm[40:80]
    src_all = np.concatenate([src, [500]]).astype(np.uint32)   # a pair past the pool: skipped
    dst_all = np.concatenate([dst, [perm[90]]]).astype(np.uint32)
    hp, _ = host_pages(pk)
    O.page_copy(hp, src, dst)
    pk.page_copy(dev_i32(src_all, gpu), dev_i32(dst_all, gpu))
    sync()
    got, _ = host_pages(pk)
    assert np.array_equal(got.k.view(np.uint8), hp.k.view(np.uint8))
    assert np.array_equal(got.v.view(np.uint8), hp.v.view(np.uint8))
    if dtype == DTYPE_Q8A:
        assert np.array_equal(got.ks, hp.ks) and np.array_equal(got.vs, hp.vs)


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_Q8A])
def test_gather_bit_exact(gpu, dtype):
    say("gather", DTYPE_NAMES[dtype])
    pk = PagedKV(64, 4, 64, dtype, gpu)
    fill_pages(pk, seed=3)
    row = np.random.default_rng(3).permutation(64).astype(np.uint32)[:20]
    row[7] = NO_PAGE  # tokens 112..127 come out as zeros
    hp, _ = host_pages(pk)
    for start, n in ((0, 320), (5, 1), (37, 200), (300, 20)):
        exp = O.gather(hp, row, start, n)
        got = pk.gather(dev_i32(row, gpu), start, n)
        sync()
        for e, g in zip(exp, got):
            if e is None:
                assert g is None
                continue
            assert np.array_equal(g.cpu().numpy().view(np.uint8), e.view(np.uint8))


def test_clear_zeroes_every_byte(gpu):
    for dtype in (DTYPE_F16, DTYPE_Q8A):
        say("clear", DTYPE_NAMES[dtype])
        pk = PagedKV(33, 3, 64, dtype, gpu)
        fill_pages(pk, seed=4)
        pk.clear()
        sync()
        assert not pk.k.view(torch.int8).any() and not pk.v.view(torch.int8).any()
        if pk.ks is not None:
            assert not pk.ks.any() and not pk.vs.any()


def test_library_owned_pools_alloc_free(gpu):
    say("pages_alloc")
    lib = _lib.lib()
    p = _lib.Pages(None, None, None, None, 16, 2, 64, DTYPE_Q8A)
    _lib.check(lib.lnskv_pages_alloc(C.byref(p)))
    assert p.k_pages and p.v_pages and p.k_scales and p.v_scales
    _lib.check(lib.lnskv_clear(C.byref(p), None))
    _lib.check(lib.lnskv_sync(None))
    _lib.check(lib.lnskv_pages_free(C.byref(p)))
    assert not p.k_pages and not p.k_scales


def test_host_tables_upload(gpu):
    """upload_block_table: the host rows arrive unchanged on the device."""
    from lnskv import BlockTables, PagePool
    pool, bt = PagePool(100), BlockTables(3, 7)
    for s, L in enumerate((5, 100, 17)):
        for pos in range(0, L, 16):
            bt.ensure_kv_page(pool, s, pos)
    dev = torch.zeros((3, 7), dtype=torch.int32, device=gpu)
    bt.upload(dev.data_ptr(), torch.cuda.current_stream(gpu).cuda_stream)
    sync()
    assert np.array_equal(dev.cpu().numpy().view(np.uint32), bt.array())


def test_host_tables_upload_snapshots(gpu):
    """Each upload carries the table as it was during the call: the host rows
    change right after every return, with several copies still queued behind a
    long kernel, and each device buffer holds its own snapshot."""
    from lnskv import BlockTables, PagePool
    say("upload snapshots")
    pool, bt = PagePool(4096), BlockTables(8, 64)
    stream = torch.cuda.current_stream(gpu)
    big = torch.ones(1 << 26, device=gpu)
    devs, want = [], []
    for it in range(6):
        big.mul_(1.0001)  # work ahead of the copy on the same stream
        for s in range(8):
            bt.ensure_kv_page(pool, s, it * 16 * (s + 1))
        dev = torch.zeros((8, 64), dtype=torch.int32, device=gpu)
        bt.upload(dev.data_ptr(), stream.cuda_stream)
        devs.append(dev)
        want.append(bt.array().copy())
    sync()
    for dev, w in zip(devs, want):
        assert np.array_equal(dev.cpu().numpy().view(np.uint32), w)
