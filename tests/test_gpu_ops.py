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
from lnskv._lib import LnskvError
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


def test_host_tables_sync_writes_the_changes(gpu):
    """lnskv_block_tables_sync keeps a device table equal to the host rows
    while writing only what changed: every entry on the first sync and after
    reset, nothing when nothing changed, a by-value patch for up to 64 changed
    entries and one span copy beyond that.  Random ensure / evict / free / fork
    steps on 6 rows, the device table (which starts as garbage) compared with
    the host rows after every sync, syncs queued behind a long kernel."""
    from lnskv import BlockTables, PagePool
    say("block table sync")
    rng = np.random.default_rng(11)
    n_seq, stride = 6, 40
    pool, bt = PagePool(2 * n_seq * stride), BlockTables(n_seq, stride)
    stream = torch.cuda.current_stream(gpu)
    dev = torch.full((n_seq, stride), 0x5A5A5A5A, dtype=torch.int32, device=gpu)
    big = torch.ones(1 << 24, device=gpu)
    assert bt.changed() == n_seq * stride
    bt.sync(dev.data_ptr(), stream.cuda_stream)
    assert bt.changed() == 0
    sync()
    assert np.array_equal(dev.cpu().numpy().view(np.uint32), bt.array())
    pos = np.zeros(n_seq, np.int64)
    kinds = set()
    for step in range(400):
        before = bt.array()
        r = rng.random()
        s = int(rng.integers(n_seq))
        if r < 0.6:
            pos[s] += int(rng.integers(1, 40))
            if pos[s] >= stride * 16:
                bt.free_sequence(pool, s)
                pos[s] = 0
            bt.ensure_kv_page(pool, s, int(pos[s]))
        elif r < 0.75:
            bt.evict_kv_pages(pool, s, int(pos[s]), int(rng.integers(1, 200)))
        elif r < 0.85:
            bt.free_sequence(pool, s)
            pos[s] = 0
        elif r < 0.95:
            c = int(rng.integers(n_seq))
            if c != s and bt.row_len(c) == 0 and bt.row_len(s) > 0:
                try:  # refused (table unchanged) when the tail page was evicted
                    bt.fork_sequence(pool, s, c, int(rng.integers(0, bt.row_len(s) * 16 + 1)))
                except LnskvError:
                    pass
        else:  # a burst: many rows at once (more than one patch holds)
            for t in range(n_seq):
                bt.free_sequence(pool, t)
                pos[t] = int(rng.integers(300, 600))
                for p in range(0, int(pos[t]) + 1, 16):
                    bt.ensure_kv_page(pool, t, p)
        n_diff = int((bt.array() != before).sum())
        assert bt.changed() >= n_diff
        if rng.random() < 0.5:
            n = bt.changed()
            kinds.add("none" if n == 0 else ("patch" if n <= _lib.TABLE_PATCH_MAX else "span"))
            big.mul_(1.0001)  # the sync waits behind this on the stream
            bt.sync(dev.data_ptr(), stream.cuda_stream)
            assert bt.changed() == 0
            if step % 7 == 0:
                sync()
                assert np.array_equal(dev.cpu().numpy().view(np.uint32), bt.array()), step
    bt.reset()
    assert bt.changed() == n_seq * stride
    bt.sync(dev.data_ptr(), stream.cuda_stream)
    sync()
    assert np.array_equal(dev.cpu().numpy().view(np.uint32), bt.array())
    assert kinds == {"none", "patch", "span"}, kinds


def test_block_table_patch_primitive(gpu):
    """lnskv_block_table_patch writes exactly its pairs and refuses 0 or 65."""
    dev = torch.zeros(256, dtype=torch.int32, device=gpu)
    idx = (C.c_uint32 * 64)(*range(3, 256, 4))
    val = (C.c_uint32 * 64)(*[0xFFFFFFFF - i for i in range(64)])
    stream = C.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    assert _lib.lib().lnskv_block_table_patch(C.c_void_p(dev.data_ptr()), 64, idx, val, stream) == 0
    assert _lib.lib().lnskv_block_table_patch(C.c_void_p(dev.data_ptr()), 0, idx, val, stream) == _lib.ERR_INVALID
    assert _lib.lib().lnskv_block_table_patch(C.c_void_p(dev.data_ptr()), 65, idx, val, stream) == _lib.ERR_INVALID
    sync()
    want = np.zeros(256, np.uint32)
    want[3::4] = 0xFFFFFFFF - np.arange(64)
    assert np.array_equal(dev.cpu().numpy().view(np.uint32), want)


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
