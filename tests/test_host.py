"""Host-side page bookkeeping of liblnskv (no GPU): PagePool, block tables,
ensure_kv_page / evict_kv_pages / kv_p_start, free and copy-on-write fork.

Checked against the oracle's restatement of engine.rs:20-44 and :2958-3013 on
random operation sequences, plus the error behaviour the reference has
(exhaustion message) and the two edge cases it gets wrong (table overflow,
SWA off-by-one exhaustion)."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from lnskv import NO_PAGE, BlockTables, LnskvError, PagePool, kv_p_start, window_pages
from lnskv import _lib


def test_pool_matches_oracle_on_random_ops():
    rng = np.random.default_rng(1)
    cap = 37
    a, b = PagePool(cap), O.Pool(cap)
    held = []
    for _ in range(5000):
        op = rng.integers(0, 10)
        if op < 6:
            x, y = a.alloc(), b.alloc()
            assert x == y
            if x is not None:
                held.append(x)
        elif op < 9 and held:
            i = int(rng.integers(0, len(held)))
            pid = held.pop(i)
            a.free_page(pid)
            b.free_page(pid)
        else:
            a.reset()
            b.reset()
            held.clear()
        assert a.num_free == b.num_free


def test_pool_exhaustion_and_errors():
    p = PagePool(2)
    assert p.alloc() == 0 and p.alloc() == 1 and p.alloc() is None
    with pytest.raises(LnskvError) as e:
        p.free_page(5)
    assert e.value.status == _lib.ERR_INVALID
    p.free_page(1)
    with pytest.raises(LnskvError):
        p.free_page(1)  # double free is refused (the reference would push it twice)
    assert p.capacity == 2 and p.num_free == 1


def test_refcounted_sharing():
    p = PagePool(4)
    x = p.alloc()
    p.retain(x)
    assert p.refcount(x) == 2
    p.free_page(x)
    assert p.num_free == 3 and p.refcount(x) == 1
    p.free_page(x)
    assert p.num_free == 4 and p.refcount(x) == 0


def test_ensure_and_evict_match_oracle_for_swa_decode():
    for window in (0, 16, 20, 100):
        cap = 64
        a_pool, a_bt = PagePool(cap), BlockTables(1, 64)
        lib = O.lib()
        b_pool = lib.orc_pool_new(cap)
        b_row = np.full(64, O.NO_PAGE, np.uint32)
        b_len = C.c_int(0)
        for pos in range(0, 700):
            ra = rb = 0
            try:
                a_bt.ensure_kv_page(a_pool, 0, pos, layer=3)
            except LnskvError as e:
                ra = e.status
            rb = lib.orc_ensure_kv_page(b_pool, b_row.ctypes.data, C.byref(b_len), 64, pos)
            assert (ra == 0) == (rb == 0), (window, pos)
            if ra:
                break
            a_bt.evict_kv_pages(a_pool, 0, pos, window)
            lib.orc_evict_kv_pages(b_pool, b_row.ctypes.data, b_len.value, pos, window)
            assert np.array_equal(a_bt.array()[0], b_row)
            assert kv_p_start(pos, window) == lib.orc_kv_p_start(pos, window)
        lib.orc_pool_delete(b_pool)


def test_exhaustion_message_names_layer_and_pos():
    pool, bt = PagePool(1), BlockTables(1, 8)
    bt.ensure_kv_page(pool, 0, 0, layer=5)
    with pytest.raises(LnskvError) as e:
        bt.ensure_kv_page(pool, 0, 16, layer=5)
    assert e.value.status == _lib.ERR_POOL_EXHAUSTED
    assert "KV page pool exhausted at layer 5 (pos=16)" in e.value.message


def test_swa_pool_sized_to_window_exhausts_at_pos_w():
    # engine.rs sizes the pool ceil(w/16) and calls ensure before evict
    # (engine.rs:1601-1603): at pos = w (w a multiple of 16) the window spans
    # w/16 + 1 pages and allocation fails.  The same order fails the same way.
    w = 64
    pool, bt = PagePool(w // 16), BlockTables(1, 16)
    for pos in range(w):
        bt.ensure_kv_page(pool, 0, pos)
        bt.evict_kv_pages(pool, 0, pos, w)
    with pytest.raises(LnskvError):
        bt.ensure_kv_page(pool, 0, w)
    # A window [pos-w+1, pos] that starts mid-page touches ceil(w/16)+1 pages,
    # so evicting first does not help at pos = w (p_start = 1 frees nothing);
    # a pool of ceil(w/16)+1 pages never runs out.
    bt.evict_kv_pages(pool, 0, w, w)
    with pytest.raises(LnskvError):
        bt.ensure_kv_page(pool, 0, w)
    pool2, bt2 = PagePool(w // 16 + 1), BlockTables(1, 64)
    for pos in range(1000):
        bt2.ensure_kv_page(pool2, 0, pos)
        bt2.evict_kv_pages(pool2, 0, pos, w)
        live = bt2.array()[0]
        assert (live != NO_PAGE).sum() <= w // 16 + 1


@pytest.mark.parametrize("w", [1, 2, 15, 16, 17, 31, 32, 33, 64, 100, 4096])
def test_step_pages_never_exhausts_a_window_sized_pool(w):
    # lnskv_step_pages (evict, then ensure) on a pool of window_pages(w) pages
    # runs 10k positions without exhausting it; at every position every page
    # the window [kv_p_start, pos] touches is mapped and no page outside it is
    # held.  The bound is tight: some position holds exactly window_pages(w)
    # pages, and a pool one page smaller runs dry.
    n_pos = 10_000
    need = window_pages(w)
    assert need == (w + 14) // 16 + 1
    pool, bt = PagePool(need), BlockTables(1, n_pos // 16 + 1)
    most = 0
    for pos in range(n_pos):
        bt.step_pages(pool, 0, pos, w)
        row = bt.array()[0]
        lo, hi = kv_p_start(pos, w) // 16, pos // 16
        live = np.nonzero(row != NO_PAGE)[0]
        assert live.min() == lo and live.max() == hi and len(live) == hi - lo + 1, (w, pos)
        most = max(most, len(live))
        assert pool.num_free == need - len(live)
    assert most == need
    small, bt_small = PagePool(need - 1), BlockTables(1, n_pos // 16 + 1)
    with pytest.raises(LnskvError) as e:
        for pos in range(n_pos):
            bt_small.step_pages(small, 0, pos, w, layer=3)
    assert e.value.status == _lib.ERR_POOL_EXHAUSTED and "at layer 3" in e.value.message


def test_step_pages_matches_evict_then_ensure_of_the_oracle():
    lib = O.lib()
    for window in (0, 20, 48):
        a_pool, a_bt = PagePool(48), BlockTables(1, 64)
        b_pool = lib.orc_pool_new(48)
        b_row = np.full(64, NO_PAGE, np.uint32)
        b_len = C.c_int(0)
        for pos in range(700):
            a_bt.step_pages(a_pool, 0, pos, window)
            lib.orc_evict_kv_pages(b_pool, b_row.ctypes.data, b_len.value, pos, window)
            assert lib.orc_ensure_kv_page(b_pool, b_row.ctypes.data, C.byref(b_len), 64, pos) == 0
            assert np.array_equal(a_bt.array()[0], b_row), (window, pos)
        lib.orc_pool_delete(b_pool)
    assert window_pages(0) == 0 and window_pages(-5) == 0


def test_table_overflow_is_an_error_not_a_write():
    pool, bt = PagePool(64), BlockTables(2, 4)
    with pytest.raises(LnskvError) as e:
        bt.ensure_kv_page(pool, 0, 4 * 16)
    assert e.value.status == _lib.ERR_INVALID
    assert (bt.array() == NO_PAGE).all()


def test_free_sequence_and_fork():
    pool, bt = PagePool(32), BlockTables(3, 8)
    for pos in range(0, 40, 16):
        bt.ensure_kv_page(pool, 0, pos)   # pages 0,1,2 for 40 tokens
    assert bt.row_len(0) == 3
    cp = bt.fork_sequence(pool, 0, 1, 40)  # 40 = 2 full pages + 8-token tail
    t = bt.array()
    assert t[1, :2].tolist() == t[0, :2].tolist()
    assert cp == (t[0, 2], t[1, 2]) and t[1, 2] not in t[0, :3]
    assert pool.refcount(int(t[0, 0])) == 2 and pool.refcount(int(t[0, 2])) == 1
    assert bt.fork_sequence(pool, 0, 2, 32) is None  # page-aligned: nothing to copy
    free_before = pool.num_free
    bt.free_sequence(pool, 0)
    assert pool.num_free == free_before + 1  # only the unshared tail returns
    assert bt.row_len(0) == 0 and (bt.array()[0] == NO_PAGE).all()
    bt.free_sequence(pool, 1)
    bt.free_sequence(pool, 2)
    assert pool.num_free == 32


def test_fork_refuses_nonempty_child():
    pool, bt = PagePool(8), BlockTables(2, 4)
    bt.ensure_kv_page(pool, 0, 0)
    bt.ensure_kv_page(pool, 1, 0)
    with pytest.raises(LnskvError):
        bt.fork_sequence(pool, 0, 1, 5)


def test_reset_clears_rows():
    pool, bt = PagePool(8), BlockTables(2, 4)
    bt.ensure_kv_page(pool, 1, 20)
    bt.reset()
    pool.reset()
    assert (bt.array() == NO_PAGE).all() and bt.row_len(1) == 0 and pool.num_free == 8


def test_sync_counts_every_entry_until_the_first_sync():
    """lnskv_block_tables_changed before any sync (and after reset): the whole
    table, whatever changed since; the sync itself needs a device and is
    checked in test_gpu_ops.py."""
    pool, bt = PagePool(16), BlockTables(3, 5)
    assert bt.changed() == 15
    bt.ensure_kv_page(pool, 1, 40)
    assert bt.changed() == 15
    bt.reset()
    assert bt.changed() == 15
    assert _lib.lib().lnskv_block_tables_changed(None) == 0
    # the patch primitive refuses NULL pointers and counts outside [1, 64]
    # before touching any device
    idx = (C.c_uint32 * 65)()
    val = (C.c_uint32 * 65)()
    assert _lib.lib().lnskv_block_table_patch(None, 1, idx, val, None) == _lib.ERR_INVALID
    assert _lib.lib().lnskv_block_tables_sync(None, None, None) == _lib.ERR_INVALID
