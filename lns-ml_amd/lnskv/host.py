"""Host-side page bookkeeping through the C ABI (no GPU needed).

Python mirrors of lns-inference/src/engine.rs's names so that callers read like
the engine: PagePool (:20-44) with alloc / free_page / reset, and the engine's
page helpers ensure_kv_page / evict_kv_pages / upload_block_table /
kv_p_start (:2958-3013), batched over sequences by BlockTables.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import NO_PAGE, PAGE_SIZE, LnskvError, check, lib


class PagePool:
    """FIFO free list of physical page ids (engine.rs:20-44), with per-page
    reference counts for copy-on-write sharing."""

    def __init__(self, capacity: int):
        h = C.c_void_p()
        check(lib().lnskv_page_pool_create(capacity, C.byref(h)))
        self._h = h

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def close(self) -> None:
        if self._h:
            lib().lnskv_page_pool_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def alloc(self) -> int | None:
        """pop_front; None when exhausted, like the reference's Option<u32>."""
        out = C.c_uint32()
        rc = lib().lnskv_page_pool_alloc(self._h, C.byref(out))
        if rc != 0:
            return None
        return out.value

    def free_page(self, idx: int) -> None:
        check(lib().lnskv_page_pool_free(self._h, idx))

    def retain(self, idx: int) -> None:
        check(lib().lnskv_page_pool_retain(self._h, idx))

    def reset(self) -> None:
        lib().lnskv_page_pool_reset(self._h)

    def refcount(self, idx: int) -> int:
        return lib().lnskv_page_pool_refcount(self._h, idx)

    @property
    def num_free(self) -> int:
        return lib().lnskv_page_pool_num_free(self._h)

    @property
    def capacity(self) -> int:
        return lib().lnskv_page_pool_capacity(self._h)


class BlockTables:
    """n_seq block-table rows of max_pages entries (NO_PAGE = unallocated)."""

    def __init__(self, n_seq: int, max_pages: int):
        h = C.c_void_p()
        check(lib().lnskv_block_tables_create(n_seq, max_pages, C.byref(h)))
        self._h = h
        self.n_seq = n_seq
        self.max_pages = max_pages

    @property
    def handle(self) -> C.c_void_p:
        return self._h

    def close(self) -> None:
        if self._h:
            lib().lnskv_block_tables_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def array(self) -> np.ndarray:
        """Copy of the [n_seq][max_pages] u32 table."""
        ptr = lib().lnskv_block_tables_host(self._h)
        flat = np.ctypeslib.as_array(ptr, shape=(self.n_seq * self.max_pages,))
        return flat.reshape(self.n_seq, self.max_pages).copy()

    def row_len(self, seq: int) -> int:
        return lib().lnskv_block_tables_len(self._h, seq)

    def reset(self) -> None:
        lib().lnskv_block_tables_reset(self._h)

    def ensure_kv_page(self, pool: PagePool, seq: int, pos: int, layer: int = 0) -> None:
        check(lib().lnskv_ensure_kv_page(self._h, pool.handle, layer, seq, pos))

    def evict_kv_pages(self, pool: PagePool, seq: int, pos: int, window: int) -> None:
        check(lib().lnskv_evict_kv_pages(self._h, pool.handle, seq, pos, window))

    def step_pages(self, pool: PagePool, seq: int, pos: int, window: int, layer: int = 0) -> None:
        """lnskv_step_pages: evict_kv_pages then ensure_kv_page, the order that
        needs only window_pages(window) pages per sequence."""
        check(lib().lnskv_step_pages(self._h, pool.handle, layer, seq, pos, window))

    def free_sequence(self, pool: PagePool, seq: int) -> None:
        check(lib().lnskv_free_sequence(self._h, pool.handle, seq))

    def fork_sequence(self, pool: PagePool, parent: int, child: int, n_tok: int):
        """Returns (src, dst) of the tail page the device must copy, or None."""
        src, dst, n = C.c_uint32(), C.c_uint32(), C.c_int32()
        check(lib().lnskv_fork_sequence(self._h, pool.handle, parent, child, n_tok,
                                        C.byref(src), C.byref(dst), C.byref(n)))
        return (src.value, dst.value) if n.value else None

    def upload(self, dst_dev_ptr: int, stream: int = 0) -> None:
        check(lib().lnskv_block_tables_upload(self._h, C.c_void_p(dst_dev_ptr), C.c_void_p(stream)))

    def sync(self, dst_dev_ptr: int, stream: int = 0) -> None:
        """Write only the entries changed since the last sync to the same device table."""
        check(lib().lnskv_block_tables_sync(self._h, C.c_void_p(dst_dev_ptr), C.c_void_p(stream)))

    def changed(self) -> int:
        """Entries the next sync writes (every entry before the first sync and after reset)."""
        return int(lib().lnskv_block_tables_changed(self._h))


def kv_p_start(pos: int, window: int) -> int:
    return lib().lnskv_kv_p_start(pos, window)


def window_pages(window: int) -> int:
    """Pages per sequence that lnskv_step_pages needs for a sliding window
    (0 for full attention)."""
    return lib().lnskv_window_pages(window)


__all__ = ["PagePool", "BlockTables", "kv_p_start", "window_pages", "LnskvError", "NO_PAGE", "PAGE_SIZE"]
