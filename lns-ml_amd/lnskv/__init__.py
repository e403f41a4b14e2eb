"""lnskv — MI355X (gfx950) paged KV cache for lns-ml's decode path.

Python surface over liblnskv.so (C ABI in include/lnskv.h):
  host     PagePool / BlockTables, the engine's page helpers (no GPU needed)
  device   PagedKV: append, decode, append_decode, attention_paged, page_copy,
           gather, clear on device pools held as torch tensors
  configs  seeded workloads for the five benchmark configurations
"""
from ._lib import (DTYPE_F16, DTYPE_F32, DTYPE_NAMES, DTYPE_Q8A, LIB_PATH, NO_PAGE, PAGE_SIZE,
                   SIGNATURES, LnskvError, lib)
from .host import BlockTables, PagePool, kv_p_start, window_pages

__all__ = ["DTYPE_F16", "DTYPE_F32", "DTYPE_Q8A", "DTYPE_NAMES", "LIB_PATH", "NO_PAGE", "PAGE_SIZE",
           "SIGNATURES", "LnskvError", "lib", "BlockTables", "PagePool", "kv_p_start", "window_pages"]
