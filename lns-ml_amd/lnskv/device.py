"""Device-side entry points of liblnskv over torch tensors.

torch is used only for device memory and the current HIP stream; every
operation runs the library's HIP kernels through the C ABI.  Shapes, dtypes,
devices and contiguity are checked here before any launch, because the C ABI
receives raw pointers and the kernels index from the stated geometry.
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import (DTYPE_F16, DTYPE_F32, DTYPE_Q8A, PAGE_SIZE, Pages, Rope, check, lib)

TORCH_DTYPE = {DTYPE_F32: torch.float32, DTYPE_F16: torch.float16, DTYPE_Q8A: torch.int8}


def _ptr(t: torch.Tensor | None) -> C.c_void_p:
    return C.c_void_p(t.data_ptr() if t is not None else 0)


def _stream(device: torch.device) -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _need(t: torch.Tensor, name: str, dtype, numel: int, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() != numel:
        raise ValueError(f"{name} must have {numel} elements, got {t.numel()}")


def split_gated_query(qg: torch.Tensor, n_heads: int, head_dim: int, q_out=None, gate_out=None):
    """lnskv_split_gated_query: qg [n_rows][n_heads][2*head_dim] -> (q, sigmoid(gate))."""
    n_rows = qg.numel() // (2 * n_heads * head_dim)
    _need(qg, "qg", torch.float32, n_rows * n_heads * 2 * head_dim, qg.device)
    if q_out is None:
        q_out = torch.empty((n_rows, n_heads, head_dim), dtype=torch.float32, device=qg.device)
    if gate_out is None:
        gate_out = torch.empty((n_rows, n_heads, head_dim), dtype=torch.float32, device=qg.device)
    _need(q_out, "q_out", torch.float32, n_rows * n_heads * head_dim, qg.device)
    _need(gate_out, "gate_out", torch.float32, n_rows * n_heads * head_dim, qg.device)
    check(lib().lnskv_split_gated_query(_ptr(qg), _ptr(q_out), _ptr(gate_out), n_rows, n_heads, head_dim,
                                        _stream(qg.device)))
    return q_out, gate_out


class PagedKV:
    """One layer's paged K/V pools in the reference layout
    [num_pages][16][n_kv_heads][head_dim] (+ Q8A scales [num_pages*16][n_kv]),
    held as torch tensors, with the library's operations on them."""

    def __init__(self, num_pages: int, n_kv_heads: int, head_dim: int, dtype: int,
                 device: str | torch.device = "cuda"):
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.num_pages, self.n_kv, self.head_dim, self.dtype = num_pages, n_kv_heads, head_dim, dtype
        shape = (num_pages, PAGE_SIZE, n_kv_heads, head_dim)
        td = TORCH_DTYPE[dtype]
        self.k = torch.zeros(shape, dtype=td, device=self.device)
        self.v = torch.zeros(shape, dtype=td, device=self.device)
        if dtype == DTYPE_Q8A:
            self.ks = torch.zeros((num_pages * PAGE_SIZE, n_kv_heads), dtype=torch.float32, device=self.device)
            self.vs = torch.zeros_like(self.ks)
        else:
            self.ks = self.vs = None
        self.desc = Pages(self.k.data_ptr(), self.v.data_ptr(),
                          self.ks.data_ptr() if self.ks is not None else None,
                          self.vs.data_ptr() if self.vs is not None else None,
                          num_pages, n_kv_heads, head_dim, dtype)

    # -- helpers -------------------------------------------------------------
    @property
    def row_elems(self) -> int:
        return self.n_kv * self.head_dim

    def _tables(self, tables: torch.Tensor, n_seq: int) -> int:
        if tables.dim() != 2 or tables.shape[0] != n_seq:
            raise ValueError(f"block tables must be [n_seq={n_seq}][stride], got {tuple(tables.shape)}")
        _need(tables, "block_tables", torch.int32 if tables.dtype == torch.int32 else torch.uint32,
              tables.numel(), self.device)
        return int(tables.shape[1])

    # -- operations ----------------------------------------------------------
    def clear(self) -> None:
        check(lib().lnskv_clear(C.byref(self.desc), _stream(self.device)))

    def append(self, k_new, v_new, tok_seq, tok_pos, tables) -> None:
        n_tok = int(tok_seq.numel())
        _need(k_new, "k_new", torch.float32, n_tok * self.row_elems, self.device)
        _need(v_new, "v_new", torch.float32, n_tok * self.row_elems, self.device)
        _need(tok_seq, "tok_seq", torch.int32, n_tok, self.device)
        _need(tok_pos, "tok_pos", torch.int32, n_tok, self.device)
        if tables.dim() != 2:
            raise ValueError("block tables must be 2-D")
        _need(tables, "block_tables", tables.dtype, tables.numel(), self.device)
        # rows outside the table are skipped by the kernel (no host sync here)
        check(lib().lnskv_append(C.byref(self.desc), _ptr(k_new), _ptr(v_new), _ptr(tok_seq),
                                 _ptr(tok_pos), n_tok, _ptr(tables), int(tables.shape[1]),
                                 int(tables.shape[0]), _stream(self.device)))

    def workspace_size(self, n_seq: int, n_heads: int, max_kv_len: int, split: int = 0) -> int:
        out = C.c_size_t()
        check(lib().lnskv_decode_workspace_size(C.byref(self.desc), n_seq, n_heads, max_kv_len, split,
                                                C.byref(out)))
        return out.value

    def _decode_common(self, q, tables, kv_len, p_start, n_heads):
        n_seq = int(kv_len.numel())
        _need(q, "q", torch.float32, n_seq * n_heads * self.head_dim, self.device)
        _need(kv_len, "kv_len", torch.int32, n_seq, self.device)
        if p_start is not None:
            _need(p_start, "p_start", torch.int32, n_seq, self.device)
        stride = self._tables(tables, n_seq)
        return n_seq, stride

    def decode(self, q, tables, kv_len, *, n_heads: int, max_kv_len: int, scale: float,
               p_start=None, split: int = 0, workspace=None, out=None) -> torch.Tensor:
        n_seq, stride = self._decode_common(q, tables, kv_len, p_start, n_heads)
        if out is None:
            out = torch.empty((n_seq, n_heads, self.head_dim), dtype=torch.float32, device=self.device)
        _need(out, "out", torch.float32, n_seq * n_heads * self.head_dim, self.device)
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(lib().lnskv_decode(C.byref(self.desc), _ptr(q), _ptr(out), _ptr(tables), stride,
                                 _ptr(kv_len), _ptr(p_start), n_seq, n_heads, max_kv_len, scale, split,
                                 _ptr(workspace), ws_bytes, _stream(self.device)))
        return out

    def append_decode(self, q, k_new, v_new, tables, kv_len, *, n_heads: int, max_kv_len: int,
                      scale: float, p_start=None, split: int = 0, workspace=None,
                      out=None) -> torch.Tensor:
        n_seq, stride = self._decode_common(q, tables, kv_len, p_start, n_heads)
        _need(k_new, "k_new", torch.float32, n_seq * self.row_elems, self.device)
        _need(v_new, "v_new", torch.float32, n_seq * self.row_elems, self.device)
        if out is None:
            out = torch.empty((n_seq, n_heads, self.head_dim), dtype=torch.float32, device=self.device)
        _need(out, "out", torch.float32, n_seq * n_heads * self.head_dim, self.device)
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(lib().lnskv_append_decode(C.byref(self.desc), _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(out),
                                        _ptr(tables), stride, _ptr(kv_len), _ptr(p_start), n_seq, n_heads,
                                        max_kv_len, scale, split, _ptr(workspace), ws_bytes,
                                        _stream(self.device)))
        return out

    def rope_decode_workspace_size(self, rope: "RopeTable", n_seq: int, n_heads: int, max_kv_len: int,
                                   split: int = 0) -> int:
        """Bytes of workspace lnskv_rope_append_decode / lnskv_gated_append_decode
        with this rope need (the decode's partials, then the rotated rows)."""
        out = C.c_size_t()
        check(lib().lnskv_rope_decode_workspace_size(C.byref(self.desc), C.byref(rope.desc), n_seq, n_heads,
                                                     max_kv_len, split, C.byref(out)))
        return out.value

    def rope_append_workspace_size(self, rope: "RopeTable", n_tok: int) -> int:
        out = C.c_size_t()
        check(lib().lnskv_rope_append_workspace_size(C.byref(self.desc), C.byref(rope.desc), n_tok, C.byref(out)))
        return out.value

    def rope_append(self, rope: "RopeTable", k_new, v_new, tok_seq, tok_pos, tables, workspace=None) -> None:
        """lnskv_rope_append: lnskv_append with K turned by tok_pos first
        (workspace None: the library's buffer for shapes that rotate first)."""
        n_tok = int(tok_seq.numel())
        _need(k_new, "k_new", torch.float32, n_tok * self.row_elems, self.device)
        _need(v_new, "v_new", torch.float32, n_tok * self.row_elems, self.device)
        _need(tok_seq, "tok_seq", torch.int32, n_tok, self.device)
        _need(tok_pos, "tok_pos", torch.int32, n_tok, self.device)
        if tables.dim() != 2:
            raise ValueError("block tables must be 2-D")
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(lib().lnskv_rope_append(C.byref(self.desc), C.byref(rope.desc), _ptr(k_new), _ptr(v_new),
                                      _ptr(tok_seq), _ptr(tok_pos), n_tok, _ptr(tables), int(tables.shape[1]),
                                      int(tables.shape[0]), _ptr(workspace), ws_bytes, _stream(self.device)))

    def rope_append_decode(self, rope: "RopeTable", q, k_new, v_new, tables, kv_len, *, n_heads: int,
                           max_kv_len: int, scale: float, p_start=None, split: int = 0, workspace=None,
                           out=None) -> torch.Tensor:
        """lnskv_rope_append_decode: q and k_new before RoPE; both turn by the
        new token's position kv_len-1, then append + decode."""
        n_seq, stride = self._decode_common(q, tables, kv_len, p_start, n_heads)
        _need(k_new, "k_new", torch.float32, n_seq * self.row_elems, self.device)
        _need(v_new, "v_new", torch.float32, n_seq * self.row_elems, self.device)
        if out is None:
            out = torch.empty((n_seq, n_heads, self.head_dim), dtype=torch.float32, device=self.device)
        _need(out, "out", torch.float32, n_seq * n_heads * self.head_dim, self.device)
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(lib().lnskv_rope_append_decode(C.byref(self.desc), C.byref(rope.desc), _ptr(q), _ptr(k_new),
                                             _ptr(v_new), _ptr(out), _ptr(tables), stride, _ptr(kv_len),
                                             _ptr(p_start), n_seq, n_heads, max_kv_len, scale, split,
                                             _ptr(workspace), ws_bytes, _stream(self.device)))
        return out

    def gated_append_decode(self, gate, q, k_new, v_new, tables, kv_len, *, n_heads: int, max_kv_len: int,
                            scale: float, rope: "RopeTable | None" = None, p_start=None, split: int = 0,
                            workspace=None, out=None) -> torch.Tensor:
        """lnskv_gated_append_decode: append + decode (RoPE first when `rope`
        is given) with the output multiplied by `gate` [n_seq][n_heads][d]."""
        n_seq, stride = self._decode_common(q, tables, kv_len, p_start, n_heads)
        _need(gate, "gate", torch.float32, n_seq * n_heads * self.head_dim, self.device)
        _need(k_new, "k_new", torch.float32, n_seq * self.row_elems, self.device)
        _need(v_new, "v_new", torch.float32, n_seq * self.row_elems, self.device)
        if out is None:
            out = torch.empty((n_seq, n_heads, self.head_dim), dtype=torch.float32, device=self.device)
        _need(out, "out", torch.float32, n_seq * n_heads * self.head_dim, self.device)
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(lib().lnskv_gated_append_decode(C.byref(self.desc), C.byref(rope.desc) if rope is not None else None,
                                              _ptr(gate), _ptr(q), _ptr(k_new), _ptr(v_new), _ptr(out),
                                              _ptr(tables), stride, _ptr(kv_len), _ptr(p_start), n_seq, n_heads,
                                              max_kv_len, scale, split, _ptr(workspace), ws_bytes,
                                              _stream(self.device)))
        return out

    def prefill_attention(self, q, chunks, tables, *, n_heads: int, scale: float, p_start=None, window: int = 0,
                          out=None) -> torch.Tensor:
        """lnskv_prefill_attention: q [n_tok][n_heads][d]; chunks int32
        [n_chunks][4] = (table row, first position, length, first token);
        window > 0: each query attends its own sliding window."""
        n_tok = q.numel() // (n_heads * self.head_dim)
        _need(q, "q", torch.float32, n_tok * n_heads * self.head_dim, self.device)
        if chunks.dtype != torch.int32 or chunks.dim() != 2 or chunks.shape[1] != 4 or not chunks.is_contiguous():
            raise ValueError("chunks must be a contiguous int32 [n_chunks][4] tensor")
        if tables.dim() != 2:
            raise ValueError("tables must be [n_rows][stride]")
        if out is None:
            out = torch.empty((n_tok, n_heads, self.head_dim), dtype=torch.float32, device=self.device)
        _need(out, "out", torch.float32, n_tok * n_heads * self.head_dim, self.device)
        check(lib().lnskv_prefill_attention(C.byref(self.desc), _ptr(q), _ptr(out), _ptr(chunks),
                                            int(chunks.shape[0]), n_tok, _ptr(tables), int(tables.shape[1]),
                                            int(tables.shape[0]), _ptr(p_start), window, n_heads, scale,
                                            _stream(self.device)))
        return out

    def attention_paged(self, q, k_in, v_in, block_table, pos: int, n_heads: int, p_start: int = 0,
                        out=None, dispatch: bool = False) -> torch.Tensor:
        """The reference's single-sequence call (encode_attention_paged_q8a,
        lns-metal/src/lib.rs:997-1043): append token `pos`, attend [p_start, pos]."""
        _need(q, "q", torch.float32, n_heads * self.head_dim, self.device)
        _need(k_in, "k_in", torch.float32, self.row_elems, self.device)
        _need(v_in, "v_in", torch.float32, self.row_elems, self.device)
        if block_table.numel() < pos // PAGE_SIZE + 1:
            raise ValueError("block table shorter than pos/16 + 1")
        _need(block_table, "block_table", block_table.dtype, block_table.numel(), self.device)
        if out is None:
            out = torch.empty((n_heads, self.head_dim), dtype=torch.float32, device=self.device)
        _need(out, "out", torch.float32, n_heads * self.head_dim, self.device)
        fn = lib().lnskv_dispatch_attention_paged if dispatch else lib().lnskv_attention_paged
        check(fn(_ptr(q), _ptr(k_in), _ptr(v_in), C.byref(self.desc), _ptr(block_table), _ptr(out), pos,
                 self.head_dim, n_heads, self.n_kv, p_start, _stream(self.device)))
        return out

    def page_copy(self, src, dst) -> None:
        n = int(src.numel())
        _need(src, "src", src.dtype, n, self.device)
        _need(dst, "dst", dst.dtype, n, self.device)
        check(lib().lnskv_page_copy(C.byref(self.desc), _ptr(src), _ptr(dst), n, _stream(self.device)))

    def gather(self, block_table_row, start: int, n_tok: int):
        """Tokens [start, start+n_tok) of one sequence as contiguous
        [n_tok][n_kv][d] tensors in page dtype (+ Q8A scales [n_tok][n_kv])."""
        if block_table_row.numel() * PAGE_SIZE < start + n_tok:
            raise ValueError("block table row shorter than the gathered range")
        _need(block_table_row, "block_table_row", block_table_row.dtype, block_table_row.numel(), self.device)
        td = TORCH_DTYPE[self.dtype]
        ko = torch.empty((n_tok, self.n_kv, self.head_dim), dtype=td, device=self.device)
        vo = torch.empty_like(ko)
        kso = vso = None
        if self.dtype == DTYPE_Q8A:
            kso = torch.empty((n_tok, self.n_kv), dtype=torch.float32, device=self.device)
            vso = torch.empty_like(kso)
        check(lib().lnskv_gather(C.byref(self.desc), _ptr(block_table_row), start, n_tok, _ptr(ko), _ptr(vo),
                                 _ptr(kso), _ptr(vso), _stream(self.device)))
        return ko, vo, kso, vso


class RopeTable:
    """The model's RoPE table on the device: inverse frequencies from
    lnskv_rope_inv_freqs (compute_rope_inv_freqs, engine.rs:139-195)."""

    def __init__(self, rotary_dim: int, theta: float, mode: int = 0, params=(1.0,), device="cuda"):
        import numpy as np

        p = np.zeros(4, np.float32)
        p[:len(params)] = params
        host = np.zeros(rotary_dim // 2, np.float32)
        check(lib().lnskv_rope_inv_freqs(rotary_dim, theta, mode, p.ctypes.data_as(C.c_void_p),
                                         host.ctypes.data_as(C.c_void_p)))
        self.rotary_dim = rotary_dim
        self.inv_freqs_host = host
        self.inv_freqs = torch.from_numpy(host).to(device)
        self.desc = Rope(self.inv_freqs.data_ptr(), rotary_dim)


class Q4LMatrix:
    """A rows x cols Q4_L weight matrix on the device: the disk super-blocks
    (134 bytes per 256 weights, row-major) repacked by lnskv_q4l_prepare
    (MetalContext::prepare_tensor, lns-metal/src/lib.rs:1255-1320)."""

    def __init__(self, disk_blocks, rows: int, cols: int, device="cuda"):
        import numpy as np

        disk = np.ascontiguousarray(disk_blocks, np.uint8).reshape(-1)
        n = rows * ((cols + 255) // 256)
        host = np.zeros(n * 144, np.uint8)
        check(lib().lnskv_q4l_prepare(disk.ctypes.data_as(C.c_void_p), disk.nbytes, rows, cols,
                                      host.ctypes.data_as(C.c_void_p)))
        self.rows, self.cols = rows, cols
        self.device = torch.device(device)
        self.blocks = torch.from_numpy(host).to(self.device)

    def workspace_size(self, n_vec: int) -> int:
        out = C.c_size_t()
        check(lib().lnskv_q4l_workspace_size(self.cols, n_vec, C.byref(out)))
        return out.value

    def gemv_accumulate(self, x: torch.Tensor, y: torch.Tensor, workspace=None) -> torch.Tensor:
        """lnskv_q4l_gemv_accumulate: y[v] += W x[v] for every row v of x
        [n_vec][>= cols] into y [n_vec][>= rows] (rows of both unit-stride);
        workspace None: the library's buffer."""
        if x.dim() != 2 or y.dim() != 2 or x.shape[0] != y.shape[0]:
            raise ValueError("x and y must be [n_vec][...] with the same n_vec")
        if x.dtype != torch.float32 or y.dtype != torch.float32 or x.stride(1) != 1 or y.stride(1) != 1:
            raise ValueError("x and y must be float32 with unit-stride rows")
        if x.shape[1] < self.cols or y.shape[1] < self.rows:
            raise ValueError("x rows need >= cols entries and y rows >= rows entries")
        ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
        check(lib().lnskv_q4l_gemv_accumulate(self.blocks.data_ptr(), x.data_ptr(), y.data_ptr(), self.rows,
                                              self.cols, int(x.shape[0]), int(x.stride(0)), int(y.stride(0)),
                                              _ptr(workspace), ws_bytes, _stream(self.device)))
        return y


def sync(device=None) -> None:
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    check(lib().lnskv_sync(_stream(dev)))


__all__ = ["PagedKV", "sync", "DTYPE_F32", "DTYPE_F16", "DTYPE_Q8A", "TORCH_DTYPE"]
