"""Python loader of the CPU oracle (oracle/liblnskv_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, always as the checker, never as the thing
measured on the GPU or shipped.  The C source (lnskv_oracle.c) restates the
reference algorithm and cites the reference lines it follows.

All arrays are host numpy arrays.  Page pools use the reference layout
[num_pages][16][n_kv][d] (f32, f16 bits as uint16, or int8 + f32 scales).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblnskv_oracle.so")

F32, F16, Q8A = 0, 1, 2
NP_DTYPE = {F32: np.float32, F16: np.uint16, Q8A: np.int8}
NO_PAGE = 0xFFFFFFFF


class OrcPages(C.Structure):
    _fields_ = [("k_pages", C.c_void_p), ("v_pages", C.c_void_p), ("k_scales", C.c_void_p),
                ("v_scales", C.c_void_p), ("num_pages", C.c_uint32), ("n_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("dtype", C.c_int32)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i32, u32 = C.c_void_p, C.c_int, C.c_uint32
        P = C.POINTER(OrcPages)
        sig = {
            "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
            "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
            "orc_f16_check_range": (C.c_uint64, [C.c_uint64, C.c_uint64, i32]),
            "orc_q8a_quantize": (None, [vp, i32, vp, vp]),
            "orc_f32_to_f16_array": (None, [vp, C.c_size_t, vp, i32]),
            "orc_f16_of_patterns": (None, [C.c_uint64, C.c_size_t, vp, i32]),
            "orc_pool_new": (vp, [u32]),
            "orc_pool_delete": (None, [vp]),
            "orc_pool_alloc": (i32, [vp, C.POINTER(u32)]),
            "orc_pool_free_page": (None, [vp, u32]),
            "orc_pool_reset": (None, [vp]),
            "orc_pool_num_free": (u32, [vp]),
            "orc_ensure_kv_page": (i32, [vp, vp, C.POINTER(i32), i32, i32]),
            "orc_evict_kv_pages": (None, [vp, vp, i32, i32, i32]),
            "orc_kv_p_start": (i32, [i32, i32]),
            "orc_append": (i32, [P, vp, vp, vp, vp, i32, vp, i32, i32]),
            "orc_gather": (i32, [P, vp, i32, i32, vp, vp, vp, vp]),
            "orc_page_copy": (None, [P, vp, vp, i32]),
            "orc_decode_refscan": (None, [P, vp, vp, vp, i32, vp, vp, i32, i32, C.c_float, i32]),
            "orc_decode_f64": (None, [P, vp, vp, vp, i32, vp, vp, i32, i32, C.c_double, i32]),
            "orc_decode_split_f64": (None, [P, vp, vp, vp, i32, vp, vp, i32, i32, C.c_double, i32]),
            "orc_append_decode_refscan": (None, [P, vp, vp, vp, vp, vp, i32, vp, vp, i32, i32, C.c_float, i32]),
            "orc_max_threads": (i32, []),
            "orc_rope_inv_freqs": (None, [i32, C.c_float, i32, vp, vp]),
            "orc_rope_apply": (None, [vp, i32, i32, i32, i32, vp, i32, vp]),
            "orc_rope_sincos": (None, [C.c_float, vp, vp]),
            "orc_split_gated_query": (None, [vp, vp, vp, i32, i32, i32]),
            "orc_q4l_prepare": (None, [vp, i32, vp]),
            "orc_q4l_decode_block": (None, [vp, vp]),
            "orc_q4l_gemv_f64": (None, [vp, vp, i32, vp, i32, vp, i32, i32, i32]),
            "orc_q4l_decode_matrix": (None, [vp, i32, i32, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None) -> C.c_void_p:
    if a is None:
        return C.c_void_p(0)
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the oracle must be C-contiguous"
    return C.c_void_p(a.ctypes.data)


class HostPages:
    """Host copy of one layer's pools, in the reference layout."""

    def __init__(self, k, v, ks=None, vs=None, dtype=F16):
        self.k = np.ascontiguousarray(k)
        self.v = np.ascontiguousarray(v)
        self.ks = None if ks is None else np.ascontiguousarray(ks, dtype=np.float32)
        self.vs = None if vs is None else np.ascontiguousarray(vs, dtype=np.float32)
        self.dtype = dtype
        num_pages, page, n_kv, d = self.k.shape
        assert page == 16
        self.num_pages, self.n_kv, self.head_dim = num_pages, n_kv, d
        self.desc = OrcPages(self.k.ctypes.data, self.v.ctypes.data,
                             self.ks.ctypes.data if self.ks is not None else None,
                             self.vs.ctypes.data if self.vs is not None else None,
                             num_pages, n_kv, d, dtype)

    @classmethod
    def zeros(cls, num_pages, n_kv, d, dtype):
        shape = (num_pages, 16, n_kv, d)
        k = np.zeros(shape, NP_DTYPE[dtype])
        v = np.zeros(shape, NP_DTYPE[dtype])
        ks = vs = None
        if dtype == Q8A:
            ks = np.zeros((num_pages * 16, n_kv), np.float32)
            vs = np.zeros((num_pages * 16, n_kv), np.float32)
        return cls(k, v, ks, vs, dtype)

    def copy(self):
        return HostPages(self.k.copy(), self.v.copy(), None if self.ks is None else self.ks.copy(),
                         None if self.vs is None else self.vs.copy(), self.dtype)


def f32_to_f16_bits(x: np.ndarray, n_threads: int | None = None) -> np.ndarray:
    """Round-to-nearest-even binary16 bits of f32 values."""
    flat = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(flat.shape, np.uint16)
    lib().orc_f32_to_f16_array(_p(flat), flat.size, _p(out), n_threads or os.cpu_count())
    return out.reshape(np.shape(x))


def f16_of_patterns(lo: int, n: int, n_threads: int | None = None) -> np.ndarray:
    """binary16 bits of the f32 bit patterns lo, lo+1, ..., lo+n-1."""
    out = np.empty(n, np.uint16)
    lib().orc_f16_of_patterns(lo, n, _p(out), n_threads or os.cpu_count())
    return out


def f16_check_range(lo: int, hi: int, n_threads: int | None = None) -> int:
    """Mismatches of the restatement vs the x86 F16C converter over [lo, hi)."""
    return int(lib().orc_f16_check_range(lo, hi, n_threads or os.cpu_count()))


def q8a_quantize(x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    q = np.zeros(x.shape, np.int8)
    sc = np.zeros(1, np.float32)
    lib().orc_q8a_quantize(_p(x), x.size, _p(q), _p(sc))
    return q, float(sc[0])


def append(pages: HostPages, k_new, v_new, tok_seq, tok_pos, tables) -> int:
    k_new = np.ascontiguousarray(k_new, np.float32)
    v_new = np.ascontiguousarray(v_new, np.float32)
    tok_seq = np.ascontiguousarray(tok_seq, np.int32)
    tok_pos = np.ascontiguousarray(tok_pos, np.int32)
    tables = np.ascontiguousarray(tables, np.uint32)
    return lib().orc_append(C.byref(pages.desc), _p(k_new), _p(v_new), _p(tok_seq), _p(tok_pos),
                            len(tok_seq), _p(tables), tables.shape[1], tables.shape[0])


def gather(pages: HostPages, bt_row, start: int, n_tok: int):
    bt_row = np.ascontiguousarray(bt_row, np.uint32)
    shape = (n_tok, pages.n_kv, pages.head_dim)
    ko = np.zeros(shape, pages.k.dtype)
    vo = np.zeros(shape, pages.v.dtype)
    kso = vso = None
    if pages.dtype == Q8A:
        kso = np.zeros((n_tok, pages.n_kv), np.float32)
        vso = np.zeros((n_tok, pages.n_kv), np.float32)
    lib().orc_gather(C.byref(pages.desc), _p(bt_row), start, n_tok, _p(ko), _p(vo), _p(kso), _p(vso))
    return ko, vo, kso, vso


def page_copy(pages: HostPages, src, dst) -> None:
    src = np.ascontiguousarray(src, np.uint32)
    dst = np.ascontiguousarray(dst, np.uint32)
    lib().orc_page_copy(C.byref(pages.desc), _p(src), _p(dst), len(src))


def _dec_args(q, tables, kv_len, p_start):
    q = np.ascontiguousarray(q, np.float32)
    tables = np.ascontiguousarray(tables, np.uint32)
    kv_len = np.ascontiguousarray(kv_len, np.int32)
    p_start = None if p_start is None else np.ascontiguousarray(p_start, np.int32)
    return q, tables, kv_len, p_start


def decode_refscan(pages: HostPages, q, tables, kv_len, p_start=None, scale=None, n_threads=None):
    """Reference-order f32 online softmax (lns_decode.metal:595-645)."""
    q, tables, kv_len, p_start = _dec_args(q, tables, kv_len, p_start)
    n_seq, n_heads, d = q.shape
    out = np.zeros_like(q)
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    lib().orc_decode_refscan(C.byref(pages.desc), _p(q), _p(out), _p(tables), tables.shape[1], _p(kv_len),
                             _p(p_start), n_seq, n_heads, scale, n_threads or os.cpu_count())
    return out


def decode_f64(pages: HostPages, q, tables, kv_len, p_start=None, scale=None, n_threads=None):
    """f64 softmax(q.K^T*scale).V over the exact stored values (ground truth)."""
    q, tables, kv_len, p_start = _dec_args(q, tables, kv_len, p_start)
    n_seq, n_heads, d = q.shape
    out = np.zeros(q.shape, np.float64)
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    lib().orc_decode_f64(C.byref(pages.desc), _p(q), _p(out), _p(tables), tables.shape[1], _p(kv_len),
                         _p(p_start), n_seq, n_heads, scale, n_threads or os.cpu_count())
    return out


def decode_split_f64(pages: HostPages, q, tables, kv_len, split: int, p_start=None, scale=None):
    q, tables, kv_len, p_start = _dec_args(q, tables, kv_len, p_start)
    n_seq, n_heads, d = q.shape
    out = np.zeros(q.shape, np.float64)
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    lib().orc_decode_split_f64(C.byref(pages.desc), _p(q), _p(out), _p(tables), tables.shape[1], _p(kv_len),
                               _p(p_start), n_seq, n_heads, scale, split)
    return out


def append_decode_refscan(pages: HostPages, q, k_new, v_new, tables, kv_len, p_start=None, scale=None,
                          n_threads=None):
    q, tables, kv_len, p_start = _dec_args(q, tables, kv_len, p_start)
    k_new = np.ascontiguousarray(k_new, np.float32)
    v_new = np.ascontiguousarray(v_new, np.float32)
    n_seq, n_heads, d = q.shape
    out = np.zeros_like(q)
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    lib().orc_append_decode_refscan(C.byref(pages.desc), _p(q), _p(k_new), _p(v_new), _p(out), _p(tables),
                                    tables.shape[1], _p(kv_len), _p(p_start), n_seq, n_heads, scale,
                                    n_threads or os.cpu_count())
    return out


def stored_values(pages: HostPages, which_v: bool) -> np.ndarray:
    """Pool contents as f64 values [num_pages*16][n_kv][d] (Q8A dequantized)."""
    a = pages.v if which_v else pages.k
    if pages.dtype == F32:
        return a.reshape(-1, pages.n_kv, pages.head_dim).astype(np.float64)
    if pages.dtype == F16:
        return a.view(np.float16).reshape(-1, pages.n_kv, pages.head_dim).astype(np.float64)
    sc = pages.vs if which_v else pages.ks
    return a.reshape(-1, pages.n_kv, pages.head_dim).astype(np.float64) * sc[:, :, None].astype(np.float64)


def rel_err_elements(out, ref, floor: float = 1e-6) -> np.ndarray:
    """Element-wise relative error |o_i - r_i| / max(|r_i|, floor)."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(out - ref) / np.maximum(np.abs(ref), floor)


def rel_err_rows(out, ref) -> np.ndarray:
    """Per (sequence, query head) row: max_i |o_i - r_i| / max(max_i |r_i|, 1e-30)."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    num = np.abs(out - ref).max(axis=-1)
    den = np.maximum(np.abs(ref).max(axis=-1), 1e-30)
    return num / den


class Pool:
    """The oracle's PagePool (engine.rs:20-44)."""

    def __init__(self, capacity: int):
        self.h = lib().orc_pool_new(capacity)

    def __del__(self):
        try:
            lib().orc_pool_delete(self.h)
        except Exception:
            pass

    def alloc(self):
        out = C.c_uint32()
        return out.value if lib().orc_pool_alloc(self.h, C.byref(out)) == 0 else None

    def free_page(self, idx: int) -> None:
        lib().orc_pool_free_page(self.h, idx)

    def reset(self) -> None:
        lib().orc_pool_reset(self.h)

    @property
    def num_free(self) -> int:
        return lib().orc_pool_num_free(self.h)


ROPE_DEFAULT, ROPE_LINEAR, ROPE_LLAMA3, ROPE_YARN = 0, 1, 2, 3


def rope_inv_freqs(rotary_dim: int, theta: float, mode: int = ROPE_DEFAULT, params=(1.0,)) -> np.ndarray:
    """compute_rope_inv_freqs (engine.rs:139-195): float32[rotary_dim // 2]."""
    p = np.zeros(4, np.float32)
    p[:len(params)] = params
    out = np.zeros(rotary_dim // 2, np.float32)
    lib().orc_rope_inv_freqs(rotary_dim, theta, mode, _p(p), _p(out))
    return out


def rope_sincos(theta) -> tuple[np.ndarray, np.ndarray]:
    """orc_rope_sincos over an array of f32 angles: (sin, cos) float32."""
    th = np.ascontiguousarray(theta, np.float32).ravel()
    sn = np.empty_like(th)
    cs = np.empty_like(th)
    a, b = C.c_float(), C.c_float()
    for i, t in enumerate(th):
        lib().orc_rope_sincos(float(t), C.byref(a), C.byref(b))
        sn[i], cs[i] = a.value, b.value
    return sn, cs


def rope_apply(x, rotary_dim: int, inv_freqs, pos) -> np.ndarray:
    """apply_cpu_rope_with_freqs (engine.rs:200-229) on a copy of x
    [rows][heads][head_dim] (float32); row r rotated by position pos[r]."""
    y = np.array(x, dtype=np.float32, copy=True, order="C")
    rows, heads, d = y.shape
    inv = np.ascontiguousarray(inv_freqs, np.float32)
    p = np.ascontiguousarray(pos, np.int32)
    assert p.shape == (rows,)
    lib().orc_rope_apply(_p(y), rows, heads, d, rotary_dim, _p(inv), len(inv), _p(p))
    return y


def split_gated_query(x, heads: int, head_dim: int):
    """split_gated_query_interleaved (engine.rs:287-307): x [rows][heads][2*head_dim]
    float32 -> (q, gate) [rows][heads][head_dim], gate = 1/(1+exp(-logit)) in f32."""
    a = np.ascontiguousarray(x, np.float32).reshape(-1, heads, 2 * head_dim)
    rows = a.shape[0]
    q = np.empty((rows, heads, head_dim), np.float32)
    g = np.empty((rows, heads, head_dim), np.float32)
    lib().orc_split_gated_query(_p(a), _p(q), _p(g), rows, heads, head_dim)
    return q, g


Q4L_DISK_BYTES, Q4L_DEV_BYTES = 134, 144


def q4l_prepare(disk) -> np.ndarray:
    """prepare_tensor's Q4L repack (lns-metal/src/lib.rs:1296-1315): disk
    super-blocks (134 bytes each) -> device blocks (144 bytes each)."""
    d = np.ascontiguousarray(disk, np.uint8).reshape(-1)
    n = d.size // Q4L_DISK_BYTES
    out = np.zeros(n * Q4L_DEV_BYTES, np.uint8)
    lib().orc_q4l_prepare(_p(d), n, _p(out))
    return out


def q4l_decode_block(dev_block) -> np.ndarray:
    """The kernel's weights of one device block (lns_decode_byte, lns_decode.metal:38-48)."""
    b = np.ascontiguousarray(dev_block, np.uint8).reshape(-1)
    assert b.size == Q4L_DEV_BYTES
    w = np.zeros(256, np.float32)
    lib().orc_q4l_decode_block(_p(b), _p(w))
    return w


def q4l_gemv_f64(dev_blocks, x, y_in, rows: int, cols: int) -> np.ndarray:
    """y_in + W x in float64 for every vector of x [n_vec][cols] (W: rows x cols device blocks)."""
    blk = np.ascontiguousarray(dev_blocks, np.uint8).reshape(-1)
    xv = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
    yv = np.ascontiguousarray(y_in, np.float32).reshape(-1, rows)
    n_vec = xv.shape[0]
    assert yv.shape[0] == n_vec and blk.size == rows * (cols // 256) * Q4L_DEV_BYTES
    out = np.zeros((n_vec, rows), np.float64)
    lib().orc_q4l_gemv_f64(_p(blk), _p(xv), cols, _p(yv), rows, _p(out), rows, cols, n_vec)
    return out


def q4l_decode_matrix(dev_blocks, rows: int, cols: int) -> np.ndarray:
    """The kernel's weights of a rows x cols device matrix (float32)."""
    blk = np.ascontiguousarray(dev_blocks, np.uint8).reshape(-1)
    assert blk.size == rows * (cols // 256) * Q4L_DEV_BYTES
    w = np.zeros((rows, cols), np.float32)
    lib().orc_q4l_decode_matrix(_p(blk), rows, cols, _p(w))
    return w
