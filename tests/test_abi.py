"""The C ABI without a GPU: the library loads, exports every symbol the header
declares, and rejects bad arguments before touching the device."""
import ctypes as C
import os
import re

import pytest

from lnskv import _lib
from lnskv._lib import Pages

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lnskv.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lnskv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_api():
    syms = declared_symbols()
    assert "lnskv_append_decode" in syms and "lnskv_page_pool_alloc" in syms
    assert len(syms) >= 30


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_version_and_page_bytes():
    lib = _lib.lib()
    assert b"gfx950" in lib.lnskv_version()
    p = Pages(None, None, None, None, 16384, 8, 128, _lib.DTYPE_F16)
    assert lib.lnskv_page_bytes(C.byref(p)) == 16 * 8 * 128 * 2


def _status(fn, *args):
    return fn(*args), _lib.last_error()


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = _lib.lib()
    bad_dim = Pages(1, 1, None, None, 64, 4, 96, _lib.DTYPE_F16)
    rc, msg = _status(lib.lnskv_decode, C.byref(bad_dim), 1, 1, 1, 4, 1, None, 1, 32, 16, 0.1, 0, None, 0, None)
    assert rc == _lib.ERR_UNSUPPORTED and "head_dim" in msg
    good = Pages(1, 1, None, None, 64, 4, 64, _lib.DTYPE_F16)
    rc, msg = _status(lib.lnskv_decode, C.byref(good), 1, 1, 1, 4, 1, None, 1, 30, 16, 0.1, 0, None, 0, None)
    assert rc == _lib.ERR_INVALID and "multiple" in msg
    rc, msg = _status(lib.lnskv_decode, C.byref(good), 1, 1, 1, 4, 1, None, 1, 32, 16, 0.1, 24, None, 0, None)
    assert rc == _lib.ERR_INVALID and "split" in msg
    rc, msg = _status(lib.lnskv_decode, C.byref(good), 1, 1, 1, 4, 1, None, 1, 32, 16, -1.0, 0, None, 0, None)
    assert rc == _lib.ERR_INVALID and "scale" in msg
    rc, _ = _status(lib.lnskv_decode, C.byref(good), None, 1, 1, 4, 1, None, 1, 32, 16, 0.1, 0, None, 0, None)
    assert rc == _lib.ERR_INVALID
    q8_no_scales = Pages(1, 1, None, None, 64, 4, 64, _lib.DTYPE_Q8A)
    rc, msg = _status(lib.lnskv_append, C.byref(q8_no_scales), 1, 1, 1, 1, 1, 1, 4, 1, None)
    assert rc == _lib.ERR_INVALID and "scales" in msg
    rc, msg = _status(lib.lnskv_attention_paged, 1, 1, 1, C.byref(good), 1, 1, 10, 128, 32, 4, 0, None)
    assert rc == _lib.ERR_INVALID and "differ" in msg
    rc, _ = _status(lib.lnskv_gather, C.byref(good), 1, 0, 4, 1, 1, 1, 1, None)
    assert rc == _lib.ERR_INVALID  # scale outputs only for Q8A
    # the load probe reads 256-byte kv-head rows only (f16 x 64 dims: 128 bytes)
    rc, msg = _status(lib.lnskv_read_units, C.byref(good), 1, 1, 1, 4, 1, None)
    assert rc == _lib.ERR_UNSUPPORTED and "256" in msg
    rc, _ = _status(lib.lnskv_read_units, C.byref(good), 1, 1, 1, 0, 1, None)
    assert rc == _lib.ERR_INVALID
    # the read ceiling: size, alignment, depth and occupancy are checked before any launch
    rc, msg = _status(lib.lnskv_read_stream, 16, 24, 4, 4, 16, None)
    assert rc == _lib.ERR_INVALID and "multiple of 16" in msg
    rc, msg = _status(lib.lnskv_read_stream, 8, 32, 4, 4, 16, None)
    assert rc == _lib.ERR_INVALID and "aligned" in msg
    rc, msg = _status(lib.lnskv_read_stream, 16, 32, 4, 9, 16, None)
    assert rc == _lib.ERR_INVALID and "blocks_per_cu" in msg
    rc, _ = _status(lib.lnskv_read_stream, None, 32, 4, 4, 16, None)
    assert rc == _lib.ERR_INVALID
    rc, msg = _status(lib.lnskv_gated_append_decode, C.byref(good), None, None, 1, 1, 1, 1, 1, 4, 1, None, 1,
                      32, 16, 0.1, 0, None, 0, None)
    assert rc == _lib.ERR_INVALID and "gate" in msg
    rc, _ = _status(lib.lnskv_split_gated_query, 1, 1, 1, 0, 4, 64, None)
    assert rc == _lib.ERR_INVALID
    # chunked prefill: head_dim 128 or 256 only; Q8A scale arrays must stay under 2 GiB
    # (num_pages * 16 * n_kv * 4 bytes: 2^22 pages x 8 kv heads is exactly 2 GiB)
    for pages, dt, d, want, text in ((64, _lib.DTYPE_F16, 64, _lib.ERR_UNSUPPORTED, "head_dim"),
                                     (1 << 22, _lib.DTYPE_Q8A, 128, _lib.ERR_UNSUPPORTED, "2 GiB"),
                                     (64, _lib.DTYPE_F32, 128, _lib.ERR_UNSUPPORTED, "f16 and Q8A")):
        desc = Pages(16, 16, 16, 16, pages, 8, d, dt)
        rc, msg = _status(lib.lnskv_prefill_attention, C.byref(desc), 16, 16, 16, 1, 1, 16, 1, 1, None, 0, 32,
                          0.1, None)
        assert rc == want and text in msg, (rc, msg)


def test_workspace_header_constant_matches_the_header():
    text = open(os.path.join(ROOT, "include", "lnskv.h")).read()
    m = re.search(r"#define LNSKV_WORKSPACE_HEADER_BYTES (\d+)", text)
    assert m and int(m.group(1)) == _lib.WORKSPACE_HEADER_BYTES


def test_workspace_size_formula():
    lib = _lib.lib()
    p = Pages(None, None, None, None, 16384, 8, 128, _lib.DTYPE_F16)
    out = C.c_size_t()
    assert lib.lnskv_decode_workspace_size(C.byref(p), 32, 32, 4097, 256, C.byref(out)) == 0
    # the counter header, then partial numerators + (max, sum)
    assert out.value == _lib.WORKSPACE_HEADER_BYTES + 32 * 32 * 17 * (128 + 2) * 4
    assert lib.lnskv_decode_workspace_size(C.byref(p), 4, 32, 200, 256, C.byref(out)) == 0
    assert out.value == 0  # one partition: no partials


def test_q4l_workspace_size_formula():
    """The Q4L GEMV workspace: none below 8 blocks a row (no split); else the
    arrival counts, then partial sums for fewer than 2 x 256 workgroups of
    64 rows (32 rows with one tile) x 16 vectors per tile (up to 4 tiles a
    launch)."""
    lib = _lib.lib()
    out = C.c_size_t()
    for cols, n_vec, want in [(256, 1, 0), (1792, 64, 0),
                              (2048, 1, 512), (4096, 16, 512), (4096, 17, 2 * 1024),
                              (4096, 32, 2 * 1024), (4096, 64, 4 * 1024), (4096, 300, 4 * 1024)]:
        assert lib.lnskv_q4l_workspace_size(cols, n_vec, C.byref(out)) == 0
        assert out.value == (0 if want == 0 else _lib.WORKSPACE_HEADER_BYTES + 2 * 256 * want * 4), (cols, n_vec)
    assert lib.lnskv_q4l_workspace_size(300, 1, C.byref(out)) == _lib.ERR_UNSUPPORTED


@pytest.mark.parametrize("name", ["lnskv_last_error", "lnskv_version"])
def test_string_entry_points(name):
    assert isinstance(getattr(_lib.lib(), name)(), bytes)


def test_rope_workspace_queries_and_reserve_arguments():
    lib = _lib.lib()
    pages = Pages(None, None, None, None, 64, 8, 128, _lib.DTYPE_Q8A)
    out = C.c_size_t(123)
    rc, msg = _status(lib.lnskv_rope_decode_workspace_size, C.byref(pages), None, 4, 32, 100, 0, C.byref(out))
    assert rc == _lib.ERR_INVALID and "rope" in msg and out.value == 0
    rope = _lib.Rope(C.c_void_p(256), 128)
    assert lib.lnskv_rope_append_workspace_size(C.byref(pages), C.byref(rope), 10, C.byref(out)) == 0
    assert out.value == 10 * 8 * 128 * 4          # the rotated K rows
    odd = _lib.Rope(C.c_void_p(256), 127)
    rc, msg = _status(lib.lnskv_rope_append_workspace_size, C.byref(pages), C.byref(odd), 10, C.byref(out))
    assert rc == _lib.ERR_INVALID and "rotary_dim" in msg
