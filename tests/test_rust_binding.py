"""The Rust drop-in crate (lns-ml_amd/lns-kv-hip) against the C ABI, without
cargo (neither this image nor the GPU box has a Rust toolchain): its
`extern "C"` block must declare every entry point of include/lnskv.h with the
header's parameter names, C types mapped one to one, and return types; its
constants and #[repr(C)] structs must equal the header's; the safe layer may
call only what sys.rs declares; the crate builds offline (no crates.io
dependencies) and links liblnskv and the HIP runtime."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lnskv.h")
CRATE = os.path.join(ROOT, "lns-ml_amd", "lns-kv-hip")

STRUCTS = {"lnskv_pages": "LnskvPages", "lnskv_rope": "LnskvRope", "lnskv_page_pool": "LnskvPagePool",
           "lnskv_block_tables": "LnskvBlockTables"}
SCALARS = {"int": "c_int", "int32_t": "i32", "int64_t": "i64", "uint32_t": "u32", "size_t": "usize",
           "float": "f32", "void": "c_void", "char": "c_char"}


def rust_type(c: str) -> str:
    c = " ".join(c.split())
    if c == "lnskv_stream_t":
        return "HipStream"
    const = c.startswith("const ")
    if const:
        c = c[len("const "):]
    stars = c.count("*")
    base = STRUCTS.get(c.replace("*", "").strip()) or SCALARS[c.replace("*", "").strip()]
    for i in range(stars):
        base = ("*const " if (i == 0 and const) else "*mut ") + base
    return base


def header_decls():
    t = open(HEADER).read()
    t = re.sub(r"/\*.*?\*/", "", t, flags=re.S)
    t = re.sub(r"#.*", "", t)
    out = {}
    for full, name, args in re.findall(r"([A-Za-z_][\w\s\*]*?\b(lnskv_\w+)\s*\(([^;{]*?)\)\s*;)", t, flags=re.S):
        ret = " ".join(full[:full.index(name)].split())
        params = []
        args = " ".join(args.split())
        if args != "void":
            for a in args.split(","):
                m = re.match(r"(.*?)(\w+)$", a.strip())
                params.append((m.group(2), rust_type(m.group(1))))
        out[name] = (params, None if ret == "void" else rust_type(ret))
    return out


def rust_decls():
    t = open(os.path.join(CRATE, "src", "sys.rs")).read()
    block = t[t.index('extern "C" {'):]
    out = {}
    for name, args, ret in re.findall(r"pub fn (lnskv_\w+)\((.*?)\)\s*(?:->\s*([^;]+?))?\s*;", block, flags=re.S):
        params = []
        for a in [x.strip() for x in args.split(",") if x.strip()]:
            n, ty = a.split(":", 1)
            params.append((n.strip(), " ".join(ty.split())))
        out[name] = (params, ret.strip() if ret else None)
    return out


def test_every_header_entry_point_is_declared_identically():
    h, r = header_decls(), rust_decls()
    assert len(h) >= 50
    assert sorted(h) == sorted(r), (sorted(set(h) ^ set(r)))
    for name, (params, ret) in h.items():
        assert r[name] == (params, ret), name


def test_declarations_follow_the_header_order():
    h = list(header_decls())
    r = list(rust_decls())
    assert h == r


def _c_consts():
    """#define'd numbers and enum constants of the header."""
    vals = {}
    for line in open(HEADER):
        m = re.match(r"#define (LNSKV_\w+)[ \t]+(\S.*?)\s*(?:/\*.*)?$", line)
        if not m:
            continue
        v = m.group(2).replace("(size_t)", "")
        v = re.sub(r"(0x[0-9A-Fa-f]+)u\b", r"\1", v)
        vals[m.group(1)] = int(eval(v, {}))
    body = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, v in re.findall(r"\b(LNSKV_[A-Z0-9_]+)\s*=\s*(-?\d+)", body):
        vals[name] = int(v)
    return vals


def test_constants_match_the_header():
    c = _c_consts()
    t = open(os.path.join(CRATE, "src", "sys.rs")).read()
    r = {}
    for name, v in re.findall(r"pub const (LNSKV_\w+):\s*[\w:]+\s*=\s*([^;]+);", t):
        r[name] = eval(v.replace("_", ""), {}) if name != "LNSKV_NO_PAGE" else int(v.replace("_", ""), 0)
    assert len(c) >= 19
    for name, v in c.items():
        assert name in r, name
        assert r[name] == v, (name, r[name], v)


def _c_struct(name):
    t = open(HEADER).read()
    body = re.search(r"typedef struct " + name + r" \{(.*?)\}", t, flags=re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for decl in [d.strip() for d in body.split(";") if d.strip()]:
        m = re.match(r"(.*?)(\w+)$", decl)
        fields.append((m.group(2), rust_type(m.group(1))))
    return fields


def _rust_struct(name):
    t = open(os.path.join(CRATE, "src", "sys.rs")).read()
    m = re.search(r"#\[repr\(C\)\][^{]*?pub struct " + name + r" \{(.*?)\}", t, flags=re.S)
    return [(n, " ".join(ty.split())) for n, ty in re.findall(r"pub (\w+):\s*([^,]+),", m.group(1))]


@pytest.mark.parametrize("c_name", ["lnskv_pages", "lnskv_rope"])
def test_repr_c_structs_match(c_name):
    assert _rust_struct(STRUCTS[c_name]) == _c_struct(c_name)


def test_safe_layer_calls_only_declared_functions():
    declared = set(rust_decls())
    for f in ("lib.rs", "paging.rs", "hip.rs"):
        src = open(os.path.join(CRATE, "src", f)).read()
        used = set(re.findall(r"sys::(lnskv_\w+)", src))
        assert used <= declared, (f, used - declared)
    lib_rs = open(os.path.join(CRATE, "src", "lib.rs")).read()
    # the reference's call and its waiting form are wrapped with its argument order
    for fn in ("attention_paged", "dispatch_attention_paged"):
        sig = re.search(r"pub fn " + fn + r"\(\s*&self,(.*?)\)\s*->", lib_rs, flags=re.S).group(1)
        names = [a.split(":")[0].strip() for a in sig.split(",") if a.strip()]
        assert names == ["q", "k_in", "v_in", "block_table_dev", "out", "pos", "head_dim", "n_heads",
                         "n_kv_heads", "p_start", "stream"], fn


def test_q4l_wrapper_follows_the_engine_call():
    """Q4lMatrix::gemv_accumulate takes gemv_accumulate_multirow_enc's
    operands in its order (attn_out, then the x it adds to, engine.rs:
    3433-3446) and passes the header's dense strides; its workspace is zeroed
    before first use (the arrival counts)."""
    lib_rs = open(os.path.join(CRATE, "src", "lib.rs")).read()
    sig = re.search(r"pub fn gemv_accumulate\(\s*&mut self,(.*?)\)\s*->", lib_rs, flags=re.S).group(1)
    names = [a.split(":")[0].strip() for a in sig.split(",") if a.strip()]
    assert names == ["attn_out_dev", "x_dev", "n_vec", "stream"]
    body = lib_rs.split("pub fn gemv_accumulate(", 1)[1]
    assert "DeviceBuffer::zeroed" in body and "sys::lnskv_q4l_workspace_size" in body
    assert "sys::lnskv_q4l_prepare" in lib_rs.split("pub fn prepare(", 1)[1]


def test_crate_builds_offline_and_links_the_library():
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    deps = toml.split("[dependencies]", 1)[1]
    assert not [ln for ln in deps.splitlines() if ln.strip() and not ln.strip().startswith("#")]
    build = open(os.path.join(CRATE, "build.rs")).read()
    assert "rustc-link-lib=dylib=lnskv" in build and "rustc-link-lib=dylib=amdhip64" in build
    for f in ("src/lib.rs", "src/sys.rs", "src/paging.rs", "src/hip.rs", "tests/gpu_attention.rs"):
        assert os.path.exists(os.path.join(CRATE, f)), f


def test_paging_mirrors_the_host_library_constants():
    src = open(os.path.join(CRATE, "src", "paging.rs")).read()
    assert "pub const PAGE_SIZE: usize = 16;" in src and "pub const NO_PAGE: u32 = u32::MAX;" in src
    # the exhaustion message is the reference's text (engine.rs:2969-2971)
    assert 'format!("KV page pool exhausted at layer {layer} (pos={pos})")' in src
