"""The cross-workgroup merge protocol's code generation (CPU only: hipcc
cross-compiles gfx950 assembly here).

decode_wg_kernel (partial rows and arrival counts) and q4l_gemv_acc_kernel
(split partial sums) rely on relaxed agent-scope atomics instead of
release/acquire fences, whose agent-scope forms on gfx950 write back or
invalidate a whole XCD's L2.  That is sound only while the primitives compile
as checked here, with the library's own device flags: the row stores and loads
carry sc1 (through to the memory side every XCD shares), the count is a
returning atomic issued after an s_waitcnt vmcnt(0) that follows the row
stores, and no L2 write-back or invalidate appears.  tests/native/
merge_protocol.hip holds the primitives in the kernels' order."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"
DEVFLAGS = ["-O3", "-std=c++17", "-fno-fast-math", "--offload-arch=gfx950", "--cuda-device-only",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-fhip-fp32-correctly-rounded-divide-sqrt", "-mllvm", "-amdgpu-mfma-vgpr-form"]


def _makefile_devflags() -> str:
    with open(os.path.join(ROOT, "lns-ml_amd", "Makefile")) as f:
        text = f.read()
    m = re.search(r"^DEVFLAGS := (.*?)(?<!\\)\n", text, re.S | re.M)
    assert m, "DEVFLAGS not found in the Makefile"
    return " ".join(m.group(1).replace("\\\n", " ").split())


def test_probe_uses_the_library_device_flags():
    flags = _makefile_devflags()
    for f in ("--cuda-device-only", "-packed-fp32-ops", "-fhip-fp32-correctly-rounded-divide-sqrt",
              "-amdgpu-mfma-vgpr-form"):
        assert f in flags, f


@pytest.mark.skipif(not (os.path.exists(HIPCC) or shutil.which("hipcc")), reason="hipcc not installed")
def test_merge_primitives_codegen(tmp_path):
    out = tmp_path / "probe.s"
    cmd = [HIPCC if os.path.exists(HIPCC) else "hipcc", *DEVFLAGS, "-S", "-o", str(out),
           os.path.join(ROOT, "tests", "native", "merge_protocol.hip")]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    asm = out.read_text()
    m = re.search(r"^merge_protocol_probe:[^\n]*\n(.*?)s_endpgm", asm, re.S | re.M)
    assert m, "probe kernel not found in the assembly"
    lines = [ln.strip() for ln in m.group(1).splitlines() if ln.strip() and not ln.strip().startswith(";")]
    idx = {name: [i for i, ln in enumerate(lines) if ln.startswith(name)] for name in
           ("global_store_dword", "global_atomic_add", "global_load_dword", "s_waitcnt vmcnt(0)")}
    row_store, count, row_load = idx["global_store_dword"][0], idx["global_atomic_add"], idx["global_load_dword"]
    assert lines[row_store].endswith("sc1"), lines[row_store]            # written through
    assert len(count) == 1 and re.search(r"\bsc0\b", lines[count[0]]), count  # returning atomic
    assert any(row_store < w < count[0] for w in idx["s_waitcnt vmcnt(0)"]), "count not after the stores' wait"
    assert row_load and all(lines[i].endswith("sc1") for i in row_load), [lines[i] for i in row_load]
    assert row_load[0] > count[0]
    assert not any(ln.startswith(("buffer_wbl2", "buffer_inv")) for ln in lines)
