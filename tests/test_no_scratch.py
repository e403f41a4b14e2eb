"""Every kernel of the built library runs without scratch memory (CPU only).

A kernel that spills registers to scratch reads and writes per-lane private
memory inside its loops; the decode, prefill and GEMV kernels are designed
not to.  The device code objects that `make -C lns-ml_amd` embeds in
liblnskv.so are unbundled from `lns-ml_amd/_build/*.hipfb` and their kernel
metadata read with the ROCm LLVM tools: every kernel must have
`.private_segment_fixed_size: 0`."""
import glob
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LLVM = "/opt/rocm/llvm/bin"
BUNDLES = sorted(glob.glob(os.path.join(ROOT, "lns-ml_amd", "_build", "*.hipfb")))


@pytest.mark.skipif(not BUNDLES, reason="library not built in-tree (no _build/*.hipfb)")
@pytest.mark.skipif(not os.path.exists(os.path.join(LLVM, "llvm-readelf")), reason="ROCm LLVM tools absent")
def test_every_kernel_has_zero_scratch(tmp_path):
    kernels, spilling = 0, []
    for b in BUNDLES:
        obj = tmp_path / (os.path.basename(b) + ".o")
        subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--type=o", f"--input={b}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={obj}", "--unbundle"],
                       check=True, capture_output=True, timeout=120)
        notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", str(obj)], check=True,
                               capture_output=True, text=True, timeout=120).stdout
        for block in notes.split("- .agpr_count:")[1:]:
            name = re.search(r"\.name:\s+(\S+)", block).group(1)
            scratch = int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", block).group(1))
            kernels += 1
            if scratch:
                spilling.append((name, scratch))
    assert kernels > 100, kernels
    assert not spilling, spilling
