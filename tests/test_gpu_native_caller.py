"""The C ABI from compiled C++ alone (tests/native/engine_loop.cpp, built by
__graft_entry__.build()): the reference engine's per-token loop on Q8A pages
with a sliding window -- lnskv_step_pages, lnskv_block_tables_upload,
lnskv_dispatch_attention_paged, then the o_proj lnskv_q4l_gemv_accumulate over
a 4096 x 4096 Q4_L matrix -- checked inside the program against a host
restatement (stored codes and scales bit-exact, rows within 1e-5 of f64, the
o_proj within 2e-6 of sum |w x| of f64)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "native", "engine_loop")


def test_engine_loop_from_cpp(gpu):
    assert os.path.exists(BIN), "tests/native/engine_loop is missing: run __graft_entry__.build() first"
    print(f"[gpu] running {BIN}", flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("engine_loop ok"), r.stdout
