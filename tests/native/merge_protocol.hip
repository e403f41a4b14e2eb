// Code-generation probe for the cross-workgroup merge of the decode and Q4L
// kernels (lnskv_decode_mfma.hip: decode_wg_kernel's partial rows and counts;
// lnskv_q4l.hip: the split partial sums).  It is compiled to gfx950 assembly
// with the library's device flags by tests/test_codegen_merge.py and never
// run.  The protocol, in the primitives the kernels use:
//   1. each workgroup stores its partial rows as relaxed agent-scope atomic
//      stores;
//   2. it waits until those stores have completed (s_waitcnt vmcnt(0));
//   3. one lane counts the workgroup in with a relaxed agent-scope fetch_add;
//   4. the workgroup that saw the last count reads every row with relaxed
//      agent-scope atomic loads.
// On gfx950 the L2 of one XCD is not coherent with the others.  The protocol
// holds because (1) and (4) compile to stores and loads with the sc1 bit
// (written through to, and read from, the memory side that every XCD shares)
// and (3) is issued only after (2).  The test fails if a compiler change
// drops those bits or moves the count before the wait.
#include <hip/hip_runtime.h>

extern "C" __global__ void merge_protocol_probe(float* rows, unsigned* cnt, float* out, int n) {
  const int t = (int)threadIdx.x;
  __hip_atomic_store(rows + blockIdx.x * 64 + t, (float)t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  unsigned old = 0;
  if (t == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
  if (old == gridDim.x - 1) {
    float s = 0.0f;
    for (int b = 0; b < n; ++b)
      s += __hip_atomic_load(rows + b * 64 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out[t] = s;
  }
}
