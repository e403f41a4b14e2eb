// Device-side pieces shared by the decode kernels of liblnskv (gfx950).
//
// Reference semantics (lns-metal/src/shaders/lns_decode.metal):
//   slot math                :541-545   slot = block_table[pos/16]*16 + pos%16
//   Q8A append (K, V)        :547-593   absmax scale, round-half-away, clamp 127
//   f16 append               :284-287   (half)x, round to nearest even
//   online softmax scan      :595-645   m=-1e38, alpha/beta recurrence, acc/l
//   GQA head mapping         :536-537   kv_h = hid / (n_heads / n_kv_heads)
// The reference scans one query head per threadgroup, token by token, with two
// barriers per token; here one workgroup owns (sequence, kv head, split-K
// partition), holds all query heads of the group, and streams whole pages.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "lnskv_internal.h"

namespace lnskv {

constexpr int kPage = LNSKV_PAGE_SIZE;
constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr float kLog2e = 1.4426950408889634f;
// Running-max start value, finite like the reference's -1e38 (metal:600) so
// that an all-masked page leaves alpha = exp2(0) = 1 instead of NaN.
constexpr float kMInit = -1e30f;
constexpr int kSkMaxSeqs = kWave * kWave;  // stream-K: 64 groups of 64 sequences
// Every decode workspace starts with this many bytes of per-workgroup counts
// (the workgroup schedule's), zero before the first call and after every
// call; the other schedules leave them alone.
constexpr size_t kWsHeaderBytes = LNSKV_WORKSPACE_HEADER_BYTES;
constexpr int kWgMaxGroups = (int)(kWsHeaderBytes / 4);
// The workgroup schedule serves batches of at most this many (sequence, kv
// head, page) units per workgroup (upper bound from max_kv_len); stream-K the
// larger ones.
constexpr int kWgSmallPages = 8;

// ---------------------------------------------------------------------------
// Storage traits: bytes per element.
template <int DT> struct Storage;
template <> struct Storage<LNSKV_DTYPE_F32> { static constexpr int kBytes = 4; };
template <> struct Storage<LNSKV_DTYPE_F16> { static constexpr int kBytes = 2; };
template <> struct Storage<LNSKV_DTYPE_Q8A> { static constexpr int kBytes = 1; };

// ---------------------------------------------------------------------------
// Cross-lane helpers.  DPP moves stay inside 16-lane rows; quad_perm and the
// two mirrors make a butterfly whose every lane ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppRowShl = 0x100;     // + n: lane i reads lane i+n of its row
constexpr int kDppRowShr = 0x110;     // + n: lane i reads lane i-n of its row
constexpr int kDppRowNewBcast = 0x150;  // + n: every lane reads lane n of its row

// Sum over aligned groups of N lanes (N = 1..64, power of two).
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_mov<kDppXor1>(x);
  if constexpr (N >= 4) x += dpp_mov<kDppXor2>(x);
  if constexpr (N >= 8) x += dpp_mov<kDppHalfMirror>(x);
  if constexpr (N >= 16) x += dpp_mov<kDppMirror>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16);
  if constexpr (N >= 64) x += __shfl_xor(x, 32);
  return x;
}
template <int N>
__device__ __forceinline__ float group_max(float x) {
  if constexpr (N >= 2) x = fmaxf(x, dpp_mov<kDppXor1>(x));
  if constexpr (N >= 4) x = fmaxf(x, dpp_mov<kDppXor2>(x));
  if constexpr (N >= 8) x = fmaxf(x, dpp_mov<kDppHalfMirror>(x));
  if constexpr (N >= 16) x = fmaxf(x, dpp_mov<kDppMirror>(x));
  if constexpr (N >= 32) x = fmaxf(x, __shfl_xor(x, 16));
  if constexpr (N >= 64) x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}
// Sum / max across lanes that are STRIDE apart (STRIDE power of two): combines
// the rows of a wave that share a column.
template <int STRIDE>
__device__ __forceinline__ float cross_sum(float x) {
#pragma unroll
  for (int o = STRIDE; o < kWave; o <<= 1) x += __shfl_xor(x, o);
  return x;
}
template <int STRIDE>
__device__ __forceinline__ float cross_max(float x) {
#pragma unroll
  for (int o = STRIDE; o < kWave; o <<= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// RoPE's sine and cosine of the f32 angle theta (pos * inv_freq, the
// reference's angle), each rounded once to f32 from an f64 evaluation:
// Cody-Waite reduction by pi/2 (pi/2 split into two 26-bit parts and a 53-bit
// tail, so that k times a part is exact for |k| < 2^27), then Taylor
// polynomials in r^2 on |r| <= pi/4 (sine to r^17, cosine to r^18:
// truncation below 1e-19), every step one IEEE f64 operation or fma, none
// contracted.  The oracle evaluates the same steps in the same order, so the
// rotated values agree bit for bit; both equal the correctly rounded sin/cos
// unless the exact value lies within ~1e-16 (relative) of an f32 rounding
// boundary.
__device__ __forceinline__ void rope_sincos(float theta, float* s, float* c) {
#pragma clang fp contract(off)
  const double t = (double)theta;
  const double k = rint(t * 0x1.45f306dc9c883p-1);  // nearest multiple of pi/2
  const double r = ((t - k * 0x1.921fb5p+0) - k * 0x1.110b46p-26) - k * 0x1.1a62633145c07p-54;
  const double z = r * r;
  double ps = 0x1.952c77030ad4ap-49;  // 1/17!
  ps = fma(ps, z, -0x1.ae7f3e733b81fp-41);
  ps = fma(ps, z, 0x1.6124613a86d09p-33);
  ps = fma(ps, z, -0x1.ae64567f544e4p-26);
  ps = fma(ps, z, 0x1.71de3a556c734p-19);
  ps = fma(ps, z, -0x1.a01a01a01a01ap-13);
  ps = fma(ps, z, 0x1.1111111111111p-7);
  ps = fma(ps, z, -0x1.5555555555555p-3);  // -1/3!
  const double sr = fma(r * z, ps, r);
  double pc = -0x1.6827863b97d97p-53;  // -1/18!
  pc = fma(pc, z, 0x1.ae7f3e733b81fp-45);
  pc = fma(pc, z, -0x1.93974a8c07c9dp-37);
  pc = fma(pc, z, 0x1.1eed8eff8d898p-29);
  pc = fma(pc, z, -0x1.27e4fb7789f5cp-22);
  pc = fma(pc, z, 0x1.a01a01a01a01ap-16);
  pc = fma(pc, z, -0x1.6c16c16c16c17p-10);
  pc = fma(pc, z, 0x1.5555555555555p-5);
  pc = fma(pc, z, -0x1.0000000000000p-1);  // -1/2!
  const double cr = fma(z, pc, 1.0);
  const int q = (int)((long long)k & 3);
  const double sv = q == 0 ? sr : (q == 1 ? cr : (q == 2 ? -sr : -cr));
  const double cv = q == 0 ? cr : (q == 1 ? -sr : (q == 2 ? -cr : sr));
  *s = (float)sv;
  *c = (float)cv;
}

// One RoPE pair (x0, x1) = (dim i, dim i + half) turned by (s, c): x0 c - x1 s
// and x0 s + x1 c, each product and each sum rounded once (no fused
// multiply-add), as the oracle computes them.
__device__ __forceinline__ void rope_turn(float x0, float x1, float s, float c, float* y0, float* y1) {
#pragma clang fp contract(off)
  *y0 = x0 * c - x1 * s;
  *y1 = x0 * s + x1 * c;
}

// Converts one f32 to the page dtype's bits; Q8A needs the head's scale.
// f16: v_cvt_f16_f32 under the default round-to-nearest-even mode for numbers.
// Q8A: IEEE division (HIP's correctly rounded f32 divide), roundf = half away
// from zero, clamp to [-127, 127] (metal:562-567).
// A NaN becomes the quiet f16 NaN with its sign and the top 10 bits of its
// payload (the IEEE conversion's narrowing; the hardware conversion would
// return its own canonical NaN).
__device__ __forceinline__ uint32_t to_f16_bits(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const uint32_t h = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
  return (u & 0x7FFFFFFFu) > 0x7F800000u ? (((u >> 16) & 0x8000u) | 0x7E00u | ((u >> 13) & 0x3FFu)) : h;
}
__device__ __forceinline__ int32_t to_q8(float x, float sc) {
  float r = roundf(x / sc);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int32_t)r;
}

// ---------------------------------------------------------------------------
struct DecodeArgs {
  const uint8_t* k_pages;
  const uint8_t* v_pages;
  const float* k_scales;
  const float* v_scales;
  uint8_t* k_pages_w;  // fused append writes (same pools)
  uint8_t* v_pages_w;
  float* k_scales_w;
  float* v_scales_w;
  const float* q;
  float* out;
  const float* k_new;
  const float* v_new;
  const uint32_t* bt;
  const int32_t* kv_len;
  const int32_t* p_start;
  float* ws_acc;        // [n_seq][n_heads][max_parts][D] partial numerators
  float* ws_ml;         // [n_seq][n_heads][max_parts][2] partial (max, sum)
  int4* sk_desc;        // stream-K: per wave, the segment its first piece closes
  uint32_t* wg_cnt;     // workgroup schedule: per workgroup, a count of the workgroups done
                        // with the segment that starts in it (zero between calls)
  uint32_t* ws_err;     // host word set to 1 when a count exceeds what a call can reach
                        // (a header that was not zero); nullptr: not checked
  const float* gate;      // gated attention: out *= gate ([n_seq][n_heads][D]); nullptr: none
  const float* rope_inv;  // fused RoPE in the MFMA kernels: inverse frequencies
  int32_t rope_half;      // fused RoPE: rotary_dim / 2, 32 or 64; 0: none (the kernels without RoPE run)
  int32_t kv_len_scalar;   // used when kv_len == nullptr
  int32_t p_start_scalar;  // used when p_start == nullptr
  int32_t bt_stride;
  int32_t n_kv;
  int32_t n_heads;
  int32_t split;
  int32_t max_parts;
  int32_t max_kv_len;
  uint32_t num_pages;
  float scale_log2;  // softmax scale * log2(e): scores live in the exp2 domain
};

// The value stored at out[idx]: the attention output, multiplied by the
// caller's gate when the call is gated (the reference's mul_inplace after the
// attention, applied as the row is written).
__device__ __forceinline__ float gated(const DecodeArgs& a, size_t idx, float v) {
  return a.gate ? v * a.gate[idx] : v;
}

struct SeqWindow {
  int L;       // kv_len; 0 when it is past what the grid or the table row can address
  int p0;      // window start
  int jf;      // first partition index
  int nparts;  // partitions of this sequence
};

template <bool FUSED>
__device__ __forceinline__ SeqWindow seq_window(const DecodeArgs& a, int s) {
  SeqWindow w;
  int L = a.kv_len ? a.kv_len[s] : a.kv_len_scalar;
  // a length past what the grid or the table row can address marks the
  // sequence out of range: empty window, nothing stored
  L = L > min(a.max_kv_len, a.bt_stride * kPage) ? 0 : max(L, 0);
  int p0 = a.p_start ? a.p_start[s] : a.p_start_scalar;
  p0 = min(max(p0, 0), L);
  int lo = p0;
  if (FUSED && L > 0) lo = min(lo, L - 1);
  if (L <= lo) {
    w.jf = 0;
    w.nparts = 1;
  } else {
    w.jf = lo / a.split;
    w.nparts = (L - 1) / a.split - w.jf + 1;
  }
  w.L = L;
  w.p0 = p0;
  return w;
}

// ---------------------------------------------------------------------------
// Block epilogue shared by the decode kernels.  On entry the LDS arrays hold,
// per wave, the running max m (log2 domain), the sum l and the numerator acc
// of every query head of the group, and a __syncthreads() has passed.
//  - one partition: out = sum_w 2^(m_w-M) acc_w / sum_w 2^(m_w-M) l_w
//  - several: the block's (M, L, A) goes to the workspace and combine_kernel
//    (launched next on the same stream) merges the partitions of each
//    (sequence, kv head) with the same log-sum-exp weights.
// (Merging in the last-finishing block instead needs an agent-scope release
// per block, i.e. an L2 writeback on every XCD, which measured slower than a
// second launch.)
template <int REP, int D>
struct EpilogueLds {
  float acc[kWavesPerBlock][REP][D];
  float m[kWavesPerBlock][REP];
  float l[kWavesPerBlock][REP];
};

template <int REP, int D>
__device__ __forceinline__ void finish_block(const DecodeArgs& a, EpilogueLds<REP, D>& sm, const SeqWindow& w,
                                             int s, int kvh, int part) {
  const int h0 = kvh * REP;
  const bool single = w.nparts == 1;
  for (int idx = threadIdx.x; idx < REP * D; idx += kBlock) {
    const int h = idx / D, i = idx % D;
    float M = sm.m[0][h];
#pragma unroll
    for (int q = 1; q < kWavesPerBlock; ++q) M = fmaxf(M, sm.m[q][h]);
    float A = 0.0f, Ls = 0.0f;
#pragma unroll
    for (int q = 0; q < kWavesPerBlock; ++q) {
      const float wq = fast_exp2(sm.m[q][h] - M);
      A = fmaf(wq, sm.acc[q][h][i], A);
      Ls = fmaf(wq, sm.l[q][h], Ls);
    }
    const size_t hrow = (size_t)s * a.n_heads + h0 + h;
    if (single) {
      a.out[hrow * D + i] = gated(a, hrow * D + i, Ls > 0.0f ? A / Ls : 0.0f);
    } else {
      const size_t pidx = hrow * a.max_parts + part;
      a.ws_acc[pidx * D + i] = A;
      if (i == 0) {
        a.ws_ml[pidx * 2 + 0] = M;
        a.ws_ml[pidx * 2 + 1] = Ls;
      }
    }
  }
}

// Merges np partial rows (m, l) = ml[row(j)], acc = acc[row(j) * D ...] of
// one query head into out[D]; one block of kBlock threads.  Wave w takes
// partials w, w+4, w+8, ..., CHUNK of them per round with all their loads in
// flight together; lane l holds columns l + 64c.  The four waves' (M, L, A)
// then merge through LDS with the same log-sum-exp weights.  A head whose
// partials are all empty (l = 0) gets zeros.
// One wave's share: partials first, first + STEP, ... below np, CHUNK per
// round of loads; lane l accumulates columns l + 64c into (M, Ls, A).
template <int D, int STEP, int CHUNK, class Row>
__device__ __forceinline__ void merge_wave(const float2* ml, const float* acc, int first, int np, Row row,
                                           float& M, float& Ls, float (&A)[D / kWave]) {
  constexpr int C = D / kWave;
  const int lane = threadIdx.x % kWave;
  M = kMInit;
  Ls = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) A[c] = 0.0f;
  for (int j0 = first; j0 < np; j0 += STEP * CHUNK) {
    float2 pm[CHUNK];
    float pa[CHUNK][C];
#pragma unroll
    for (int u = 0; u < CHUNK; ++u) {
      const int j = j0 + u * STEP;
      const bool in = j < np;
      const size_t r = in ? row(j) : 0;
      pm[u] = in ? ml[r] : make_float2(kMInit, 0.0f);
#pragma unroll
      for (int c = 0; c < C; ++c) pa[u][c] = in ? acc[r * D + c * kWave + lane] : 0.0f;
    }
    float Mc = M;
#pragma unroll
    for (int u = 0; u < CHUNK; ++u) Mc = fmaxf(Mc, pm[u].x);
    const float r = fast_exp2(M - Mc);
    Ls *= r;
#pragma unroll
    for (int c = 0; c < C; ++c) A[c] *= r;
#pragma unroll
    for (int u = 0; u < CHUNK; ++u) {
      const float wj = fast_exp2(pm[u].x - Mc);
      Ls = fmaf(wj, pm[u].y, Ls);
#pragma unroll
      for (int c = 0; c < C; ++c) A[c] = fmaf(wj, pa[u][c], A[c]);
    }
    M = Mc;
  }
}

template <int D, class Row>
__device__ __forceinline__ void merge_partials(const float2* ml, const float* acc, int np, Row row,
                                               float* out, const float* gate) {
  constexpr int C = D / kWave;
  __shared__ float s_acc[kWavesPerBlock][D];
  __shared__ float s_m[kWavesPerBlock], s_l[kWavesPerBlock];
  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  float M, Ls, A[C];
  merge_wave<D, kWavesPerBlock, 16>(ml, acc, wv, np, row, M, Ls, A);
#pragma unroll
  for (int c = 0; c < C; ++c) s_acc[wv][c * kWave + lane] = A[c];
  if (lane == 0) {
    s_m[wv] = M;
    s_l[wv] = Ls;
  }
  __syncthreads();
  if (wv != 0) return;
  float Mt = s_m[0];
#pragma unroll
  for (int q = 1; q < kWavesPerBlock; ++q) Mt = fmaxf(Mt, s_m[q]);
  float wq[kWavesPerBlock], Lt = 0.0f;
#pragma unroll
  for (int q = 0; q < kWavesPerBlock; ++q) {
    wq[q] = fast_exp2(s_m[q] - Mt);
    Lt = fmaf(wq[q], s_l[q], Lt);
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    float At = 0.0f;
#pragma unroll
    for (int q = 0; q < kWavesPerBlock; ++q) At = fmaf(wq[q], s_acc[q][c * kWave + lane], At);
    const float v = Lt > 0.0f ? At / Lt : 0.0f;
    out[c * kWave + lane] = gate ? v * gate[c * kWave + lane] : v;
  }
}

template <int REP, int D, bool FUSED>
__global__ __launch_bounds__(kBlock) void combine_kernel(DecodeArgs a) {
  const int kvh = blockIdx.x, s = blockIdx.y, h = blockIdx.z;
  const SeqWindow w = seq_window<FUSED>(a, s);
  if (w.nparts <= 1) return;  // block-uniform: the decode kernel wrote the output
  const int np = min(w.nparts, a.max_parts);
  const size_t hrow = (size_t)s * a.n_heads + (size_t)kvh * REP + h;
  const size_t base = hrow * a.max_parts;
  merge_partials<D>(reinterpret_cast<const float2*>(a.ws_ml), a.ws_acc, np,
                    [base](int j) { return base + (size_t)j; }, a.out + hrow * D,
                    a.gate ? a.gate + hrow * D : nullptr);
}

template <int REP, int D, bool FUSED>
inline void launch_combine(const DecodeArgs& a, int n_seq, hipStream_t st) {
  if (a.max_parts > 1)
    combine_kernel<REP, D, FUSED><<<dim3((unsigned)a.n_kv, (unsigned)n_seq, REP), kBlock, 0, st>>>(a);
}

// Launchers (defined in the decode translation units).
template <int DT, bool FUSED>
int launch_decode_valu(const DecodeArgs& a, int d, int rep, int n_seq, hipStream_t st);
// Matrix-core decode of f16 pages, split-K schedule (head_dim d of 128 or 256).
template <bool FUSED>
int launch_decode_mfma_f16(const DecodeArgs& a, int rep, int d, int n_seq, hipStream_t st);
// Stream-K schedule of the MFMA kernel (n_seq <= kSkMaxSeqs): n_waves single-wave
// blocks, workspace of n_waves * 2 * rep partial rows.  q8: Q8A pages.
template <bool FUSED>
int launch_decode_mfma_sk(const DecodeArgs& a, int rep, int d, int n_seq, int n_waves, bool q8, hipStream_t st);
// Waves of the stream-K kernel resident at once on the current device.
// rope: the fused kernel that turns RoPE in registers.
int mfma_sk_waves(int rep, int d, bool fused, bool q8, bool rope, int* waves);
// Workgroup schedule of the MFMA kernels (n_seq <= kSkMaxSeqs): up to n_wg
// workgroups (mfma_wg_count: two per CU); the workspace holds the header of
// kWsHeaderBytes (a count per workgroup, zero between calls) and then 2 * rep
// partial rows per workgroup.
template <bool FUSED>
int launch_decode_mfma_wg(const DecodeArgs& a, int rep, int d, int n_seq, int n_wg, bool q8, hipStream_t st);
int mfma_wg_count(int* n_wg);

// Chunked prefill over f16 or Q8A pages with head_dim 128 or 256
// (lnskv_prefill_attention).
struct PrefillArgs {
  const uint8_t* k_pages;
  const uint8_t* v_pages;
  const float* k_scales;   // Q8A pages: per (slot, kv head) scales; nullptr for f16
  const float* v_scales;
  const float* q;          // [n_tok][n_heads][head_dim]
  float* out;              // [n_tok][n_heads][head_dim]
  const int4* chunks;      // [n_chunks]: {table row, first position, length, first token}
  const uint32_t* bt;      // [n_rows][bt_stride]
  const int32_t* p_start;  // [n_rows] window starts, or nullptr (0)
  int32_t window;          // > 0: sliding window, query P starts at max(p_start, P - window + 1)
  int32_t n_chunks;
  int32_t n_tok;
  int32_t n_rows;
  int32_t bt_stride;
  int32_t n_kv;
  int32_t n_heads;
  uint32_t num_pages;
  float scale_log2;
};
// Queries per tile of the prefill kernel (a workgroup per tile and kv head).
int prefill_queries_per_tile(int rep, int head_dim);
int launch_prefill_mfma(const PrefillArgs& a, int rep, int head_dim, int n_tiles, hipStream_t st);

int hip_check(const char* what);
// A device buffer the library keeps per device: 0 the decode workspace, 1
// RoPE'd q/k rows, 2 the Q4L GEMV's x operands.  Growing it allocates a new
// buffer and keeps the old one until lnskv_workspace_release (no device
// synchronization inside a call); during stream capture it fails with
// LNSKV_ERR_WORKSPACE instead.  Calls that share one must not overlap in time.
int library_buffer(int which, size_t need, void** out, hipStream_t stream);

}  // namespace lnskv
