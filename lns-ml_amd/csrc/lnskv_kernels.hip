// liblnskv device side: paged K/V append, single-query paged decode attention
// (GQA-grouped, split-K with log-sum-exp combine), page copy, gather, clear.
// Written for gfx950 (CDNA4): 64-lane wavefronts, 16-byte coalesced loads of
// page rows, DPP row reductions, one read of every K/V page per kv-head group.
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
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "lnskv_internal.h"

namespace lnskv {
namespace {

constexpr int kPage = LNSKV_PAGE_SIZE;
constexpr int kWave = 64;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr float kLog2e = 1.4426950408889634f;
// Running-max start value, finite like the reference's -1e38 (metal:600) so
// that an all-masked page leaves alpha = exp2(0) = 1 instead of NaN.
constexpr float kMInit = -1e30f;

// ---------------------------------------------------------------------------
// Storage traits: bytes per element, elements per 16-byte lane load.
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
constexpr int kDppXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

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

// ---------------------------------------------------------------------------
// Element (un)packing from a 16-byte lane chunk.
template <int DT>
__device__ __forceinline__ float elem(const uint4& raw, int e) {
  const uint32_t w = (&raw.x)[(e * Storage<DT>::kBytes) / 4];
  if constexpr (DT == LNSKV_DTYPE_F32) {
    return __builtin_bit_cast(float, w);
  } else if constexpr (DT == LNSKV_DTYPE_F16) {
    const uint16_t h = (uint16_t)(w >> (16 * (e & 1)));
    return (float)__builtin_bit_cast(_Float16, h);
  } else {
    return (float)(int8_t)(w >> (8 * (e & 3)));
  }
}

// Converts one f32 to the page dtype's bits; Q8A needs the head's scale.
// f16: v_cvt_f16_f32 under the default round-to-nearest-even mode.
// Q8A: IEEE division (HIP's correctly rounded f32 divide), roundf = half away
// from zero, clamp to [-127, 127] (metal:562-567).
__device__ __forceinline__ uint32_t to_f16_bits(float x) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
}
__device__ __forceinline__ int32_t to_q8(float x, float sc) {
  float r = roundf(x / sc);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int32_t)r;
}

// ---------------------------------------------------------------------------
// Append kernel.  One wave per (token, kv head); lane i holds elements
// [i*EPT, (i+1)*EPT) of the head, EPT = D/64.
struct AppendArgs {
  uint8_t* k_pages;
  uint8_t* v_pages;
  float* k_scales;
  float* v_scales;
  const float* k_new;
  const float* v_new;
  const int32_t* tok_seq;
  const int32_t* tok_pos;
  const uint32_t* bt;
  int32_t bt_stride;
  int32_t n_tok;
  int32_t n_kv;
  uint32_t num_pages;
};

template <int DT, int D>
__device__ __forceinline__ void store_head_row(uint8_t* pages, float* scales, size_t row_elem,
                                               size_t scale_idx, const float* x, int lane) {
  constexpr int EPT = D / kWave;
  float v[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) v[e] = x[lane * EPT + e];
  if constexpr (DT == LNSKV_DTYPE_F32) {
    float* dst = reinterpret_cast<float*>(pages) + row_elem + lane * EPT;
#pragma unroll
    for (int e = 0; e < EPT; ++e) dst[e] = v[e];
  } else if constexpr (DT == LNSKV_DTYPE_F16) {
    uint16_t* dst = reinterpret_cast<uint16_t*>(pages) + row_elem + lane * EPT;
#pragma unroll
    for (int e = 0; e < EPT; ++e) dst[e] = (uint16_t)to_f16_bits(v[e]);
  } else {
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) amax = fmaxf(amax, fabsf(v[e]));
    amax = group_max<kWave>(amax);
    const float sc = amax == 0.0f ? 1.0f : amax / 127.0f;
    int8_t* dst = reinterpret_cast<int8_t*>(pages) + row_elem + lane * EPT;
#pragma unroll
    for (int e = 0; e < EPT; ++e) dst[e] = (int8_t)to_q8(v[e], sc);
    if (lane == 0) scales[scale_idx] = sc;
  }
}

template <int DT, int D>
__global__ __launch_bounds__(kBlock) void append_kernel(AppendArgs a) {
  const int lane = threadIdx.x % kWave;
  const int64_t item = (int64_t)blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (item >= (int64_t)a.n_tok * a.n_kv) return;  // wave-uniform
  const int t = (int)(item / a.n_kv), h = (int)(item % a.n_kv);
  const int seq = a.tok_seq[t], pos = a.tok_pos[t];
  if (seq < 0 || pos < 0 || pos / kPage >= a.bt_stride) return;
  const uint32_t phys = a.bt[(size_t)seq * a.bt_stride + pos / kPage];
  if (phys >= a.num_pages) return;  // LNSKV_NO_PAGE or outside the pool
  const size_t slot = (size_t)phys * kPage + (size_t)(pos % kPage);
  const size_t row = (slot * a.n_kv + h) * D;
  const size_t src = ((size_t)t * a.n_kv + h) * D;
  store_head_row<DT, D>(a.k_pages, a.k_scales, row, slot * a.n_kv + h, a.k_new + src, lane);
  store_head_row<DT, D>(a.v_pages, a.v_scales, row, slot * a.n_kv + h, a.v_new + src, lane);
}

// ---------------------------------------------------------------------------
// Decode attention.
//
// Grid (partition, kv head, sequence); 256 threads = 4 waves.  The block's
// token range [ta, tb) is its partition of `split` tokens intersected with the
// window [p_start, kv_len) (minus the newest token when the append is fused).
// Pages of the range go round-robin to the 4 waves.
//
// Lane layout for a page (rows of D*ES bytes, one per token and kv head):
//   LPR = D*ES/16 lanes cover one row with 16-byte loads, RPL = 64/LPR rows
//   per wave load, NLOAD = 16/RPL loads per page.  Lane (r, c) = (lane/LPR,
//   lane%LPR) holds elements [c*EPL, (c+1)*EPL) of token j*RPL + r for load j.
// Query heads of the group live in registers in the same column layout, so a
// score is a per-lane partial dot plus a DPP sum over the row's LPR lanes, and
// the P.V update needs no data exchange at all: acc[h][e] accumulates per row
// and rows are summed once at the end.
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
  float* ws_acc;  // [n_seq][n_heads][max_parts][D]
  float* ws_ml;   // [n_seq][n_heads][max_parts][2]
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

struct SeqWindow {
  int L;      // kv_len clamped to what the grid and the table can address
  int p0;     // window start
  int jf;     // first partition index
  int nparts; // partitions of this sequence
};

template <bool FUSED>
__device__ __forceinline__ SeqWindow seq_window(const DecodeArgs& a, int s) {
  SeqWindow w;
  int L = a.kv_len ? a.kv_len[s] : a.kv_len_scalar;
  L = min(max(L, 0), min(a.max_kv_len, a.bt_stride * kPage));
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

template <int DT, int D, int REP>
struct Geo {
  static constexpr int ES = Storage<DT>::kBytes;
  static constexpr int EPL = 16 / ES;        // elements per lane per load
  static constexpr int LPR = D * ES / 16;    // lanes per row
  static constexpr int RPL = kWave / LPR;    // rows per load
  static constexpr int NLOAD = kPage / RPL;  // loads per page
  static_assert(LPR >= 4 && LPR <= 64, "row must span 4..64 lanes");
};

// Loads one page (K and V chunks of this lane, plus Q8A per-token scales).
template <int DT, int D, int REP>
struct PageRegs {
  using G = Geo<DT, D, REP>;
  uint4 k[G::NLOAD];
  uint4 v[G::NLOAD];
  float ks[G::NLOAD];
  float vs[G::NLOAD];
};

template <int DT, int D, int REP>
__device__ __forceinline__ void load_page(const DecodeArgs& a, uint32_t phys, int kvh, int r, int c,
                                          PageRegs<DT, D, REP>& pr) {
  using G = Geo<DT, D, REP>;
#pragma unroll
  for (int j = 0; j < G::NLOAD; ++j) {
    const size_t slot = (size_t)phys * kPage + (size_t)(j * G::RPL + r);
    const size_t off = ((slot * a.n_kv + kvh) * D) * G::ES + (size_t)c * 16;
    pr.k[j] = *reinterpret_cast<const uint4*>(a.k_pages + off);
    pr.v[j] = *reinterpret_cast<const uint4*>(a.v_pages + off);
    if constexpr (DT == LNSKV_DTYPE_Q8A) {
      pr.ks[j] = a.k_scales[slot * a.n_kv + kvh];
      pr.vs[j] = a.v_scales[slot * a.n_kv + kvh];
    }
  }
}

template <int DT, int D, int REP>
struct WaveState {
  using G = Geo<DT, D, REP>;
  float q[REP][G::EPL];
  float acc[REP][G::EPL];
  float m[REP];
  float l[REP];
};

// One page through the online softmax.  `full` means every token of the page
// is inside [ta, tb) and the page is valid; otherwise token validity is
// checked per row and masked V chunks are zeroed (unwritten slots may hold any
// bits, NaN included).
template <int DT, int D, int REP>
__device__ __forceinline__ void consume_page(WaveState<DT, D, REP>& st, const PageRegs<DT, D, REP>& pr,
                                             bool full, bool valid, int tok0, int ta, int tb, int r) {
  using G = Geo<DT, D, REP>;
  float s[G::NLOAD][REP];
#pragma unroll
  for (int j = 0; j < G::NLOAD; ++j) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float part = 0.0f;
#pragma unroll
      for (int e = 0; e < G::EPL; ++e) part = fmaf(elem<DT>(pr.k[j], e), st.q[h][e], part);
      s[j][h] = group_sum<G::LPR>(part);
      if constexpr (DT == LNSKV_DTYPE_Q8A) s[j][h] *= pr.ks[j];
    }
  }
  bool tok_ok[G::NLOAD];
#pragma unroll
  for (int j = 0; j < G::NLOAD; ++j) {
    const int t = tok0 + j * G::RPL + r;
    tok_ok[j] = full || (valid && t >= ta && t < tb);
    if (!tok_ok[j]) {
#pragma unroll
      for (int h = 0; h < REP; ++h) s[j][h] = -INFINITY;
    }
  }
  float alpha[REP];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float mx = s[0][h];
#pragma unroll
    for (int j = 1; j < G::NLOAD; ++j) mx = fmaxf(mx, s[j][h]);
    mx = cross_max<G::LPR>(mx);
    const float m_new = fmaxf(st.m[h], mx);
    alpha[h] = fast_exp2(st.m[h] - m_new);
    st.m[h] = m_new;
    float lsum = 0.0f;
#pragma unroll
    for (int j = 0; j < G::NLOAD; ++j) {
      s[j][h] = fast_exp2(s[j][h] - m_new);  // now p
      lsum += s[j][h];
    }
    st.l[h] = fmaf(alpha[h], st.l[h], lsum);
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) st.acc[h][e] *= alpha[h];
  }
#pragma unroll
  for (int j = 0; j < G::NLOAD; ++j) {
    float pj[REP];
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      pj[h] = s[j][h];
      if constexpr (DT == LNSKV_DTYPE_Q8A) pj[h] *= pr.vs[j];
    }
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      float ve = elem<DT>(pr.v[j], e);
      if (!full) ve = tok_ok[j] ? ve : 0.0f;
#pragma unroll
      for (int h = 0; h < REP; ++h) st.acc[h][e] = fmaf(pj[h], ve, st.acc[h][e]);
    }
  }
}

// The newest token (fused append): lanes of row 0 convert k_new/v_new to the
// page dtype, store them to the token's slot, and feed the stored values to
// the online softmax.  All lanes run the cross-lane steps; only row 0 loads,
// stores and accumulates.
template <int DT, int D, int REP>
__device__ __forceinline__ void fused_new_token(const DecodeArgs& a, WaveState<DT, D, REP>& st, int s,
                                                int kvh, int pos, bool attend, int lane) {
  using G = Geo<DT, D, REP>;
  const int r = lane / G::LPR, c = lane % G::LPR;
  const bool row0 = r == 0;
  const int lp = pos / kPage;
  const uint32_t phys = a.bt[(size_t)s * a.bt_stride + lp];
  const bool valid = phys < a.num_pages;
  const size_t slot = (size_t)phys * kPage + (size_t)(pos % kPage);
  const size_t src = ((size_t)s * a.n_kv + kvh) * D + (size_t)c * G::EPL;
  float kx[G::EPL], vx[G::EPL];
#pragma unroll
  for (int e = 0; e < G::EPL; ++e) {
    kx[e] = row0 ? a.k_new[src + e] : 0.0f;
    vx[e] = row0 ? a.v_new[src + e] : 0.0f;
  }
  // Convert to stored values, keep them as floats for the attention update.
  float kst[G::EPL], vst[G::EPL];
  float ksc = 1.0f, vsc = 1.0f;
  uint32_t kw[4] = {0, 0, 0, 0}, vw[4] = {0, 0, 0, 0};
  if constexpr (DT == LNSKV_DTYPE_F32) {
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      kst[e] = kx[e];
      vst[e] = vx[e];
      kw[e] = __builtin_bit_cast(uint32_t, kx[e]);
      vw[e] = __builtin_bit_cast(uint32_t, vx[e]);
    }
  } else if constexpr (DT == LNSKV_DTYPE_F16) {
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      const _Float16 hk = (_Float16)kx[e], hv = (_Float16)vx[e];
      kst[e] = (float)hk;
      vst[e] = (float)hv;
      kw[e / 2] |= (uint32_t)__builtin_bit_cast(uint16_t, hk) << (16 * (e & 1));
      vw[e / 2] |= (uint32_t)__builtin_bit_cast(uint16_t, hv) << (16 * (e & 1));
    }
  } else {
    float ka = 0.0f, va = 0.0f;
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      ka = fmaxf(ka, fabsf(kx[e]));
      va = fmaxf(va, fabsf(vx[e]));
    }
    ka = group_max<G::LPR>(ka);
    va = group_max<G::LPR>(va);
    ksc = ka == 0.0f ? 1.0f : ka / 127.0f;
    vsc = va == 0.0f ? 1.0f : va / 127.0f;
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      const int32_t kq = to_q8(kx[e], ksc), vq = to_q8(vx[e], vsc);
      kst[e] = (float)kq;
      vst[e] = (float)vq;
      kw[e / 4] |= ((uint32_t)kq & 0xFFu) << (8 * (e & 3));
      vw[e / 4] |= ((uint32_t)vq & 0xFFu) << (8 * (e & 3));
    }
  }
  if (row0 && valid) {
    const size_t off = ((slot * a.n_kv + kvh) * D) * G::ES + (size_t)c * 16;
    *reinterpret_cast<uint4*>(a.k_pages_w + off) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
    *reinterpret_cast<uint4*>(a.v_pages_w + off) = make_uint4(vw[0], vw[1], vw[2], vw[3]);
    if constexpr (DT == LNSKV_DTYPE_Q8A) {
      if (c == 0) {
        a.k_scales_w[slot * a.n_kv + kvh] = ksc;
        a.v_scales_w[slot * a.n_kv + kvh] = vsc;
      }
    }
  }
  if (!(attend && valid)) return;  // wave-uniform
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) part = fmaf(kst[e], st.q[h][e], part);
    float sc = group_sum<G::LPR>(part);
    if constexpr (DT == LNSKV_DTYPE_Q8A) sc *= ksc;
    sc = __shfl(sc, 0);  // row 0's score, wave-uniform
    const float m_new = fmaxf(st.m[h], sc);
    const float alpha = fast_exp2(st.m[h] - m_new);
    const float p = fast_exp2(sc - m_new);
    st.m[h] = m_new;
    const float pv = (DT == LNSKV_DTYPE_Q8A) ? p * vsc : p;
    st.l[h] = alpha * st.l[h] + (row0 ? p : 0.0f);
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) st.acc[h][e] = alpha * st.acc[h][e] + (row0 ? pv * vst[e] : 0.0f);
  }
}

template <int DT, int D, int REP, bool FUSED>
__global__ __launch_bounds__(kBlock) void decode_kernel(DecodeArgs a) {
  using G = Geo<DT, D, REP>;
  __shared__ float sm_acc[kWavesPerBlock][REP][D];
  __shared__ float sm_m[kWavesPerBlock][REP];
  __shared__ float sm_l[kWavesPerBlock][REP];

  const int part = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
  const SeqWindow w = seq_window<FUSED>(a, s);
  if (part >= w.nparts) return;  // block-uniform
  const int j = w.jf + part;
  const int tread_end = FUSED ? max(w.L - 1, 0) : w.L;  // newest token comes from registers
  const int ta = max(w.p0, j * a.split);
  const int tb = min(tread_end, (j + 1) * a.split);

  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int r = lane / G::LPR, c = lane % G::LPR;

  WaveState<DT, D, REP> st;
  const int h0 = kvh * REP;
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const float* qh = a.q + ((size_t)s * a.n_heads + h0 + h) * D + (size_t)c * G::EPL;
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) {
      st.q[h][e] = qh[e] * a.scale_log2;
      st.acc[h][e] = 0.0f;
    }
    st.m[h] = kMInit;
    st.l[h] = 0.0f;
  }

  const uint32_t* bt_row = a.bt + (size_t)s * a.bt_stride;
  if (ta < tb) {
    const int pg_first = ta / kPage, pg_last = (tb - 1) / kPage;
    int pg = pg_first + wave;
    if (pg <= pg_last) {
      auto page_phys = [&](int p, bool& valid) {
        const uint32_t ph = bt_row[p];
        valid = ph < a.num_pages;
        return valid ? ph : 0u;  // in-bounds dummy for missing pages, fully masked
      };
      bool valid;
      uint32_t phys = page_phys(pg, valid);
      PageRegs<DT, D, REP> cur;
      load_page<DT, D, REP>(a, phys, kvh, r, c, cur);
      for (; pg <= pg_last; pg += kWavesPerBlock) {
        const int nxt = pg + kWavesPerBlock;
        PageRegs<DT, D, REP> nx;
        bool nvalid = false;
        if (nxt <= pg_last) {
          const uint32_t nphys = page_phys(nxt, nvalid);
          load_page<DT, D, REP>(a, nphys, kvh, r, c, nx);
        }
        const int tok0 = pg * kPage;
        const bool full = valid && tok0 >= ta && tok0 + kPage <= tb;
        consume_page<DT, D, REP>(st, cur, full, valid, tok0, ta, tb, r);
        cur = nx;
        valid = nvalid;
      }
    }
  }

  if constexpr (FUSED) {
    if (wave == 0 && w.L > 0 && part == w.nparts - 1) {
      const int pos = w.L - 1;
      fused_new_token<DT, D, REP>(a, st, s, kvh, pos, pos >= w.p0, lane);
    }
  }

  // Rows -> wave totals (every row holds the same m).
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    st.l[h] = cross_sum<G::LPR>(st.l[h]);
#pragma unroll
    for (int e = 0; e < G::EPL; ++e) st.acc[h][e] = cross_sum<G::LPR>(st.acc[h][e]);
  }
  if (r == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h)
#pragma unroll
      for (int e = 0; e < G::EPL; ++e) sm_acc[wave][h][c * G::EPL + e] = st.acc[h][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      sm_m[wave][h] = st.m[h];
      sm_l[wave][h] = st.l[h];
    }
  }
  __syncthreads();

  // Waves -> block result, log-sum-exp weighted.
  const bool single = w.nparts == 1;
  for (int idx = threadIdx.x; idx < REP * D; idx += kBlock) {
    const int h = idx / D, i = idx % D;
    float M = sm_m[0][h];
#pragma unroll
    for (int q = 1; q < kWavesPerBlock; ++q) M = fmaxf(M, sm_m[q][h]);
    float A = 0.0f, Ls = 0.0f;
#pragma unroll
    for (int q = 0; q < kWavesPerBlock; ++q) {
      const float wq = fast_exp2(sm_m[q][h] - M);
      A = fmaf(wq, sm_acc[q][h][i], A);
      Ls = fmaf(wq, sm_l[q][h], Ls);
    }
    const size_t hrow = (size_t)s * a.n_heads + h0 + h;
    if (single) {
      a.out[hrow * D + i] = Ls > 0.0f ? A / Ls : 0.0f;
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

// Split-K combine: one wave per (query head, sequence), lanes over head_dim.
// out = sum_j 2^(m_j - M) acc_j / sum_j 2^(m_j - M) l_j  (scores in log2 units).
template <int D, bool FUSED>
__global__ __launch_bounds__(kWave) void combine_kernel(DecodeArgs a) {
  const int h = blockIdx.x, s = blockIdx.y, lane = threadIdx.x;
  const SeqWindow w = seq_window<FUSED>(a, s);
  if (w.nparts <= 1) return;
  const int np = min(w.nparts, a.max_parts);
  const size_t hrow = (size_t)s * a.n_heads + h;
  const float* ml = a.ws_ml + hrow * a.max_parts * 2;
  float M = kMInit;
  for (int j = lane; j < np; j += kWave) M = fmaxf(M, ml[2 * j]);
  M = group_max<kWave>(M);
  float Ls = 0.0f;
  for (int j = lane; j < np; j += kWave) Ls += fast_exp2(ml[2 * j] - M) * ml[2 * j + 1];
  Ls = group_sum<kWave>(Ls);
  constexpr int EPT = D / kWave;
  float A[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) A[e] = 0.0f;
  const float* acc = a.ws_acc + hrow * a.max_parts * D;
  for (int j = 0; j < np; ++j) {
    const float wj = fast_exp2(ml[2 * j] - M);
#pragma unroll
    for (int e = 0; e < EPT; ++e) A[e] = fmaf(wj, acc[(size_t)j * D + e * kWave + lane], A[e]);
  }
  const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
#pragma unroll
  for (int e = 0; e < EPT; ++e) a.out[hrow * D + e * kWave + lane] = A[e] * inv;
}

// ---------------------------------------------------------------------------
// Page copy: block (pair, pool) copies one page with 16-byte moves; pool 0/1 =
// K/V data, 2/3 = K/V scales (Q8A).
struct CopyArgs {
  uint8_t* pool[4];
  size_t page_bytes[4];
  const uint32_t* src;
  const uint32_t* dst;
  int32_t n;
  uint32_t num_pages;
};

__global__ __launch_bounds__(kBlock) void page_copy_kernel(CopyArgs a) {
  const int i = blockIdx.x, which = blockIdx.y;
  if (i >= a.n) return;
  const uint32_t sp = a.src[i], dp = a.dst[i];
  if (sp >= a.num_pages || dp >= a.num_pages) return;
  const size_t pb = a.page_bytes[which];
  if (pb == 0) return;
  const uint8_t* from = a.pool[which] + (size_t)sp * pb;
  uint8_t* to = a.pool[which] + (size_t)dp * pb;
  if (pb % 16 == 0) {
    for (size_t o = (size_t)threadIdx.x * 16; o < pb; o += (size_t)kBlock * 16)
      *reinterpret_cast<uint4*>(to + o) = *reinterpret_cast<const uint4*>(from + o);
  } else {
    for (size_t o = (size_t)threadIdx.x * 4; o < pb; o += (size_t)kBlock * 4)
      *reinterpret_cast<uint32_t*>(to + o) = *reinterpret_cast<const uint32_t*>(from + o);
  }
}

// Gather: one wave per token; the token's whole row (all kv heads) is
// row_bytes contiguous bytes in a slot.
struct GatherArgs {
  const uint8_t* k_pages;
  const uint8_t* v_pages;
  const float* k_scales;
  const float* v_scales;
  uint8_t* k_out;
  uint8_t* v_out;
  float* ks_out;
  float* vs_out;
  const uint32_t* bt;
  int32_t start;
  int32_t n_tok;
  int32_t n_kv;
  uint32_t num_pages;
  size_t row_bytes;  // multiple of 16
};

__global__ __launch_bounds__(kBlock) void gather_kernel(GatherArgs a) {
  const int lane = threadIdx.x % kWave;
  const int t = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (t >= a.n_tok) return;
  const int pos = a.start + t;
  const uint32_t phys = a.bt[pos / kPage];
  const bool valid = phys < a.num_pages;
  const size_t slot = (size_t)phys * kPage + (size_t)(pos % kPage);
  uint8_t* ko = a.k_out + (size_t)t * a.row_bytes;
  uint8_t* vo = a.v_out + (size_t)t * a.row_bytes;
  for (size_t o = (size_t)lane * 16; o < a.row_bytes; o += kWave * 16) {
    uint4 kv = make_uint4(0, 0, 0, 0), vv = make_uint4(0, 0, 0, 0);
    if (valid) {
      kv = *reinterpret_cast<const uint4*>(a.k_pages + slot * a.row_bytes + o);
      vv = *reinterpret_cast<const uint4*>(a.v_pages + slot * a.row_bytes + o);
    }
    *reinterpret_cast<uint4*>(ko + o) = kv;
    *reinterpret_cast<uint4*>(vo + o) = vv;
  }
  if (a.ks_out && a.vs_out) {
    for (int h = lane; h < a.n_kv; h += kWave) {
      a.ks_out[(size_t)t * a.n_kv + h] = valid ? a.k_scales[slot * a.n_kv + h] : 0.0f;
      a.vs_out[(size_t)t * a.n_kv + h] = valid ? a.v_scales[slot * a.n_kv + h] : 0.0f;
    }
  }
}

// Zero fill (used instead of hipMemsetAsync so a caller may capture it).
__global__ __launch_bounds__(kBlock) void zero_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n16; i += (size_t)gridDim.x * kBlock)
    p[i] = make_uint4(0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
int hip_check(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LNSKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return LNSKV_OK;
}

template <int DT>
int launch_append_dt(const AppendArgs& a, int d, hipStream_t st) {
  const unsigned blocks = (unsigned)(((int64_t)a.n_tok * a.n_kv + kWavesPerBlock - 1) / kWavesPerBlock);
  switch (d) {
    case 64: append_kernel<DT, 64><<<blocks, kBlock, 0, st>>>(a); break;
    case 128: append_kernel<DT, 128><<<blocks, kBlock, 0, st>>>(a); break;
    case 256: append_kernel<DT, 256><<<blocks, kBlock, 0, st>>>(a); break;
    default: return fail(LNSKV_ERR_UNSUPPORTED, "head_dim %d", d);
  }
  return hip_check("append kernel launch");
}

template <int DT, int D, int REP, bool FUSED>
void launch_decode_t(const DecodeArgs& a, int n_seq, hipStream_t st) {
  const dim3 grid((unsigned)a.max_parts, (unsigned)a.n_kv, (unsigned)n_seq);
  decode_kernel<DT, D, REP, FUSED><<<grid, kBlock, 0, st>>>(a);
  if (a.max_parts > 1) {
    const dim3 cgrid((unsigned)a.n_heads, (unsigned)n_seq);
    combine_kernel<D, FUSED><<<cgrid, kWave, 0, st>>>(a);
  }
}

template <int DT, int D, bool FUSED>
int launch_decode_rep(const DecodeArgs& a, int rep, int n_seq, hipStream_t st) {
  switch (rep) {
    case 1: launch_decode_t<DT, D, 1, FUSED>(a, n_seq, st); break;
    case 2: launch_decode_t<DT, D, 2, FUSED>(a, n_seq, st); break;
    case 4: launch_decode_t<DT, D, 4, FUSED>(a, n_seq, st); break;
    case 8: launch_decode_t<DT, D, 8, FUSED>(a, n_seq, st); break;
    default: return fail(LNSKV_ERR_UNSUPPORTED, "n_heads/n_kv_heads = %d not supported (1, 2, 4, 8)", rep);
  }
  return hip_check("decode kernel launch");
}

template <int DT, bool FUSED>
int launch_decode_d(const DecodeArgs& a, int d, int rep, int n_seq, hipStream_t st) {
  switch (d) {
    case 64: return launch_decode_rep<DT, 64, FUSED>(a, rep, n_seq, st);
    case 128: return launch_decode_rep<DT, 128, FUSED>(a, rep, n_seq, st);
    case 256: return launch_decode_rep<DT, 256, FUSED>(a, rep, n_seq, st);
    default: return fail(LNSKV_ERR_UNSUPPORTED, "head_dim %d", d);
  }
}

template <bool FUSED>
int launch_decode(const DecodeArgs& a, int dtype, int d, int rep, int n_seq, hipStream_t st) {
  switch (dtype) {
    case LNSKV_DTYPE_F32: return launch_decode_d<LNSKV_DTYPE_F32, FUSED>(a, d, rep, n_seq, st);
    case LNSKV_DTYPE_F16: return launch_decode_d<LNSKV_DTYPE_F16, FUSED>(a, d, rep, n_seq, st);
    case LNSKV_DTYPE_Q8A: return launch_decode_d<LNSKV_DTYPE_Q8A, FUSED>(a, d, rep, n_seq, st);
    default: return fail(LNSKV_ERR_INVALID, "dtype %d", dtype);
  }
}

// Tokens per split-K partition when the caller passes 0: keep whole pages,
// aim for a few thousand workgroups (256 CUs), never split below 64 tokens.
int choose_split(int n_seq, int n_kv, int max_kv_len) {
  const int64_t pairs = (int64_t)n_seq * n_kv;
  int split = 256;
  while (split < 1024 && pairs * ((max_kv_len + split - 1) / split) > 16384) split *= 2;
  while (split > 64 && pairs * ((max_kv_len + split - 1) / split) < 1024) split /= 2;
  return split;
}

size_t workspace_bytes(int n_seq, int n_heads, int d, int max_parts) {
  if (max_parts <= 1) return 0;
  return (size_t)n_seq * n_heads * max_parts * ((size_t)d + 2) * sizeof(float);
}

// Library-kept workspace per device, grown on demand.
struct DeviceWorkspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::vector<DeviceWorkspace> g_ws;

int library_workspace(size_t need, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LNSKV_ERR_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  if ((int)g_ws.size() <= dev) g_ws.resize((size_t)dev + 1);
  DeviceWorkspace& w = g_ws[(size_t)dev];
  if (w.bytes < need) {
    if (w.ptr) {
      // Kernels queued earlier may still use the old buffer.
      if (hipDeviceSynchronize() != hipSuccess) return fail(LNSKV_ERR_HIP, "hipDeviceSynchronize failed");
      (void)hipFree(w.ptr);
      w.ptr = nullptr;
      w.bytes = 0;
    }
    const size_t grow = std::max(need, (size_t)1 << 20);
    if (hipMalloc(&w.ptr, grow) != hipSuccess) {
      w.ptr = nullptr;
      return fail(LNSKV_ERR_NOMEM, "workspace of %zu bytes: hipMalloc failed", grow);
    }
    w.bytes = grow;
  }
  *out = w.ptr;
  return LNSKV_OK;
}

template <bool FUSED>
int decode_entry(const lnskv_pages* c, const float* q, const float* k_new, const float* v_new,
                 float* out, const uint32_t* bt, int32_t bt_stride, const int32_t* kv_len,
                 int32_t kv_len_scalar, const int32_t* p_start, int32_t p_start_scalar,
                 int32_t n_seq, int32_t n_heads, int32_t max_kv_len, float scale, int32_t split,
                 void* ws, size_t ws_bytes, lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (!q || !out || !bt) return fail(LNSKV_ERR_INVALID, "q, out and block tables must be non-null");
  if (FUSED && (!k_new || !v_new)) return fail(LNSKV_ERR_INVALID, "k_new and v_new must be non-null");
  if (n_seq <= 0 || n_seq > 65535) return fail(LNSKV_ERR_INVALID, "n_seq %d out of range [1, 65535]", n_seq);
  if (n_heads <= 0 || n_heads % (int)c->n_kv_heads != 0)
    return fail(LNSKV_ERR_INVALID, "n_heads %d is not a multiple of n_kv_heads %u", n_heads, c->n_kv_heads);
  if (bt_stride <= 0) return fail(LNSKV_ERR_INVALID, "bt_stride %d must be positive", bt_stride);
  if (max_kv_len < 0) return fail(LNSKV_ERR_INVALID, "max_kv_len %d is negative", max_kv_len);
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(LNSKV_ERR_INVALID, "scale must be positive and finite");
  if (split == 0) split = choose_split(n_seq, (int)c->n_kv_heads, max_kv_len);
  if (split < kPage || split % kPage != 0)
    return fail(LNSKV_ERR_INVALID, "split_tokens %d must be a positive multiple of 16", split);
  const int rep = n_heads / (int)c->n_kv_heads;
  const int max_parts = std::max(1, (max_kv_len + split - 1) / split);
  const size_t need = workspace_bytes(n_seq, n_heads, (int)c->head_dim, max_parts);
  if (need > 0) {
    if (ws == nullptr) {
      if (int rc = library_workspace(need, &ws)) return rc;
    } else if (ws_bytes < need) {
      return fail(LNSKV_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed", ws_bytes, need);
    }
  }
  DecodeArgs a{};
  a.k_pages = static_cast<const uint8_t*>(c->k_pages);
  a.v_pages = static_cast<const uint8_t*>(c->v_pages);
  a.k_scales = c->k_scales;
  a.v_scales = c->v_scales;
  a.k_pages_w = static_cast<uint8_t*>(c->k_pages);
  a.v_pages_w = static_cast<uint8_t*>(c->v_pages);
  a.k_scales_w = c->k_scales;
  a.v_scales_w = c->v_scales;
  a.q = q;
  a.out = out;
  a.k_new = k_new;
  a.v_new = v_new;
  a.bt = bt;
  a.kv_len = kv_len;
  a.p_start = p_start;
  a.kv_len_scalar = kv_len_scalar;
  a.p_start_scalar = p_start_scalar;
  a.bt_stride = bt_stride;
  a.n_kv = (int32_t)c->n_kv_heads;
  a.n_heads = n_heads;
  a.split = split;
  a.max_parts = max_parts;
  a.max_kv_len = max_kv_len;
  a.num_pages = c->num_pages;
  a.scale_log2 = scale * kLog2e;
  float* wsf = static_cast<float*>(ws);
  a.ws_acc = wsf;
  a.ws_ml = wsf ? wsf + (size_t)n_seq * n_heads * max_parts * c->head_dim : nullptr;
  return launch_decode<FUSED>(a, c->dtype, (int)c->head_dim, rep, n_seq, (hipStream_t)stream);
}

}  // namespace
}  // namespace lnskv

using namespace lnskv;

extern "C" {

int lnskv_pages_alloc(lnskv_pages* c) {
  clear_error();
  if (int rc = check_geometry(c)) return rc;
  const size_t pb = lnskv_page_bytes(c) * c->num_pages;
  const size_t sb = c->dtype == LNSKV_DTYPE_Q8A ? (size_t)c->num_pages * kPage * c->n_kv_heads * 4 : 0;
  void* ptrs[4] = {nullptr, nullptr, nullptr, nullptr};
  const size_t sizes[4] = {pb, pb, sb, sb};
  for (int i = 0; i < 4; ++i) {
    if (sizes[i] == 0) continue;
    if (hipMalloc(&ptrs[i], sizes[i]) != hipSuccess || hipMemset(ptrs[i], 0, sizes[i]) != hipSuccess) {
      for (int k = 0; k < 4; ++k)
        if (ptrs[k]) (void)hipFree(ptrs[k]);
      return fail(LNSKV_ERR_NOMEM, "page pool allocation of %zu bytes failed", sizes[i]);
    }
  }
  c->k_pages = ptrs[0];
  c->v_pages = ptrs[1];
  c->k_scales = static_cast<float*>(ptrs[2]);
  c->v_scales = static_cast<float*>(ptrs[3]);
  return LNSKV_OK;
}

int lnskv_pages_free(lnskv_pages* c) {
  clear_error();
  if (!c) return fail(LNSKV_ERR_INVALID, "page descriptor is NULL");
  void* ptrs[4] = {c->k_pages, c->v_pages, c->k_scales, c->v_scales};
  for (void* p : ptrs)
    if (p && hipFree(p) != hipSuccess) return fail(LNSKV_ERR_HIP, "hipFree failed");
  c->k_pages = c->v_pages = nullptr;
  c->k_scales = c->v_scales = nullptr;
  return LNSKV_OK;
}

int lnskv_clear(const lnskv_pages* c, lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  const size_t pb = lnskv_page_bytes(c) * c->num_pages;
  const size_t sb = c->dtype == LNSKV_DTYPE_Q8A ? (size_t)c->num_pages * kPage * c->n_kv_heads * 4 : 0;
  void* ptrs[4] = {c->k_pages, c->v_pages, c->k_scales, c->v_scales};
  const size_t sizes[4] = {pb, pb, sb, sb};
  for (int i = 0; i < 4; ++i) {
    if (!sizes[i]) continue;
    // Page bytes are multiples of 64, scale arrays multiples of 64 (16 slots * 4 B).
    const size_t n16 = sizes[i] / 16;
    const unsigned blocks = (unsigned)std::min<size_t>((n16 + kBlock - 1) / kBlock, 16384);
    zero_kernel<<<blocks, kBlock, 0, (hipStream_t)stream>>>(static_cast<uint4*>(ptrs[i]), n16);
  }
  return hip_check("clear kernel launch");
}

int lnskv_append(const lnskv_pages* c, const float* k_new, const float* v_new,
                 const int32_t* tok_seq, const int32_t* tok_pos, int32_t n_tok,
                 const uint32_t* bt, int32_t bt_stride, lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (n_tok < 0) return fail(LNSKV_ERR_INVALID, "n_tok %d is negative", n_tok);
  if (n_tok == 0) return LNSKV_OK;
  if (!k_new || !v_new || !tok_seq || !tok_pos || !bt)
    return fail(LNSKV_ERR_INVALID, "append arguments must be non-null");
  if (bt_stride <= 0) return fail(LNSKV_ERR_INVALID, "bt_stride %d must be positive", bt_stride);
  if ((int64_t)n_tok * c->n_kv_heads > (int64_t)1 << 33)
    return fail(LNSKV_ERR_INVALID, "too many tokens (%d)", n_tok);
  AppendArgs a{};
  a.k_pages = static_cast<uint8_t*>(c->k_pages);
  a.v_pages = static_cast<uint8_t*>(c->v_pages);
  a.k_scales = c->k_scales;
  a.v_scales = c->v_scales;
  a.k_new = k_new;
  a.v_new = v_new;
  a.tok_seq = tok_seq;
  a.tok_pos = tok_pos;
  a.bt = bt;
  a.bt_stride = bt_stride;
  a.n_tok = n_tok;
  a.n_kv = (int32_t)c->n_kv_heads;
  a.num_pages = c->num_pages;
  const hipStream_t st = (hipStream_t)stream;
  switch (c->dtype) {
    case LNSKV_DTYPE_F32: return launch_append_dt<LNSKV_DTYPE_F32>(a, (int)c->head_dim, st);
    case LNSKV_DTYPE_F16: return launch_append_dt<LNSKV_DTYPE_F16>(a, (int)c->head_dim, st);
    default: return launch_append_dt<LNSKV_DTYPE_Q8A>(a, (int)c->head_dim, st);
  }
}

int lnskv_decode_workspace_size(const lnskv_pages* c, int32_t n_seq, int32_t n_heads,
                                int32_t max_kv_len, int32_t split_tokens, size_t* bytes) {
  clear_error();
  if (!bytes) return fail(LNSKV_ERR_INVALID, "bytes is NULL");
  *bytes = 0;
  if (int rc = check_geometry(c)) return rc;
  if (n_seq <= 0 || n_heads <= 0 || max_kv_len < 0) return fail(LNSKV_ERR_INVALID, "bad shape");
  const int split = split_tokens ? split_tokens : choose_split(n_seq, (int)c->n_kv_heads, max_kv_len);
  if (split < kPage || split % kPage) return fail(LNSKV_ERR_INVALID, "split_tokens %d", split_tokens);
  const int max_parts = std::max(1, (max_kv_len + split - 1) / split);
  *bytes = workspace_bytes(n_seq, n_heads, (int)c->head_dim, max_parts);
  return LNSKV_OK;
}

int lnskv_decode(const lnskv_pages* c, const float* q, float* out, const uint32_t* bt,
                 int32_t bt_stride, const int32_t* kv_len, const int32_t* p_start, int32_t n_seq,
                 int32_t n_heads, int32_t max_kv_len, float scale, int32_t split_tokens,
                 void* ws, size_t ws_bytes, lnskv_stream_t stream) {
  if (!kv_len) return fail(LNSKV_ERR_INVALID, "kv_len must be non-null");
  return decode_entry<false>(c, q, nullptr, nullptr, out, bt, bt_stride, kv_len, 0, p_start, 0, n_seq,
                             n_heads, max_kv_len, scale, split_tokens, ws, ws_bytes, stream);
}

int lnskv_append_decode(const lnskv_pages* c, const float* q, const float* k_new, const float* v_new,
                        float* out, const uint32_t* bt, int32_t bt_stride, const int32_t* kv_len,
                        const int32_t* p_start, int32_t n_seq, int32_t n_heads, int32_t max_kv_len,
                        float scale, int32_t split_tokens, void* ws, size_t ws_bytes,
                        lnskv_stream_t stream) {
  if (!kv_len) return fail(LNSKV_ERR_INVALID, "kv_len must be non-null");
  return decode_entry<true>(c, q, k_new, v_new, out, bt, bt_stride, kv_len, 0, p_start, 0, n_seq,
                            n_heads, max_kv_len, scale, split_tokens, ws, ws_bytes, stream);
}

int lnskv_attention_paged(const float* q, const float* k_in, const float* v_in, const lnskv_pages* c,
                          const uint32_t* block_table, float* out, uint32_t pos, uint32_t head_dim,
                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t p_start,
                          lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (head_dim != c->head_dim || n_kv_heads != c->n_kv_heads)
    return fail(LNSKV_ERR_INVALID, "head_dim/n_kv_heads (%u/%u) differ from the cache (%u/%u)", head_dim,
                n_kv_heads, c->head_dim, c->n_kv_heads);
  if (pos >= (1u << 30) || p_start > pos) return fail(LNSKV_ERR_INVALID, "pos %u / p_start %u", pos, p_start);
  const int32_t L = (int32_t)pos + 1;
  const int32_t stride = (int32_t)(pos / kPage) + 1;
  // metal:539 qk_scale = rsqrt(head_dim)
  const float scale = 1.0f / std::sqrt((float)head_dim);
  return decode_entry<true>(c, q, k_in, v_in, out, block_table, stride, nullptr, L, nullptr,
                            (int32_t)p_start, 1, (int32_t)n_heads, L, scale, 0, nullptr, 0, stream);
}

int lnskv_dispatch_attention_paged(const float* q, const float* k_in, const float* v_in,
                                   const lnskv_pages* c, const uint32_t* block_table, float* out,
                                   uint32_t pos, uint32_t head_dim, uint32_t n_heads,
                                   uint32_t n_kv_heads, uint32_t p_start, lnskv_stream_t stream) {
  if (int rc = lnskv_attention_paged(q, k_in, v_in, c, block_table, out, pos, head_dim, n_heads,
                                     n_kv_heads, p_start, stream))
    return rc;
  return lnskv_sync(stream);
}

int lnskv_page_copy(const lnskv_pages* c, const uint32_t* src, const uint32_t* dst, int32_t n,
                    lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (n < 0 || n > 65535 * 64) return fail(LNSKV_ERR_INVALID, "n %d out of range", n);
  if (n == 0) return LNSKV_OK;
  if (!src || !dst) return fail(LNSKV_ERR_INVALID, "src/dst are NULL");
  CopyArgs a{};
  a.pool[0] = static_cast<uint8_t*>(c->k_pages);
  a.pool[1] = static_cast<uint8_t*>(c->v_pages);
  a.pool[2] = reinterpret_cast<uint8_t*>(c->k_scales);
  a.pool[3] = reinterpret_cast<uint8_t*>(c->v_scales);
  const size_t pb = lnskv_page_bytes(c);
  const size_t sb = c->dtype == LNSKV_DTYPE_Q8A ? (size_t)kPage * c->n_kv_heads * 4 : 0;
  a.page_bytes[0] = pb;
  a.page_bytes[1] = pb;
  a.page_bytes[2] = sb;
  a.page_bytes[3] = sb;
  a.src = src;
  a.dst = dst;
  a.n = n;
  a.num_pages = c->num_pages;
  const dim3 grid((unsigned)n, sb ? 4u : 2u);
  page_copy_kernel<<<grid, kBlock, 0, (hipStream_t)stream>>>(a);
  return hip_check("page copy kernel launch");
}

int lnskv_gather(const lnskv_pages* c, const uint32_t* bt, int32_t start, int32_t n_tok, void* k_out,
                 void* v_out, float* ks_out, float* vs_out, lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (start < 0 || n_tok < 0) return fail(LNSKV_ERR_INVALID, "start %d / n_tok %d", start, n_tok);
  if (n_tok == 0) return LNSKV_OK;
  if (!bt || !k_out || !v_out) return fail(LNSKV_ERR_INVALID, "gather arguments must be non-null");
  if ((ks_out || vs_out) && c->dtype != LNSKV_DTYPE_Q8A)
    return fail(LNSKV_ERR_INVALID, "scale outputs are only defined for Q8A pages");
  GatherArgs a{};
  a.k_pages = static_cast<const uint8_t*>(c->k_pages);
  a.v_pages = static_cast<const uint8_t*>(c->v_pages);
  a.k_scales = c->k_scales;
  a.v_scales = c->v_scales;
  a.k_out = static_cast<uint8_t*>(k_out);
  a.v_out = static_cast<uint8_t*>(v_out);
  a.ks_out = ks_out;
  a.vs_out = vs_out;
  a.bt = bt;
  a.start = start;
  a.n_tok = n_tok;
  a.n_kv = (int32_t)c->n_kv_heads;
  a.num_pages = c->num_pages;
  a.row_bytes = (size_t)c->n_kv_heads * c->head_dim * dtype_bytes(c->dtype);
  const unsigned blocks = (unsigned)((n_tok + kWavesPerBlock - 1) / kWavesPerBlock);
  gather_kernel<<<blocks, kBlock, 0, (hipStream_t)stream>>>(a);
  return hip_check("gather kernel launch");
}

int lnskv_sync(lnskv_stream_t stream) {
  clear_error();
  const hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return fail(LNSKV_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  return LNSKV_OK;
}

}  // extern "C"
