// Decode kernel for f16 pages with head_dim 128 (Llama-3 / Mixtral shapes):
// both products of the online softmax on the matrix cores, one wave per
// (kv head, split-K partition, sequence).
//
// A wave streams the pages of its partition with two pages in flight: K of a
// page goes straight to registers in the MFMA A-operand layout, V goes to a
// two-slot LDS ring by LDS DMA (global_load_lds_dwordx4), so prefetched V
// costs no registers.  Page loads are issued before q is prepared, so the
// first HBM round trip overlaps the wave's set-up.  A single-wave workgroup
// needs no barrier and frees its slot the moment it finishes.
//
// Lane (g, n) = (lane/16, lane%16).  For one page (16 tokens x 128 dims of
// one kv head):
//  Q.K^T  S^T[16 tok][16 col] = K[16 tok][128] . Qc[128][16 col] as four
//         v_mfma_f32_16x16x32_f16.  Columns 0..REP-1 hold the query heads'
//         f16 "hi" parts, columns REP..2REP-1 the "lo" remainders
//         (q = hi + lo to ~2^-22 relative), and a DPP row shift adds the two,
//         so scores keep f32-level accuracy with f16 operands.  Lane (g, n)
//         loads token n, dims 32j + 8g + 0..7 for MFMA j (instruction j reads
//         bytes [64j, 64j+64) of all 16 token rows).  Result: lane (g, n)
//         holds S^T[token 4g+ii][col n], ii = 0..3.
//  softmax  page max: in-lane max of 4, then permlane32/16 swaps (VALU); the
//         running max is raised only when a page exceeds it by more than 8
//         (log2 units), so rescaling is rare and p <= 2^8 otherwise.
//  P.V    O[16 row][128] = P[16 row][16 tok] . V[16 tok][128] as eight
//         v_mfma_f32_16x16x16_f16.  The A operand wants lane (g, n) to hold
//         P[row n][tokens 4g..4g+3] -- exactly the lane's four softmax
//         weights: rows 0..REP-1 are f16(p), rows REP..2REP-1 the f16
//         remainders p - f16(p) (from lane n-REP by DPP).  The B operand
//         comes from the V slot via ds_read_b64_tr_b16: within a 16-lane
//         group q, lane 4b+c receives element c of the 8-byte chunks that
//         lanes b, b+4, b+8, b+12 point at; pointing lane 16q+r at token
//         4q + r/4, dims d0 + 4*(r%4) gives lane 16q+4b+c the values
//         V[4q..4q+3][d0+4b+c], the B layout.  Rows r and r+REP (hi and lo
//         of one head) are summed at the end of the partition.
//
// V slot layout: LDS DMA instruction j writes lane l's 16 bytes at 16*l, so
// lane (g, n) lands in LDS row R = 4j+g, 16-byte chunk n; it fetches token
// 4g+j, chunk n ^ sw(R) with sw(R) = 2*(((R>>2)&3) | ((R&1)<<2)).  The XOR
// keeps every 4-lane group on one 64-byte global segment and spreads the 16
// rows that one transposed read touches over distinct LDS banks.
//
// Fused append: the wave whose partition holds the newest token converts it
// (f16, round to nearest even), stores it to its page slot, and substitutes
// it into its own registers / V slot when it reaches that page, so the scan
// never reads the slot back.  Partitions are merged by combine_kernel.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>
#include "lnskv_device.h"

namespace lnskv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef int int4v __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef unsigned int uint2v __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) short4v lds_short4v;
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) half8 lds_half8;

// Heads of 128 dims (Llama-3 / Mixtral) and of 256 (lns-ml's Qwen3.5
// full-attention layers, model_config.rs:563-593): a 256-wide head is two
// 128-dim halves (NH = 2) that share one softmax; every per-half layout below
// (K operand lanes, V slot, transposed reads, output lanes) is the 128-dim one.
constexpr int kD = 128;                    // dims of one half
constexpr int kRowBytes = kD * 2;         // one half-row of f16
constexpr int kVSlot = kPage * kRowBytes;  // one half-page of V in LDS (swizzled rows)
constexpr float kRescaleSlack = 8.0f;     // log2 units the running max may lag
constexpr int kSkMinPages = 4;            // stream-K: fewest pages per wave
// Buffer resource word 3 for raw dword access on gfx9-family parts
// (DATA_FORMAT = 32-bit; no swizzle, no index stride).
constexpr int kBufferFormat = 0x00020000;

// permlane32_swap(x, x) yields (x[l & ~32], x[l | 32]), permlane16_swap(x, x)
// yields (x[l & ~16], x[l | 16]): a max or sum of the pair reduces across
// halves / across adjacent 16-lane rows on the VALU.
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (int)r[0]), __builtin_bit_cast(float, (int)r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
  return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
  return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
}

// x of lane H of this lane's 16-lane row (DPP row_newbcast).  Per-head
// values are picked with compile-time lane numbers: a select between two
// elements of a local array, taken inside a loop, becomes one load at a
// select of indices and leaves the array in scratch.
template <int H>
__device__ __forceinline__ float row_value(float x) {
  return dpp_mov<kDppRowNewBcast + H>(x);
}

// f(integral_constant<int, I>) for I = 0..N-1, each with a compile-time I.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

__device__ __forceinline__ uint32_t v_swz(int R) { return 2u * (uint32_t)(((R >> 2) & 3) | ((R & 1) << 2)); }

// Waits until at most N vector-memory loads of this wave are outstanding
// (gfx9 s_waitcnt: vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left open).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int REP, int NH = 1>
struct WaveState {
  // Q8A pages: int8 products; the B columns are REP heads x 3 limbs
  static constexpr int kSets = (3 * REP + 15) / 16;
  half8 qb[4 * NH];  // B operand of Q.K^T per 32-dim block, column lane%16
  // Q8A pages: q as three int8 limbs (B operand of the int8 products, 2 per
  // set and half: qi[2 kSets h + 2 set + j]): column c = 16*set + lane%16
  // holds limb c/REP of head c%REP; qsc takes the limb sums of head lane%16
  // back to scaled scores
  u32x4 qi[2 * kSets * NH];
  float qsc;
  float4v acc[8 * NH];  // P.V result: lane (g, n) holds O[row 4g+ii][16*nb + n]
  float m;          // lanes with lane%16 < REP: running max of head lane%16
  float l;          // partial softmax sum over this lane's tokens
  float qexp;       // 2^E undoing the per-head normalisation of q
  // Q8A pages: acc holds the P.V sums divided by vnorm, a power of two that
  // follows the pages' largest V scale (0 until a page sets it); vinv = 1/vnorm
  float vnorm;
  float vinv;
};

// Multiplies the result rows 4g+ii of this lane by their head's alpha: row r
// belongs to head r % REP, whose alpha sits in lane (r % REP) of every
// 16-lane row (all rows agree).
template <int REP, int NH, int II = 0>
__device__ __forceinline__ void scale_rows(WaveState<REP, NH>& st, float alpha, int g) {
  if constexpr (II < 4) {
    float f = row_value<II % REP>(alpha);
    if constexpr (REP == 8) f = (g & 1) ? row_value<4 + II>(alpha) : f;
#pragma unroll
    for (int nb = 0; nb < 8 * NH; ++nb) st.acc[nb][II] *= f;
    scale_rows<REP, NH, II + 1>(st, alpha, g);
  }
}

// Per-wave constants of the page streaming.
struct Stream {
  const uint8_t* k_pages;
  const uint8_t* v_pages;
  lds_u8* vring;       // ring of page slots of kVSlot bytes
  uint32_t koff;       // K: token n row + 16g
  uint32_t voff[4];    // V DMA, instruction j: token 4g+j row + 16*(n ^ sw(4j+g))
  uint32_t vr_off;     // transposed read: row 4*(n>>2)+g, (chunk ^ sw) folded per nb
  uint32_t vr_swz;     // sw of that row
  uint32_t vr_half;    // 8 * (n & 1)
  uint32_t vr_sub;     // (n & 3) >> 1: chunk within the 2-chunk pair
  uint32_t num_pages;
  uint32_t kvh_off;    // kvh * NH * kRowBytes
  uint32_t page_bytes; // 16 * n_kv * NH * kRowBytes
};

// Issues the loads of page `ph` (physical id, wave-uniform): K into
// registers, V by DMA into slot `slot` (NH half-slots of kVSlot bytes).
// Returns the page validity.  Exactly 8 NH vector-memory instructions.
template <int NH>
__device__ __forceinline__ bool issue_page(const Stream& sm, uint32_t ph, int slot, half8 (&k)[4 * NH]) {
  const bool valid = ph < sm.num_pages;
  // a missing page reads page 0 (in bounds) and all its tokens are masked
  const size_t base = (size_t)(valid ? ph : 0u) * sm.page_bytes + sm.kvh_off;
  const uint8_t* kb = sm.k_pages + base;
  const uint8_t* vb = sm.v_pages + base;
#pragma unroll
  for (int j = 0; j < 4 * NH; ++j) k[j] = *reinterpret_cast<const half8*>(kb + sm.koff + 64 * j);
  // V goes through a buffer-resource DMA (MUBUF `lds` form) whose base is this
  // page's row block (wave-uniform).  The FLAT form (global_load_lds) would
  // make the compiler drain all vector loads before any dependent use, since
  // it counts it as a flat access to both global memory and LDS.
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0, (int)sm.page_bytes, kBufferFormat);
  lds_u8* dst = sm.vring + slot * (NH * kVSlot);
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(dst + h * kVSlot + 1024 * j),
                                               16, (int)(sm.voff[j] + h * kRowBytes), 0, 0, 0);
  return valid;
}

// Scores of tokens 4g+ii of a page of f16 rows (log2 units), lanes n < REP.
template <int REP, int NH>
__device__ __forceinline__ void page_scores(const WaveState<REP, NH>& st, const half8 (&k)[4 * NH], float (&s)[4]) {
  float4v sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 4 * NH; ++j) sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[j], st.qb[j], sacc, 0, 0, 0);
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) s[ii] = (sacc[ii] + dpp_mov<kDppRowShl + REP>(sacc[ii])) * st.qexp;
}

// The int32 x of lane n + H of this lane's 16-lane row, as a float (exact:
// the limb sums stay below 2^24).
template <int H>
__device__ __forceinline__ float row_up_i32(int x) {
  if constexpr (H == 0) return (float)x;
  else return (float)__builtin_amdgcn_update_dpp(0, x, kDppRowShl + H, 0xF, 0xF, false);
}

// Q8A pages: scores of tokens 4g+ii from the page's int8 K codes as they
// were loaded (kc[j]: token n, dims 32g + 16j .. +15, the A operand of the
// int8 product) and the int8 limbs of q.  The products and their sums over
// the 128 dims are exact integers D_L (|D_L| <= 127*127*128); the score is
// qsc * ks * (D_0 + D_1/254 + D_2/254^2), lanes n < REP.
template <int REP, int NH>
__device__ __forceinline__ void page_scores_q8(const WaveState<REP, NH>& st, const u32x4 (&kc)[2 * NH],
                                               const float4v& ksc, float (&s)[4]) {
  constexpr int NS = WaveState<REP, NH>::kSets;
  int4v d[NS];
#pragma unroll
  for (int S = 0; S < NS; ++S) {
    d[S] = int4v{0, 0, 0, 0};
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        d[S] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(int4v, kc[2 * h + j]),
                                                    __builtin_bit_cast(int4v, st.qi[2 * NS * h + 2 * S + j]), d[S], 0,
                                                    0, 0);
  }
  // limb L of head h sits in set (L*REP)/16, lane h + (L*REP)%16
  constexpr int S1 = REP / 16, H1 = REP % 16, S2 = 2 * REP / 16, H2 = 2 * REP % 16;
  constexpr float kInv254 = 1.0f / 254.0f;
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const float c0 = (float)d[0][ii];
    const float c1 = row_up_i32<H1>(d[S1][ii]);
    const float c2 = row_up_i32<H2>(d[S2][ii]);
    s[ii] = fmaf(fmaf(c2, kInv254, c1), kInv254, c0) * (st.qsc * ksc[ii]);
  }
}

// One page's softmax update and P.V product, given its scores s (lanes
// n < REP, tokens 4g+ii).
// SC (Q8A pages): the V slot holds int8 codes as f16 (finite, so masked rows
// need no clearing: their weights are exact zeros); the weights that
// multiply V are multiplied by the V scale vsc[ii] (the sums l stay
// unscaled).
template <int REP, bool FULL, bool SC = false, int NH = 1>
__device__ __forceinline__ void consume_scores(WaveState<REP, NH>& st, const Stream& sm, float (&s)[4], int slot,
                                               int tok0, bool valid, int ta, int tb, int g, int n,
                                               float4v vsc = float4v{1.0f, 1.0f, 1.0f, 1.0f}) {
  lds_u8* vslot = sm.vring + slot * (NH * kVSlot);
  if constexpr (!FULL && !SC) {
    // rows of masked tokens (and of a missing page) must not carry NaN bits
    // into the matrix product: zero them in the slot
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = tok0 + 4 * g + j;
      if (!(valid && t >= ta && t < tb))
#pragma unroll
        for (int h = 0; h < NH; ++h)
          *(lds_u32x4*)(vslot + h * kVSlot + (4 * j + g) * kRowBytes + 16 * n) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  if constexpr (!FULL) {
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int t = tok0 + 4 * g + ii;
      if (!(valid && t >= ta && t < tb)) s[ii] = -INFINITY;
    }
  }
  float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  mx = max_xor16(max_xor32(mx));
  const bool need = n < REP && mx > st.m + kRescaleSlack;
  if (__builtin_amdgcn_ballot_w64(need)) {  // wave-uniform
    const float m_new = need ? mx : st.m;
    const float alpha = fast_exp2(st.m - m_new);
    st.m = m_new;
    st.l *= alpha;
    scale_rows<REP, NH>(st, alpha, g);
  }
  float pr[4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) pr[ii] = fast_exp2(s[ii] - st.m);
  st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);

  // A operand of P.V: row n < REP: f16(p) of head n; REP <= n < 2REP: the
  // remainder of head n-REP; other rows zero.
  // SC: the weights carry vs / vnorm, vnorm the power of two at or just above
  // the largest V scale seen (kept within 16x of each page's largest), so that
  // their f16 lo parts stay normal numbers; acc accumulates in units of vnorm
  // and is rescaled, exactly, only when a page's largest scale leaves
  // [vnorm/16, vnorm].  Masked tokens' scales (stale bytes) are left out.
  if constexpr (SC) {
    if constexpr (!FULL) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const int t = tok0 + 4 * g + ii;
        if (!(valid && t >= ta && t < tb)) vsc[ii] = 0.0f;
      }
    }
    float vmax = fmaxf(fmaxf(vsc[0], vsc[1]), fmaxf(vsc[2], vsc[3]));
    vmax = max_xor16(max_xor32(vmax));  // over the page's 16 tokens; wave-uniform
    if ((vmax > st.vnorm || vmax * 16.0f < st.vnorm) && vmax > 0.0f) {
      int e = 0;
      (void)frexpf(vmax, &e);
      const float nn = ldexpf(1.0f, e);  // >= vmax, < 2 vmax
      if (st.vnorm > 0.0f) {
        const float r = st.vnorm * ldexpf(1.0f, -e);  // a power of two: exact
#pragma unroll
        for (int nb = 0; nb < 8 * NH; ++nb)
#pragma unroll
          for (int q = 0; q < 4; ++q) st.acc[nb][q] *= r;
      }
      st.vnorm = nn;
      st.vinv = ldexpf(1.0f, -e);
    }
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) pr[ii] *= vsc[ii] * st.vinv;
  }
  half4 pa;
#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    const float from = dpp_mov<kDppRowShr + REP>(pr[ii]);  // lane n-REP
    const float lo = from - (float)(_Float16)from;
    const float v = n < REP ? pr[ii] : (n < 2 * REP ? lo : 0.0f);
    pa[ii] = (_Float16)v;
  }
  // The transposed reads are issued as inline asm: the compiler cannot tell
  // which slot an LDS DMA writes and would otherwise wait for every DMA in
  // flight (the next page's too) before reading.  This slot's DMA is already
  // complete (the caller's vmcnt wait); the lgkmcnt wait below, tied to the
  // results, completes the reads before any use and before the next DMA
  // into this slot is issued.
  // (Half h of a 256-wide head: its own half-slot, accumulators 8h .. 8h+7.)
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    const uint32_t vbase = (uint32_t)(size_t)(vslot + h * kVSlot + sm.vr_off + sm.vr_half);
    short4v bv[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const uint32_t chunk = ((uint32_t)(2 * nb) + sm.vr_sub) ^ sm.vr_swz;
      asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(bv[nb]) : "v"(vbase + 16u * chunk) : "memory");
    }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(bv[0]), "+v"(bv[1]), "+v"(bv[2]), "+v"(bv[3]), "+v"(bv[4]), "+v"(bv[5]), "+v"(bv[6]),
                   "+v"(bv[7])
                 :
                 : "memory");
#pragma unroll
    for (int nb = 0; nb < 8; ++nb)
      st.acc[8 * h + nb] =
          __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4, bv[nb]), st.acc[8 * h + nb], 0, 0, 0);
  }
}

// One page of f16 rows: K in registers (k), V in LDS slot `slot`.
template <int REP, bool FULL, int NH>
__device__ __forceinline__ void consume_page(WaveState<REP, NH>& st, const Stream& sm, const half8 (&k)[4 * NH],
                                             int slot, int tok0, bool valid, int ta, int tb, int g, int n) {
  float s[4];
  page_scores<REP, NH>(st, k, s);
  consume_scores<REP, FULL, false, NH>(st, sm, s, slot, tok0, valid, ta, tb, g, n);
}

// Loads of one piece that do not depend on the sequence's length, issued
// oldest first in the order they are needed: the table window (64 entries
// from table index `tbl`), q and, for a fused call, the new token's row.
template <int REP, int NH = 1>
struct PieceLoads {
  uint32_t btv;  // lane j: block-table entry tbl + j (0 past the row's end)
  int tbl;
  float4v qv[8 * NH];      // 8 float4 per 128-dim half
  float2v knew[NH], vnew[NH];  // new token, half h: elements 128h + 2 lane, +1
};

// Q8: the order of the Q8A kernel, where lane (g, n) holds dims 32g .. 32g+31
// of head n % REP (a contiguous 32-dim slice per lane, so that a page row's
// codes come in two 16-byte loads); otherwise dims 32j + 8g .. 32j + 8g + 7
// for product j of head n (n < REP) or n - REP (n < 2 REP).  Half h of a
// 256-wide head: the same, 128h further (qv[8h ..]).
template <int REP, bool FUSED, bool ROPE, bool Q8 = false, int NH = 1>
__device__ __forceinline__ void piece_loads(const DecodeArgs& a, int s, int kvh, int tbl, PieceLoads<REP, NH>& pl) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int g = lane >> 4, n = lane & 15;
  const int e = tbl + lane;
  pl.btv = e < a.bt_stride ? a.bt[(size_t)s * a.bt_stride + e] : 0u;
  pl.tbl = tbl;
  const bool qcol = n < 2 * REP;
  // other columns load some head and drop it
  const int hq = Q8 ? n % REP : (qcol ? (n < REP ? n : n - REP) : 0);
  const float4v* qh = reinterpret_cast<const float4v*>(
      a.q + ((size_t)s * a.n_heads + (size_t)kvh * REP + hq) * (NH * kD) + (Q8 ? 32 * g : 8 * g));
#pragma unroll
  for (int h = 0; h < NH; ++h)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pl.qv[8 * h + 2 * j] = qh[32 * h + (Q8 ? 2 * j : 8 * j)];
      pl.qv[8 * h + 2 * j + 1] = qh[32 * h + (Q8 ? 2 * j + 1 : 8 * j + 1)];
    }
  // Every piece of a fused call loads the new token's row (the same 1 KiB
  // per sequence and kv head, so the repeats hit L2): a load under a branch
  // would make the compiler wait for it right there.
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    pl.knew[h] = float2v{0.0f, 0.0f};
    pl.vnew[h] = float2v{0.0f, 0.0f};
  }
  if constexpr (FUSED) {
    const size_t src = ((size_t)s * a.n_kv + kvh) * (NH * kD) + 2 * lane;
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      pl.knew[h] = *reinterpret_cast<const float2v*>(a.k_new + src + h * kD);
      pl.vnew[h] = *reinterpret_cast<const float2v*>(a.v_new + src + h * kD);
    }
  }
}

// RoPE: the wave's table in LDS (kRopeTableBytes): the inverse frequencies
// (floats 0..63, copied once per wave), then the (sin, cos) pairs of the
// current piece's position (pair i at floats 64 + 2i), read where the
// rotation needs them so that no table values are held in registers while
// the pages are in flight.
constexpr int kRopeTableBytes = 3 * 64 * 4;
// The wave's copy of the inverse frequencies in LDS, in two steps: the load
// issued at the kernel's start, the LDS store once the layout's own loads are
// in (storing at once would wait for this load before they are issued).
template <bool ROPE>
__device__ __forceinline__ float rope_inv_load(const DecodeArgs& a) {
  if constexpr (ROPE) {
    const int lane = (int)(threadIdx.x & (kWave - 1));
    return lane < a.rope_half ? a.rope_inv[lane] : 0.0f;
  }
  return 0.0f;
}
template <bool ROPE>
__device__ __forceinline__ void rope_inv_store(lds_u8* table, float v) {
  if constexpr (ROPE) ((__attribute__((address_space(3))) float*)table)[threadIdx.x & (kWave - 1)] = v;
}
template <bool ROPE>
__device__ __forceinline__ void stage_rope_table(const DecodeArgs& a, lds_u8* table) {
  rope_inv_store<ROPE>(table, rope_inv_load<ROPE>(a));
}

// The sines and cosines of one position: lane i < half evaluates angle i
// (pos * inv_freq[i], the reference's f32 product) once, for every head and
// lane that turns a pair of that frequency.
__device__ __forceinline__ void rope_angles(lds_u8* table, int half, float fpos) {
  typedef __attribute__((address_space(3))) float lds_f32;
  lds_f32* t = (lds_f32*)table;
  const int lane = (int)(threadIdx.x & (kWave - 1));
  if (lane < half) {
    float sn, cs;
    rope_sincos(fpos * t[lane], &sn, &cs);
    t[64 + 2 * lane] = sn;
    t[65 + 2 * lane] = cs;
  }
  __builtin_amdgcn_wave_barrier();
}

// (sin, cos) of frequencies fi and fi + 1 (fi even): one 16-byte LDS read.
__device__ __forceinline__ float4v rope_pairs(const lds_u8* table, int fi) {
  typedef __attribute__((address_space(3))) float4v lds_float4v;
  return ((const lds_float4v*)(table + 256))[fi >> 1];
}

// The new token's K in the f16 lane order (lane: elements 2 lane, 2 lane + 1
// of half 0) turned by the table's position: the partner of element i sits
// half/2 lanes away; elements past the rotary width stay.
__device__ __forceinline__ void rope_new_k(float2v& kn, int half, const lds_u8* table) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int mlane = half / 2;
  const bool first = (lane & mlane) == 0;
  const float p0 = __shfl_xor(kn.x, mlane, kWave);
  const float p1 = __shfl_xor(kn.y, mlane, kWave);
  if (half == 64 || lane < 32) {  // half 32: elements 64.. stay
    const float4v sc = rope_pairs(table, 2 * (lane & (mlane - 1)));
    float a0, b0, a1, b1;
    // first half: (x, partner) -> x c - partner s; second: (partner, x) -> partner s + x c
    rope_turn(first ? kn.x : p0, first ? p0 : kn.x, sc[0], sc[1], &a0, &b0);
    rope_turn(first ? kn.y : p1, first ? p1 : kn.y, sc[2], sc[3], &a1, &b1);
    kn.x = first ? a0 : b0;
    kn.y = first ? a1 : b1;
  }
}

// Where a piece's result goes: the normalised output rows, or partial rows
// (numerator, running max, sum) for a later merge, head hh of the group in
// partial row pbase + hh * pstride.
struct PieceOut {
  bool final;
  size_t pbase;
  int pstride;
  // in_lds: partial rows go to the LDS array `lds` instead, row r at
  // lds + r * (D + 2): acc[D], then m, then l (D the head dim).  (A flag, not
  // a null test: an LDS array may sit at address 0.)
  bool in_lds = false;
  __attribute__((address_space(3))) float* lds = nullptr;
};

// q -> B operand: column n < REP is hi of head n, REP <= n < 2REP lo of head
// n-REP, others zero.  Each head is first scaled by 2^-E (E from its max
// |q*scale|) so hi/lo stay in f16 range; the scores are scaled back by 2^E.
template <int REP, int NH>
__device__ __forceinline__ void init_wave_state(const DecodeArgs& a, const PieceLoads<REP, NH>& pl,
                                                WaveState<REP, NH>& st, int n) {
  const bool qcol = n < 2 * REP;
  {
    float x[4 * NH][8];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4 * NH; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float qe = pl.qv[2 * j + (e >> 2)][e & 3];
        x[j][e] = qcol ? qe * a.scale_log2 : 0.0f;
        amax = fmaxf(amax, fabsf(x[j][e]));
      }
    amax = max_xor16(max_xor32(amax));
    int E = 0;
    if (amax > 0.0f && amax < INFINITY) (void)frexpf(amax, &E);
    const float inv = ldexpf(1.0f, -E);
    st.qexp = ldexpf(1.0f, E);
#pragma unroll
    for (int j = 0; j < 4 * NH; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = x[j][e] * inv;
        const _Float16 hi = (_Float16)y;
        const _Float16 lo = (_Float16)(y - (float)hi);
        st.qb[j][e] = n < REP ? hi : (qcol ? lo : (_Float16)0.0f);
      }
#pragma unroll
    for (int nb = 0; nb < 8 * NH; ++nb) st.acc[nb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    st.m = kMInit;
    st.l = 0.0f;
    st.vnorm = 0.0f;
    st.vinv = 0.0f;
  }
}

// Q8A pages: q -> three int8 limbs per element.  y = q*scale*127/amax, amax
// the head's largest |q*scale| (so |y| <= 127); limb 0 = rint(y), limb 1 =
// rint(254 r), limb 2 = rint(254 (254 r - limb 1)) with r = y - limb 0, each
// in [-127, 127]; y = limb0 + limb1/254 + limb2/254^2 to within 0.5/254^2.
template <int REP, int NH>
__device__ __forceinline__ void init_wave_state_q8(const DecodeArgs& a, const PieceLoads<REP, NH>& pl,
                                                   WaveState<REP, NH>& st, int n) {
  constexpr int NS = WaveState<REP, NH>::kSets;
  float x[32 * NH];
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 32 * NH; ++e) {
    x[e] = pl.qv[e >> 2][e & 3] * a.scale_log2;
    amax = fmaxf(amax, fabsf(x[e]));
  }
  amax = max_xor16(max_xor32(amax));  // over the head's dims
  // a head whose largest |q*scale| is below 2^-100 scores zero (127 / amax
  // could overflow; the products it drops are below 2^-93 |k|)
  const float inv = amax >= 0x1p-100f ? 127.0f / amax : 0.0f;
  st.qsc = amax / 127.0f;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    uint32_t w[NS][8];
#pragma unroll
    for (int S = 0; S < NS; ++S)
#pragma unroll
      for (int i = 0; i < 8; ++i) w[S][i] = 0u;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float y = x[32 * h + e] * inv;
      const float l0 = rintf(y);
      const float r1 = (y - l0) * 254.0f;
      const float l1 = rintf(r1);
      const float l2 = rintf((r1 - l1) * 254.0f);
#pragma unroll
      for (int S = 0; S < NS; ++S) {
        const int c = 16 * S + n;
        const float v = c < REP ? l0 : (c < 2 * REP ? l1 : (c < 3 * REP ? l2 : 0.0f));
        w[S][e >> 2] |= ((uint32_t)(int)v & 0xFFu) << (8 * (e & 3));
      }
    }
#pragma unroll
    for (int S = 0; S < NS; ++S) {
      st.qi[2 * NS * h + 2 * S] = u32x4{w[S][0], w[S][1], w[S][2], w[S][3]};
      st.qi[2 * NS * h + 2 * S + 1] = u32x4{w[S][4], w[S][5], w[S][6], w[S][7]};
    }
  }
#pragma unroll
  for (int nb = 0; nb < 8 * NH; ++nb) st.acc[nb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  st.m = kMInit;
  st.l = 0.0f;
  st.qexp = 1.0f;
  st.vnorm = 0.0f;
  st.vinv = 0.0f;
}

// The end of a piece: sums over the lanes, then the normalised output rows
// or the partial rows the piece leaves for a merge.
// SC (Q8A pages): acc is in units of st.vnorm.
template <int REP, bool SC = false, int NH = 1>
__device__ __forceinline__ void finish_piece(const DecodeArgs& a, WaveState<REP, NH>& st, int s, int kvh,
                                             const PieceOut& po, int g, int n) {
  constexpr int D = NH * kD;
  // Denominators: sum this head's lanes over the four 16-lane rows.
  st.l = sum_xor16(sum_xor32(st.l));
  // Numerators: result row r (hi) and r + REP (lo) belong to head r.  After
  // the sums, lanes g == 0 hold heads 0..min(REP,4)-1 and, for REP == 8,
  // lanes g == 1 hold heads 4..7, at dims 16*nb + n.
  constexpr int HL = REP < 4 ? REP : 4;  // heads a lane writes
  float o[HL][8 * NH];
#pragma unroll
  for (int nb = 0; nb < 8 * NH; ++nb) {
    if constexpr (REP == 1) {
      o[0][nb] = st.acc[nb][0] + st.acc[nb][1];
    } else if constexpr (REP == 2) {
      o[0][nb] = st.acc[nb][0] + st.acc[nb][2];
      o[1][nb] = st.acc[nb][1] + st.acc[nb][3];
    } else if constexpr (REP == 4) {  // hi rows in lanes g=0, lo rows in g=1
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) o[ii][nb] = sum_xor16(st.acc[nb][ii]);
    } else {  // REP == 8: hi rows in g=0,1, lo rows in g=2,3
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) o[ii][nb] = sum_xor32(st.acc[nb][ii]);
    }
  }
  // l and m of the heads this lane writes (REP == 8: lanes g == 1 hold heads
  // 4..7), broadcast while every lane is active: DPP reads of inactive lanes
  // return nothing useful.
  float lsel[HL], msel[HL];
  static_for<HL>([&](auto c) {
    constexpr int ii = decltype(c)::value;
    lsel[ii] = (REP == 8 && g == 1) ? row_value<(4 + ii) % REP>(st.l) : row_value<ii>(st.l);
    msel[ii] = (REP == 8 && g == 1) ? row_value<(4 + ii) % REP>(st.m) : row_value<ii>(st.m);
  });
  if (g == 0 || (REP == 8 && g == 1)) {
    const int hb = REP == 8 ? 4 * g : 0;
    static_for<HL>([&](auto c) {
      constexpr int ii = decltype(c)::value;
      const float lh = lsel[ii], mh = msel[ii];
      if (po.final) {
        const size_t hrow = (size_t)s * a.n_heads + (size_t)kvh * REP + hb + ii;
        const float inv = lh > 0.0f ? (SC ? st.vnorm : 1.0f) / lh : 0.0f;
#pragma unroll
        for (int nb = 0; nb < 8 * NH; ++nb)
          a.out[hrow * D + 16 * nb + n] = gated(a, hrow * D + 16 * nb + n, o[ii][nb] * inv);
      } else {
        const size_t pidx = po.pbase + (size_t)(hb + ii) * po.pstride;
        if (po.in_lds) {
          __attribute__((address_space(3))) float* row = po.lds + pidx * (D + 2);
#pragma unroll
          for (int nb = 0; nb < 8 * NH; ++nb) row[16 * nb + n] = SC ? o[ii][nb] * st.vnorm : o[ii][nb];
          if (n == 0) {
            row[D] = mh;
            row[D + 1] = lh;
          }
        } else {
#pragma unroll
          for (int nb = 0; nb < 8 * NH; ++nb)
            a.ws_acc[pidx * D + 16 * nb + n] = SC ? o[ii][nb] * st.vnorm : o[ii][nb];
          if (n == 0) {
            a.ws_ml[pidx * 2 + 0] = mh;
            a.ws_ml[pidx * 2 + 1] = lh;
          }
        }
      }
    });
  }
}

// Attends tokens [ta, tb) of sequence s for the REP query heads of kv head
// kvh, streaming the pages with DEPTH of them in flight (K in registers, V
// in a DEPTH-slot LDS ring), and writes the
// result as `po` says.  `append` (fused calls): this piece holds position
// pos = L-1; it stores the new token to its page slot and substitutes it in
// the page data it reads.  `tbl_ok`: pl.btv holds the table window from
// pl.tbl; the window is reloaded when that is not so or does not cover the
// piece's first page.
template <int REP, bool FUSED, int DEPTH, bool ROPE, int NH = 1>
__device__ __forceinline__ void run_piece(const DecodeArgs& a, lds_u8* vring, lds_u8* newtok,
                                          PieceLoads<REP, NH>& pl, bool tbl_ok, int s, int kvh, int ta, int tb,
                                          bool append, int pos, const PieceOut& po, lds_u8* rope_table = nullptr) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int g = lane >> 4, n = lane & 15;
  constexpr int kRow = NH * kRowBytes;  // one (token, kv head) row of f16

  Stream sm;
  sm.k_pages = a.k_pages;
  sm.v_pages = a.v_pages;
  sm.vring = vring;
  sm.num_pages = a.num_pages;
  sm.kvh_off = (uint32_t)kvh * kRow;
  const uint32_t rs = (uint32_t)a.n_kv * kRow;  // bytes between token rows
  sm.page_bytes = kPage * rs;
  sm.koff = (uint32_t)n * rs + 16u * g;
#pragma unroll
  for (int j = 0; j < 4; ++j) sm.voff[j] = (uint32_t)(4 * g + j) * rs + 16u * ((uint32_t)n ^ v_swz(4 * j + g));
  {
    const int R = 4 * (n >> 2) + g;  // transposed read: token 4g + n/4 lives in row 4*(n/4) + g
    sm.vr_off = (uint32_t)R * kRowBytes;
    sm.vr_swz = v_swz(R);
    sm.vr_half = 8u * (n & 1);
    sm.vr_sub = (uint32_t)((n & 3) >> 1);
  }

  // Table window: btv lane j holds entry base + win + j; pages are read from
  // it with v_readlane and the next 64 entries are loaded when the walk
  // leaves the window.
  const uint32_t* bt_row = a.bt + (size_t)s * a.bt_stride;
  const int pg_first = ta / kPage;
  const int npg = ta < tb ? (tb - 1) / kPage - pg_first + 1 : 0;
  int base = pl.tbl;
  int win = 0;
  auto load_window = [&]() {
    const int e = base + win + lane;
    pl.btv = e < a.bt_stride ? bt_row[e] : 0u;
    wait_vmcnt<0>();  // rare: a sliding window, or a piece of more than 64 pages
  };
  if (!tbl_ok || pg_first < base || pg_first - base >= 64) {
    base = pg_first;
    load_window();
  }
  const int off = pg_first - base;  // first page of the piece within the window
  auto phys_of = [&](int i) -> uint32_t {
    int idx = off + i - win;
    if (idx >= 64) {
      win += 64;
      idx -= 64;
      load_window();
    }
    return __builtin_amdgcn_readlane(pl.btv, idx);
  };

  // Keeps the loads of piece_loads ahead of the page loads (the scheduler
  // would sink them towards their uses, behind the pages).
  asm volatile("" : "+v"(pl.btv) : : "memory");

  // The first DEPTH pages are issued unconditionally, for the same reason: a
  // piece with fewer pages loads pool page 0 as a stand-in (in bounds, never
  // consumed; drained before the epilogue).
  half8 kbuf[DEPTH][4 * NH];
  bool vld[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) vld[d] = issue_page<NH>(sm, phys_of(d), d, kbuf[d]) && npg > d;
  // Uses of q and of the new token start here, with the pages in flight.
#pragma unroll
  for (int h = 0; h < NH; ++h)
    asm volatile(""
                 : "+v"(pl.qv[8 * h + 0]), "+v"(pl.qv[8 * h + 1]), "+v"(pl.qv[8 * h + 2]), "+v"(pl.qv[8 * h + 3]),
                   "+v"(pl.qv[8 * h + 4]), "+v"(pl.qv[8 * h + 5]), "+v"(pl.qv[8 * h + 6]), "+v"(pl.qv[8 * h + 7]),
                   "+v"(pl.knew[h]), "+v"(pl.vnew[h]));

  // Fused RoPE: turn q (every piece) and the new K (the appending piece) by
  // the new token's position before they are used.  A rotary width of 64 or
  // 128 lies in the first 128 dims (half 0 of a 256-wide head).
  if constexpr (FUSED && ROPE) {
    {
      rope_angles(rope_table, a.rope_half, (float)max(pos, 0));
      // this lane's q holds elements 8g + 32j + e, and element i < half pairs
      // with i + half (j and j+2 when half is 64, j = 0 and 1 when it is 32)
      const int i1 = a.rope_half == 64 ? 8 * g + 32 : 8 * g;
      // q pairs: vectors (v0, v1) hold the first halves, (w0, w1) the
      // partners: (j, j+2) for half 64, (0, 1) for half 32; x[e] turns with
      // frequency fi + e
      auto turn4 = [&](float4v& x, float4v& y, int fi) {
        const float4v p01 = rope_pairs(rope_table, fi), p23 = rope_pairs(rope_table, fi + 2);
        const float sn[4] = {p01[0], p01[2], p23[0], p23[2]};
        const float cs[4] = {p01[1], p01[3], p23[1], p23[3]};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float y0, y1;
          rope_turn(x[e], y[e], sn[e], cs[e], &y0, &y1);
          x[e] = y0;
          y[e] = y1;
        }
      };
      // Partners are picked by value, not by array index: a branch on the
      // rotary width that names different elements of pl.qv gets merged into
      // a dynamically indexed (scratch) array.  Width 32 turns j = 2, 3 as
      // well and discards the result.
      const bool h64 = a.rope_half == 64;
      float4v y0 = h64 ? pl.qv[4] : pl.qv[2];
      float4v y1 = h64 ? pl.qv[5] : pl.qv[3];
      float4v x2 = pl.qv[2], x3 = pl.qv[3], y2 = pl.qv[6], y3 = pl.qv[7];
      turn4(pl.qv[0], y0, 8 * g);
      turn4(pl.qv[1], y1, 8 * g + 4);
      turn4(x2, y2, i1);
      turn4(x3, y3, i1 + 4);
      pl.qv[2] = h64 ? x2 : y0;
      pl.qv[3] = h64 ? x3 : y1;
      pl.qv[4] = h64 ? y0 : pl.qv[4];
      pl.qv[5] = h64 ? y1 : pl.qv[5];
      pl.qv[6] = h64 ? y2 : pl.qv[6];
      pl.qv[7] = h64 ? y3 : pl.qv[7];
      if (append) rope_new_k(pl.knew[0], a.rope_half, rope_table);
    }
  }

  // Fused append: convert the new token, store it to its page slot, and
  // stage it in LDS for substitution.
  if constexpr (FUSED) {
    if (append) {
      typedef __attribute__((address_space(3))) uint32_t lds_u32;
      uint32_t kb[NH], vb[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        kb[h] = to_f16_bits(pl.knew[h].x) | (to_f16_bits(pl.knew[h].y) << 16);
        vb[h] = to_f16_bits(pl.vnew[h].x) | (to_f16_bits(pl.vnew[h].y) << 16);
        ((lds_u32*)newtok)[64 * h + lane] = kb[h];
        ((lds_u32*)(newtok + kRow))[64 * h + lane] = vb[h];
      }
      const int ip = pos / kPage - base - win;  // the page is normally in the table window
      const uint32_t ph = ip >= 0 && ip < 64 && pos / kPage - pg_first < npg ? __builtin_amdgcn_readlane(pl.btv, ip)
                                                                              : bt_row[pos / kPage];
      if (ph < a.num_pages) {
        const size_t row = ((size_t)ph * kPage + (size_t)(pos % kPage)) * a.n_kv + kvh;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          *reinterpret_cast<uint32_t*>(a.k_pages_w + row * kRow + h * kRowBytes + 4 * lane) = kb[h];
          *reinterpret_cast<uint32_t*>(a.v_pages_w + row * kRow + h * kRowBytes + 4 * lane) = vb[h];
        }
      }
    }
  }
  const bool attend_new = append && pos >= ta;

  WaveState<REP, NH> st;
  init_wave_state<REP, NH>(a, pl, st, n);

  // Page i: wait for its loads (those of the pages issued after it may stay
  // in flight), patch in the new token if it lives there, consume, refill the
  // slot with page i + DEPTH.  `steady` asserts pages i+1 .. i+DEPTH exist,
  // which lets the compiler's wait counting see exactly DEPTH pages in
  // flight; the other steps use the masked consume only.
  auto step = [&](int i, half8(&k)[4 * NH], bool& valid, int slot, bool steady) {
    const int ahead = steady ? DEPTH - 1 : min(npg - 1 - i, DEPTH - 1);  // pages issued after page i
    constexpr int kLoads = 8 * NH;  // vector-memory instructions per page
    if (ahead >= 3) wait_vmcnt<3 * kLoads>();
    else if (ahead == 2) wait_vmcnt<2 * kLoads>();
    else if (ahead == 1) wait_vmcnt<kLoads>();
    else wait_vmcnt<0>();
    const int tok0 = (pg_first + i) * kPage;
    if (attend_new && pos / kPage == pg_first + i) {
      const int t = pos % kPage;
      if (n == t) {
#pragma unroll
        for (int j = 0; j < 4 * NH; ++j) k[j] = *(lds_half8*)(newtok + 64 * j + 16 * g);
      }
      const int R = 4 * (t & 3) + (t >> 2);
      if (g == (R & 3)) {
        lds_u8* vslot = vring + slot * (NH * kVSlot);
#pragma unroll
        for (int h = 0; h < NH; ++h)
          *(lds_u32x4*)(vslot + h * kVSlot + R * kRowBytes + 16 * n) =
              *(lds_u32x4*)(newtok + kRow + h * kRowBytes + 16 * ((uint32_t)n ^ v_swz(R)));
      }
      __builtin_amdgcn_wave_barrier();
    }
    if (steady && valid && tok0 >= ta && tok0 + kPage <= tb)
      consume_page<REP, true, NH>(st, sm, k, slot, tok0, valid, ta, tb, g, n);
    else
      consume_page<REP, false, NH>(st, sm, k, slot, tok0, valid, ta, tb, g, n);
    if (steady || i + DEPTH < npg) valid = issue_page<NH>(sm, phys_of(i + DEPTH), slot, k);
  };
  int i = 0;
  for (; i + 2 * DEPTH - 1 < npg; i += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) step(i + d, kbuf[d], vld[d], d, true);
  }
  // the last one to 2*DEPTH-1 pages
#pragma unroll
  for (int d = 0; d < 2 * DEPTH - 1; ++d)
    if (i + d < npg) step(i + d, kbuf[d % DEPTH], vld[d % DEPTH], d % DEPTH, false);
  wait_vmcnt<0>();  // stand-in pages of a piece with fewer than DEPTH pages
  // the slots and the staged token are reused by the next piece
  __builtin_amdgcn_wave_barrier();

  finish_piece<REP, false, NH>(a, st, s, kvh, po, g, n);
}

// ---------------------------------------------------------------------------
// Q8A pages (the reference's paged type: int8 codes, one f32 scale per
// (slot, kv head), lns_decode.metal:547-593, 611-634) on the same matrix-core
// pipeline.  A page's K rows (16 x 128 bytes) and V rows come to registers
// as int8 codes with 16-byte buffer loads, plus the K and V scales of the
// lane's token.  K codes are the A operand of v_mfma_i32_16x16x64_i8 as
// loaded (each lane a contiguous 32-dim slice), against q split into three
// int8 limbs: exact integer dot products, scaled back per token
// (page_scores_q8).  V codes become f16 exactly and go to the LDS slot in the
// layout the transposed reads expect; the softmax weights are multiplied by
// the V scale in the P.V product (the reference's q.(k8 ks) and (beta vs)
// v8).  A fused call quantizes the new token in the wave that holds it.
// ---------------------------------------------------------------------------

// Exact int8 -> f16 of the four signed bytes of w: the f16 with bits
// 0x6400 | (b + 128) is 1024 + b + 128, and subtracting 1152 leaves b.
__device__ __forceinline__ half4 i8x4_to_f16(uint32_t w) {
  typedef _Float16 half2q __attribute__((ext_vector_type(2)));
  const uint32_t u = w ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // bytes u0, 0x64, u1, 0x64
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // bytes u2, 0x64, u3, 0x64
  const half2q c = {(_Float16)1152.0f, (_Float16)1152.0f};
  const half2q x = __builtin_bit_cast(half2q, lo) - c;
  const half2q y = __builtin_bit_cast(half2q, hi) - c;
  return half4{x[0], x[1], y[0], y[1]};
}

__device__ __forceinline__ half8 i8x8_to_f16(uint2v w) {
  const half4 a = i8x4_to_f16(w[0]), b = i8x4_to_f16(w[1]);
  return half8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// One Q8A page in flight: K codes of token n, dims 32g .. 32g+31 (int8
// product j takes dims 32g + 16j ..); V codes of token 8h + lane/8, dims
// 16 (lane%8) .. +15 for load h; the K and V scales of token 4g + n%4.  Half
// hh of a 256-wide head: the same, 128hh further (k[2hh ..], v[2hh ..]).
template <int NH>
struct PageQ8 {
  u32x4 k[2 * NH];
  u32x4 v[2 * NH];
  float ks, vs;
};

// RoPE on the Q8A lane order (lane (g, n): dims 32g .. 32g+31 of half 0):
// rotary width 2H (H = 32: dims 0..63, H = 64: dims 0..127), dim i < H pairs
// with i + H, which lives in lane g ^ (H/32) at the same element; dim i turns
// with frequency i % H, whose (sin, cos) the table holds.
template <int H>
__device__ __forceinline__ void rope_q8_lanes(float4v (&qv)[8], const lds_u8* rope_table, int g) {
  static_assert(H == 32 || H == 64, "rotary half-width");
  const int lane = (int)(threadIdx.x & (kWave - 1));
  constexpr bool h64 = H == 64;
  const bool rotated = h64 || g < 2;
  const bool first = h64 ? g < 2 : g == 0;
  const int fb = h64 ? 32 * (g & 1) : 0;  // frequency of this lane's element 0
  // one pair of elements at a time, the next pair's (sin, cos) read while
  // this pair turns: unbounded, the scheduler would hoist every table read
  // and lane swap of the 32 elements at once
  float4v sc_next = rope_pairs(rope_table, fb);
#pragma unroll
  for (int e = 0; e < 32; e += 2) {
    __builtin_amdgcn_sched_barrier(0);
    const float4v sc = sc_next;
    if (e + 2 < 32) sc_next = rope_pairs(rope_table, fb + e + 2);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float x = qv[(e + u) >> 2][(e + u) & 3];
      // the value of lane ^ H/2 (the swap returns the pair in lane order)
      float p;
      if constexpr (h64) {
        const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x),
                                                        false, false);
        p = __builtin_bit_cast(float, (int)((lane & 32) ? r[0] : r[1]));
      } else {
        const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x),
                                                        false, false);
        p = __builtin_bit_cast(float, (int)((lane & 16) ? r[0] : r[1]));
      }
      float y0, y1;
      rope_turn(first ? x : p, first ? p : x, sc[2 * u], sc[2 * u + 1], &y0, &y1);
      qv[(e + u) >> 2][(e + u) & 3] = rotated ? (first ? y0 : y1) : x;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// FUSED: when `append`, this piece holds position pos = L-1; the wave
// quantizes the new token (the quantizer of append_kernel: absmax / 127,
// IEEE divide, round half away from zero, clamp 127), stores its codes and
// scales to the slot, and substitutes them into the page data it loaded.
// ROPE (fused calls): q and the new K are turned by pos first, so the codes
// stored are those of the rotated K (the engine's rotate, then attend).
template <int REP, int DEPTH, bool FUSED, int NH = 1, bool ROPE = false>
__device__ __forceinline__ void run_piece_q8(const DecodeArgs& a, lds_u8* vslot, lds_u8* newtok,
                                             PieceLoads<REP, NH>& pl, bool tbl_ok, int s, int kvh, int ta, int tb,
                                             bool append, int pos, const PieceOut& po,
                                             lds_u8* rope_table = nullptr) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int g = lane >> 4, n = lane & 15;
  constexpr int kRowQ8 = NH * kD;  // one (token, kv head) row of int8 codes

  Stream sm{};
  sm.vring = vslot;
  {
    const int R = 4 * (n >> 2) + g;
    sm.vr_off = (uint32_t)R * kRowBytes;
    sm.vr_swz = v_swz(R);
    sm.vr_half = 8u * (n & 1);
    sm.vr_sub = (uint32_t)((n & 3) >> 1);
  }
  const uint32_t rs = (uint32_t)a.n_kv * kRowQ8;  // bytes between token rows
  const size_t page_bytes = (size_t)kPage * rs;
  const uint32_t kvh_off = (uint32_t)kvh * kRowQ8;
  const uint32_t koff = (uint32_t)n * rs + 32u * g;
  // V load h: token 8h + lane/8, 16 codes from dim 16 * (lane % 8); they go
  // to the LDS row of that token (row 4 (t % 4) + t / 4, the layout of the
  // transposed reads) as f16 chunks 2c and 2c + 1, each at chunk ^ sw(row)
  const int vc = lane & 7;
  uint32_t voff[2], vlds[2][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int t = 8 * h + (lane >> 3);
    const int R = 4 * (t & 3) + (t >> 2);
    voff[h] = (uint32_t)t * rs + 16u * (uint32_t)vc;
    vlds[h][0] = (uint32_t)R * kRowBytes + 16u * ((uint32_t)(2 * vc) ^ v_swz(R));
    vlds[h][1] = (uint32_t)R * kRowBytes + 16u * ((uint32_t)(2 * vc + 1) ^ v_swz(R));
  }
  const uint32_t soff = (uint32_t)(4 * g + (n & 3)) * (uint32_t)a.n_kv + (uint32_t)kvh;

  const uint32_t* bt_row = a.bt + (size_t)s * a.bt_stride;
  const int pg_first = ta / kPage;
  const int npg = ta < tb ? (tb - 1) / kPage - pg_first + 1 : 0;
  int base = pl.tbl;
  int win = 0;
  auto load_window = [&]() {
    const int e = base + win + lane;
    pl.btv = e < a.bt_stride ? bt_row[e] : 0u;
    wait_vmcnt<0>();
  };
  if (!tbl_ok || pg_first < base || pg_first - base >= 64) {
    base = pg_first;
    load_window();
  }
  const int off = pg_first - base;
  auto phys_of = [&](int i) -> uint32_t {
    int idx = off + i - win;
    if (idx >= 64) {
      win += 64;
      idx -= 64;
      load_window();
    }
    return __builtin_amdgcn_readlane(pl.btv, idx);
  };
  asm volatile("" : "+v"(pl.btv) : : "memory");

  // exactly 4 NH + 2 vector-memory loads; a missing page reads page 0
  // (masked).  Buffer resources on the page's rows and scales (scalar bases,
  // 32-bit lane offsets), each ending where this kv head's last row of the
  // page does.
  auto issue = [&](uint32_t ph, PageQ8<NH>& pg) -> bool {
    const bool valid = ph < a.num_pages;
    const size_t pb = (size_t)(valid ? ph : 0u);
    const int rows = (int)(page_bytes - kvh_off);
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.k_pages + pb * page_bytes + kvh_off), (short)0, rows, kBufferFormat);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.v_pages + pb * page_bytes + kvh_off), (short)0, rows, kBufferFormat);
    const size_t sb = pb * kPage * (size_t)a.n_kv;
    const int sbytes = kPage * a.n_kv * (int)sizeof(float);
    const __amdgpu_buffer_rsrc_t ksr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.k_scales + sb), (short)0, sbytes, kBufferFormat);
    const __amdgpu_buffer_rsrc_t vsr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a.v_scales + sb), (short)0, sbytes, kBufferFormat);
#pragma unroll
    for (int hh = 0; hh < NH; ++hh)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        pg.k[2 * hh + h] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, (int)(koff + kD * hh + 16u * h), 0, 0));
#pragma unroll
    for (int hh = 0; hh < NH; ++hh)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        pg.v[2 * hh + h] =
            __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, (int)(voff[h] + kD * hh), 0, 0));
    pg.ks = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ksr, (int)(4u * soff), 0, 0));
    pg.vs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vsr, (int)(4u * soff), 0, 0));
    return valid;
  };

  PageQ8<NH> pbuf[DEPTH];
  bool vld[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) vld[d] = issue(phys_of(d), pbuf[d]) && npg > d;
#pragma unroll
  for (int h = 0; h < NH; ++h)
    asm volatile(""
                 : "+v"(pl.qv[8 * h + 0]), "+v"(pl.qv[8 * h + 1]), "+v"(pl.qv[8 * h + 2]), "+v"(pl.qv[8 * h + 3]),
                   "+v"(pl.qv[8 * h + 4]), "+v"(pl.qv[8 * h + 5]), "+v"(pl.qv[8 * h + 6]), "+v"(pl.qv[8 * h + 7]),
                   "+v"(pl.knew[h]), "+v"(pl.vnew[h]));

  // Fused RoPE: turn q and, in the appending piece, the new K (the f16
  // kernels' lane order for it: elements 2 lane, 2 lane + 1 of half 0) by the
  // new token's position.
  if constexpr (FUSED && ROPE) {
    rope_angles(rope_table, a.rope_half, (float)max(pos, 0));
    float4v q0[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q0[j] = pl.qv[j];
    if (a.rope_half == 64)
      rope_q8_lanes<64>(q0, rope_table, g);
    else
      rope_q8_lanes<32>(q0, rope_table, g);
#pragma unroll
    for (int j = 0; j < 8; ++j) pl.qv[j] = q0[j];
    if (append) rope_new_k(pl.knew[0], a.rope_half, rope_table);
  }

  // Fused append: quantize the new token (lane: elements 2*lane, 2*lane+1 of
  // each half), store codes and scales to its slot, stage the codes in LDS.
  float new_ks = 1.0f, new_vs = 1.0f;
  if constexpr (FUSED) {
    if (append) {
      auto quant = [&](const float2v (&x)[NH], float& sc, uint32_t (&c)[NH]) {
        float m = 0.0f;
#pragma unroll
        for (int h = 0; h < NH; ++h) m = fmaxf(m, fmaxf(fabsf(x[h].x), fabsf(x[h].y)));
        const float amax = group_max<kWave>(m);
        sc = amax == 0.0f ? 1.0f : amax / 127.0f;
#pragma unroll
        for (int h = 0; h < NH; ++h)
          c[h] = ((uint32_t)to_q8(x[h].x, sc) & 0xFFu) | (((uint32_t)to_q8(x[h].y, sc) & 0xFFu) << 8);
      };
      uint32_t kc[NH], vcd[NH];
      quant(pl.knew, new_ks, kc);
      quant(pl.vnew, new_vs, vcd);
      typedef __attribute__((address_space(3))) uint16_t lds_u16;
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        ((lds_u16*)newtok)[64 * h + lane] = (uint16_t)kc[h];
        ((lds_u16*)(newtok + kRowQ8))[64 * h + lane] = (uint16_t)vcd[h];
      }
      const int ip = pos / kPage - base - win;  // the page is normally in the table window
      const uint32_t ph = ip >= 0 && ip < 64 && pos / kPage - pg_first < npg ? __builtin_amdgcn_readlane(pl.btv, ip)
                                                                              : bt_row[pos / kPage];
      if (ph < a.num_pages) {
        const size_t row = ((size_t)ph * kPage + (size_t)(pos % kPage)) * a.n_kv + kvh;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          *reinterpret_cast<uint16_t*>(a.k_pages_w + row * kRowQ8 + kD * h + 2 * lane) = (uint16_t)kc[h];
          *reinterpret_cast<uint16_t*>(a.v_pages_w + row * kRowQ8 + kD * h + 2 * lane) = (uint16_t)vcd[h];
        }
        if (lane == 0) {
          a.k_scales_w[row] = new_ks;
          a.v_scales_w[row] = new_vs;
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  const bool attend_new = FUSED && append && pos >= ta;

  WaveState<REP, NH> st;
  init_wave_state_q8<REP, NH>(a, pl, st, n);

  auto step = [&](int i, PageQ8<NH>& pg, bool& valid, bool steady) {
    const int ahead = steady ? DEPTH - 1 : min(npg - 1 - i, DEPTH - 1);  // pages issued after page i
    constexpr int kLoads = 4 * NH + 2;  // vector-memory loads per page
    static_assert(kLoads * (DEPTH - 1) < 64, "vmcnt range");
    static_for<DEPTH>([&](auto c) {
      constexpr int k = decltype(c)::value;
      if (ahead == DEPTH - 1 - k) wait_vmcnt<kLoads * (DEPTH - 1 - k)>();
    });
    const int tok0 = (pg_first + i) * kPage;
    if (attend_new && pos / kPage == pg_first + i) {
      // the loads may predate the store: take the new token's codes and
      // scales from the staged copy
      const int t = pos % kPage;
      if (n == t) {
#pragma unroll
        for (int hh = 0; hh < NH; ++hh)
#pragma unroll
          for (int h = 0; h < 2; ++h) pg.k[2 * hh + h] = *(const lds_u32x4*)(newtok + kD * hh + 32 * g + 16 * h);
      }
#pragma unroll
      for (int hh = 0; hh < NH; ++hh)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          if (8 * h + (lane >> 3) == t) pg.v[2 * hh + h] = *(const lds_u32x4*)(newtok + kRowQ8 + kD * hh + 16 * vc);
      if (4 * g + (n & 3) == t) {
        pg.ks = new_ks;
        pg.vs = new_vs;
      }
    }
#pragma unroll
    for (int hh = 0; hh < NH; ++hh)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        *(lds_half8*)(vslot + hh * kVSlot + vlds[h][0]) = i8x8_to_f16(uint2v{pg.v[2 * hh + h][0], pg.v[2 * hh + h][1]});
        *(lds_half8*)(vslot + hh * kVSlot + vlds[h][1]) = i8x8_to_f16(uint2v{pg.v[2 * hh + h][2], pg.v[2 * hh + h][3]});
      }
    // scales of tokens 4g+ii: lane 4*(n/4) + ii of this row holds them
    float4v ksc, vsc;
    ksc[0] = dpp_mov<0x00>(pg.ks);
    ksc[1] = dpp_mov<0x55>(pg.ks);
    ksc[2] = dpp_mov<0xAA>(pg.ks);
    ksc[3] = dpp_mov<0xFF>(pg.ks);
    vsc[0] = dpp_mov<0x00>(pg.vs);
    vsc[1] = dpp_mov<0x55>(pg.vs);
    vsc[2] = dpp_mov<0xAA>(pg.vs);
    vsc[3] = dpp_mov<0xFF>(pg.vs);
    float sc[4];
    page_scores_q8<REP, NH>(st, pg.k, ksc, sc);
    if (steady && valid && tok0 >= ta && tok0 + kPage <= tb)
      consume_scores<REP, true, true, NH>(st, sm, sc, 0, tok0, valid, ta, tb, g, n, vsc);
    else
      consume_scores<REP, false, true, NH>(st, sm, sc, 0, tok0, valid, ta, tb, g, n, vsc);
    if (steady || i + DEPTH < npg) valid = issue(phys_of(i + DEPTH), pg);
  };
  int i = 0;
  for (; i + 2 * DEPTH - 1 < npg; i += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) step(i + d, pbuf[d], vld[d], true);
  }
#pragma unroll
  for (int d = 0; d < 2 * DEPTH - 1; ++d)
    if (i + d < npg) step(i + d, pbuf[d % DEPTH], vld[d % DEPTH], false);
  wait_vmcnt<0>();  // stand-in pages of a piece with fewer than DEPTH pages
  __builtin_amdgcn_wave_barrier();
  finish_piece<REP, true, NH>(a, st, s, kvh, po, g, n);
}

// Split-K schedule: block (kv head, partition, sequence) attends one
// partition of `split` tokens.  Partial rows: [sequence][head][partition].
template <int REP, bool FUSED, bool ROPE, int NH = 1>
__global__ __launch_bounds__(kWave) void decode_mfma_kernel(DecodeArgs a) {
  static_assert(2 * REP <= 16, "hi and lo columns must fit one 16-wide MFMA tile");
  __shared__ __attribute__((aligned(16))) uint8_t vring_[2 * NH * kVSlot];
  __shared__ __attribute__((aligned(16))) uint8_t newtok_[2 * NH * kRowBytes];  // K row, V row (f16)
  const int kvh = blockIdx.x, part = blockIdx.y, s = blockIdx.z;
  // The table window guesses that the partitions start at position 0 (no
  // sliding window), so that every load of the piece is issued before the
  // sequence's length is known; a wrong guess reloads it.
  PieceLoads<REP, NH> pl;
  __shared__ __attribute__((aligned(16))) uint8_t rope_table_[ROPE ? kRopeTableBytes : 16];
  stage_rope_table<ROPE>(a, (lds_u8*)rope_table_);
  piece_loads<REP, FUSED, ROPE, false, NH>(a, s, kvh, part * (a.split / kPage), pl);
  const SeqWindow w = seq_window<FUSED>(a, s);
  if (part >= w.nparts) return;  // wave-uniform
  const int jp = w.jf + part;
  const int ta = max(w.p0, jp * a.split);
  const int tb = min(w.L, (jp + 1) * a.split);
  PieceOut po;
  po.final = w.nparts == 1;
  po.pbase = ((size_t)s * a.n_heads + (size_t)kvh * REP) * a.max_parts + part;
  po.pstride = a.max_parts;
  run_piece<REP, FUSED, 2, ROPE, NH>(a, (lds_u8*)vring_, (lds_u8*)newtok_, pl, w.jf == 0, s, kvh, ta, tb,
                                     FUSED && part == w.nparts - 1 && w.L > 0, w.L - 1, po, (lds_u8*)rope_table_);
}

// ---------------------------------------------------------------------------
// Stream-K schedule.  The units of work are the (sequence, kv head, page)
// triples of every sequence's attention window, ordered by sequence, then kv
// head, then page: each (sequence, kv head) is a contiguous segment.  Wave w
// of W takes units [w*C, (w+1)*C) with C = max(kSkMinPages, ceil(T/W)), so
// all waves carry the same load and the launch fills the GPU exactly once.
// A wave's run of a segment is a piece; a piece that is a whole segment
// writes the output, the others leave partial rows (slot 0: the wave's first
// piece, slot 1: its last) that combine_sk_kernel merges.

// Sequences are taken 64 at a time: group g holds sequences 64g .. 64g+63,
// one per lane.  Per-lane view of sequence 64g + lane (past n_seq: empty).
struct SkSeq {
  int L;     // length, 0 when out of range (as in seq_window)
  int p0;    // window start
  int lo;    // first position that owns a page of the segment
  int np;    // pages per (sequence, kv head) segment
  int cnt;   // units of the sequence: np * n_kv
  int incl;  // units of every sequence up to and including this one
};

template <bool FUSED>
__device__ __forceinline__ SkSeq sk_fields(const DecodeArgs& a, int s, int n_seq) {
  SkSeq q;
  int L = 0, p0 = 0;
  if (s < n_seq) {
    L = a.kv_len ? a.kv_len[s] : a.kv_len_scalar;
    p0 = a.p_start ? a.p_start[s] : a.p_start_scalar;
  }
  // a length past what the grid or the table row can address marks the
  // sequence out of range: empty window, nothing stored
  L = L > min(a.max_kv_len, a.bt_stride * kPage) ? 0 : max(L, 0);
  p0 = min(max(p0, 0), L);
  int lo = p0;
  if (FUSED && L > 0) lo = min(lo, L - 1);
  q.L = L;
  q.p0 = p0;
  q.lo = lo;
  q.np = L > lo ? (L - 1) / kPage - lo / kPage + 1 : 0;
  q.cnt = q.np * a.n_kv;
  q.incl = 0;
  return q;
}

// Three inclusive scans over the wave's lanes, their steps interleaved.
__device__ __forceinline__ void wave_incl_scan3(int& x, int& y, int& z) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int xs = __shfl_up(x, d, kWave);
    const int ys = __shfl_up(y, d, kWave);
    const int zs = __shfl_up(z, d, kWave);
    if (lane >= d) {
      x += xs;
      y += ys;
      z += zs;
    }
  }
}

__device__ __forceinline__ int wave_incl_scan(int x) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(x, d, kWave);
    if (lane >= d) x += y;
  }
  return x;
}

// Group g with `base` units before it.
template <bool FUSED>
__device__ __forceinline__ SkSeq sk_group(const DecodeArgs& a, int n_seq, int g, int base) {
  SkSeq q = sk_fields<FUSED>(a, g * kWave + (int)(threadIdx.x & (kWave - 1)), n_seq);
  q.incl = base + wave_incl_scan(q.cnt);
  return q;
}

// More than 64 sequences: lane g (< number of groups, at most 64) returns the
// units before group g; *total gets all units.  Eight groups' lengths are
// loaded together.
template <bool FUSED>
__device__ __forceinline__ int sk_group_bases(const DecodeArgs& a, int n_seq, int* total) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int G = (n_seq + kWave - 1) / kWave;
  int mine = 0;
  for (int g0 = 0; g0 < G; g0 += 8) {
    int c[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) c[u] = sk_fields<FUSED>(a, (g0 + u) * kWave + lane, n_seq).cnt;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      int t = c[u];
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) t += __shfl_xor(t, o, kWave);
      if (lane == g0 + u) mine = t;
    }
  }
  const int incl = wave_incl_scan(mine);
  *total = __builtin_amdgcn_readlane(incl, kWave - 1);
  return incl - mine;
}

// The group holding unit cur (cur < total): the last one whose base is <= cur.
__device__ __forceinline__ int sk_find_group(int gb, int n_groups, int cur) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  return (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(lane < n_groups && gb <= cur)) - 1;
}

__device__ __forceinline__ int sk_chunk(int total, int n_waves) {
  return max(kSkMinPages, (total + n_waves - 1) / n_waves);
}

template <int REP, bool FUSED, int DEPTH, bool ROPE, bool Q8 = false, int NH = 1>
// Q8A pages with 128-wide heads run two waves per SIMD: the register budget
// is held to 256 so that the RoPE variant (whose rotation the compiler would
// otherwise schedule with every pair and sine/cosine live at once, 370
// registers) keeps that occupancy too.
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(Q8 && NH == 1 ? 2 : 1)))
void decode_sk_kernel(DecodeArgs a, int n_seq, int n_waves) {
  static_assert(2 * REP <= 16, "hi and lo columns must fit one 16-wide MFMA tile");
  __shared__ __attribute__((aligned(16))) uint8_t vring_[DEPTH * NH * kVSlot];
  __shared__ __attribute__((aligned(16))) uint8_t newtok_[2 * NH * kRowBytes];  // K row, V row (f16)
  __shared__ __attribute__((aligned(16))) uint8_t rope_table_[ROPE ? kRopeTableBytes : 16];
  const float rinv = rope_inv_load<ROPE>(a);
  const int wv = blockIdx.x;
  const int n_groups = (n_seq + kWave - 1) / kWave;
  int total = 0, gb = 0, g = 0;
  SkSeq q;
  if (n_groups == 1) {
    q = sk_group<FUSED>(a, n_seq, 0, 0);
    total = __builtin_amdgcn_readlane(q.incl, kWave - 1);
  } else {
    gb = sk_group_bases<FUSED>(a, n_seq, &total);
  }
  rope_inv_store<ROPE>((lds_u8*)rope_table_, rinv);
  const int chunk = sk_chunk(total, n_waves);
  int cur = wv * chunk;
  const int end = min(total, cur + chunk);
  if (n_groups > 1 && cur < end) {
    g = sk_find_group(gb, n_groups, cur);
    q = sk_group<FUSED>(a, n_seq, g, __builtin_amdgcn_readlane(gb, g));
  }
  int slot = 0;
  // the segment that this wave's first piece closes when it began in an
  // earlier wave: (sequence, kv head, its first wave, 2 * waves + slot of
  // that wave's piece); w = 0: none
  int4 desc = make_int4(0, 0, 0, 0);
  while (cur < end) {  // wave-uniform
    // the sequence holding unit cur: lanes whose inclusive prefix is <= cur
    int si = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(q.incl <= cur));
    if (si == kWave) {  // cur is past this group (more than 64 sequences only)
      g = sk_find_group(gb, n_groups, cur);
      q = sk_group<FUSED>(a, n_seq, g, __builtin_amdgcn_readlane(gb, g));
      si = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(q.incl <= cur));
    }
    const int s = g * kWave + si;
    const int np = __builtin_amdgcn_readlane(q.np, si);
    const int L = __builtin_amdgcn_readlane(q.L, si);
    const int p0 = __builtin_amdgcn_readlane(q.p0, si);
    const int pg0 = __builtin_amdgcn_readlane(q.lo, si) / kPage;  // the segment's first page
    const int sbase = __builtin_amdgcn_readlane(q.incl, si) - __builtin_amdgcn_readlane(q.cnt, si);
    const int kvh = (cur - sbase) / np;
    const int seg0 = sbase + kvh * np;
    const int pend = min(end, seg0 + np);
    const int i0 = cur - seg0, i1 = pend - seg0;  // pages [i0, i1) of the segment
    if (slot == 0 && i0 > 0 && i1 == np) {
      const int wa = seg0 / chunk;
      desc = make_int4(s, kvh, wa, (wv - wa + 1) * 2 + (seg0 == wa * chunk ? 0 : 1));
    }
    PieceLoads<REP, NH> pl;
    piece_loads<REP, FUSED, ROPE, Q8, NH>(a, s, kvh, pg0 + i0, pl);
    PieceOut po;
    po.final = i0 == 0 && i1 == np;
    po.pbase = ((size_t)wv * 2 + slot) * REP;
    po.pstride = 1;
    if constexpr (Q8)
      run_piece_q8<REP, DEPTH, FUSED, NH, ROPE>(a, (lds_u8*)vring_, (lds_u8*)newtok_, pl, true, s, kvh,
                                                max(p0, (pg0 + i0) * kPage), min(L, (pg0 + i1) * kPage),
                                                FUSED && i1 == np && L > 0, L - 1, po, (lds_u8*)rope_table_);
    else
      run_piece<REP, FUSED, DEPTH, ROPE, NH>(a, (lds_u8*)vring_, (lds_u8*)newtok_, pl, true, s, kvh,
                                             max(p0, (pg0 + i0) * kPage), min(L, (pg0 + i1) * kPage),
                                             FUSED && i1 == np && L > 0, L - 1, po, (lds_u8*)rope_table_);
    cur = pend;
    slot = 1;
  }
  if ((threadIdx.x & (kWave - 1)) == 0) a.sk_desc[wv] = desc;
}

// Block w merges the segment whose last piece is wave w's first piece, when
// that segment began in an earlier wave (the descriptor the decode kernel
// left), and writes zeros for the empty windows of sequences w, w + W, ...
// Wave h of the block merges query heads h, h + 4, ... of the segment.
template <int REP, bool FUSED, int NH = 1>
__global__ __launch_bounds__(kBlock) void combine_sk_kernel(DecodeArgs a, int n_seq, int n_waves) {
  constexpr int D = NH * kD;
  constexpr int C = D / kWave;
  const int w = blockIdx.x, wv = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int4 d = a.sk_desc[w];
  for (int s = w; s < n_seq; s += n_waves) {  // block-uniform
    if (sk_fields<FUSED>(a, s, n_seq).np == 0)
      for (int i = threadIdx.x; i < a.n_heads * D; i += kBlock) a.out[(size_t)s * a.n_heads * D + i] = 0.0f;
  }
  if (d.w == 0) return;
  const int s = d.x, kvh = d.y, wa = d.z, nw = d.w >> 1, first_slot = d.w & 1;
  for (int h = wv; h < REP; h += kWavesPerBlock) {
    const size_t row = ((size_t)s * a.n_heads + (size_t)kvh * REP + h) * D;
    float gv[C];  // the gate, loaded before the partial rows
#pragma unroll
    for (int c = 0; c < C; ++c) gv[c] = a.gate ? a.gate[row + c * kWave + lane] : 1.0f;
    float M, Ls, A[C];
    merge_wave<D, 1, 8>(reinterpret_cast<const float2*>(a.ws_ml), a.ws_acc, 0, nw,
                        [=](int j) { return ((size_t)(wa + j) * 2 + (j == 0 ? first_slot : 0)) * REP + h; },
                        M, Ls, A);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float v = Ls > 0.0f ? A[c] / Ls : 0.0f;
      a.out[row + c * kWave + lane] = a.gate ? v * gv[c] : v;
    }
  }
}


// ---------------------------------------------------------------------------
// Workgroup schedule (small batches): G workgroups of NW waves (two per CU
// at most; only as many as the batch can fill).  The units (sequence,
// kv head, page) are ordered as for stream-K.  When the batch is at most 64
// sequences and the grid holds it, each (sequence, kv head) segment gets
// workgroups of its own that split its pages evenly (segment-aligned
// ranges; the reference's one-sequence call always runs so); otherwise
// workgroup g of G takes units [A, B) = [g C, g C + C) with C = max(NW
// kWgMinPages, ceil(T / G)).  The waves split [A, B) equally (wave i:
// [A + i Cw, A + (i + 1) Cw)).  Each
// wave runs its pieces exactly as stream-K does, except that a piece that is
// not a whole segment leaves its partial rows in LDS (slot 0 for the wave's
// first piece, slot 1 for its last).  After a barrier the workgroup merges,
// in wave order, every segment that one of its wave boundaries (or its own
// boundaries A, B) cuts:
//  - a segment inside [A, B): the output rows are written;
//  - a segment that crosses A or B: the merged rows go to the workgroup's
//    partial slot in the workspace (0: the segment crossing A, 1: the one
//    crossing B) as device-scope stores, and wg_cnt[ga] (ga the segment's
//    first workgroup) counts the workgroups done with it once those stores
//    have completed.  The last one merges every workgroup's rows with
//    device-scope loads, in workgroup order, writes the output, and sets the
//    count back to zero for the next call.  (Device-scope accesses of the
//    rows themselves instead of agent-scope fences: each such fence writes
//    back or invalidates the whole L2 of an XCD.)
// No workgroup waits for another (the last to finish does the merge), and the
// result does not depend on which one that is: the merge order is fixed.
// ---------------------------------------------------------------------------
constexpr int kWgMinPages = 2;  // fewest pages per wave
// the last merge's rows in flight per wave: one round of loads for up to 32
// workgroups per segment (registers: 32 x (2 + D / 64), 128 at D = 128 and
// 192 at D = 256, whose one wave per SIMD has 512)
constexpr int kWgMergeRows = 32;

// Workgroups of a segment of np pages in the segment-aligned ranges (S the
// fewest pages of a workgroup): ceil(np / S), or floor(np / S) when that
// keeps the last merge to one round.
__host__ __device__ constexpr int wg_seg_ceil(int np, int S) {
  return (np + S - 1) / S > kWgMergeRows && np / S <= kWgMergeRows ? np / S : (np + S - 1) / S;
}

__device__ __forceinline__ int wg_chunk(int total, int n_wg, int nw) {
  return max(nw * kWgMinPages, (total + n_wg - 1) / n_wg);
}

// The segment holding unit u (u < total) as (sequence, kv head, [x0, x1)).
// (g, q) is the caller's current group of 64 sequences; it moves forward as
// u does (more than 64 sequences only).
struct WgSeg {
  int s, kvh, x0, x1;
};

template <bool FUSED>
__device__ __forceinline__ WgSeg wg_seg_at(const DecodeArgs& a, int n_seq, int n_groups, int gb, int& g,
                                           SkSeq& q, int u) {
  if (n_groups > 1) {
    const int gg = sk_find_group(gb, n_groups, u);
    if (gg != g) {
      g = gg;
      q = sk_group<FUSED>(a, n_seq, g, __builtin_amdgcn_readlane(gb, g));
    }
  }
  const int si = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(q.incl <= u));
  const int np = __builtin_amdgcn_readlane(q.np, si);
  const int sbase = __builtin_amdgcn_readlane(q.incl, si) - __builtin_amdgcn_readlane(q.cnt, si);
  WgSeg x;
  x.s = g * kWave + si;
  x.kvh = (u - sbase) / np;
  x.x0 = sbase + x.kvh * np;
  x.x1 = x.x0 + np;
  return x;
}

template <int REP, bool FUSED, int DEPTH, bool ROPE, bool Q8, int NW, int NH = 1>
// (As for stream-K; the RoPE variant at REP 8 would spill within 256
// registers, so it keeps its registers and the occupancy they allow.)
__global__ __launch_bounds__(kWave* NW)
__attribute__((amdgpu_waves_per_eu(Q8 && NH == 1 && !(ROPE && REP == 8) ? 2 : 1)))
void decode_wg_kernel(DecodeArgs a, int n_seq, int n_wg, int n_cu) {
  static_assert(2 * REP <= 16, "hi and lo columns must fit one 16-wide MFMA tile");
  constexpr int kSlots = Q8 ? 1 : DEPTH;
  constexpr int D = NH * kD;                    // head dim
  constexpr int CL = D / kWave;                 // elements a lane merges per row
  constexpr int kRow = D + 2;                   // an LDS partial row: acc, m, l
  typedef __attribute__((address_space(3))) float lds_f32;
  __shared__ __attribute__((aligned(16))) uint8_t vring_[NW][kSlots * NH * kVSlot];
  __shared__ __attribute__((aligned(16))) uint8_t newtok_[NW][2 * NH * kRowBytes];
  __shared__ __attribute__((aligned(16))) uint8_t rope_table_[NW][ROPE ? kRopeTableBytes : 16];
  __shared__ __attribute__((aligned(16))) float part_[NW * 2 * REP * kRow];
  __shared__ int split_[NW + 1][4];  // cut segments: s, kv head, x0, x1
  __shared__ int n_split_;
  __shared__ int last_[2];           // cut segments this workgroup merges last (index or -1)
  const int wi = (int)(threadIdx.x / kWave), lane = (int)(threadIdx.x % kWave);
  const int wg = blockIdx.x;
  const float rinv = rope_inv_load<ROPE>(a);

  // the layout (every wave computes it)
  const int n_groups = (n_seq + kWave - 1) / kWave;
  // Segment-aligned ranges when the batch is one group and the grid holds
  // them: segment (s, h) gets kseg[s] workgroups of its own, which split its
  // pages evenly, so no workgroup or wave holds the end of one segment and
  // the start of the next (two pieces in a row on one wave, two merges on one
  // workgroup).  kseg = ceil(np / S) (S = NW kWgMinPages, the fewest units
  // of a workgroup; floor(np / S) where that keeps the last merge to one
  // round) while those workgroups have a CU each, else max(1, floor(np / S)):
  // a wave with one more page costs less than two workgroups on one CU or a
  // second round of row loads.  Otherwise workgroup g takes [g C, g C + C).
  constexpr int kMinShare = NW * kWgMinPages;
  int total = 0, gb = 0, g = 0;
  int kseg = 0, kincl = 0;
  bool aligned = false;
  SkSeq q;
  if (n_groups == 1) {
    q = sk_fields<FUSED>(a, lane, n_seq);
    const int kc = wg_seg_ceil(q.np, kMinShare), kf = q.np > 0 ? max(1, q.np / kMinShare) : 0;
    int ic = kc * a.n_kv, iflo = kf * a.n_kv;
    q.incl = q.cnt;
    wave_incl_scan3(q.incl, ic, iflo);  // units and both workgroup counts in one pass
    total = __builtin_amdgcn_readlane(q.incl, kWave - 1);
    const bool ceil_fits = __builtin_amdgcn_readlane(ic, kWave - 1) <= n_cu;
    kseg = ceil_fits ? kc : kf;
    kincl = ceil_fits ? ic : iflo;
    aligned = __builtin_amdgcn_readlane(kincl, kWave - 1) <= n_wg;
  } else {
    gb = sk_group_bases<FUSED>(a, n_seq, &total);
    q = sk_group<FUSED>(a, n_seq, 0, 0);
  }
  rope_inv_store<ROPE>((lds_u8*)rope_table_[wi], rinv);
  const int C = wg_chunk(total, n_wg, NW);
  int A, B;
  if (aligned) {
    const int si = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(kincl <= wg));
    A = B = total;
    if (si < kWave) {
      const int k = __builtin_amdgcn_readlane(kseg, si);
      const int kb = __builtin_amdgcn_readlane(kincl, si) - k * a.n_kv;
      const int np = __builtin_amdgcn_readlane(q.np, si);
      const int h = (wg - kb) / k, j = (wg - kb) - h * k;
      const int x0 = __builtin_amdgcn_readlane(q.incl, si) - __builtin_amdgcn_readlane(q.cnt, si) + h * np;
      A = x0 + j * np / k;
      B = x0 + (j + 1) * np / k;
    }
  } else {
    A = min(total, wg * C);
    B = min(total, A + C);
  }
  const int Cw = (B - A + NW - 1) / NW;  // wave i: [A + i Cw, A + (i + 1) Cw) within [A, B)
  // the first and last workgroup of segment (s, kvh) = units [x0, x1)
  auto seg_wgs = [&](int s, int kvh, int x0, int x1, int& ga, int& gz) {
    if (aligned) {
      const int sl = __builtin_amdgcn_readfirstlane(s);
      const int k = __builtin_amdgcn_readlane(kseg, sl);
      ga = __builtin_amdgcn_readlane(kincl, sl) - k * a.n_kv + kvh * k;
      gz = ga + k - 1;
    } else {
      ga = x0 / C;
      gz = (x1 - 1) / C;
    }
  };
  int cur = min(B, A + wi * Cw);
  const int end = min(B, cur + Cw);
  if (n_groups > 1 && cur < end) {
    g = sk_find_group(gb, n_groups, cur);
    q = sk_group<FUSED>(a, n_seq, g, __builtin_amdgcn_readlane(gb, g));
  }
  int slot = 0;
  while (cur < end) {  // wave-uniform
    int si = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(q.incl <= cur));
    if (si == kWave) {  // cur is past this group (more than 64 sequences only)
      g = sk_find_group(gb, n_groups, cur);
      q = sk_group<FUSED>(a, n_seq, g, __builtin_amdgcn_readlane(gb, g));
      si = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(q.incl <= cur));
    }
    const int s = g * kWave + si;
    const int np = __builtin_amdgcn_readlane(q.np, si);
    const int L = __builtin_amdgcn_readlane(q.L, si);
    const int p0 = __builtin_amdgcn_readlane(q.p0, si);
    const int pg0 = __builtin_amdgcn_readlane(q.lo, si) / kPage;
    const int sbase = __builtin_amdgcn_readlane(q.incl, si) - __builtin_amdgcn_readlane(q.cnt, si);
    const int kvh = (cur - sbase) / np;
    const int seg0 = sbase + kvh * np;
    const int pend = min(end, seg0 + np);
    const int i0 = cur - seg0, i1 = pend - seg0;  // pages [i0, i1) of the segment
    PieceLoads<REP, NH> pl;
    piece_loads<REP, FUSED, ROPE, Q8, NH>(a, s, kvh, pg0 + i0, pl);
    PieceOut po;
    po.final = i0 == 0 && i1 == np;
    po.pbase = ((size_t)wi * 2 + slot) * REP;
    po.pstride = 1;
    po.in_lds = true;
    po.lds = (lds_f32*)part_;
    if constexpr (Q8)
      run_piece_q8<REP, DEPTH, FUSED, NH, ROPE>(a, (lds_u8*)vring_[wi], (lds_u8*)newtok_[wi], pl, true, s, kvh,
                                                max(p0, (pg0 + i0) * kPage), min(L, (pg0 + i1) * kPage),
                                                FUSED && i1 == np && L > 0, L - 1, po, (lds_u8*)rope_table_[wi]);
    else
      run_piece<REP, FUSED, DEPTH, ROPE, NH>(a, (lds_u8*)vring_[wi], (lds_u8*)newtok_[wi], pl, true, s, kvh,
                                             max(p0, (pg0 + i0) * kPage), min(L, (pg0 + i1) * kPage),
                                             FUSED && i1 == np && L > 0, L - 1, po, (lds_u8*)rope_table_[wi]);
    cur = pend;
    slot = 1;
  }

  // The segments cut by a boundary A + i Cw (i = 0 .. NW, the last being B),
  // in order, each once: wave 0 lists them.
  if (wi == 0) {
    int ns = 0;
    int prev_x0 = -1;
    for (int i = 0; i <= NW; ++i) {
      const int b = min(B, A + i * Cw);
      if (b <= 0 || b >= total || (i > 0 && b == min(B, A + (i - 1) * Cw))) continue;
      const WgSeg x = wg_seg_at<FUSED>(a, n_seq, n_groups, gb, g, q, b);
      if (x.x0 >= b || x.x0 == prev_x0) continue;  // starts at b, or listed already
      prev_x0 = x.x0;
      if (lane == 0) {
        split_[ns][0] = x.s;
        split_[ns][1] = x.kvh;
        split_[ns][2] = x.x0;
        split_[ns][3] = x.x1;
      }
      ++ns;
    }
    if (lane == 0) {
      n_split_ = ns;
      last_[0] = last_[1] = -1;
    }
  }
  __syncthreads();

  // Merge each cut segment's pieces held in LDS (wave e takes segments e,
  // e + NW, ...), head by head; lane l holds acc elements l + 64 c.
  const int n_split = n_split_;
  for (int e = wi; e < n_split; e += NW) {  // wave-uniform
    const int s = split_[e][0], kvh = split_[e][1], x0 = split_[e][2], x1 = split_[e][3];
    const int lo = max(x0, A), hi = min(x1, B);
    const int w1 = (lo - A) / Cw, w2 = (hi - 1 - A) / Cw;  // the waves holding pieces of it
    const bool inside = x0 >= A && x1 <= B;
    const int side = x0 < A ? 0 : 1;
    for (int h = 0; h < REP; ++h) {
      float M = kMInit, Ls = 0.0f, Av[CL];
#pragma unroll
      for (int c = 0; c < CL; ++c) Av[c] = 0.0f;
      for (int w = w1; w <= w2; ++w) {
        const int sl = (w == w1 && x0 > A + w1 * Cw) ? 1 : 0;
        const lds_f32* row = (const lds_f32*)part_ + ((size_t)(w * 2 + sl) * REP + h) * kRow;
        const float m = row[D], l = row[D + 1];
        const float Mn = fmaxf(M, m);
        const float ra = fast_exp2(M - Mn), rb = fast_exp2(m - Mn);
        Ls = Ls * ra + l * rb;
#pragma unroll
        for (int c = 0; c < CL; ++c) Av[c] = Av[c] * ra + row[lane + c * kWave] * rb;
        M = Mn;
      }
      if (inside) {
        const size_t orow = ((size_t)s * a.n_heads + (size_t)kvh * REP + h) * D;
        const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
#pragma unroll
        for (int c = 0; c < CL; ++c) a.out[orow + c * kWave + lane] = gated(a, orow + c * kWave + lane, Av[c] * inv);
      } else {
        // device-scope stores: written through to where every XCD reads
        const size_t r = ((size_t)wg * 2 + side) * REP + h;
#pragma unroll
        for (int c = 0; c < CL; ++c)
          __hip_atomic_store(a.ws_acc + r * D + c * kWave + lane, Av[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lane == 0) {
          __hip_atomic_store(a.ws_ml + r * 2 + 0, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(a.ws_ml + r * 2 + 1, Ls, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    if (!inside) {
      // Count this workgroup done once its rows are stored.  The rows are
      // device-scope stores and the merge reads them with device-scope loads,
      // so no cache-wide write-back or invalidate is needed: the wait for the
      // stores to complete orders them before the count.
      int ga, gz;
      seg_wgs(s, kvh, x0, x1, ga, gz);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      uint32_t old = 0;
      if (lane == 0) old = __hip_atomic_fetch_add(a.wg_cnt + ga, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      old = __builtin_amdgcn_readfirstlane(old);
      // a count above gz - ga cannot happen on a header that was zero: flag it
      // for the host (lnskv_sync reports it); the count is left as it is, so
      // every later call on this header is flagged too
      if (old > (uint32_t)(gz - ga) && lane == 0 && a.ws_err)
        __hip_atomic_store(a.ws_err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      if (old == (uint32_t)(gz - ga)) {  // every other workgroup is done: this one merges
        if (lane == 0) {
          __hip_atomic_store(a.wg_cnt + ga, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          last_[side] = e;
        }
      }
    }
  }
  __syncthreads();

  // Cut segments this workgroup finished last: merge every workgroup's rows
  // (workgroup ga's from its slot 1, the others' from slot 0) in workgroup
  // order, with device-scope loads.  Wave v takes query head v % REP and the
  // rows j with j % HP == v / REP (HP = NW / REP parts per head), every load
  // of up to 32 rows in flight before any is used (one round of loads for the
  // 32 workgroups that share a 256-page segment); wave h < REP then merges
  // the HP parts of head h through LDS, in part order.
  constexpr int HP = NW >= REP ? NW / REP : 1;  // parts per head
  constexpr int HW = NW >= REP ? 1 : REP / NW;  // heads per wave
  constexpr int kChunk = kWgMergeRows;
  lds_f32* prow = (lds_f32*)part_;  // free again: row v of wave v, acc then m, l
#pragma unroll
  for (int side = 0; side < 2; ++side) {
    const int e = last_[side];
    if (e < 0) continue;  // block-uniform
    const int s = split_[e][0], kvh = split_[e][1], x0 = split_[e][2], x1 = split_[e][3];
    int ga, gz;
    seg_wgs(s, kvh, x0, x1, ga, gz);
    const int nwg = gz - ga + 1;
    for (int hh = 0; hh < HW; ++hh) {
      const int h = NW >= REP ? wi % REP : wi + hh * NW;
      const int part = NW >= REP ? wi / REP : 0;
      const size_t orow = ((size_t)s * a.n_heads + (size_t)kvh * REP + h) * D;
      // the gate of the row this wave writes, loaded before the rows (its
      // round trip overlaps theirs instead of following the merge)
      float gv[CL];
#pragma unroll
      for (int c = 0; c < CL; ++c) gv[c] = HP == 1 && a.gate ? a.gate[orow + c * kWave + lane] : 1.0f;
      float M = kMInit, Ls = 0.0f, Av[CL];
#pragma unroll
      for (int c = 0; c < CL; ++c) Av[c] = 0.0f;
      for (int j0 = part; j0 < nwg; j0 += kChunk * HP) {  // wave-uniform
        float m[kChunk], l[kChunk], v[kChunk][CL];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
          const int j = j0 + u * HP;
          m[u] = kMInit;
          l[u] = 0.0f;
#pragma unroll
          for (int c = 0; c < CL; ++c) v[u][c] = 0.0f;
          if (j < nwg) {
            const size_t r = ((size_t)(ga + j) * 2 + (j == 0 ? 1 : 0)) * REP + h;
            m[u] = __hip_atomic_load(a.ws_ml + r * 2 + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            l[u] = __hip_atomic_load(a.ws_ml + r * 2 + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int c = 0; c < CL; ++c)
              v[u][c] = __hip_atomic_load(a.ws_acc + r * D + c * kWave + lane, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        float Mc = M;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) Mc = fmaxf(Mc, m[u]);
        const float ra = fast_exp2(M - Mc);
        Ls *= ra;
#pragma unroll
        for (int c = 0; c < CL; ++c) Av[c] *= ra;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
          const float wgt = fast_exp2(m[u] - Mc);
          Ls = fmaf(wgt, l[u], Ls);
#pragma unroll
          for (int c = 0; c < CL; ++c) Av[c] = fmaf(wgt, v[u][c], Av[c]);
        }
        M = Mc;
      }
      if constexpr (HP == 1) {
        const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
#pragma unroll
        for (int c = 0; c < CL; ++c) {
          const float v = Av[c] * inv;
          a.out[orow + c * kWave + lane] = a.gate ? v * gv[c] : v;
        }
      } else {
#pragma unroll
        for (int c = 0; c < CL; ++c) prow[wi * kRow + c * kWave + lane] = Av[c];
        if (lane == 0) {
          prow[wi * kRow + D] = M;
          prow[wi * kRow + D + 1] = Ls;
        }
      }
    }
    if constexpr (HP > 1) {
      __syncthreads();
      if (wi < REP) {
        float Mt = kMInit;
#pragma unroll
        for (int q = 0; q < HP; ++q) Mt = fmaxf(Mt, prow[(wi + q * REP) * kRow + D]);
        float Lt = 0.0f, T[CL];
#pragma unroll
        for (int c = 0; c < CL; ++c) T[c] = 0.0f;
#pragma unroll
        for (int q = 0; q < HP; ++q) {
          const lds_f32* row = prow + (wi + q * REP) * kRow;
          const float wgt = fast_exp2(row[D] - Mt);
          Lt = fmaf(wgt, row[D + 1], Lt);
#pragma unroll
          for (int c = 0; c < CL; ++c) T[c] = fmaf(wgt, row[c * kWave + lane], T[c]);
        }
        const size_t orow = ((size_t)s * a.n_heads + (size_t)kvh * REP + wi) * D;
        const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
#pragma unroll
        for (int c = 0; c < CL; ++c) a.out[orow + c * kWave + lane] = gated(a, orow + c * kWave + lane, T[c] * inv);
      }
      __syncthreads();
    }
  }

  // zero rows for the sequences with empty windows (wg, wg + G, ...)
  for (int s = wg; s < n_seq; s += n_wg) {  // block-uniform
    if (sk_fields<FUSED>(a, s, n_seq).np == 0)
      for (int i = threadIdx.x; i < a.n_heads * D; i += kWave * NW) a.out[(size_t)s * a.n_heads * D + i] = 0.0f;
  }
}

}  // namespace

namespace {
// RoPE variants exist for fused calls only (a.rope_half > 0).
template <int REP, bool FUSED, int NH>
void launch_mfma_rep(const DecodeArgs& a, int n_seq, hipStream_t st) {
  const dim3 grid((unsigned)a.n_kv, (unsigned)a.max_parts, (unsigned)n_seq);
  if (FUSED && a.rope_half > 0)
    decode_mfma_kernel<REP, FUSED, FUSED, NH><<<grid, kWave, 0, st>>>(a);
  else
    decode_mfma_kernel<REP, FUSED, false, NH><<<grid, kWave, 0, st>>>(a);
  launch_combine<REP, NH * kD, FUSED>(a, n_seq, st);
}

// rep (1, 2, 4, 8) and head dim (128: NH = 1, 256: NH = 2) as compile-time
// constants: f(rep_c, nh_c).
template <typename F>
int with_rep_nh(int rep, int d, F&& f) {
  if (d != 128 && d != 256) return fail(LNSKV_ERR_UNSUPPORTED, "head_dim %d: the matrix-core decode takes 128 or 256", d);
  auto go = [&](auto rep_c) {
    if (d == 256) f(rep_c, std::integral_constant<int, 2>{});
    else f(rep_c, std::integral_constant<int, 1>{});
  };
  switch (rep) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 4: go(std::integral_constant<int, 4>{}); break;
    case 8: go(std::integral_constant<int, 8>{}); break;
    default: return fail(LNSKV_ERR_UNSUPPORTED, "n_heads/n_kv_heads = %d not supported (1, 2, 4, 8)", rep);
  }
  return LNSKV_OK;
}
}  // namespace

template <bool FUSED>
int launch_decode_mfma_f16(const DecodeArgs& a, int rep, int d, int n_seq, hipStream_t st) {
  if (int rc = with_rep_nh(rep, d, [&](auto rep_c, auto nh_c) {
        launch_mfma_rep<decltype(rep_c)::value, FUSED, decltype(nh_c)::value>(a, n_seq, st);
      }))
    return rc;
  return hip_check("decode kernel launch");
}

template int launch_decode_mfma_f16<false>(const DecodeArgs&, int, int, int, hipStream_t);
template int launch_decode_mfma_f16<true>(const DecodeArgs&, int, int, int, hipStream_t);

namespace {
// Stream-K launch shape: two pages in flight per wave and four waves per CU
// (one per SIMD).  Measured on the c2 shape: one wave per SIMD matches two
// (2-4 pages in flight each) within noise, and avoids the older-wave-first
// issue arbitration that runs the second wave of a SIMD about 30% slower.
constexpr int kSkDepth = 2;
constexpr int kSkWavesPerCu = 4;
// Q8A pages: half the bytes per page and more work per byte (int8 -> f16,
// scales), so two waves per SIMD hide each other's per-page dependency chain:
// c2-shaped Q8A step 57.2 us with four waves per CU, 53.7 with eight; two,
// three or four pages in flight per wave measured the same.
// Measured against codes by LDS DMA into a ring of code slots (no registers
// for pages in flight): 56.4 us per c2 Q8A step with one wave per SIMD and six
// pages in flight, 51.0-51.4 with two waves and three, against 49.5 here.
constexpr int kSkDepthQ8 = 2;
constexpr int kSkWavesPerCuQ8 = 8;
// 256-wide heads (one wave per SIMD on either page type): also two pages
// in flight; at the Qwen3.5 shape three and four measured 57.8 and 61.6 us
// per Q8A step (RoPE, gated) against 53.0, and 73.0 and 73.3 per f16 step
// against 70.4-72.1.
constexpr int kSkDepthWide = 2;
template <bool Q8, int NH>
constexpr int sk_depth() {
  return NH == 2 ? kSkDepthWide : (Q8 ? kSkDepthQ8 : kSkDepth);
}

// Resident waves of one stream-K kernel (ROPE: the fused variant that turns
// RoPE in registers, whose extra registers may fit fewer waves), capped at
// the launch shape's waves per CU.
template <int REP, bool FUSED, bool Q8, int NH, bool ROPE>
int sk_waves_of(int cus, int* waves) {
  int per_cu = 0;
  constexpr int depth = sk_depth<Q8, NH>();
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_sk_kernel<REP, FUSED, depth, ROPE, Q8, NH>, kWave,
                                                   0) != hipSuccess)
    per_cu = 0;
  if (per_cu <= 0) return fail(LNSKV_ERR_HIP, "occupancy query of the stream-K decode kernel failed");
  *waves = cus * std::min(per_cu, Q8 ? kSkWavesPerCuQ8 : kSkWavesPerCu);
  return LNSKV_OK;
}

template <int REP, bool FUSED, int NH>
void launch_sk_rep(const DecodeArgs& a, int n_seq, int n_waves, bool q8, hipStream_t st) {
  const bool rope = FUSED && a.rope_half > 0;
  constexpr int dq = sk_depth<true, NH>(), df = sk_depth<false, NH>();
  if (q8 && rope)
    decode_sk_kernel<REP, FUSED, dq, FUSED, true, NH><<<n_waves, kWave, 0, st>>>(a, n_seq, n_waves);
  else if (q8)
    decode_sk_kernel<REP, FUSED, dq, false, true, NH><<<n_waves, kWave, 0, st>>>(a, n_seq, n_waves);
  else if (rope)
    decode_sk_kernel<REP, FUSED, df, FUSED, false, NH><<<n_waves, kWave, 0, st>>>(a, n_seq, n_waves);
  else
    decode_sk_kernel<REP, FUSED, df, false, false, NH><<<n_waves, kWave, 0, st>>>(a, n_seq, n_waves);
  combine_sk_kernel<REP, FUSED, NH><<<n_waves, kBlock, 0, st>>>(a, n_seq, n_waves);
}
}  // namespace

int mfma_sk_waves(int rep, int d, bool fused, bool q8, bool rope, int* waves) {
  // resident waves used per launch on the current device, kept per
  // (device, rep, head dim, fused, q8, rope)
  static std::mutex mu;
  static std::map<std::tuple<int, int, int, bool, bool, bool>, int> cache;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LNSKV_ERR_HIP, "hipGetDevice failed");
  rope = rope && fused;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(dev, rep, d, fused, q8, rope);
  const auto it = cache.find(key);
  if (it != cache.end()) {
    *waves = it->second;
    return LNSKV_OK;
  }
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return fail(LNSKV_ERR_HIP, "compute-unit count query failed");
  int rc = LNSKV_OK;
  if (int r = with_rep_nh(rep, d, [&](auto rep_c, auto nh_c) {
        constexpr int R = decltype(rep_c)::value, NH = decltype(nh_c)::value;
        auto of = [&](auto q8_c) {
          constexpr bool Q = decltype(q8_c)::value;
          if (!fused) return sk_waves_of<R, false, Q, NH, false>(cus, waves);
          return rope ? sk_waves_of<R, true, Q, NH, true>(cus, waves) : sk_waves_of<R, true, Q, NH, false>(cus, waves);
        };
        rc = q8 ? of(std::true_type{}) : of(std::false_type{});
      }))
    return r;
  if (rc == LNSKV_OK) cache[key] = *waves;
  return rc;
}

template <bool FUSED>
int launch_decode_mfma_sk(const DecodeArgs& a, int rep, int d, int n_seq, int n_waves, bool q8, hipStream_t st) {
  if (n_seq > kSkMaxSeqs)
    return fail(LNSKV_ERR_INVALID, "stream-K decode serves at most %d sequences", kSkMaxSeqs);
  if (int rc = with_rep_nh(rep, d, [&](auto rep_c, auto nh_c) {
        launch_sk_rep<decltype(rep_c)::value, FUSED, decltype(nh_c)::value>(a, n_seq, n_waves, q8, st);
      }))
    return rc;
  return hip_check("stream-K decode kernel launch");
}

template int launch_decode_mfma_sk<false>(const DecodeArgs&, int, int, int, int, bool, hipStream_t);
template int launch_decode_mfma_sk<true>(const DecodeArgs&, int, int, int, int, bool, hipStream_t);

namespace {
// Workgroup schedule launch shape: two workgroups per CU, of two waves (f16
// pages) or four (Q8A pages), two pages in flight per wave.  Measured on the
// reference's one-sequence call (Q8A, 4096 tokens): 13.8 us per call against
// 15.7 with one workgroup of four / eight waves per CU and 19.6 for stream-K.
constexpr int kWgWaves = 2;
constexpr int kWgWavesQ8 = 4;
constexpr int kWgPerCu = 2;

template <int REP, bool FUSED, int NH>
void launch_wg_rep(const DecodeArgs& a, int n_seq, int n_wg, int n_cu, bool q8, hipStream_t st) {
  const bool rope = FUSED && a.rope_half > 0;
  if (q8 && rope)
    decode_wg_kernel<REP, FUSED, kSkDepthQ8, FUSED, true, kWgWavesQ8, NH>
        <<<n_wg, kWave * kWgWavesQ8, 0, st>>>(a, n_seq, n_wg, n_cu);
  else if (q8)
    decode_wg_kernel<REP, FUSED, kSkDepthQ8, false, true, kWgWavesQ8, NH>
        <<<n_wg, kWave * kWgWavesQ8, 0, st>>>(a, n_seq, n_wg, n_cu);
  else if (rope)
    decode_wg_kernel<REP, FUSED, kSkDepth, FUSED, false, kWgWaves, NH>
        <<<n_wg, kWave * kWgWaves, 0, st>>>(a, n_seq, n_wg, n_cu);
  else
    decode_wg_kernel<REP, FUSED, kSkDepth, false, false, kWgWaves, NH>
        <<<n_wg, kWave * kWgWaves, 0, st>>>(a, n_seq, n_wg, n_cu);
}
}  // namespace

int mfma_wg_count(int* n_wg) {
  // kWgPerCu workgroups per CU of the current device (at most kWgMaxGroups)
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LNSKV_ERR_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(mu);
  const auto it = cache.find(dev);
  if (it != cache.end()) {
    *n_wg = it->second;
    return LNSKV_OK;
  }
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return fail(LNSKV_ERR_HIP, "compute-unit count query failed");
  const int n = std::min(cus * kWgPerCu, kWgMaxGroups);
  cache[dev] = n;
  *n_wg = n;
  return LNSKV_OK;
}

template <bool FUSED>
int launch_decode_mfma_wg(const DecodeArgs& a, int rep, int d, int n_seq, int n_wg, bool q8, hipStream_t st) {
  if (n_seq > kSkMaxSeqs)
    return fail(LNSKV_ERR_INVALID, "the workgroup schedule serves at most %d sequences", kSkMaxSeqs);
  if (n_wg <= 0 || n_wg > kWgMaxGroups) return fail(LNSKV_ERR_INVALID, "%d workgroups", n_wg);
  // Launch only the workgroups the batch can fill: with at most `bound`
  // units (from max_kv_len), groups of NW * kWgMinPages units each cover
  // them, so the kernel's chunk C = max(NW * kWgMinPages, ceil(T / G)) stays
  // at its minimum and [0, G * C) still holds every unit; one more per
  // segment lets the segment-aligned ranges (ceil(np / C) or fewer
  // workgroups per segment, at most T / C + n_seq n_kv in all) fit the grid.
  const int nw = q8 ? kWgWavesQ8 : kWgWaves;
  const int64_t bound = (int64_t)n_seq * a.n_kv * ((int64_t)a.max_kv_len / kPage + 1);
  const int64_t per = (int64_t)nw * kWgMinPages;
  const int n_cu = n_wg / kWgPerCu;
  int64_t want = (bound + per - 1) / per + (int64_t)n_seq * a.n_kv;
  if (!a.kv_len && !a.p_start) {
    // every sequence has the scalar window (the reference's one-sequence
    // call): exactly the kernel's segment-aligned count, np as in sk_fields
    int L = a.kv_len_scalar;
    L = L > std::min(a.max_kv_len, a.bt_stride * kPage) ? 0 : std::max(L, 0);
    const int p0 = std::min(std::max(a.p_start_scalar, 0), L);
    const int lo = FUSED && L > 0 ? std::min(p0, L - 1) : p0;
    const int64_t np = L > lo ? (L - 1) / kPage - lo / kPage + 1 : 0;
    const int64_t segs = (int64_t)n_seq * a.n_kv;
    want = segs * wg_seg_ceil((int)np, (int)per);
    if (want > n_cu) want = segs * (np > 0 ? std::max<int64_t>(1, np / per) : 0);
  }
  const int groups = (int)std::max<int64_t>(1, std::min<int64_t>(n_wg, want));
  if (int rc = with_rep_nh(rep, d, [&](auto rep_c, auto nh_c) {
        launch_wg_rep<decltype(rep_c)::value, FUSED, decltype(nh_c)::value>(a, n_seq, groups, n_cu, q8, st);
      }))
    return rc;
  return hip_check("workgroup decode kernel launch");
}

template int launch_decode_mfma_wg<false>(const DecodeArgs&, int, int, int, int, bool, hipStream_t);
template int launch_decode_mfma_wg<true>(const DecodeArgs&, int, int, int, int, bool, hipStream_t);


// ---------------------------------------------------------------------------
// Chunked prefill over pages.  The chunk's K/V are already in the pages; a
// query at position P attends the window [p_start, P] of its sequence, as the
// decode would with kv_len = P + 1 -- or, for a sliding window w > 0,
// [max(p_start, P - w + 1), P], the reference's per-token kv_p_start.
//
// Workgroup = (tile of QT queries of one chunk, kv head), eight waves.  The
// workgroup streams the tile's window two pages (32 tokens) at a time through
// a three-slot LDS ring: each wave DMAs a quarter of two of the pair's four
// page regions (K and V of each page), a barrier publishes the pair, and all
// waves read it from LDS, so a page is fetched once per tile.  Wave w serves
// the 16 queries of query group w / WPQ and HW = min(REP, 2) query heads
// (head set w % WPQ); the K and V operands it reads from LDS serve all HW
// heads.  QT = 64 queries for REP <= 4, 32 for REP = 8.
//
// Per pair and head, lane (g, n) = (lane / 16, lane % 16):
//  Q.K^T  per page, S^T[16 tok][16 query] = K . Q^T as 4 x 2
//         v_mfma_f32_16x16x32_f16 (q as f16 hi and lo parts, each query and
//         head scaled by 2^-E); lane (g, n) receives S^T[token 4g+ii][query n].
//  softmax  per query over the pair's 32 tokens; the running max is raised
//         only past a slack of 8 (log2 units); tokens after the query's
//         position, outside the window or on a missing page are masked.
//  P.V    O[16 query][128] += P[16 query][32 tok] . V[32 tok][128] as 8 x 2
//         v_mfma_f32_16x16x32_f16 (p as f16 hi and lo).  The contraction
//         index k = 8g + e is page 0's token 4g+e for e < 4 and page 1's token
//         4g+e-4 otherwise, so the A operand is the lane's own eight weights
//         and the B operand is two transposed LDS reads, one per page.  Lane
//         (g, n) accumulates O[query 4g+ii][16 nb + n].
//
// LDS slot = K page 0 | K page 1 | V page 0 | V page 1, 4 KiB each.  K row r
// holds token r with its 16-byte chunk c at chunk c ^ r, so the A-operand
// reads (16 lanes: 16 tokens, one logical chunk) hit 16 distinct bank groups.
// V rows use the decode's swizzled layout for ds_read_b64_tr_b16.
//
// Blocks are numbered (tile, kv head) with the kv head fastest.  Consecutive
// blocks go to the 8 XCDs in turn, so with 8 kv heads every tile of one
// (chunk, kv head) runs on the same XCD and re-reads its pages from that
// XCD's L2, and every XCD gets an equal share of each chunk.
// ---------------------------------------------------------------------------
namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
// K and V of two pages, per 128-wide half of the head: [K p0 | K p1 | V p0 | V p1]
template <int NH>
constexpr int kPfSlot = NH * 4 * kVSlot;

// Two query heads per wave and eight waves per workgroup (two per SIMD, 256
// VGPRs each): measured against four heads with four waves (one per SIMD,
// 20% slower), one head with eight waves (16% slower) and two heads with
// four waves, two workgroups per CU (35% slower) on c2's pages.
// 256-wide heads (NH = 2 halves): one query head per wave (the accumulators
// and operands of a second would not fit in 256 VGPRs) and one pair per
// barrier (a pair's slot is twice as large).
template <int REP, int NH = 1>
struct PfShape {
  static constexpr int HW = NH == 2 ? 1 : (REP < 2 ? REP : 2);  // query heads per wave
  static constexpr int WPQ = REP / HW;                          // waves per 16 queries
  static constexpr int NW = 8;                                  // waves per workgroup
  static constexpr int QT = 16 * (NW / WPQ);                    // queries per tile
  static constexpr int RPW = 16 * NH / NW;                      // quarter regions a wave DMAs per pair
  static constexpr int kBatch = NH == 2 ? 1 : 2;                // pairs consumed per barrier (1 to 3)
  static constexpr int kDepth = 3 * kBatch;  // ring slots: a batch consumed, a batch in flight, a batch issued
};

// Workgroup barrier after this wave's LDS accesses have completed.  No
// release fence: that would also wait for the DMAs still in flight.  The
// memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void pf_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Per-lane constants of the pair DMA and the LDS operand reads.
// The K and V read offsets of operand j / nb are rebuilt from two registers
// each (a constant XOR and an add) instead of being held per operand: with
// two waves per SIMD the kernel has 256 VGPRs, and twelve held offsets
// spilled.  K operand j reads chunk (4j + g) ^ n of row n, at
// krow + ((64 j) ^ kx) with kx = 64 (n >> 2) and krow = 256 n + 16 (g ^ (n & 3));
// V operand nb (dims 16 nb ..) reads chunk (2 nb + sub) ^ sw(Rv) of row
// Rv = 4 (n >> 2) + g, at vrow + ((32 nb) ^ vx) with vx = 16 sw(Rv) (sw is
// even) and vrow = 256 Rv + 8 (n & 1) + 16 sub, sub = (n & 3) >> 1.
struct PfLanes {
  uint32_t koff;    // K DMA: token 4w+g, chunk n ^ (4w+g)
  uint32_t voff;    // V DMA: token 4g+w, chunk n ^ sw(4w+g)
  uint32_t lds_q;   // 1024 w: this wave's quarter of a page region
  uint32_t krow, kx;
  uint32_t vrow, vx;
};

// DMA of this wave's share of pages ph0 and ph1 into `slot`: quarter w % 4
// of page regions (w / 4) * RPW .. + RPW - 1 (region r: half r / 4 of the
// head; within it K of page r % 4 for r % 4 < 2, V of page r % 4 - 2
// otherwise), RPW vector-memory instructions.  A missing page reads page 0
// (in bounds); its tokens are masked and its V rows zeroed before use.
template <int RPW>
__device__ __forceinline__ void pf_issue(const PrefillArgs& a, const PfLanes& pl, uint32_t page_bytes,
                                         uint32_t kvh_off, lds_u8* slot, uint32_t ph0, uint32_t ph1, int w) {
#pragma unroll
  for (int t = 0; t < RPW; ++t) {
    const int r = (w >> 2) * RPW + t;  // wave-uniform
    // region within the half, and the half (one half: r < 4, eight waves)
    const int rr = RPW == 2 ? r : r & 3, hf = RPW == 2 ? 0 : r >> 2;
    const uint32_t ph = (rr & 1) ? ph1 : ph0;
    const size_t base = (size_t)(ph < a.num_pages ? ph : 0u) * page_bytes + kvh_off + (size_t)hf * kRowBytes;
    const uint8_t* src = (rr >> 1) ? a.v_pages : a.k_pages;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void*)(src + base), (short)0, (int)page_bytes, kBufferFormat);
    // the offset as a value select (a select of the two fields' addresses
    // would keep pl in memory)
    const uint32_t off = pl.koff + ((rr >> 1) ? pl.voff - pl.koff : 0u);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(slot + r * kVSlot + pl.lds_q),
                                             16, (int)off, 0, 0, 0);
  }
}

// Q8A pages.  A pair's int8 codes (per 128-wide half of the head, four
// 2 KiB regions: K of page 0, K of page 1, V of page 0, V of page 1, 16 rows
// of 128 codes each) come by DMA in 1 KiB pieces: piece i = NH w + t (t <
// NH) of wave w is half i & 1 (rows 8 (i & 1) ..) of region i >> 1 (region r:
// half r / 4, region r % 4), so lane l fetches row 8 (i & 1) + l / 8, codes
// 16 (l % 8) .. + 15 of that region -- the same 16 bytes it converts to f16
// afterwards; each wave also DMAs its own copy of the pair's 32 K and 32 V
// scales (lane l: page (l / 16) & 1, token l % 16).  NH + 2 vector-memory
// instructions per wave and pair.
template <int NH>
constexpr int kPfCodeSlot = NH * 4 * 2048;                           // the codes of a pair
constexpr int kPfScaleWave = 512;                                    // K scales [0, 256), V scales [256, 512)
template <int NH>
constexpr int kPfQ8Slot = kPfCodeSlot<NH> + 8 * kPfScaleWave;        // codes, then eight waves' scale copies

template <int NH>
__device__ __forceinline__ void pf_issue_q8(const PrefillArgs& a, uint32_t rs, uint32_t kvh, lds_u8* slot,
                                            uint32_t ph0, uint32_t ph1, int w) {
  typedef __attribute__((address_space(3))) void lds_void;
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const uint32_t page_bytes = kPage * rs;
#pragma unroll
  for (int t = 0; t < NH; ++t) {
    // wave-uniform; with one half, r < 4 (eight waves)
    const int i = NH * w + t, r = i >> 1, rr = NH == 1 ? r : r & 3, hf = NH == 1 ? 0 : r >> 2;
    const uint32_t ph = (rr & 1) ? ph1 : ph0;
    const size_t base = (size_t)(ph < a.num_pages ? ph : 0u) * page_bytes + (size_t)kvh * (NH * kD) +
                        (size_t)hf * kD;
    const uint8_t* src = (rr >> 1) ? a.v_pages : a.k_pages;
    const __amdgpu_buffer_rsrc_t rsc =
        __builtin_amdgcn_make_buffer_rsrc((void*)(src + base), (short)0, (int)page_bytes, kBufferFormat);
    const uint32_t row = 8u * (uint32_t)(i & 1) + (uint32_t)(lane >> 3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsc, (lds_void*)(slot + r * 2048 + (i & 1) * 1024), 16,
                                             (int)(row * rs + 16u * (uint32_t)(lane & 7)), 0, 0, 0);
  }
  // scales: token lane % 16 of page (lane / 16) & 1 (a missing page: page 0)
  const uint32_t sp = ((lane >> 4) & 1) ? ph1 : ph0;
  const uint32_t sidx = ((sp < a.num_pages ? sp : 0u) * kPage + (uint32_t)(lane & 15)) * (uint32_t)a.n_kv + kvh;
  const int sbytes = (int)min((size_t)a.num_pages * kPage * (size_t)a.n_kv * 4, (size_t)0x7FFFFFF0);
  const __amdgpu_buffer_rsrc_t ksr = __builtin_amdgcn_make_buffer_rsrc((void*)a.k_scales, (short)0, sbytes, kBufferFormat);
  const __amdgpu_buffer_rsrc_t vsr = __builtin_amdgcn_make_buffer_rsrc((void*)a.v_scales, (short)0, sbytes, kBufferFormat);
  lds_u8* sc = slot + kPfCodeSlot<NH> + w * kPfScaleWave;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(ksr, (lds_void*)sc, 4, (int)(4u * sidx), 0, 0, 0);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(vsr, (lds_void*)(sc + 256), 4, (int)(4u * sidx), 0, 0, 0);
}

// This wave's codes of the pair (the NH pieces it DMA'd) to f16 in the f16
// pair slot `dst` (the layout pf_consume reads, per half): K token t's chunk
// c at c ^ t of row t, V token t in row R = 4 (t % 4) + t / 4 with chunk c at
// c ^ sw(R).  The codes are exact in f16.
template <int NH>
__device__ __forceinline__ void pf_convert_q8(const lds_u8* codes, lds_u8* dst, int w) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const uint32_t d = (uint32_t)(size_t)dst;
#pragma unroll
  for (int tt = 0; tt < NH; ++tt) {
    const int i = NH * w + tt, r = i >> 1, rr = NH == 1 ? r : r & 3, hf = NH == 1 ? 0 : r >> 2;
    const int t = 8 * (i & 1) + (lane >> 3), c16 = lane & 7;
    u32x4 x;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                 : "=v"(x)
                 : "v"((uint32_t)(size_t)(codes + r * 2048 + (i & 1) * 1024 + 16 * lane))
                 : "memory");
    const half8 lo = i8x8_to_f16(uint2v{x[0], x[1]}), hi = i8x8_to_f16(uint2v{x[2], x[3]});
    const int p = rr & 1;
    const uint32_t hb = (uint32_t)hf * (uint32_t)kPfSlot<1>;  // this half's 16 KiB
    uint32_t o0, o1;
    if (rr < 2) {  // K
      o0 = hb + (uint32_t)(p * kVSlot + t * kRowBytes) + 16u * ((uint32_t)(2 * c16) ^ (uint32_t)t);
      o1 = hb + (uint32_t)(p * kVSlot + t * kRowBytes) + 16u * ((uint32_t)(2 * c16 + 1) ^ (uint32_t)t);
    } else {  // V
      const int R = 4 * (t & 3) + (t >> 2);
      o0 = hb + (uint32_t)((2 + p) * kVSlot + R * kRowBytes) + 16u * ((uint32_t)(2 * c16) ^ v_swz(R));
      o1 = hb + (uint32_t)((2 + p) * kVSlot + R * kRowBytes) + 16u * ((uint32_t)(2 * c16 + 1) ^ v_swz(R));
    }
    // inline asm stores: the compiler would otherwise wait for every DMA in
    // flight before a plain LDS store (it cannot tell which slot a DMA writes)
    asm volatile("ds_write_b128 %0, %1" : : "v"(d + o0), "v"(lo) : "memory");
    asm volatile("ds_write_b128 %0, %1" : : "v"(d + o1), "v"(hi) : "memory");
  }
}

// MODE 0: every token of the pair is attended by every query of the wave;
// 1: per-query masks only (causal, and the query's own sliding window
// [qlo, qpos]); 2: some tokens are outside the tile's window or on a missing
// page: mask them and zero their V rows (stale LDS or page bytes may hold NaN
// patterns, and 0 * NaN would reach the accumulators).
// Q8 (Q8A pages): `slot` holds the pair's codes as f16 and `scales` this
// wave's copy of their K and V scales.  The K scale of each token multiplies
// its scores; the V scale multiplies its weights before P.V, over vnorm, a
// power of two at or just above the largest V scale seen (kept within 16x of
// each pair's largest; acc is rescaled exactly when it moves), so that the
// f16 lo parts of the weights stay normal numbers; l sums the unscaled
// weights and the output is acc * vnorm / l.
// NH = 2 (256-wide heads): the slot holds the two halves' pairs one after the
// other (16 KiB apart); q operand 4 hf + j and accumulator 8 hf + nb belong
// to half hf.  Both halves' K operands are read first (the scores sum over
// them), then both halves' V operands, which stay in flight during the
// softmax.
template <int HW, int MODE, bool Q8 = false, int NH = 1>
__device__ __forceinline__ void pf_consume(float4v (&acc)[HW][8 * NH], float (&m)[HW], float (&l)[HW],
                                           const half8 (&qh)[HW][4 * NH], const half8 (&ql)[HW][4 * NH],
                                           const float (&qexp)[HW], const PfLanes& pl, lds_u8* slot, int tok0,
                                           bool v0, bool v1, int ta, int tb, int qpos, int qlo, bool qok, int g,
                                           int n, const lds_u8* scales = nullptr, float* vnorm = nullptr) {
  static_assert(NH == 1 || HW == 1, "256-wide heads: one query head per wave");
  if constexpr (MODE == 2 && !Q8) {
#pragma unroll
    for (int hf = 0; hf < NH; ++hf)
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = tok0 + 16 * p + 4 * g + j;
          if (!((p ? v1 : v0) && t >= ta && t < tb))
            *(lds_u32x4*)(slot + hf * kPfSlot<1> + (2 + p) * kVSlot + (4 * j + g) * kRowBytes + 16 * n) =
                u32x4{0u, 0u, 0u, 0u};
        }
  }
  float4v sacc[HW][2];
  short4v bv[2][8];
  if constexpr (NH == 1) {
    // K operands of both pages, then the V operands of both pages; the reads
    // are inline asm because the compiler cannot tell which slot a DMA writes
    // and would wait for every DMA in flight before a plain LDS read.  This
    // slot's DMAs have completed (vmcnt wait and barrier before the call).
    // the XOR bases pass through an empty asm so that the compiler rebuilds
    // the offsets here instead of hoisting all twelve out of the pair loop
    uint32_t kx = pl.kx, vx = pl.vx;
    asm volatile("" : "+v"(kx), "+v"(vx));
    const uint32_t kb = (uint32_t)(size_t)slot + pl.krow;
    half8 k[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t ka = kb + ((64u * (uint32_t)j) ^ kx);
      asm volatile("ds_read_b128 %0, %1" : "=v"(k[0][j]) : "v"(ka) : "memory");
      asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(k[1][j]) : "v"(ka) : "memory");
    }
    const uint32_t vb = (uint32_t)(size_t)slot + 2 * kVSlot + pl.vrow;
    auto read_v = [&](int nb) {
      const uint32_t a0 = vb + ((32u * (uint32_t)nb) ^ vx);
      asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(bv[0][nb]) : "v"(a0) : "memory");
      asm volatile("ds_read_b64_tr_b16 %0, %1 offset:4096" : "=v"(bv[1][nb]) : "v"(a0) : "memory");
    };
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) read_v(nb);
    // LDS reads complete in order: the 8 V reads just issued may be outstanding
    asm volatile("s_waitcnt lgkmcnt(8)"
                 : "+v"(k[0][0]), "+v"(k[0][1]), "+v"(k[0][2]), "+v"(k[0][3]), "+v"(k[1][0]), "+v"(k[1][1]),
                   "+v"(k[1][2]), "+v"(k[1][3])
                 :
                 : "memory");
#pragma unroll
    for (int nb = 4; nb < 8; ++nb) read_v(nb);
#pragma unroll
    for (int hh = 0; hh < HW; ++hh)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        float4v s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[p][j], qh[hh][j], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[p][j], ql[hh][j], s, 0, 0, 0);
        }
        sacc[hh][p] = s;
      }
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(bv[0][0]), "+v"(bv[0][1]), "+v"(bv[0][2]), "+v"(bv[0][3]), "+v"(bv[0][4]), "+v"(bv[0][5]),
                   "+v"(bv[0][6]), "+v"(bv[0][7]), "+v"(bv[1][0]), "+v"(bv[1][1]), "+v"(bv[1][2]), "+v"(bv[1][3]),
                   "+v"(bv[1][4]), "+v"(bv[1][5]), "+v"(bv[1][6]), "+v"(bv[1][7])
                 :
                 : "memory");
  } else {
    // one half's K operands at a time (the second half's at +16 KiB), each
    // waited for before its products: the other wave on the SIMD covers the
    // read latency, and 32 operand registers fewer stay live than with both
    // halves in flight (the accumulators and q of a 256-wide head take 128)
    uint32_t kx = pl.kx;
    asm volatile("" : "+v"(kx));
    const uint32_t kb = (uint32_t)(size_t)slot + pl.krow;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      half8 k[2][4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t ka = kb + ((64u * (uint32_t)j) ^ kx);
        if (hf == 0) {
          asm volatile("ds_read_b128 %0, %1" : "=v"(k[0][j]) : "v"(ka) : "memory");
          asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(k[1][j]) : "v"(ka) : "memory");
        } else {
          asm volatile("ds_read_b128 %0, %1 offset:16384" : "=v"(k[0][j]) : "v"(ka) : "memory");
          asm volatile("ds_read_b128 %0, %1 offset:20480" : "=v"(k[1][j]) : "v"(ka) : "memory");
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(k[0][0]), "+v"(k[0][1]), "+v"(k[0][2]), "+v"(k[0][3]), "+v"(k[1][0]), "+v"(k[1][1]),
                     "+v"(k[1][2]), "+v"(k[1][3])
                   :
                   : "memory");
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        float4v sv = hf ? sacc[0][p] : float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[p][j], qh[0][4 * hf + j], sv, 0, 0, 0);
          sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[p][j], ql[0][4 * hf + j], sv, 0, 0, 0);
        }
        sacc[0][p] = sv;
      }
      __builtin_amdgcn_sched_barrier(0);  // the next half's reads follow these products
    }
  }
  // Q8: the scales of the lane's tokens 16 p + 4g + ii (e = 4p + ii)
  float ks[8], vsc[8], vinv = 1.0f;
  if constexpr (Q8) {
    float4v k0, k1, w0, w1;
    const uint32_t sa = (uint32_t)(size_t)scales + 16u * (uint32_t)g;
    asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:64\n\t"
                 "ds_read_b128 %2, %4 offset:256\n\tds_read_b128 %3, %4 offset:320\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(k0), "=&v"(k1), "=&v"(w0), "=&v"(w1)  // early clobber: the address stays live
                 : "v"(sa)
                 : "memory");
    float vmax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ks[e] = e < 4 ? k0[e] : k1[e - 4];
      vsc[e] = e < 4 ? w0[e] : w1[e - 4];
      const int t = tok0 + 16 * (e >> 2) + 4 * g + (e & 3);
      if (MODE == 2 && !(((e >> 2) ? v1 : v0) && t >= ta && t < tb)) vsc[e] = 0.0f;  // stale bytes
      vmax = fmaxf(vmax, vsc[e]);
    }
    vmax = max_xor16(max_xor32(vmax));  // over the pair's 32 tokens; wave-uniform
    if ((vmax > *vnorm || vmax * 16.0f < *vnorm) && vmax > 0.0f) {
      int ex = 0;
      (void)frexpf(vmax, &ex);
      if (*vnorm > 0.0f) {
        const float rr = *vnorm * ldexpf(1.0f, -ex);  // a power of two: exact
#pragma unroll
        for (int hh = 0; hh < HW; ++hh)
#pragma unroll
          for (int nb = 0; nb < 8 * NH; ++nb) acc[hh][nb] *= rr;
      }
      *vnorm = ldexpf(1.0f, ex);
    }
    vinv = *vnorm > 0.0f ? 1.0f / *vnorm : 0.0f;
  }
  // NH = 2: V operands of half hf into bv[.][0 .. 7] (the first half's stay
  // in flight during the softmax; the second half's are read after the
  // first half's products, into the same registers)
  auto read_v_half = [&](int hf) {
    uint32_t vx = pl.vx;
    asm volatile("" : "+v"(vx));
    const uint32_t vb = (uint32_t)(size_t)slot + 2 * kVSlot + pl.vrow;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const uint32_t a0 = vb + ((32u * (uint32_t)nb) ^ vx);
      if (hf == 0) {
        asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(bv[0][nb]) : "v"(a0) : "memory");
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:4096" : "=v"(bv[1][nb]) : "v"(a0) : "memory");
      } else {
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:16384" : "=v"(bv[0][nb]) : "v"(a0) : "memory");
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:20480" : "=v"(bv[1][nb]) : "v"(a0) : "memory");
      }
    }
  };
  auto wait_v = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(bv[0][0]), "+v"(bv[0][1]), "+v"(bv[0][2]), "+v"(bv[0][3]), "+v"(bv[0][4]), "+v"(bv[0][5]),
                   "+v"(bv[0][6]), "+v"(bv[0][7]), "+v"(bv[1][0]), "+v"(bv[1][1]), "+v"(bv[1][2]), "+v"(bv[1][3]),
                   "+v"(bv[1][4]), "+v"(bv[1][5]), "+v"(bv[1][6]), "+v"(bv[1][7])
                 :
                 : "memory");
  };
  if constexpr (NH == 2) read_v_half(0);
#pragma unroll
  for (int hh = 0; hh < HW; ++hh) {
    // raw scores (still scaled by 2^-E); masked tokens -inf
    float s[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = Q8 ? sacc[hh][e >> 2][e & 3] * ks[e] : sacc[hh][e >> 2][e & 3];
    if constexpr (MODE != 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = tok0 + 16 * (e >> 2) + 4 * g + (e & 3);
        if (!(qok && ((e >> 2) ? v1 : v0) && t >= qlo && t < tb && t <= qpos)) s[e] = -INFINITY;
      }
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
    mx = max_xor16(max_xor32(mx)) * qexp[hh];  // over the 32 tokens of query n; 2^E scaling is exact
    const bool need = mx > m[hh] + kRescaleSlack;
    if (__builtin_amdgcn_ballot_w64(need)) {  // wave-uniform
      const float m_new = need ? mx : m[hh];
      const float alpha = fast_exp2(m[hh] - m_new);
      m[hh] = m_new;
      l[hh] *= alpha;
      // result row 4g+ii is query 4g+ii, whose alpha sits in lane 16g + 4g + ii
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        const float aq = __shfl(alpha, 20 * g + ii, kWave);
#pragma unroll
        for (int nb = 0; nb < 8 * NH; ++nb) acc[hh][nb][ii] *= aq;
      }
    }
    // p = 2^(s 2^E - m) (the product is exact, so one rounding as s - m);
    // hi = f16(p) to nearest even, lo = f16(p - hi), converted in pairs
    const float nm = -m[hh];
    half8 ph, plo;
    float lsum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      float2v pp = {fast_exp2(fmaf(s[e], qexp[hh], nm)), fast_exp2(fmaf(s[e + 1], qexp[hh], nm))};
      lsum += pp[0] + pp[1];
      if constexpr (Q8) pp = float2v{pp[0] * (vsc[e] * vinv), pp[1] * (vsc[e + 1] * vinv)};
      const half2v h = __builtin_convertvector(pp, half2v);
      const float2v hf = __builtin_convertvector(h, float2v);
      const half2v lo = __builtin_convertvector(float2v{pp[0] - hf[0], pp[1] - hf[1]}, half2v);
      ph[e] = h[0];
      ph[e + 1] = h[1];
      plo[e] = lo[0];
      plo[e + 1] = lo[1];
    }
    l[hh] += lsum;
#pragma unroll
    for (int hf = 0; hf < NH; ++hf) {
      if constexpr (NH == 2) {  // one query head per wave (hh == 0)
        if (hf == 1) {
          __builtin_amdgcn_sched_barrier(0);  // after the first half's products
          read_v_half(1);
        }
        wait_v();
      }
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const half8 b = __builtin_bit_cast(half8, __builtin_shufflevector(bv[0][nb], bv[1][nb], 0, 1, 2, 3, 4, 5, 6, 7));
        acc[hh][8 * hf + nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, b, acc[hh][8 * hf + nb], 0, 0, 0);
        acc[hh][8 * hf + nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(plo, b, acc[hh][8 * hf + nb], 0, 0, 0);
      }
    }
  }
}

// Chunk i's tile count, 0 for a chunk outside the inputs (skipped).
template <int QT>
__device__ __forceinline__ int pf_tiles(const PrefillArgs& a, int i) {
  if (i >= a.n_chunks) return 0;
  const int4 ch = a.chunks[i];
  const bool ok = ch.x >= 0 && ch.x < a.n_rows && ch.y >= 0 && ch.z > 0 && ch.w >= 0 && ch.z <= a.n_tok - ch.w;
  return ok ? (ch.z + QT - 1) / QT : 0;
}

// Q8: Q8A pages (int8 codes and scales, pf_issue_q8): every wave converts the
// codes it fetched into a double-buffered f16 pair slot before the batch's
// barrier, so a batch still costs one barrier.
// NH: 128-wide halves of the head (1 or 2).
template <int REP, bool Q8 = false, int NH = 1>
__global__ __launch_bounds__((kWave * PfShape<REP, NH>::NW)) void prefill_mfma_kernel(PrefillArgs a) {
  using Sh = PfShape<REP, NH>;
  constexpr int HW = Sh::HW, WPQ = Sh::WPQ, QT = Sh::QT;
  constexpr int kPfBatch = Sh::kBatch, kPfDepth = Sh::kDepth, kSlot = kPfSlot<NH>;
  constexpr int RPW = Q8 ? NH + 2 : Sh::RPW;  // vector-memory instructions per wave and pair
  constexpr int kRingSlot = Q8 ? kPfQ8Slot<NH> : kSlot;
  __shared__ __attribute__((aligned(16))) uint8_t ring_[kPfDepth * kRingSlot];
  __shared__ __attribute__((aligned(16))) uint8_t f16buf_[Q8 ? 2 * kPfBatch * kSlot : 16];
  const int lane = (int)(threadIdx.x & (kWave - 1)), w = (int)(threadIdx.x / kWave);
  const int g = lane >> 4, n = lane & 15;

  // block -> (chunk, tile, kv head); the kv head varies fastest.  Up to 64
  // chunks are taken longest first (by the position after their last token,
  // ties by index), so that the last workgroups a CU receives are short ones;
  // more chunks are taken in index order.
  const int kvh = (int)(blockIdx.x % (unsigned)a.n_kv);
  int slot = (int)(blockIdx.x / (unsigned)a.n_kv), c = -1, tile = 0, nt_c = 0;
  if (a.n_chunks <= kWave) {
    const int nt = pf_tiles<QT>(a, lane);
    const int4 chl = a.chunks[lane < a.n_chunks ? lane : 0];
    const int key = nt > 0 ? (int)min((int64_t)chl.y + chl.z, (int64_t)INT32_MAX) : -1;
    int before = 0;  // tiles of the chunks taken before this one
    for (int j = 0; j < a.n_chunks; ++j) {
      const int kj = __builtin_amdgcn_readlane(key, j);
      const int ntj = __builtin_amdgcn_readlane(nt, j);
      if (kj > key || (kj == key && j < lane)) before += ntj;
    }
    const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < a.n_chunks && nt > 0 && before <= slot &&
                                                     slot < before + nt);
    if (hit) {
      const int idx = (int)__builtin_ctzll(hit);
      c = idx;
      nt_c = __builtin_amdgcn_readlane(nt, idx);
      tile = slot - __builtin_amdgcn_readlane(before, idx);
    }
  } else for (int c0 = 0; c0 < a.n_chunks; c0 += kWave) {  // wave-uniform; identical in every wave
    const int nt = pf_tiles<QT>(a, c0 + lane);
    const int incl = wave_incl_scan(nt);
    const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
    if (slot < total) {
      const int idx = (int)__builtin_popcountll(__builtin_amdgcn_ballot_w64(incl <= slot));
      c = c0 + idx;
      nt_c = __builtin_amdgcn_readlane(nt, idx);
      tile = slot - (__builtin_amdgcn_readlane(incl, idx) - nt_c);
      break;
    }
    slot -= total;
  }
  if (c < 0) return;  // beyond the last tile: the whole block leaves
  tile = nt_c - 1 - tile;  // a chunk's later (longer) tiles first
  const int4 ch = a.chunks[c];
  const int s = ch.x;
  const int pos0 = ch.y + QT * tile;
  const int qn = min(QT, ch.z - QT * tile);  // queries in this tile
  const int p_last = pos0 + qn - 1;
  int p0 = a.p_start ? a.p_start[s] : 0;
  // a start past the tile's last query leaves every query nothing to attend:
  // no pages are read and the rows are written as zeros
  p0 = min(max(p0, 0), p_last + 1);
  // a sliding window gives query P the start max(p0, P - window + 1); the
  // tile reads from its first query's start
  const int ta = a.window > 0 ? max(p0, pos0 - a.window + 1) : p0;
  const int tb = min(p_last + 1, a.bt_stride * kPage);

  // this wave: queries [wq, wq + qn_w) of the tile, heads h0 .. h0 + HW - 1
  const int qg = w / WPQ;
  const int qn_w = min(16, qn - 16 * qg);
  const bool active = qn_w > 0;
  const int wq = pos0 + 16 * qg;
  const int tq = ch.w + QT * tile + 16 * qg;  // q/out row of query wq
  const int h0 = kvh * REP + (w % WPQ) * HW;
  const bool qok = n < qn_w;
  const int qpos = wq + n;
  const int qlo = a.window > 0 ? max(ta, qpos - a.window + 1) : ta;  // this lane's query's window start
  // the largest window start among the wave's queries: pairs from there on
  // need no window mask
  const int wlo = a.window > 0 ? max(ta, wq + max(qn_w, 1) - a.window) : ta;

  // table window of 64 entries (lane j: entry base + j)
  const uint32_t* bt_row = a.bt + (size_t)s * a.bt_stride;
  const int pg_first = ta / kPage;
  const int npg = ta < tb ? (tb - 1) / kPage - pg_first + 1 : 0;
  const int npairs = (npg + 1) / 2;
  int base = pg_first;
  uint32_t btv = 0;
  auto load_window = [&]() {
    const int e = base + lane;
    btv = e < a.bt_stride ? bt_row[e] : 0u;
    wait_vmcnt<0>();
  };
  load_window();
  auto phys_of = [&](int i) -> uint32_t {  // i increases from call to call
    int idx = pg_first + i - base;
    if (idx >= 64) {
      base += 64;
      idx -= 64;
      load_window();
    }
    return __builtin_amdgcn_readlane(btv, idx);
  };

  // q of query n, head h0 + hh: dims 128 hf + 32j + 8g .. +7 in qraw[hh][8 hf
  // + 2j ..], loaded before the pages
  float4v qraw[HW][8 * NH];
  {
    const int trow = qok ? tq + n : ch.w;
#pragma unroll
    for (int hh = 0; hh < HW; ++hh) {
      const float4v* qsrc =
          reinterpret_cast<const float4v*>(a.q + ((size_t)trow * a.n_heads + h0 + hh) * (NH * kD) + 8 * g);
#pragma unroll
      for (int j = 0; j < 4 * NH; ++j) {
        qraw[hh][2 * j] = qsrc[8 * j];
        qraw[hh][2 * j + 1] = qsrc[8 * j + 1];
      }
    }
  }

  PfLanes pl;
  const uint32_t rs = (uint32_t)a.n_kv * (NH * kRowBytes);
  const uint32_t page_bytes = kPage * rs;
  const uint32_t kvh_off = (uint32_t)kvh * (NH * kRowBytes);
  {
    const int j = w & 3;  // this wave's quarter of a page region
    const uint32_t R = 4u * (uint32_t)j + (uint32_t)g;
    pl.koff = R * rs + 16u * ((uint32_t)n ^ R);
    pl.voff = (uint32_t)(4 * g + j) * rs + 16u * ((uint32_t)n ^ v_swz((int)R));
    pl.lds_q = 1024u * (uint32_t)j;
    pl.krow = (uint32_t)n * kRowBytes + 16u * ((uint32_t)g ^ ((uint32_t)n & 3u));
    pl.kx = 64u * ((uint32_t)n >> 2);
    const int Rv = 4 * (n >> 2) + g;
    pl.vrow = (uint32_t)Rv * kRowBytes + 8u * (n & 1) + 16u * (uint32_t)((n & 3) >> 1);
    pl.vx = 16u * v_swz(Rv);
  }
  lds_u8* ring = (lds_u8*)ring_;

  // pair i -> ring slot i % kPfDepth; validity bits of the slot's two pages
  uint32_t vbits = 0;
  auto issue = [&](int i) {
    const int sl = i % kPfDepth;
    const uint32_t ph0 = phys_of(2 * i);
    const uint32_t ph1 = 2 * i + 1 < npg ? phys_of(2 * i + 1) : 0xFFFFFFFFu;
    const uint32_t bits = (ph0 < a.num_pages ? 1u : 0u) | (ph1 < a.num_pages ? 2u : 0u);
    vbits = (vbits & ~(3u << (2 * sl))) | (bits << (2 * sl));
    if constexpr (Q8)
      pf_issue_q8<NH>(a, (uint32_t)a.n_kv * (NH * kD), (uint32_t)kvh, ring + sl * kRingSlot, ph0, ph1, w);
    else
      pf_issue<Sh::RPW>(a, pl, page_bytes, kvh_off, ring + sl * kSlot, ph0, ph1, w);
  };
#pragma unroll
  for (int i = 0; i < 2 * kPfBatch; ++i)
    if (i < npairs) issue(i);

  // q -> B operands: per query and head, scale by 2^-E (E from max |q *
  // scale|) so that hi and lo stay in f16 range; scores are scaled back by 2^E
  half8 qh[HW][4 * NH], ql[HW][4 * NH];
  float qexp[HW];
#pragma unroll
  for (int hh = 0; hh < HW; ++hh) {
    float amax = 0.0f;
#pragma unroll
    for (int r = 0; r < 8 * NH; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(qraw[hh][r][e] * a.scale_log2));
    amax = max_xor16(max_xor32(amax));  // over the 4 lanes of query n
    int E = 0;
    if (amax > 0.0f && amax < INFINITY) (void)frexpf(amax, &E);
    const float inv = ldexpf(1.0f, -E);
    qexp[hh] = ldexpf(1.0f, E);
#pragma unroll
    for (int j = 0; j < 4 * NH; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = qok ? qraw[hh][2 * j + (e >> 2)][e & 3] * a.scale_log2 * inv : 0.0f;
        const _Float16 hi = (_Float16)y;
        qh[hh][j][e] = hi;
        ql[hh][j][e] = (_Float16)(y - (float)hi);
      }
  }
  float4v acc[HW][8 * NH];
  float m[HW], l[HW];
  float vnorm = 0.0f;  // Q8: acc is in units of vnorm
#pragma unroll
  for (int hh = 0; hh < HW; ++hh) {
    m[hh] = kMInit;
    l[hh] = 0.0f;
#pragma unroll
    for (int nb = 0; nb < 8 * NH; ++nb) acc[hh][nb] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // kPfBatch pairs per barrier: pairs [i0, i0 + B) are consumed while the
  // next B are in flight and the B after those are issued into the slots of
  // [i0 - B, i0) (every wave consumed those before this barrier).
  for (int i0 = 0; i0 < npairs; i0 += kPfBatch) {
    // the pairs issued after this batch, which may stay in flight
    const int later = min(max(npairs - (i0 + kPfBatch), 0), kPfBatch);
    if constexpr (kPfBatch >= 3) {
      if (later == 3) wait_vmcnt<3 * RPW>();
    }
    if (later == 2)
      wait_vmcnt<2 * RPW>();
    else if (later == 1)
      wait_vmcnt<RPW>();
    else if (later == 0)
      wait_vmcnt<0>();
    // Q8: this wave's codes of the batch (its own DMAs, just waited for) to
    // f16 in the batch's buffer; the buffer was last read by the batch before
    // the previous one, which every wave finished before the last barrier
    lds_u8* f16b = (lds_u8*)f16buf_ + ((i0 / kPfBatch) & 1) * (kPfBatch * kSlot);
    if constexpr (Q8) {
#pragma unroll
      for (int k = 0; k < kPfBatch; ++k)
        if (i0 + k < npairs) pf_convert_q8<NH>(ring + ((i0 + k) % kPfDepth) * kRingSlot, f16b + k * kSlot, w);
    }
    pf_barrier();  // every wave's quarters of this batch landed; the previous batch is consumed
#pragma unroll
    for (int k = 0; k < kPfBatch; ++k)
      if (i0 + 2 * kPfBatch + k < npairs) issue(i0 + 2 * kPfBatch + k);
    for (int i = i0; i < min(i0 + kPfBatch, npairs); ++i) {
    if (active) {
      const int sl = i % kPfDepth;
      lds_u8* sp = Q8 ? f16b + (i - i0) * kSlot : ring + sl * kSlot;
      const lds_u8* sc = ring + sl * kRingSlot + kPfCodeSlot<NH> + w * kPfScaleWave;  // Q8: this wave's scales
      const bool v0 = (vbits >> (2 * sl)) & 1u, v1 = (vbits >> (2 * sl + 1)) & 1u;
      const int tok0 = (pg_first + 2 * i) * kPage;
      const bool whole = v0 && v1 && tok0 >= ta && tok0 + 2 * kPage <= tb;
      // 256-wide heads: no mask-free copy (its register allocation spilled)
      if (NH == 1 && whole && tok0 + 2 * kPage - 1 <= wq && tok0 >= wlo)
        pf_consume<HW, 0, Q8, NH>(acc, m, l, qh, ql, qexp, pl, sp, tok0, v0, v1, ta, tb, qpos, qlo, qok, g, n, sc, &vnorm);
      else if (whole)
        pf_consume<HW, 1, Q8, NH>(acc, m, l, qh, ql, qexp, pl, sp, tok0, v0, v1, ta, tb, qpos, qlo, qok, g, n, sc, &vnorm);
      else
        pf_consume<HW, 2, Q8, NH>(acc, m, l, qh, ql, qexp, pl, sp, tok0, v0, v1, ta, tb, qpos, qlo, qok, g, n, sc, &vnorm);
    }
    }
  }
  if (!active) return;

#pragma unroll
  for (int hh = 0; hh < HW; ++hh) {
    // l over the 32 tokens of each pair: sum the four lanes of query n
    const float lt = sum_xor16(sum_xor32(l[hh]));
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const float L = __shfl(lt, 20 * g + ii, kWave);  // query 4g + ii
      const int qq = 4 * g + ii;
      if (qq < qn_w) {
        const float inv = L > 0.0f ? (Q8 ? vnorm : 1.0f) / L : 0.0f;
        float* orow = a.out + ((size_t)(tq + qq) * a.n_heads + h0 + hh) * (NH * kD);
#pragma unroll
        for (int nb = 0; nb < 8 * NH; ++nb) orow[16 * nb + n] = acc[hh][nb][ii] * inv;
      }
    }
  }
}

template <int REP, int NH>
void launch_prefill_rep(const PrefillArgs& a, int n_tiles, hipStream_t st) {
  const unsigned blocks = (unsigned)n_tiles * (unsigned)a.n_kv;
  if (a.k_scales)
    prefill_mfma_kernel<REP, true, NH><<<blocks, kWave * PfShape<REP, NH>::NW, 0, st>>>(a);
  else
    prefill_mfma_kernel<REP, false, NH><<<blocks, kWave * PfShape<REP, NH>::NW, 0, st>>>(a);
}

template <int NH>
int prefill_qt(int rep) {
  switch (rep) {
    case 1: return PfShape<1, NH>::QT;
    case 2: return PfShape<2, NH>::QT;
    case 4: return PfShape<4, NH>::QT;
    default: return PfShape<8, NH>::QT;
  }
}

template <int NH>
void launch_prefill_nh(const PrefillArgs& a, int rep, int n_tiles, hipStream_t st) {
  switch (rep) {
    case 1: launch_prefill_rep<1, NH>(a, n_tiles, st); break;
    case 2: launch_prefill_rep<2, NH>(a, n_tiles, st); break;
    case 4: launch_prefill_rep<4, NH>(a, n_tiles, st); break;
    default: launch_prefill_rep<8, NH>(a, n_tiles, st); break;
  }
}
}  // namespace

int prefill_queries_per_tile(int rep, int head_dim) {
  return head_dim == 256 ? prefill_qt<2>(rep) : prefill_qt<1>(rep);
}

int launch_prefill_mfma(const PrefillArgs& a, int rep, int head_dim, int n_tiles, hipStream_t st) {
  switch (rep) {
    case 1:
    case 2:
    case 4:
    case 8:
      if (head_dim == 256)
        launch_prefill_nh<2>(a, rep, n_tiles, st);
      else
        launch_prefill_nh<1>(a, rep, n_tiles, st);
      break;
    default: return fail(LNSKV_ERR_UNSUPPORTED, "n_heads/n_kv_heads = %d not supported (1, 2, 4, 8)", rep);
  }
  return hip_check("prefill kernel launch");
}

}  // namespace lnskv
