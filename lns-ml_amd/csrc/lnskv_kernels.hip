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
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <vector>

#include "lnskv_device.h"

namespace lnskv {

int hip_check(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LNSKV_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return LNSKV_OK;
}

namespace {
std::mutex g_err_mutex;
std::atomic<uint32_t*> g_ws_err{nullptr};  // pinned, coherent host word; never freed
}  // namespace

uint32_t* ws_error_word(void* stream, bool allocate) {
  uint32_t* w = g_ws_err.load(std::memory_order_acquire);
  if (w || !allocate) return w;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing((hipStream_t)stream, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (cs != hipStreamCaptureStatusNone) return nullptr;
  std::lock_guard<std::mutex> lock(g_err_mutex);
  w = g_ws_err.load(std::memory_order_acquire);
  if (!w) {
    void* p = nullptr;
    if (hipHostMalloc(&p, sizeof(uint32_t), hipHostMallocCoherent) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    w = static_cast<uint32_t*>(p);
    __atomic_store_n(w, 0u, __ATOMIC_RELAXED);
    g_ws_err.store(w, std::memory_order_release);
  }
  return w;
}

int take_ws_error() {
  uint32_t* w = g_ws_err.load(std::memory_order_acquire);
  return w ? (int)__atomic_exchange_n(w, 0u, __ATOMIC_ACQ_REL) : 0;
}

namespace {

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
  int32_t n_rows;
  int32_t n_tok;
  int32_t n_kv;
  uint32_t num_pages;
  const float* rope_inv;  // append_vec_kernel: K turns by tok_pos with these inverse frequencies
  int32_t rope_half;      // rotary_dim / 2 (a multiple of 8, half/8 a power of two); 0: none
  int32_t head_dim;
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
  if (seq < 0 || seq >= a.n_rows || pos < 0 || pos / kPage >= a.bt_stride) return;
  const uint32_t phys = a.bt[(size_t)seq * a.bt_stride + pos / kPage];
  if (phys >= a.num_pages) return;  // LNSKV_NO_PAGE or outside the pool
  const size_t slot = (size_t)phys * kPage + (size_t)(pos % kPage);
  const size_t row = (slot * a.n_kv + h) * D;
  const size_t src = ((size_t)t * a.n_kv + h) * D;
  store_head_row<DT, D>(a.k_pages, a.k_scales, row, slot * a.n_kv + h, a.k_new + src, lane);
  store_head_row<DT, D>(a.v_pages, a.v_scales, row, slot * a.n_kv + h, a.v_new + src, lane);
}

// Append for f32 and f16 pages: a token's K (and V) values for all its kv
// heads, n_kv*D of them, are contiguous both in k_new/v_new and in the page
// slot, so thread i of a token converts elements [8i, 8i+8) of K and of V with
// 32-byte loads and 16-byte (f16) or 32-byte (f32) stores.  Needs k_new and
// v_new 16-byte aligned (the host checks; the per-row kernel serves the rest).
template <int DT>
__global__ __launch_bounds__(kBlock) void append_vec_kernel(AppendArgs a, int row_elems) {
  const int per_tok = row_elems / 8;
  const int64_t gid = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t t = gid / per_tok;
  if (t >= a.n_tok) return;
  const int e = (int)(gid - t * per_tok) * 8;
  const int seq = a.tok_seq[t], pos = a.tok_pos[t];
  if (seq < 0 || seq >= a.n_rows || pos < 0 || pos / kPage >= a.bt_stride) return;
  const uint32_t phys = a.bt[(size_t)seq * a.bt_stride + pos / kPage];
  if (phys >= a.num_pages) return;  // LNSKV_NO_PAGE or outside the pool
  const size_t dst = ((size_t)phys * kPage + (size_t)(pos % kPage)) * row_elems + e;
  const size_t src = (size_t)t * row_elems + e;
  float4 k0 = *reinterpret_cast<const float4*>(a.k_new + src);
  float4 k1 = *reinterpret_cast<const float4*>(a.k_new + src + 4);
  const float4 v0 = *reinterpret_cast<const float4*>(a.v_new + src);
  const float4 v1 = *reinterpret_cast<const float4*>(a.v_new + src + 4);
  if (a.rope_half > 0) {
    // RoPE on K: this thread's 8 elements hl..hl+7 of a head lie in one half
    // of the rotary part (or past it); the partner elements sit half/8
    // threads away in the same head (heads start at multiples of d/8 >= 2m)
    const int half = a.rope_half, m = half / 8;
    const int hl = e % a.head_dim;
    float x[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    float p[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) p[j] = __shfl_xor(x[j], m, kWave);
    if (hl < 2 * half) {
      const bool first = hl < half;
      const int i0 = first ? hl : hl - half;
      const float4 f0 = *reinterpret_cast<const float4*>(a.rope_inv + i0);
      const float4 f1 = *reinterpret_cast<const float4*>(a.rope_inv + i0 + 4);
      const float f[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
      const float fpos = (float)pos;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float sn, cs, y0, y1;
        rope_sincos(fpos * f[j], &sn, &cs);
        // (dim i, dim i + half) = (x, partner) in the first half, (partner, x) in the second
        rope_turn(first ? x[j] : p[j], first ? p[j] : x[j], sn, cs, &y0, &y1);
        x[j] = first ? y0 : y1;
      }
      k0 = make_float4(x[0], x[1], x[2], x[3]);
      k1 = make_float4(x[4], x[5], x[6], x[7]);
    }
  }
  if constexpr (DT == LNSKV_DTYPE_F32) {
    float4* kd = reinterpret_cast<float4*>(reinterpret_cast<float*>(a.k_pages) + dst);
    float4* vd = reinterpret_cast<float4*>(reinterpret_cast<float*>(a.v_pages) + dst);
    kd[0] = k0;
    kd[1] = k1;
    vd[0] = v0;
    vd[1] = v1;
  } else {
    auto pack = [](float lo, float hi) { return to_f16_bits(lo) | (to_f16_bits(hi) << 16); };
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(a.k_pages) + dst) =
        make_uint4(pack(k0.x, k0.y), pack(k0.z, k0.w), pack(k1.x, k1.y), pack(k1.z, k1.w));
    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(a.v_pages) + dst) =
        make_uint4(pack(v0.x, v0.y), pack(v0.z, v0.w), pack(v1.x, v1.y), pack(v1.z, v1.w));
  }
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

// RoPE for the shapes the fused kernels do not turn in place:
// y[r][h][:] = x[r][h][:] with the first 2*half elements of every head turned
// by row r's position (a decode row: kv_len[r]-1; an append row: tok_pos[r]).
// Block per row, threads over (head, element).
__global__ __launch_bounds__(kBlock) void rope_rows_kernel(const float* x, float* y, int heads, int d, int half,
                                                          const float* inv, const int32_t* kv_len,
                                                          int32_t kv_len_scalar, const int32_t* tok_pos) {
  const int r = blockIdx.x;
  const int pos = tok_pos ? tok_pos[r] : (kv_len ? kv_len[r] : kv_len_scalar) - 1;
  const float fpos = (float)max(pos, 0);
  const float* xr = x + (size_t)r * heads * d;
  float* yr = y + (size_t)r * heads * d;
  for (int idx = threadIdx.x; idx < heads * d; idx += kBlock) {
    const int h = idx / d, i = idx % d;
    float v = xr[idx];
    if (i < 2 * half) {
      const int kk = i < half ? i : i - half;
      float sn, cs, y0, y1;
      rope_sincos(fpos * inv[kk], &sn, &cs);
      rope_turn(xr[h * d + kk], xr[h * d + kk + half], sn, cs, &y0, &y1);
      v = i < half ? y0 : y1;
    }
    yr[idx] = v;
  }
}

// Zero fill (used instead of hipMemsetAsync so a caller may capture it).
__global__ __launch_bounds__(kBlock) void zero_kernel(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x; i < n16; i += (size_t)gridDim.x * kBlock)
    p[i] = make_uint4(0, 0, 0, 0);
}

// The changed entries of a block table, by value: no staging copy of host
// memory, only the kernel's arguments (4 + 8 * LNSKV_TABLE_PATCH_MAX bytes).
struct TablePatch {
  int32_t n;
  uint32_t idx[LNSKV_TABLE_PATCH_MAX];
  uint32_t val[LNSKV_TABLE_PATCH_MAX];
};
static_assert(LNSKV_TABLE_PATCH_MAX <= kWave, "one lane per changed entry");

__global__ __launch_bounds__(kWave) void table_patch_kernel(uint32_t* dst, TablePatch p) {
  const int i = (int)threadIdx.x;
  if (i < p.n) dst[p.idx[i]] = p.val[i];
}

// ---------------------------------------------------------------------------
// Host-side dispatch.
template <int DT>
int launch_append_dt(const AppendArgs& a, int d, hipStream_t st) {
  if constexpr (DT != LNSKV_DTYPE_Q8A) {
    const bool aligned = ((reinterpret_cast<uintptr_t>(a.k_new) | reinterpret_cast<uintptr_t>(a.v_new)) & 15) == 0;
    if (aligned && (d == 64 || d == 128 || d == 256)) {
      const int row_elems = a.n_kv * d;
      const int64_t threads = (int64_t)a.n_tok * (row_elems / 8);
      append_vec_kernel<DT><<<(unsigned)((threads + kBlock - 1) / kBlock), kBlock, 0, st>>>(a, row_elems);
      return hip_check("append kernel launch");
    }
  }
  const unsigned blocks = (unsigned)(((int64_t)a.n_tok * a.n_kv + kWavesPerBlock - 1) / kWavesPerBlock);
  switch (d) {
    case 64: append_kernel<DT, 64><<<blocks, kBlock, 0, st>>>(a); break;
    case 128: append_kernel<DT, 128><<<blocks, kBlock, 0, st>>>(a); break;
    case 256: append_kernel<DT, 256><<<blocks, kBlock, 0, st>>>(a); break;
    default: return fail(LNSKV_ERR_UNSUPPORTED, "head_dim %d", d);
  }
  return hip_check("append kernel launch");
}

// LNSKV_FORCE_VALU=1 routes every decode through the generic kernel (used by
// the tests to check the two kernels against each other).
bool force_valu() {
  const char* e = std::getenv("LNSKV_FORCE_VALU");
  return e && e[0] == '1';
}

// The MFMA kernels serve f16 and Q8A pages with head_dim 128 (the Llama /
// Mixtral shapes) or 256 (lns-ml's Qwen3.5 full-attention layers); every
// other combination runs the generic VALU kernel.
bool mfma_path(int dtype, int d, int rep);
bool mfma_q8_path(int dtype, int d, int rep);

template <bool FUSED>
int launch_decode(const DecodeArgs& a, int dtype, int d, int rep, int n_seq, hipStream_t st) {
  if (mfma_path(dtype, d, rep))
    return launch_decode_mfma_f16<FUSED>(a, rep, d, n_seq, st);
  switch (dtype) {
    case LNSKV_DTYPE_F32: return launch_decode_valu<LNSKV_DTYPE_F32, FUSED>(a, d, rep, n_seq, st);
    case LNSKV_DTYPE_F16: return launch_decode_valu<LNSKV_DTYPE_F16, FUSED>(a, d, rep, n_seq, st);
    case LNSKV_DTYPE_Q8A: return launch_decode_valu<LNSKV_DTYPE_Q8A, FUSED>(a, d, rep, n_seq, st);
    default: return fail(LNSKV_ERR_INVALID, "dtype %d", dtype);
  }
}

// Tokens per split-K partition when the caller passes 0: the largest power
// of two in [64, 1024] that still gives about 1024 workgroups (4 per CU) if
// sequences average half of max_kv_len.
int choose_split(int n_seq, int n_kv, int max_kv_len) {
  const int64_t pairs = (int64_t)n_seq * n_kv;
  int split = 1024;
  while (split > 64 && pairs * max_kv_len < (int64_t)2 * split * 1024) split /= 2;
  return split;
}

// Workspace (only needed when some sequence spans several split-K
// partitions): partial numerators [n_seq][n_heads][max_parts][d] f32, then
// partial (max, sum) [n_seq][n_heads][max_parts][2] f32.  No contents carry
// over between calls.
size_t workspace_bytes(int n_seq, int n_heads, int d, int max_parts) {
  if (max_parts <= 1) return 0;
  return (size_t)n_seq * n_heads * max_parts * ((size_t)d + 2) * sizeof(float);
}

bool mfma_path(int dtype, int d, int rep) {
  return dtype == LNSKV_DTYPE_F16 && (d == 128 || d == 256) && (rep == 1 || rep == 2 || rep == 4 || rep == 8) &&
         !force_valu();
}

// Q8A pages with head_dim 128 or 256 also run on the matrix cores, on the
// stream-K and workgroup schedules only (split_tokens = 0; stream-K in
// launches of at most kSkMaxSeqs sequences).
bool mfma_q8_path(int dtype, int d, int rep) {
  return dtype == LNSKV_DTYPE_Q8A && (d == 128 || d == 256) && (rep == 1 || rep == 2 || rep == 4 || rep == 8) &&
         !force_valu();
}

// Gated query split (split_gated_query_kernel, lns_decode.metal:193-209): the
// q projection holds, per (row, head), head_dim q values then head_dim gate
// logits.  Element gid of q_out / gate_out is lane gid % head_dim of global
// head gid / head_dim; gate_out = 1 / (1 + exp(-logit)).
__global__ __launch_bounds__(kBlock) void split_gated_query_kernel(const float* in, float* q_out, float* gate_out,
                                                                   int64_t n, int head_dim) {
  for (int64_t gid = (int64_t)blockIdx.x * kBlock + threadIdx.x; gid < n; gid += (int64_t)gridDim.x * kBlock) {
    const int64_t base = (gid / head_dim) * 2 * head_dim + gid % head_dim;
    q_out[gid] = in[base];
    gate_out[gid] = 1.0f / (1.0f + expf(-in[base + head_dim]));
  }
}

// The same, four elements per thread (head_dim a multiple of 4, 16-byte
// aligned buffers): 16-byte loads and stores.
__global__ __launch_bounds__(kBlock) void split_gated_query_vec_kernel(const float* in, float* q_out,
                                                                       float* gate_out, int64_t n4, int head_dim) {
  for (int64_t g4 = (int64_t)blockIdx.x * kBlock + threadIdx.x; g4 < n4; g4 += (int64_t)gridDim.x * kBlock) {
    const int64_t gid = 4 * g4;
    const int64_t base = (gid / head_dim) * 2 * head_dim + gid % head_dim;
    const float4 q = *reinterpret_cast<const float4*>(in + base);
    const float4 z = *reinterpret_cast<const float4*>(in + base + head_dim);
    float4 g;
    g.x = 1.0f / (1.0f + expf(-z.x));
    g.y = 1.0f / (1.0f + expf(-z.y));
    g.z = 1.0f / (1.0f + expf(-z.z));
    g.w = 1.0f / (1.0f + expf(-z.w));
    *reinterpret_cast<float4*>(q_out + gid) = q;
    *reinterpret_cast<float4*>(gate_out + gid) = g;
  }
}

// How one decode call runs, when the caller leaves the split to the library,
// the MFMA kernel serves the pages and there are at most kSkMaxSeqs
// sequences (Q8A pages: any number, stream-K in launches of kSkMaxSeqs): a
// small batch (at most kWgSmallPages units per workgroup) runs
// the workgroup schedule, one kernel whose workgroups merge what they share;
// a larger one stream-K (one wave per resident slot, each taking an equal
// share of all pages, then a merge kernel), which measured faster there.
// Split-K partitions of `split` tokens otherwise.
struct DecodePlan {
  int split = 0;      // split-K: tokens per partition
  int max_parts = 1;  // split-K: partitions of the longest sequence
  int sk_waves = 0;   // > 0: stream-K with this many waves
  int sk_waves_rope = 0;  // stream-K waves of a fused call that turns RoPE in the kernel
  int wg = 0;         // > 0: the workgroup schedule with this many workgroups
  size_t ws_bytes = 0;
};

// LNSKV_DECODE_SCHEDULE=stream-k or =workgroup forces that schedule wherever
// the library would choose between the two (tests, tuning); unset or any
// other value: by batch size.  Read on every plan, so that a workspace query
// and the call it sizes see the same setting.
enum { kScheduleAuto = 0, kScheduleStreamK = 1, kScheduleWorkgroup = 2 };
int schedule_setting() {
  const char* v = std::getenv("LNSKV_DECODE_SCHEDULE");
  if (v == nullptr) return kScheduleAuto;
  if (std::strcmp(v, "stream-k") == 0) return kScheduleStreamK;
  if (std::strcmp(v, "workgroup") == 0) return kScheduleWorkgroup;
  return kScheduleAuto;
}

int plan_decode(const lnskv_pages* c, int n_seq, int n_heads, int max_kv_len, int split_tokens, int fused,
                DecodePlan* p) {
  const int n_kv = (int)c->n_kv_heads, d = (int)c->head_dim, rep = n_heads / n_kv;
  *p = DecodePlan{};
  const int64_t units = (int64_t)n_seq * n_kv * ((int64_t)max_kv_len / kPage + 1);
  const bool q8 = mfma_q8_path((int)c->dtype, d, rep);
  // Q8A batches of more than kSkMaxSeqs sequences run stream-K in launches of
  // at most kSkMaxSeqs sequences each (the Q8A pages have no split-K matrix
  // kernel); f16 batches that large take the split-K matrix kernel
  if (split_tokens == 0 && (mfma_path((int)c->dtype, d, rep) || q8) && (n_seq <= kSkMaxSeqs || q8) &&
      units < ((int64_t)1 << 30)) {
    int n_wg = 0;
    if (int rc = mfma_wg_count(&n_wg)) return rc;
    const int setting = schedule_setting();
    if (n_seq <= kSkMaxSeqs &&
        (setting == kScheduleWorkgroup || (setting == kScheduleAuto && units <= (int64_t)kWgSmallPages * n_wg))) {
      // a small batch: the workgroup schedule (one kernel); the header, then
      // 2 * rep partial rows of (acc[d], m, l) per workgroup
      p->wg = n_wg;
      p->ws_bytes = kWsHeaderBytes + (size_t)n_wg * 2 * rep * ((size_t)d + 2) * sizeof(float);
      return LNSKV_OK;
    }
    // stream-K; fused < 0: either kind (the workspace query), sized for the
    // larger
    // the RoPE variants may hold more registers, so fewer of their waves
    // fit: each launch uses its own kernel's count, the workspace fits all
    int w0 = 0, w1 = 0, w1r = 0;
    if (fused <= 0)
      if (int rc = mfma_sk_waves(rep, d, false, q8, false, &w0)) return rc;
    if (fused != 0) {
      if (int rc = mfma_sk_waves(rep, d, true, q8, false, &w1)) return rc;
      if (int rc = mfma_sk_waves(rep, d, true, q8, true, &w1r)) return rc;
    }
    p->sk_waves = std::max(w0, w1);
    p->sk_waves_rope = w1r;
    const int w_most = std::max(p->sk_waves, w1r);
    // the header, then partial rows (acc, then (m, l)) of two pieces per
    // wave, then one 16-byte descriptor per wave
    p->ws_bytes = kWsHeaderBytes + (size_t)w_most * (2 * rep * ((size_t)d + 2) * sizeof(float) + 16);
    return LNSKV_OK;
  }
  p->split = split_tokens ? split_tokens : choose_split(n_seq, n_kv, max_kv_len);
  if (p->split < kPage || p->split % kPage != 0)
    return fail(LNSKV_ERR_INVALID, "split_tokens %d must be a positive multiple of 16", p->split);
  p->max_parts = std::max(1, (max_kv_len + p->split - 1) / p->split);
  if (p->max_parts > 65535)
    return fail(LNSKV_ERR_INVALID, "max_kv_len %d needs more than 65535 partitions", max_kv_len);
  const size_t part = workspace_bytes(n_seq, n_heads, d, p->max_parts);
  p->ws_bytes = part > 0 ? kWsHeaderBytes + part : 0;
  return LNSKV_OK;
}

}  // namespace

// Library-kept buffers per device: 0 decode workspace, 1 RoPE rows, 2 Q4L
// GEMV workspace (0 and 2 start with a zeroed count header).  A call that finds its buffer too small allocates a larger one and
// keeps the old one alive (kernels queued earlier may still read it) until
// lnskv_workspace_release: no call that enqueues work synchronizes the device
// or frees memory.  While the call's stream is being captured into a graph it
// allocates nothing and fails instead (reserve the buffers before capturing).
namespace {
constexpr int kLibraryBuffers = 3;
struct DeviceWorkspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::vector<DeviceWorkspace> g_ws;       // [device * kLibraryBuffers + which]
std::vector<std::pair<int, void*>> g_ws_retired;  // (device, pointer) outgrown, freed on release

const char* kBufferName[kLibraryBuffers] = {"decode workspace", "RoPE rows", "Q4L workspace"};

// grows buffer `which` of device `dev` to at least `need` bytes (lock held)
int grow_locked(int dev, int which, size_t need) {
  const size_t slot = (size_t)dev * kLibraryBuffers + (size_t)which;
  if (g_ws.size() <= slot) g_ws.resize((size_t)(dev + 1) * kLibraryBuffers);
  DeviceWorkspace& w = g_ws[slot];
  if (w.bytes >= need) return LNSKV_OK;
  const size_t grow = std::max({need, (size_t)1 << 20, w.bytes + w.bytes / 2});
  void* p = nullptr;
  if (hipMalloc(&p, grow) != hipSuccess) {
    (void)hipGetLastError();
    return fail(LNSKV_ERR_NOMEM, "library %s of %zu bytes: hipMalloc failed", kBufferName[which], grow);
  }
  if (w.ptr) g_ws_retired.emplace_back(dev, w.ptr);
  w.ptr = p;
  w.bytes = grow;
  return LNSKV_OK;
}
}  // namespace

int library_buffer(int which, size_t need, void** out, hipStream_t stream) {
  if (which < 0 || which >= kLibraryBuffers) return fail(LNSKV_ERR_INVALID, "library buffer %d", which);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LNSKV_ERR_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  const size_t slot = (size_t)dev * kLibraryBuffers + (size_t)which;
  if (g_ws.size() <= slot || g_ws[slot].bytes < need) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
      (void)hipGetLastError();
      return fail(LNSKV_ERR_HIP, "hipStreamIsCapturing failed");
    }
    if (cs != hipStreamCaptureStatusNone)
      return fail(LNSKV_ERR_WORKSPACE,
                  "the library %s holds %zu bytes, this call needs %zu, and the stream is being captured: "
                  "pass a workspace or call lnskv_workspace_reserve before capturing",
                  kBufferName[which], g_ws.size() > slot ? g_ws[slot].bytes : (size_t)0, need);
    if (int rc = grow_locked(dev, which, need)) return rc;
    // a decode or Q4L workspace starts with its counts at zero
    if ((which == 0 || which == 2) && hipMemsetAsync(g_ws[slot].ptr, 0, kWsHeaderBytes, stream) != hipSuccess)
      return fail(LNSKV_ERR_HIP, "hipMemsetAsync of the workspace header failed");
  }
  *out = g_ws[slot].ptr;
  return LNSKV_OK;
}

// ---------------------------------------------------------------------------
// Static scratch of lnskv_append_decode_noalloc: the decode workspace (the
// workgroup schedule's count header, partial rows and stream-K segment
// descriptors) for callers that cannot allocate device memory.  Every GPU the
// library runs on holds its own copy until the process ends.  The host name
// `scratch` is only a stand-in for the device array: its device address is
// looked up once per device and used from then on.  The count header starts
// at zero (static device storage is zero-initialised when the code object is
// loaded) and every call leaves it zero; every other word a call reads was
// written earlier in the same call.  Calls that overlap in time on one device
// race on it.
namespace {
constexpr size_t kNoAllocScratchBytes = LNSKV_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device
}  // namespace

// The current device's scratch address.  The first call on a device looks the
// address up and fills the host-side schedule caches the decode consults, so
// later calls allocate nothing, on the device or on the host.
int noalloc_scratch(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LNSKV_ERR_HIP, "hipGetDevice failed");
  if (dev < 0 || dev >= kMaxDevices) return fail(LNSKV_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(LNSKV_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    for (int rep : {1, 2, 4, 8})
      for (int d : {128, 256})
        for (bool q8 : {false, true}) {
          int waves = 0;
          for (bool rope : {false, true})
            if (int rc = mfma_sk_waves(rep, d, true, q8, rope, &waves)) return rc;
        }
    int n_wg = 0;
    if (int rc = mfma_wg_count(&n_wg)) return rc;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LNSKV_OK;
}

namespace {
int library_workspace(size_t need, void** out, hipStream_t st) { return library_buffer(0, need, out, st); }

// Checks a RoPE descriptor against head_dim; half = rotary_dim / 2.
int check_rope(const lnskv_rope* rope, int d, int* half) {
  if (!rope || !rope->inv_freqs_dev) return fail(LNSKV_ERR_INVALID, "rope and its inverse frequencies must be non-null");
  if (rope->rotary_dim < 2 || rope->rotary_dim % 2 != 0 || rope->rotary_dim > d)
    return fail(LNSKV_ERR_INVALID, "rotary_dim %d must be even and in [2, head_dim %d]", rope->rotary_dim, d);
  *half = rope->rotary_dim / 2;
  return LNSKV_OK;
}
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Where the rotated q/k rows of a RoPE call start in a caller's workspace:
// after the decode's part, on a 256-byte boundary.
size_t rope_rows_offset(size_t decode_bytes) { return (decode_bytes + 255) & ~(size_t)255; }

template <bool FUSED>
int decode_entry(const lnskv_pages* c, const float* q, const float* k_new, const float* v_new,
                 float* out, const uint32_t* bt, int32_t bt_stride, const int32_t* kv_len,
                 int32_t kv_len_scalar, const int32_t* p_start, int32_t p_start_scalar,
                 int32_t n_seq, int32_t n_heads, int32_t max_kv_len, float scale, int32_t split,
                 void* ws, size_t ws_bytes, lnskv_stream_t stream, const lnskv_rope* rope = nullptr,
                 const float* gate = nullptr, bool noalloc = false) {
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
  if (split < 0) return fail(LNSKV_ERR_INVALID, "split_tokens %d is negative", split);
  const int rep = n_heads / (int)c->n_kv_heads;
  const int d = (int)c->head_dim;
  // RoPE: turned inside the MFMA kernels for rotary widths 64 and 128 of
  // 128-wide heads; otherwise q and k_new are turned first into rows that the
  // decode then reads: in the caller's workspace after the decode's part, or
  // in a library buffer when the caller passes none
  int rope_half = 0;
  bool rope_rows = false;
  DecodePlan plan;
  if (int rc = plan_decode(c, n_seq, n_heads, max_kv_len, split, FUSED ? 1 : 0, &plan)) return rc;
  if (rope) {
    if (!FUSED) return fail(LNSKV_ERR_INVALID, "RoPE needs the fused append");
    if (int rc = check_rope(rope, d, &rope_half)) return rc;
    // turned in place by the matrix-core kernels (f16 pages on every
    // schedule, Q8A pages on stream-K and the workgroup schedule) for a
    // rotary width of 64 or 128 of a 128- or 256-wide head
    const bool mfma = mfma_path((int)c->dtype, d, rep) ||
                      (mfma_q8_path((int)c->dtype, d, rep) && (plan.wg > 0 || plan.sk_waves > 0));
    rope_rows = !(mfma && (rope_half == 32 || rope_half == 64) && aligned16(rope->inv_freqs_dev));
  }
  const size_t need = plan.ws_bytes;
  const size_t qn = (size_t)n_seq * n_heads * d, kn = (size_t)n_seq * c->n_kv_heads * d;
  const size_t rope_off = rope_rows_offset(need);
  const size_t rope_bytes = rope_rows ? (qn + kn) * sizeof(float) : 0;
  const hipStream_t st = (hipStream_t)stream;
  void* rope_buf = nullptr;
  if (ws == nullptr) {
    if (need > 0)
      if (int rc = library_workspace(need, &ws, st)) return rc;
    if (rope_rows)
      if (int rc = library_buffer(1, rope_bytes, &rope_buf, st)) return rc;
  } else {
    if (reinterpret_cast<uintptr_t>(ws) % 16 != 0) return fail(LNSKV_ERR_WORKSPACE, "workspace must be 16-byte aligned");
    const size_t total = rope_rows ? rope_off + rope_bytes : need;
    if (ws_bytes < total)
      return fail(LNSKV_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed%s", ws_bytes, total,
                  rope_rows ? " (decode partials, then the rotated q and k rows)" : "");
    if (rope_rows) rope_buf = static_cast<uint8_t*>(ws) + rope_off;
  }
  if (rope_rows) {
    float* qr = static_cast<float*>(rope_buf);
    float* kr = qr + qn;
    rope_rows_kernel<<<(unsigned)n_seq, kBlock, 0, st>>>(q, qr, n_heads, d, rope_half, rope->inv_freqs_dev, kv_len,
                                                        kv_len_scalar, nullptr);
    rope_rows_kernel<<<(unsigned)n_seq, kBlock, 0, st>>>(k_new, kr, (int)c->n_kv_heads, d, rope_half,
                                                        rope->inv_freqs_dev, kv_len, kv_len_scalar, nullptr);
    if (int rc = hip_check("rope kernel launch")) return rc;
    q = qr;
    k_new = kr;
    rope_half = 0;
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
  a.split = plan.split;
  a.max_parts = plan.max_parts;
  a.max_kv_len = max_kv_len;
  a.num_pages = c->num_pages;
  a.scale_log2 = scale * kLog2e;
  a.rope_half = rope_half;
  a.rope_inv = rope_half > 0 ? rope->inv_freqs_dev : nullptr;
  a.gate = gate;
  a.ws_err = ws_error_word(stream, !noalloc);
  if (plan.wg > 0) {
    a.wg_cnt = static_cast<uint32_t*>(ws);
    a.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kWsHeaderBytes);
    a.ws_ml = a.ws_acc + (size_t)plan.wg * 2 * rep * c->head_dim;
    return launch_decode_mfma_wg<FUSED>(a, rep, d, n_seq, plan.wg, c->dtype == LNSKV_DTYPE_Q8A, (hipStream_t)stream);
  }
  if (plan.sk_waves > 0) {
    const int n_waves = rope_half > 0 ? plan.sk_waves_rope : plan.sk_waves;
    a.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kWsHeaderBytes);
    a.ws_ml = a.ws_acc + (size_t)n_waves * 2 * rep * c->head_dim;
    a.sk_desc = reinterpret_cast<int4*>(a.ws_ml + (size_t)n_waves * 2 * rep * 2);
    // sequences [s0, s0 + ns) per launch; the launches share the workspace in
    // stream order (each combine has read it before the next decode writes)
    for (int s0 = 0; s0 < n_seq; s0 += kSkMaxSeqs) {
      const int ns = std::min(n_seq - s0, kSkMaxSeqs);
      DecodeArgs b = a;
      const size_t qo = (size_t)s0 * n_heads * d, ko = (size_t)s0 * c->n_kv_heads * d;
      b.q = a.q + qo;
      b.out = a.out + qo;
      b.gate = a.gate ? a.gate + qo : nullptr;
      b.k_new = a.k_new ? a.k_new + ko : nullptr;
      b.v_new = a.v_new ? a.v_new + ko : nullptr;
      b.bt = a.bt + (size_t)s0 * bt_stride;
      b.kv_len = a.kv_len ? a.kv_len + s0 : nullptr;
      b.p_start = a.p_start ? a.p_start + s0 : nullptr;
      if (int rc = launch_decode_mfma_sk<FUSED>(b, rep, d, ns, n_waves, c->dtype == LNSKV_DTYPE_Q8A,
                                                (hipStream_t)stream))
        return rc;
    }
    return LNSKV_OK;
  }
  if (need > 0) {
    a.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kWsHeaderBytes);
    a.ws_ml = a.ws_acc + (size_t)n_seq * n_heads * plan.max_parts * c->head_dim;
  }
  return launch_decode<FUSED>(a, c->dtype, (int)c->head_dim, rep, n_seq, (hipStream_t)stream);
}

}  // namespace

int table_patch(uint32_t* dst_dev, int n, const uint32_t* idx, const uint32_t* val, void* stream) {
  if (n < 1 || n > LNSKV_TABLE_PATCH_MAX) return fail(LNSKV_ERR_INVALID, "table patch of %d entries", n);
  TablePatch p{};
  p.n = n;
  for (int j = 0; j < n; ++j) {
    p.idx[j] = idx[j];
    p.val[j] = val[j];
  }
  table_patch_kernel<<<1, kWave, 0, (hipStream_t)stream>>>(dst_dev, p);
  return hip_check("block table patch launch");
}

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

namespace lnskv {
namespace {
int append_entry(const lnskv_pages* c, const lnskv_rope* rope, const float* k_new, const float* v_new,
                 const int32_t* tok_seq, const int32_t* tok_pos, int32_t n_tok, const uint32_t* bt,
                 int32_t bt_stride, int32_t n_rows, void* ws, size_t ws_bytes, lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (n_tok < 0) return fail(LNSKV_ERR_INVALID, "n_tok %d is negative", n_tok);
  if (n_tok == 0) return LNSKV_OK;
  if (!k_new || !v_new || !tok_seq || !tok_pos || !bt)
    return fail(LNSKV_ERR_INVALID, "append arguments must be non-null");
  if (bt_stride <= 0) return fail(LNSKV_ERR_INVALID, "bt_stride %d must be positive", bt_stride);
  if (n_rows < 0) return fail(LNSKV_ERR_INVALID, "n_rows %d is negative", n_rows);
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
  a.n_rows = n_rows;
  a.n_tok = n_tok;
  a.n_kv = (int32_t)c->n_kv_heads;
  a.num_pages = c->num_pages;
  a.head_dim = (int32_t)c->head_dim;
  const int d = (int)c->head_dim;
  const hipStream_t st = (hipStream_t)stream;
  if (rope) {
    // turned in the vector kernel when its lanes can pair up (half a multiple
    // of 8 with half/8 a power of two); otherwise K is turned first into rows
    // in the caller's workspace (or a library buffer when there is none)
    int half = 0;
    if (int rc = check_rope(rope, d, &half)) return rc;
    const int m = half / 8;
    const bool in_kernel = c->dtype != LNSKV_DTYPE_Q8A && (d == 64 || d == 128 || d == 256) && half % 8 == 0 &&
                           (m & (m - 1)) == 0 && aligned16(k_new) && aligned16(v_new) &&
                           aligned16(rope->inv_freqs_dev);
    if (in_kernel) {
      a.rope_inv = rope->inv_freqs_dev;
      a.rope_half = half;
    } else {
      void* buf = nullptr;
      const size_t need = (size_t)n_tok * c->n_kv_heads * d * sizeof(float);
      if (ws == nullptr) {
        if (int rc = library_buffer(1, need, &buf, st)) return rc;
      } else if (ws_bytes < need) {
        return fail(LNSKV_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed for the rotated K rows", ws_bytes, need);
      } else if (!aligned16(ws)) {
        return fail(LNSKV_ERR_WORKSPACE, "workspace must be 16-byte aligned");
      } else {
        buf = ws;
      }
      rope_rows_kernel<<<(unsigned)n_tok, kBlock, 0, st>>>(k_new, static_cast<float*>(buf), (int)c->n_kv_heads, d,
                                                          half, rope->inv_freqs_dev, nullptr, 0, tok_pos);
      if (int rc = hip_check("rope kernel launch")) return rc;
      a.k_new = static_cast<const float*>(buf);
    }
  }
  switch (c->dtype) {
    case LNSKV_DTYPE_F32: return launch_append_dt<LNSKV_DTYPE_F32>(a, d, st);
    case LNSKV_DTYPE_F16: return launch_append_dt<LNSKV_DTYPE_F16>(a, d, st);
    default: return launch_append_dt<LNSKV_DTYPE_Q8A>(a, d, st);
  }
}
}  // namespace
}  // namespace lnskv

int lnskv_append(const lnskv_pages* c, const float* k_new, const float* v_new,
                 const int32_t* tok_seq, const int32_t* tok_pos, int32_t n_tok,
                 const uint32_t* bt, int32_t bt_stride, int32_t n_rows, lnskv_stream_t stream) {
  return append_entry(c, nullptr, k_new, v_new, tok_seq, tok_pos, n_tok, bt, bt_stride, n_rows, nullptr, 0, stream);
}

int lnskv_rope_append(const lnskv_pages* c, const lnskv_rope* rope, const float* k_new, const float* v_new,
                      const int32_t* tok_seq, const int32_t* tok_pos, int32_t n_tok, const uint32_t* bt,
                      int32_t bt_stride, int32_t n_rows, void* ws, size_t ws_bytes, lnskv_stream_t stream) {
  if (!rope) {
    clear_error();
    return fail(LNSKV_ERR_INVALID, "rope must be non-null");
  }
  return append_entry(c, rope, k_new, v_new, tok_seq, tok_pos, n_tok, bt, bt_stride, n_rows, ws, ws_bytes, stream);
}

int lnskv_decode_workspace_size(const lnskv_pages* c, int32_t n_seq, int32_t n_heads,
                                int32_t max_kv_len, int32_t split_tokens, size_t* bytes) {
  clear_error();
  if (!bytes) return fail(LNSKV_ERR_INVALID, "bytes is NULL");
  *bytes = 0;
  if (int rc = check_geometry(c)) return rc;
  if (n_seq <= 0 || n_heads <= 0 || max_kv_len < 0 || split_tokens < 0 || n_heads % (int)c->n_kv_heads != 0)
    return fail(LNSKV_ERR_INVALID, "bad shape");
  DecodePlan plan;
  if (int rc = plan_decode(c, n_seq, n_heads, max_kv_len, split_tokens, -1, &plan)) return rc;
  *bytes = plan.ws_bytes;
  return LNSKV_OK;
}

int lnskv_rope_decode_workspace_size(const lnskv_pages* c, const lnskv_rope* rope, int32_t n_seq, int32_t n_heads,
                                     int32_t max_kv_len, int32_t split_tokens, size_t* bytes) {
  clear_error();
  if (!bytes) return fail(LNSKV_ERR_INVALID, "bytes is NULL");
  *bytes = 0;
  if (int rc = check_geometry(c)) return rc;
  if (n_seq <= 0 || n_heads <= 0 || max_kv_len < 0 || split_tokens < 0 || n_heads % (int)c->n_kv_heads != 0)
    return fail(LNSKV_ERR_INVALID, "bad shape");
  int half = 0;
  if (int rc = check_rope(rope, (int)c->head_dim, &half)) return rc;
  DecodePlan plan;
  if (int rc = plan_decode(c, n_seq, n_heads, max_kv_len, split_tokens, 1, &plan)) return rc;
  // room for the rotated rows whatever path the call takes
  *bytes = rope_rows_offset(plan.ws_bytes) + (size_t)n_seq * (n_heads + c->n_kv_heads) * c->head_dim * sizeof(float);
  return LNSKV_OK;
}

int lnskv_rope_append_workspace_size(const lnskv_pages* c, const lnskv_rope* rope, int32_t n_tok, size_t* bytes) {
  clear_error();
  if (!bytes) return fail(LNSKV_ERR_INVALID, "bytes is NULL");
  *bytes = 0;
  if (int rc = check_geometry(c)) return rc;
  if (n_tok < 0) return fail(LNSKV_ERR_INVALID, "n_tok %d is negative", n_tok);
  int half = 0;
  if (int rc = check_rope(rope, (int)c->head_dim, &half)) return rc;
  *bytes = (size_t)n_tok * c->n_kv_heads * c->head_dim * sizeof(float);
  return LNSKV_OK;
}

int lnskv_workspace_reserve(size_t decode_bytes, size_t rope_bytes, size_t q4l_bytes) {
  clear_error();
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LNSKV_ERR_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  const size_t want[kLibraryBuffers] = {decode_bytes, rope_bytes, q4l_bytes};
  for (int i = 0; i < kLibraryBuffers; ++i) {
    if (want[i] == 0) continue;
    const size_t slot = (size_t)dev * kLibraryBuffers + (size_t)i;
    const bool grows = g_ws.size() <= slot || g_ws[slot].bytes < want[i];
    if (int rc = grow_locked(dev, i, want[i])) return rc;
    if (grows && (i == 0 || i == 2) && hipMemset(g_ws[slot].ptr, 0, kWsHeaderBytes) != hipSuccess)
      return fail(LNSKV_ERR_HIP, "hipMemset of the workspace header failed");
  }
  return LNSKV_OK;
}

int lnskv_workspace_release(void) {
  clear_error();
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(LNSKV_ERR_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  if (hipDeviceSynchronize() != hipSuccess) return fail(LNSKV_ERR_HIP, "hipDeviceSynchronize failed");
  for (auto it = g_ws_retired.begin(); it != g_ws_retired.end();) {
    if (it->first == dev) {
      (void)hipFree(it->second);
      it = g_ws_retired.erase(it);
    } else {
      ++it;
    }
  }
  for (int i = 0; i < kLibraryBuffers; ++i) {
    const size_t slot = (size_t)dev * kLibraryBuffers + (size_t)i;
    if (slot < g_ws.size() && g_ws[slot].ptr) {
      (void)hipFree(g_ws[slot].ptr);
      g_ws[slot] = DeviceWorkspace{};
    }
  }
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

int lnskv_append_decode_noalloc(const lnskv_pages* c, const float* q, const float* k_new, const float* v_new,
                                float* out, const uint32_t* bt, int32_t bt_stride, const int32_t* kv_len,
                                const int32_t* p_start, int32_t n_seq, int32_t n_heads, int32_t max_kv_len,
                                float scale, int32_t split_tokens, lnskv_stream_t stream) {
  clear_error();
  if (!kv_len) return fail(LNSKV_ERR_INVALID, "kv_len must be non-null");
  void* ws = nullptr;
  if (int rc = noalloc_scratch(&ws)) return rc;
  return decode_entry<true>(c, q, k_new, v_new, out, bt, bt_stride, kv_len, 0, p_start, 0, n_seq, n_heads,
                            max_kv_len, scale, split_tokens, ws, kNoAllocScratchBytes, stream, nullptr, nullptr,
                            true);
}

int lnskv_rope_append_decode(const lnskv_pages* c, const lnskv_rope* rope, const float* q, const float* k_new,
                             const float* v_new, float* out, const uint32_t* bt, int32_t bt_stride,
                             const int32_t* kv_len, const int32_t* p_start, int32_t n_seq, int32_t n_heads,
                             int32_t max_kv_len, float scale, int32_t split_tokens, void* ws, size_t ws_bytes,
                             lnskv_stream_t stream) {
  clear_error();
  if (!kv_len) return fail(LNSKV_ERR_INVALID, "kv_len must be non-null");
  if (!rope) return fail(LNSKV_ERR_INVALID, "rope must be non-null");
  return decode_entry<true>(c, q, k_new, v_new, out, bt, bt_stride, kv_len, 0, p_start, 0, n_seq,
                            n_heads, max_kv_len, scale, split_tokens, ws, ws_bytes, stream, rope);
}

int lnskv_gated_append_decode(const lnskv_pages* c, const lnskv_rope* rope, const float* gate, const float* q,
                              const float* k_new, const float* v_new, float* out, const uint32_t* bt,
                              int32_t bt_stride, const int32_t* kv_len, const int32_t* p_start, int32_t n_seq,
                              int32_t n_heads, int32_t max_kv_len, float scale, int32_t split_tokens, void* ws,
                              size_t ws_bytes, lnskv_stream_t stream) {
  clear_error();
  if (!kv_len) return fail(LNSKV_ERR_INVALID, "kv_len must be non-null");
  if (!gate) return fail(LNSKV_ERR_INVALID, "gate must be non-null");
  return decode_entry<true>(c, q, k_new, v_new, out, bt, bt_stride, kv_len, 0, p_start, 0, n_seq,
                            n_heads, max_kv_len, scale, split_tokens, ws, ws_bytes, stream, rope, gate);
}

int lnskv_prefill_attention(const lnskv_pages* c, const float* q, float* out, const int32_t* chunks,
                            int32_t n_chunks, int32_t n_tok, const uint32_t* bt, int32_t bt_stride, int32_t n_rows,
                            const int32_t* p_start, int32_t window, int32_t n_heads, float scale,
                            lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (!q || !out || !chunks || !bt) return fail(LNSKV_ERR_INVALID, "q, out, chunks and block tables must be non-null");
  if (n_chunks <= 0 || n_chunks > 65535) return fail(LNSKV_ERR_INVALID, "n_chunks %d out of range [1, 65535]", n_chunks);
  if (n_tok <= 0) return fail(LNSKV_ERR_INVALID, "n_tok %d must be positive", n_tok);
  if (n_rows <= 0 || bt_stride <= 0)
    return fail(LNSKV_ERR_INVALID, "n_rows %d and bt_stride %d must be positive", n_rows, bt_stride);
  if (n_heads <= 0 || n_heads % (int)c->n_kv_heads != 0)
    return fail(LNSKV_ERR_INVALID, "n_heads %d is not a multiple of n_kv_heads %u", n_heads, c->n_kv_heads);
  if (!(scale > 0.0f) || !std::isfinite(scale)) return fail(LNSKV_ERR_INVALID, "scale must be positive and finite");
  if (window < 0) return fail(LNSKV_ERR_INVALID, "window %d is negative", window);
  if ((c->dtype != LNSKV_DTYPE_F16 && c->dtype != LNSKV_DTYPE_Q8A) || (c->head_dim != 128 && c->head_dim != 256))
    return fail(LNSKV_ERR_UNSUPPORTED, "prefill attention is built for f16 and Q8A pages with head_dim 128 or 256");
  if (!aligned16(chunks) || !aligned16(q)) return fail(LNSKV_ERR_INVALID, "chunks and q must be 16-byte aligned");
  // the Q8A kernel addresses each scale array with 32-bit byte offsets
  if (c->dtype == LNSKV_DTYPE_Q8A && (uint64_t)c->num_pages * kPage * c->n_kv_heads * sizeof(float) > 0x7FFFFFF0u)
    return fail(LNSKV_ERR_UNSUPPORTED, "prefill over Q8A pages needs scale arrays under 2 GiB (%u pages x %u kv heads)",
                c->num_pages, c->n_kv_heads);
  PrefillArgs a{};
  a.k_pages = static_cast<const uint8_t*>(c->k_pages);
  a.v_pages = static_cast<const uint8_t*>(c->v_pages);
  a.k_scales = c->dtype == LNSKV_DTYPE_Q8A ? c->k_scales : nullptr;
  a.v_scales = c->dtype == LNSKV_DTYPE_Q8A ? c->v_scales : nullptr;
  a.q = q;
  a.out = out;
  a.chunks = reinterpret_cast<const int4*>(chunks);
  a.bt = bt;
  a.p_start = p_start;
  a.window = window;
  a.n_chunks = n_chunks;
  a.n_tok = n_tok;
  a.n_rows = n_rows;
  a.bt_stride = bt_stride;
  a.n_kv = (int32_t)c->n_kv_heads;
  a.n_heads = n_heads;
  a.num_pages = c->num_pages;
  a.scale_log2 = scale * kLog2e;
  // at most one partly filled tile per chunk beyond n_tok / qt full ones;
  // blocks past the chunks' real tile count leave at once
  const int rep = n_heads / (int)c->n_kv_heads;
  const int64_t qt = prefill_queries_per_tile(rep, (int)c->head_dim);
  const int64_t tiles = ((int64_t)n_tok + qt - 1) / qt + n_chunks;
  if (tiles * c->n_kv_heads > INT32_MAX) return fail(LNSKV_ERR_INVALID, "too many query tiles");
  return launch_prefill_mfma(a, rep, (int)c->head_dim, (int)tiles, (hipStream_t)stream);
}

int lnskv_split_gated_query(const float* input, float* q_out, float* gate_out, int32_t n_rows, int32_t n_heads,
                            int32_t head_dim, lnskv_stream_t stream) {
  clear_error();
  if (!input || !q_out || !gate_out) return fail(LNSKV_ERR_INVALID, "input, q_out and gate_out must be non-null");
  if (n_rows <= 0 || n_heads <= 0 || head_dim <= 0)
    return fail(LNSKV_ERR_INVALID, "n_rows %d, n_heads %d and head_dim %d must be positive", n_rows, n_heads,
                head_dim);
  const int64_t n = (int64_t)n_rows * n_heads * head_dim;
  const hipStream_t st = (hipStream_t)stream;
  if (head_dim % 4 == 0 && aligned16(input) && aligned16(q_out) && aligned16(gate_out)) {
    const int64_t n4 = n / 4;
    const unsigned blocks = (unsigned)std::min<int64_t>((n4 + kBlock - 1) / kBlock, 65535);
    split_gated_query_vec_kernel<<<blocks, kBlock, 0, st>>>(input, q_out, gate_out, n4, head_dim);
  } else {
    const unsigned blocks = (unsigned)std::min<int64_t>((n + kBlock - 1) / kBlock, 65535);
    split_gated_query_kernel<<<blocks, kBlock, 0, st>>>(input, q_out, gate_out, n, head_dim);
  }
  return hip_check("split_gated_query kernel launch");
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
  if (take_ws_error())
    return fail(LNSKV_ERR_WORKSPACE,
                "a decode or Q4L GEMV call found an arrival count in its workspace header above what the call "
                "can reach: that header was not zero before its first use, and the results of calls on it are "
                "wrong (zero the first LNSKV_WORKSPACE_HEADER_BYTES bytes once)");
  return LNSKV_OK;
}

}  // extern "C"
