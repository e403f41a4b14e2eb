// o_proj after the attention over Q4_L weights: y[v] += W x[v] for a batch of
// vectors (the reference's q4l_gemv_accumulate_multirow, lns_decode.metal:
// 1174-1225, once per vector).  W is rows x cols in device blocks of 144 bytes
// (8 f16 effective scales, then 256 weight nibbles: bit 3 sign, bits 0-2
// magnitude m; the weight is sign * scale * 2^(m - 5), m = 0 exact zero).
//
// On the matrix cores.  Within one 32-weight sub-block a row's scale is
// constant, so the sub-block's products take the weights as the exact f16
// powers of two +-2^(m - 5) and the row's scale is applied afterwards in f32:
// no f16 rounding of small weights.  x enters as two f16 parts, hi = f16(x)
// and lo = f16(x - hi), both rounded toward zero (x = hi + lo to 2^-20):
//   D[vec][row] = sum_k A[vec][k] * B[k][row],  A = x parts, B = weight codes
// with v_mfma_f32_16x16x32_f16 over 16 vectors and 16 rows.  Lane (g, n) =
// (lane / 16, lane % 16) holds A row n (vector n of the tile) and B column n
// (weight row n), k = 8g..8g+7, and receives D[vectors 4g..4g+3][row n], so
// the scale it applies is its own row's.  The lane's dword g of a sub-block
// holds its columns 8g..8g+7; a sub-block is two products with the same B,
// the hi parts then the lo parts, chained through the accumulator (so the
// products sum (hi + lo) * w), each dword of k holding two columns:
//   B  = [ w(0, 2),    w(4, 6),    w(1, 3),    w(5, 7)  ]
//   A1 = [hi(x0, x2), hi(x4, x6), hi(x1, x3), hi(x5, x7)],  A2 the lo parts.
// Per sub-block, row tile and vector tile: two products, then four f32
// multiply-adds for the scale.
//
// Work split.  A workgroup of 4 waves owns 16 RT weight rows (RT row tiles:
// 4, or 2 for up to 16 vectors) and a range of whole blocks; wave q takes
// blocks q, q + 4, ... of the range.  Per block a wave brings the RT tiles'
// weights into its LDS by LDS DMA (the next block's while it multiplies this
// one), then for each sub-block forms the x operands once and multiplies them
// with all RT row tiles.  When there are too few row groups to fill the GPU, the blocks of a
// row are split over S workgroups: each stores its partial sums, and the last
// of the S to finish (an arrival count per row group) adds the S partials in
// split order to y.  All sums run in a fixed order (sub-blocks, waves, then
// splits), so every call gives the same bits whichever workgroup finishes
// last.
#include <algorithm>

#include "lnskv_device.h"

namespace lnskv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kQ4lBlockBytes = LNSKV_Q4L_DEVICE_BYTES;
constexpr int kQ4lTileVecs = 16;   // vectors per product (A rows)
constexpr int kQ4lMaxTiles = 4;    // vector tiles per launch (64 vectors)
constexpr int kQ4lWaves = 4;       // waves per workgroup (split of a range's blocks)
constexpr int kQ4lTargetWgs = 256; // workgroups wanted per launch: one per CU
// Buffer resource word 3 for raw dword access (DATA_FORMAT = 32-bit).
constexpr int kQ4lBufferFormat = 0x00020000;
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) uint32_t lds_u32;

// High byte of the f16 +2^(m - 5) for m = 0..7 (m = 0: zero): (m + 10) << 2,
// bytes m = 0..3 and m = 4..7, for v_perm_b32.
constexpr uint32_t kMagLo = 0x34302C00u;
constexpr uint32_t kMagHi = 0x44403C38u;

// Eight weight nibbles (one dword: weights 2i and 2i+1 in byte i) -> the f16
// codes as dwords (w0, w2), (w4, w6), (w1, w3), (w5, w7).
__device__ __forceinline__ u32x4 weight_codes(uint32_t w) {
  const uint32_t he = __builtin_amdgcn_perm(kMagHi, kMagLo, w & 0x07070707u) | ((w << 4) & 0x80808080u);
  const uint32_t ho = __builtin_amdgcn_perm(kMagHi, kMagLo, (w >> 4) & 0x07070707u) | (w & 0x80808080u);
  // f16 k (low half) and k+1 (high half) of each dword: high bytes only
  u32x4 d;
  d.x = __builtin_amdgcn_perm(he, ho, 0x050C040Cu);  // he bytes 0, 1
  d.y = __builtin_amdgcn_perm(he, ho, 0x070C060Cu);  // he bytes 2, 3
  d.z = __builtin_amdgcn_perm(he, ho, 0x010C000Cu);  // ho bytes 0, 1
  d.w = __builtin_amdgcn_perm(he, ho, 0x030C020Cu);  // ho bytes 2, 3
  return d;
}

// The hi and lo f16 parts of two x values, each as one dword (a in the low
// half): hi = f16(x) and lo = f16(x - hi), rounded toward zero.  x - hi is
// exact in f32 (hi is x with its low mantissa bits cleared), formed as one
// mixed-precision fma of the f16 hi with m1 = -1 (a value the compiler cannot
// see, so that it keeps the fma instead of a conversion and a subtraction).
__device__ __forceinline__ void x_pair_parts(float a, float b, float m1, uint32_t& hi, uint32_t& lo) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(a, b);
  const auto l = __builtin_amdgcn_cvt_pkrtz(__builtin_fmaf((float)h[0], m1, a), __builtin_fmaf((float)h[1], m1, b));
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, l);
}

// Waits until at most N vector-memory loads of this wave are outstanding
// (gfx9 s_waitcnt: vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left open).
template <int N>
__device__ __forceinline__ void q4l_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// 16-row tiles per workgroup (and per wave) for T vector tiles: each x
// operand a wave splits serves this many tiles; with one vector tile, two
// (measured faster: more row groups and a shorter merge).
constexpr int q4l_row_tiles(int T) { return T == 1 ? 2 : 4; }
// Outputs (vector, row) one workgroup produces for T vector tiles.
constexpr int q4l_wg_outputs(int T) { return T * kQ4lTileVecs * 16 * q4l_row_tiles(T); }

struct Q4lArgs {
  const uint8_t* W;
  const float* x;
  float* y;
  float* part;    // [S][groups][q4l_wg_outputs(T)] partial sums (S > 1)
  uint32_t* cnt;  // [groups] arrival counts, zero between calls (S > 1)
  uint32_t* err;  // host word set to 1 on a count above S - 1 (a header that was not zero)
  int64_t x_stride, y_stride;
  int rows, bpr, n_vec, tile0;
  int groups;     // row groups of 16 q4l_row_tiles(T) rows
  int split;      // S: workgroups per row group
  int bpw;        // blocks per workgroup (the last may hold fewer)
};

// Workgroup (row group rg, split sp) = blockIdx.x (rg fastest).
template <int T>
__global__ __launch_bounds__(kQ4lWaves * kWave) void q4l_gemv_acc_kernel(Q4lArgs a) {
  constexpr int RT = q4l_row_tiles(T);
  constexpr int RW = 16 * RT;                                // rows per workgroup
  constexpr int E = q4l_wg_outputs(T);                       // outputs per workgroup
  constexpr int kPer = E / (kQ4lWaves * kWave);              // outputs per thread
  constexpr int kChunks = RW * 9;                            // 16-byte chunks of a weight tile
  constexpr int kDma = (kChunks + kWave - 1) / kWave;        // LDS DMA instructions per tile
  constexpr int kTileStride = kDma * kWave * 16;             // LDS bytes per tile slot (padding included)
  constexpr int kRedBytes = kQ4lWaves * E * 4;
  constexpr int kTileBytes = kQ4lWaves * 2 * kTileStride;   // two slots per wave
  constexpr int kLds = kTileBytes > kRedBytes ? kTileBytes : kRedBytes;
  static_assert(E % (kQ4lWaves * kWave) == 0, "outputs per thread");
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLds];
  __shared__ int merge;

  const int tid = (int)threadIdx.x;
  // q: the wave index, made visibly uniform so that offsets derived from it
  // stay in scalar registers
  const int lane = tid & (kWave - 1), q = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane >> 4, n = lane & 15;
  const int rg = (int)blockIdx.x % a.groups, sp = (int)blockIdx.x / a.groups;
  const int row0 = rg * RW;
  const int b_end = min(a.bpr, (sp + 1) * a.bpw);

  // the y entries this thread adds to (if it is the one to add them) are
  // loaded now so that the read-modify-write adds no memory round trip at the
  // end
  float yv[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int idx = tid + u * kQ4lWaves * kWave;
    const int t = idx / (kQ4lTileVecs * RW), v = (idx / RW) % kQ4lTileVecs, r = idx % RW;
    const int vec = (a.tile0 + t) * kQ4lTileVecs + v;
    yv[u] = vec < a.n_vec && row0 + r < a.rows ? a.y[(int64_t)vec * a.y_stride + row0 + r] : 0.0f;
  }

  float4v acc[T][RT];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[t][r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.W, (short)0, (int)((int64_t)a.rows * a.bpr * kQ4lBlockBytes), kQ4lBufferFormat);
  lds_u8* const wslot = (lds_u8*)&lds[q * 2 * kTileStride];
  // this lane's x row for each tile (vectors past n_vec read vector 0; their
  // outputs are never stored), at its 8 columns of a sub-block
  const float* xrow[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int vec = (a.tile0 + t) * kQ4lTileVecs + n;
    xrow[t] = a.x + (int64_t)(vec < a.n_vec ? vec : 0) * a.x_stride + 8 * g;
  }

  float m1;
  asm volatile("v_mov_b32 %0, -1.0" : "=v"(m1));
  // The RT tiles of block b (RW rows x 144 bytes, chunk 9 r + c) into LDS by
  // LDS DMA; lanes past the tile load its first chunk into the padding.  Rows
  // past the matrix read row 0 of the group (their outputs are never stored).
  auto weight_dma = [&](int b, lds_u8* dst) {
#pragma unroll
    for (int k = 0; k < kDma; ++k) {
      const int idx = kWave * k + lane;
      const int r = idx < kChunks ? idx / 9 : 0, c = idx < kChunks ? idx % 9 : 0;
      const int rr = row0 + r < a.rows ? row0 + r : row0;
      const int off = (int)(((int64_t)rr * a.bpr + b) * kQ4lBlockBytes + 16 * c);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wrsrc, (__attribute__((address_space(3))) void*)(dst + 1024 * k), 16,
                                               off, 0, 0, 0);
    }
  };
  // Two tile slots per wave: the next block's tiles are on their way while
  // this block is multiplied (its slot's LDS reads are all consumed by then).
  int b = sp * a.bpw + q;
  if (b < b_end) weight_dma(b, wslot);
  for (int i = 0; b < b_end; b += kQ4lWaves, ++i) {  // wave-uniform
    lds_u8* const wl = wslot + (i & 1) * kTileStride;
    const bool more = b + kQ4lWaves < b_end;
    __builtin_amdgcn_sched_barrier(0);
    if (more) weight_dma(b + kQ4lWaves, wslot + ((i + 1) & 1) * kTileStride);
    // x of sub-block j + 1 is loaded while sub-block j is multiplied
    float4v xb[2][T][2];
    auto load_x = [&](int j, float4v (&dst)[T][2]) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        dst[t][0] = *reinterpret_cast<const float4v*>(xrow[t] + 256 * b + 32 * j);
        dst[t][1] = *reinterpret_cast<const float4v*>(xrow[t] + 256 * b + 32 * j + 4);
      }
    };
    __builtin_amdgcn_sched_barrier(0);
    load_x(0, xb[0]);
    // The compiler does not order LDS reads after an LDS DMA: this block's
    // DMAs were issued before the next block's and sub-block 0's x loads, and
    // loads complete in order, so once no more than those are outstanding the
    // tiles are in LDS.
    __builtin_amdgcn_sched_barrier(0);
    if (more)
      q4l_wait_vmcnt<kDma + T * 2>();
    else
      q4l_wait_vmcnt<T * 2>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j + 1 < 8) load_x(j + 1, xb[(j + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      // x columns 8g + 0..7 of vector n (p: 0..3, v: 4..7), hi parts in
      // A1, lo parts in A2, in the k order of weight_codes
      half8 a1[T], a2[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const float4v p = xb[j & 1][t][0], v = xb[j & 1][t][1];
        uint32_t h0, h1, h2, h3, l0, l1, l2, l3;
        x_pair_parts(p[0], p[2], m1, h0, l0);
        x_pair_parts(v[0], v[2], m1, h1, l1);
        x_pair_parts(p[1], p[3], m1, h2, l2);
        x_pair_parts(v[1], v[3], m1, h3, l3);
        a1[t] = __builtin_bit_cast(half8, u32x4{h0, h1, h2, h3});
        a2[t] = __builtin_bit_cast(half8, u32x4{l0, l1, l2, l3});
      }
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        const lds_u8* trow = wl + kQ4lBlockBytes * (16 * r + n);
        const uint32_t wj = *(const lds_u32*)(trow + 16 + 16 * j + 4 * g);
        const uint32_t sw = *(const lds_u32*)(trow + 4 * (j >> 1));
        const half8 codes = __builtin_bit_cast(half8, weight_codes(wj));
        const float scale = (float)__builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
#pragma unroll
        for (int t = 0; t < T; ++t) {
          float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1[t], codes, float4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2[t], codes, d, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[t][r][e] = fmaf(scale, d[e], acc[t][r][e]);
        }
      }
    }
  }

  // lane (g, n): vectors 4g..4g+3 of each tile, row n of each row tile.  The
  // weight tiles are dead once every wave is past its products.
  __syncthreads();
  float* red = reinterpret_cast<float*>(lds);  // [wave][t][vector][row]
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[((q * T + t) * kQ4lTileVecs + 4 * g + e) * RW + 16 * r + n] = acc[t][r][e];
  __syncthreads();
  float sum[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int idx = tid + u * kQ4lWaves * kWave;
    float s = red[idx];
#pragma unroll
    for (int w = 1; w < kQ4lWaves; ++w) s += red[w * E + idx];
    sum[u] = s;
  }
  if (a.split > 1) {
    // Store this workgroup's partials as device-scope stores (written through
    // to where every XCD reads), wait until they have completed, then count
    // the workgroup in; the last of the row group's S adds them up.
    float* mine = a.part + ((int64_t)sp * a.groups + rg) * E;
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      __hip_atomic_store(mine + tid + u * kQ4lWaves * kWave, sum[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const uint32_t old = __hip_atomic_fetch_add(a.cnt + rg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = old == (uint32_t)(a.split - 1);
      if (old > (uint32_t)(a.split - 1) && a.err)  // not a zeroed header: flagged for lnskv_sync
        __hip_atomic_store(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      if (last) __hip_atomic_store(a.cnt + rg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      merge = last;
    }
    __syncthreads();
    if (!merge) return;  // workgroup-uniform
    for (int s0 = 0; s0 < a.split; ++s0) {  // split order
      const float* ps = a.part + ((int64_t)s0 * a.groups + rg) * E;
      float pv[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u)
        pv[u] = __hip_atomic_load(ps + tid + u * kQ4lWaves * kWave, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int u = 0; u < kPer; ++u) sum[u] = s0 == 0 ? pv[u] : sum[u] + pv[u];
    }
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int idx = tid + u * kQ4lWaves * kWave;
    const int t = idx / (kQ4lTileVecs * RW), v = (idx / RW) % kQ4lTileVecs, r = idx % RW;
    const int vec = (a.tile0 + t) * kQ4lTileVecs + v;
    if (vec >= a.n_vec || row0 + r >= a.rows) continue;
    a.y[(int64_t)vec * a.y_stride + row0 + r] = yv[u] + sum[u];
  }
}

// The launch plan for rw rows per workgroup: row groups, split and blocks per
// workgroup.
void q4l_plan(int rows, int bpr, int rw, int* groups, int* split, int* bpw) {
  const int G = (rows + rw - 1) / rw;
  int S = 1;
  if (G < kQ4lTargetWgs) S = std::max(1, std::min((kQ4lTargetWgs + G - 1) / G, bpr / kQ4lWaves));
  const int per = (bpr + S - 1) / S;
  *groups = G;
  *split = (bpr + per - 1) / per;
  *bpw = per;
}

template <int T>
void launch_q4l(Q4lArgs a, hipStream_t st) {
  q4l_plan(a.rows, a.bpr, 16 * q4l_row_tiles(T), &a.groups, &a.split, &a.bpw);
  q4l_gemv_acc_kernel<T><<<(unsigned)(a.groups * a.split), kQ4lWaves * kWave, 0, st>>>(a);
}

// Workspace: the arrival counts (LNSKV_WORKSPACE_HEADER_BYTES, zero between
// calls) and the partial sums of a split launch.  A split needs fewer than
// kQ4lTargetWgs row groups, so S * groups < 2 kQ4lTargetWgs whatever the rows
// (q4l_wg_outputs grows with T, so the launch with the most tiles is largest);
// with fewer than 2 kQ4lWaves blocks a row there is no split and no workspace.
size_t q4l_ws_bytes(int cols, int n_vec) {
  const int bpr = cols / 256;
  if (bpr < 2 * kQ4lWaves) return 0;
  const int T = std::min((n_vec + kQ4lTileVecs - 1) / kQ4lTileVecs, kQ4lMaxTiles);
  return kWsHeaderBytes + (size_t)2 * kQ4lTargetWgs * (size_t)q4l_wg_outputs(T) * sizeof(float);
}

// What the launches of one call use: 0 when none of them splits (then the
// call needs no workspace at all), else at most q4l_ws_bytes(cols, n_vec).
size_t q4l_call_ws_bytes(int rows, int cols, int n_vec) {
  const int bpr = cols / 256;
  const int n_tiles = (n_vec + kQ4lTileVecs - 1) / kQ4lTileVecs;
  size_t most = 0;
  for (int t0 = 0; t0 < n_tiles; t0 += kQ4lMaxTiles) {
    const int T = std::min(n_tiles - t0, kQ4lMaxTiles);
    int groups = 0, split = 0, bpw = 0;
    q4l_plan(rows, bpr, 16 * q4l_row_tiles(T), &groups, &split, &bpw);
    if (split > 1) most = std::max(most, (size_t)split * groups * (size_t)q4l_wg_outputs(T) * sizeof(float));
  }
  return most > 0 ? kWsHeaderBytes + most : 0;
}

}  // namespace
}  // namespace lnskv

using namespace lnskv;

extern "C" int lnskv_q4l_workspace_size(int32_t cols, int32_t n_vec, size_t* bytes) {
  clear_error();
  if (!bytes) return fail(LNSKV_ERR_INVALID, "bytes must be non-null");
  if (cols <= 0 || n_vec <= 0) return fail(LNSKV_ERR_INVALID, "cols %d and n_vec %d must be positive", cols, n_vec);
  if (cols % 256 != 0) return fail(LNSKV_ERR_UNSUPPORTED, "cols %d must be a multiple of 256", cols);
  *bytes = q4l_ws_bytes(cols, n_vec);
  return LNSKV_OK;
}

extern "C" int lnskv_q4l_gemv_accumulate(const void* blocks_dev, const float* x_dev, float* y_dev, int32_t rows,
                                         int32_t cols, int32_t n_vec, int32_t x_stride, int32_t y_stride,
                                         void* ws, size_t ws_bytes, lnskv_stream_t stream) {
  clear_error();
  if (!blocks_dev || !x_dev || !y_dev) return fail(LNSKV_ERR_INVALID, "blocks, x and y must be non-null");
  if (rows <= 0 || cols <= 0 || n_vec <= 0)
    return fail(LNSKV_ERR_INVALID, "rows %d, cols %d and n_vec %d must be positive", rows, cols, n_vec);
  if (cols % 256 != 0) return fail(LNSKV_ERR_UNSUPPORTED, "cols %d must be a multiple of 256", cols);
  if (x_stride < cols || y_stride < rows)
    return fail(LNSKV_ERR_INVALID, "x_stride %d must be >= cols %d and y_stride %d >= rows %d", x_stride, cols,
                y_stride, rows);
  if ((int64_t)rows * (cols / 256) * LNSKV_Q4L_DEVICE_BYTES > INT32_MAX)
    return fail(LNSKV_ERR_UNSUPPORTED, "a Q4L matrix over 2 GiB of blocks (%d x %d)", rows, cols);
  if (x_stride % 4 != 0 || (reinterpret_cast<uintptr_t>(x_dev) & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(blocks_dev) & 15) != 0)
    return fail(LNSKV_ERR_INVALID, "x and the blocks must be 16-byte aligned and x_stride a multiple of 4");
  const hipStream_t st = (hipStream_t)stream;
  const size_t need = q4l_call_ws_bytes(rows, cols, n_vec);
  if (need > 0) {
    if (ws == nullptr) {
      if (int rc = library_buffer(2, need, &ws, st)) return rc;
    } else if (ws_bytes < need) {
      return fail(LNSKV_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed", ws_bytes, need);
    } else if ((reinterpret_cast<uintptr_t>(ws) & 15) != 0) {
      return fail(LNSKV_ERR_WORKSPACE, "workspace must be 16-byte aligned");
    }
  }
  Q4lArgs a{};
  a.W = static_cast<const uint8_t*>(blocks_dev);
  a.x = x_dev;
  a.y = y_dev;
  a.cnt = need > 0 ? static_cast<uint32_t*>(ws) : nullptr;
  a.part = need > 0 ? reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + kWsHeaderBytes) : nullptr;
  a.err = need > 0 ? ws_error_word(stream, true) : nullptr;
  a.x_stride = x_stride;
  a.y_stride = y_stride;
  a.rows = rows;
  a.bpr = cols / 256;
  a.n_vec = n_vec;
  // up to 4 tiles (64 vectors) per launch
  const int n_tiles = (n_vec + kQ4lTileVecs - 1) / kQ4lTileVecs;
  for (int t0 = 0; t0 < n_tiles; t0 += kQ4lMaxTiles) {
    a.tile0 = t0;
    switch (std::min(n_tiles - t0, kQ4lMaxTiles)) {
      case 1: launch_q4l<1>(a, st); break;
      case 2: launch_q4l<2>(a, st); break;
      case 3: launch_q4l<3>(a, st); break;
      default: launch_q4l<4>(a, st); break;
    }
  }
  return hip_check("q4l gemv kernel launch");
}
