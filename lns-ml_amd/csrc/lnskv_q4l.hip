// o_proj after the attention over Q4_L weights: y[v] += W x[v] for a batch of
// vectors (the reference's q4l_gemv_accumulate_multirow, lns_decode.metal:
// 1174-1225, once per vector).  W is rows x cols in device blocks of 144 bytes
// (8 f16 effective scales, then 256 weight nibbles: bit 3 sign, bits 0-2
// magnitude m; the weight is sign * scale * 2^(m - 5), m = 0 exact zero).
//
// On the matrix cores.  Within one 32-weight sub-block a row's scale is
// constant, so one v_mfma_f32_16x16x32_f16 per (sub-block, 8 vectors) takes
// the weights as the exact f16 powers of two +-2^(m - 5) and the row's scale is
// applied afterwards in f32: no f16 rounding of small weights.  x enters as two
// f16 parts, hi = f16(x) and lo = f16(x - hi) (x = hi + lo to ~2^-22), in the
// A operand's rows 0-7 and 8-15:
//   D[slot][row] = sum_k A[slot][k] * B[k][row],  A = x parts, B = weight codes
// lane (g, n) = (lane / 16, lane % 16) holds B column n (weight row n of the
// 16-row tile, k = 8g..8g+7) and receives D[slots 4g..4g+3][row n], so the
// scale it applies is its own row's.  The k order inside a lane's 8 weights is
// even nibbles then odd (w0 w2 w4 w6 w1 w3 w5 w7); x is permuted to match.
//
// Up to 8 vectors: each lane loads half of its 8 x values and swaps halves
// with its hi/lo partner lane (n ^ 8).  More: x is split into its A operands
// once per call (q4l_x_operands_kernel, into a workspace: 16 bytes per lane,
// tile and sub-block) and loaded ready-made.  A workgroup of 4 waves owns 16
// weight rows; wave q takes blocks q, q + 4, ... of those rows, four blocks at
// a time: their 16-row tiles go to LDS by LDS DMA (3 instructions a block) and
// the x operands are loaded up to 16 sub-blocks ahead.  The four waves'
// partial sums are added in LDS in a fixed order, so every call gives the same
// bits.
#include <algorithm>
#include <type_traits>

#include "lnskv_device.h"

namespace lnskv {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kQ4lBlockBytes = LNSKV_Q4L_DEVICE_BYTES;
constexpr int kQ4lWaves = 4;     // waves per workgroup (K split)
constexpr int kQ4lRows = 16;     // weight rows per workgroup
constexpr int kQ4lMaxTiles = 8;  // 8-vector tiles per launch (64 vectors)

// High byte of the f16 +2^(m - 5) for m = 0..7 (m = 0: zero): (m + 10) << 2,
// bytes m = 0..3 and m = 4..7, for v_perm_b32.
constexpr uint32_t kMagLo = 0x34302C00u;
constexpr uint32_t kMagHi = 0x44403C38u;

// Eight weight nibbles (one dword: weights 2i and 2i+1 in byte i) -> the f16
// codes in k order w0 w2 w4 w6 w1 w3 w5 w7.
__device__ __forceinline__ half8 weight_codes(uint32_t w) {
  const uint32_t he = __builtin_amdgcn_perm(kMagHi, kMagLo, w & 0x07070707u) | ((w << 4) & 0x80808080u);
  const uint32_t ho = __builtin_amdgcn_perm(kMagHi, kMagLo, (w >> 4) & 0x07070707u) | (w & 0x80808080u);
  // f16 k (low half) and k+1 (high half) of each dword: high bytes only
  u32x4 d;
  d.x = __builtin_amdgcn_perm(he, ho, 0x050C040Cu);  // he bytes 0, 1
  d.y = __builtin_amdgcn_perm(he, ho, 0x070C060Cu);  // he bytes 2, 3
  d.z = __builtin_amdgcn_perm(he, ho, 0x010C000Cu);  // ho bytes 0, 1
  d.w = __builtin_amdgcn_perm(he, ho, 0x030C020Cu);  // ho bytes 2, 3
  return __builtin_bit_cast(half8, d);
}

// A operand of one 8-vector tile for the 8 columns c, c+1, ..., c+7 of the
// lane's sub-block chunk: slot n < 8 holds f16(x) of vector n, slot n >= 8 the
// remainder f16(x - f16(x)) of vector n - 8 (zero past n_vec), in the k order
// of weight_codes.
// The A-operand parts of 8 x values (columns c..c+3 in p, c+4..c+7 in q), in
// the k order of weight_codes: f16(x) when !lo, f16(x - f16(x)) when lo; zero
// when !valid.
__device__ __forceinline__ half8 x_parts(const float4v& p, const float4v& q, bool valid, bool lo) {
  const float v[8] = {p[0], p[2], q[0], q[2], p[1], p[3], q[1], q[3]};
  half8 a;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float xv = valid ? v[e] : 0.0f;
    const _Float16 h = (_Float16)xv;
    a[e] = lo ? (_Float16)(xv - (float)h) : h;
  }
  return a;
}

__device__ __forceinline__ half8 x_operand(const float* x, int64_t x_stride, int vec, bool valid, bool lo,
                                           int col) {
  // branch-free: a vector past n_vec reads vector 0 (always present) and is
  // zeroed, so callers stay straight-line code
  const int64_t base = (int64_t)(valid ? vec : 0) * x_stride + col;
  const float4v p = *reinterpret_cast<const float4v*>(x + base);
  const float4v q = *reinterpret_cast<const float4v*>(x + base + 4);
  return x_parts(p, q, valid, lo);
}

// x operands: xa[(t * nsb + sb) * 64 + lane] for 8-vector tile t, sub-block
// sb (columns 32 sb .. 32 sb + 31) and lane (g, n): slot n, columns 8g..8g+7.
__global__ __launch_bounds__(kBlock) void q4l_x_operands_kernel(const float* __restrict__ x, int64_t x_stride,
                                                                int n_vec, int nsb, int64_t n_ops,
                                                                half8* __restrict__ xa) {
  const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (idx >= n_ops) return;
  const int lane = (int)(idx & (kWave - 1));
  const int64_t ts = idx / kWave;
  const int sb = (int)(ts % nsb), t = (int)(ts / nsb);
  const int g = lane >> 4, n = lane & 15;
  const int vec = 8 * t + (n & 7);
  xa[idx] = x_operand(x, x_stride, vec, vec < n_vec, n >= 8, 32 * sb + 8 * g);
}

constexpr int kQ4lBatch = 4;     // blocks whose weight tiles a wave loads together
constexpr int kQ4lGroup = 2;     // sub-blocks per operand group
constexpr int kWTile = 3 * 1024;  // LDS bytes per weight tile: 2304 used, the rest catches padding DMA
// Buffer resource word 3 for raw dword access (DATA_FORMAT = 32-bit).
constexpr int kQ4lBufferFormat = 0x00020000;
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) uint32_t lds_u32;
// Waits until at most N vector-memory loads of this wave are outstanding
// (gfx9 s_waitcnt: vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left open).
template <int N>
__device__ __forceinline__ void q4l_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <bool INLINE_X>
using XOp = typename std::conditional<INLINE_X, float4v, half8>::type;  // an operand as loaded

// INLINE_X (one tile only): the A operands are formed from x here instead of
// read from the workspace (no separate operand pass for up to 8 vectors).
template <int T, bool INLINE_X>
__global__ __launch_bounds__(kQ4lWaves * kWave) void q4l_gemv_acc_kernel(const uint8_t* __restrict__ W,
                                                                          const half8* __restrict__ xa,
                                                                          const float* __restrict__ x,
                                                                          int64_t x_stride, float* __restrict__ y,
                                                                          int rows, int bpr, int n_vec, int tile0,
                                                                          int64_t y_stride) {
  static_assert(!INLINE_X || T == 1, "operands are formed in the kernel for one tile only");
  constexpr int kPerThread = (T * 8 * kQ4lRows + kQ4lWaves * kWave - 1) / (kQ4lWaves * kWave);
  __shared__ float red[kQ4lWaves][T][8][kQ4lRows];
  __shared__ __attribute__((aligned(16))) uint8_t wtile[kQ4lWaves][kQ4lBatch][kWTile];
  // q: the wave index, made visibly uniform so that block and sub-block
  // offsets derived from it stay in scalar registers
  const int lane = (int)(threadIdx.x & (kWave - 1)), q = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int g = lane >> 4, n = lane & 15;
  const int row0 = (int)blockIdx.x * kQ4lRows;
  const int row = row0 + n;
  const bool row_ok = row < rows;
  const int nsb = bpr * 8;

  // the y entries this thread adds to at the end, loaded now so that the
  // read-modify-write does not add a memory round trip after the products
  float yv[kPerThread];
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int idx = (int)threadIdx.x + u * kQ4lWaves * kWave;
    const int t = idx / (8 * kQ4lRows), v = (idx / kQ4lRows) % 8, r = idx % kQ4lRows;
    const int vec = (tile0 + t) * 8 + v;
    const bool ok = idx < T * 8 * kQ4lRows && vec < n_vec && row0 + r < rows;
    yv[u] = ok ? y[(int64_t)vec * y_stride + row0 + r] : 0.0f;
  }

  float4v acc[T];
#pragma unroll
  for (int t = 0; t < T; ++t) acc[t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

  // Per batch: the weight tiles of kQ4lBatch blocks (16 rows x 144 bytes
  // each) go to this wave's LDS by LDS DMA, 16 bytes per lane (3 instructions
  // a block instead of 9 scattered dword loads), and the operands are read
  // back from LDS.  The batch body is straight-line code: blocks past the
  // row's end load a valid block and contribute zero codes.
  const __amdgpu_buffer_rsrc_t wrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)((int64_t)rows * bpr * kQ4lBlockBytes),
                                        kQ4lBufferFormat);
  lds_u8* wl = (lds_u8*)&wtile[q][0][0];
  // The x operands of this launch's tiles through a buffer resource: the
  // offset of (tile, sub-block) is wave-uniform (a scalar register) and the
  // lane's 16 bytes a constant vector offset, so the loads need no 64-bit
  // address arithmetic per lane.  The host keeps T * nsb * 1024 below 2^31.
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      INLINE_X ? (void*)x : (void*)(xa + (int64_t)tile0 * nsb * kWave), (short)0,
      INLINE_X ? 0 : T * nsb * kWave * (int)sizeof(half8), kQ4lBufferFormat);
  for (int b0 = q; b0 < bpr; b0 += kQ4lWaves * kQ4lBatch) {
    int bb[kQ4lBatch];
    bool bok[kQ4lBatch];
#pragma unroll
    for (int i = 0; i < kQ4lBatch; ++i) {
      const int b = b0 + kQ4lWaves * i;
      bok[i] = row_ok && b < bpr;
      bb[i] = b < bpr ? b : b0;
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        // 16-byte chunk idx = 9 * row + chunk of the tile (idx >= 144: padding)
        const int idx = 64 * k + lane;
        const int r = idx < 144 ? idx / 9 : 15, c = idx < 144 ? idx % 9 : 8;
        const int rr = row0 + r < rows ? row0 + r : row0;
        const int off = (int)(((int64_t)rr * bpr + bb[i]) * kQ4lBlockBytes + 16 * c);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wrsrc, (__attribute__((address_space(3))) void*)(wl + kWTile * i + 1024 * k),
                                                 16, off, 0, 0, 0);
      }
    }
    // operands in groups of kQ4lGroup sub-blocks, D groups ahead in a ring
    // of D + 1 buffers: group k + D is loaded (raw) before group k is
    // multiplied, enough to cover an L2 round trip; the scheduling barriers
    // keep the compiler from sinking the loads to their use
    constexpr int NG = kQ4lBatch * 8 / kQ4lGroup;
    constexpr int D = T == 1 ? NG : (T == 2 ? 8 : (T <= 4 ? 4 : 2));
    XOp<INLINE_X> xb[D + 1][kQ4lGroup][T];
    auto load_group = [&](int k, XOp<INLINE_X> (&dst)[kQ4lGroup][T]) {
#pragma unroll
      for (int u = 0; u < kQ4lGroup; ++u) {
        const int sbi = k * kQ4lGroup + u;
        const int sb = bb[sbi / 8] * 8 + sbi % 8;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          if constexpr (INLINE_X) {
            // lane n < 8: columns 8g..8g+3 of vector n; lane n + 8: 8g+4..8g+7
            const int vec = tile0 * 8 + (n & 7);
            const int64_t base = (int64_t)(vec < n_vec ? vec : 0) * x_stride + 32 * sb + 8 * g + 4 * (n >> 3);
            dst[u][t] = *reinterpret_cast<const float4v*>(x + base);
          } else {
            dst[u][t] = __builtin_bit_cast(
                half8, __builtin_amdgcn_raw_buffer_load_b128(xrsrc, lane * (int)sizeof(half8),
                                                             (t * nsb + sb) * kWave * (int)sizeof(half8), 0));
          }
        }
      }
    };
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < D && k < NG; ++k) load_group(k, xb[k]);
    // The compiler does not order LDS reads after an LDS DMA, so wait here:
    // the tile DMAs were issued before the first D groups' loads and
    // vector-memory loads complete in order, so once no more than those are
    // in flight the tiles are in LDS.  The barriers keep every load on its
    // side of the wait.
    __builtin_amdgcn_sched_barrier(0);
    q4l_wait_vmcnt<(D < NG ? D : NG) * kQ4lGroup * T>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      if (k + D < NG) load_group(k + D, xb[(k + D) % (D + 1)]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kQ4lGroup; ++u) {
        const int sbi = k * kQ4lGroup + u, i = sbi / 8, j = sbi % 8;
        const lds_u8* trow = wl + kWTile * i + kQ4lBlockBytes * n;
        const uint32_t wj = *(const lds_u32*)(trow + 16 + 16 * j + 4 * g);
        const uint32_t sw = *(const lds_u32*)(trow + 4 * (j >> 1));
        const half8 codes = weight_codes(bok[i] ? wj : 0u);
        const float scale =
            (float)__builtin_bit_cast(_Float16, (uint16_t)((j & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
#pragma unroll
        for (int t = 0; t < T; ++t) {
          half8 a;
          if constexpr (INLINE_X) {
            const float4v mine = xb[k % (D + 1)][u][t];
            float4v other;
#pragma unroll
            for (int e = 0; e < 4; ++e) other[e] = __shfl_xor(mine[e], 8, kWave);
            const bool second = n >= 8;
            const float4v p = second ? other : mine, qv = second ? mine : other;
            const bool valid = tile0 * 8 + (n & 7) < n_vec;
            a = x_parts(p, qv, valid, second);
          } else {
            a = xb[k % (D + 1)][u][t];
          }
          const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, codes, float4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[t][e] = fmaf(scale, d[e], acc[t][e]);
        }
      }
    }
  }

  // slots 4g..4g+3: g = 0, 1 the hi parts of vectors 4g + e, g = 2, 3 the lo
  // parts of vectors 4(g - 2) + e; lane l + 32 holds the lo part of lane l's
#pragma unroll
  for (int t = 0; t < T; ++t) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float other = __shfl_xor(acc[t][e], 32, kWave);
      if (g < 2) red[q][t][4 * g + e][n] = acc[t][e] + other;
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kPerThread; ++u) {
    const int idx = (int)threadIdx.x + u * kQ4lWaves * kWave;
    const int t = idx / (8 * kQ4lRows), v = (idx / kQ4lRows) % 8, r = idx % kQ4lRows;
    const int vec = (tile0 + t) * 8 + v;
    if (idx >= T * 8 * kQ4lRows || vec >= n_vec || row0 + r >= rows) continue;
    float s = red[0][t][v][r];
#pragma unroll
    for (int w = 1; w < kQ4lWaves; ++w) s += red[w][t][v][r];
    y[(int64_t)vec * y_stride + row0 + r] = yv[u] + s;
  }
}

template <int T>
void launch_q4l(const uint8_t* W, const half8* xa, float* y, int rows, int bpr, int n_vec, int tile0, int64_t ys,
                hipStream_t st) {
  const unsigned grid = (unsigned)((rows + kQ4lRows - 1) / kQ4lRows);
  q4l_gemv_acc_kernel<T, false><<<grid, kQ4lWaves * kWave, 0, st>>>(W, xa, nullptr, 0, y, rows, bpr, n_vec, tile0,
                                                                   ys);
}

// Up to 8 vectors take their operands from x inside the GEMV kernel and need
// no workspace; more go through q4l_x_operands_kernel.
size_t q4l_ws_bytes(int cols, int n_vec) {
  if (n_vec <= 8) return 0;
  return (size_t)((n_vec + 7) / 8) * (size_t)(cols / 32) * kWave * sizeof(half8);
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
  // one launch's x operands (up to kQ4lMaxTiles tiles) are addressed with 32-bit offsets
  if ((int64_t)kQ4lMaxTiles * (cols / 32) * kWave * (int64_t)sizeof(half8) > INT32_MAX)
    return fail(LNSKV_ERR_UNSUPPORTED, "cols %d: one launch's x operands exceed 2 GiB", cols);
  if (x_stride % 4 != 0 || (reinterpret_cast<uintptr_t>(x_dev) & 15) != 0 ||
      (reinterpret_cast<uintptr_t>(blocks_dev) & 15) != 0)
    return fail(LNSKV_ERR_INVALID, "x and the blocks must be 16-byte aligned and x_stride a multiple of 4");
  const hipStream_t st = (hipStream_t)stream;
  const uint8_t* W = static_cast<const uint8_t*>(blocks_dev);
  const int bpr = cols / 256, nsb = cols / 32;
  if (n_vec <= 8) {
    const unsigned grid = (unsigned)((rows + kQ4lRows - 1) / kQ4lRows);
    q4l_gemv_acc_kernel<1, true><<<grid, kQ4lWaves * kWave, 0, st>>>(W, nullptr, x_dev, x_stride, y_dev, rows,
                                                                     bpr, n_vec, 0, y_stride);
    return hip_check("q4l gemv kernel launch");
  }
  const size_t need = q4l_ws_bytes(cols, n_vec);
  if (ws == nullptr) {
    if (int rc = library_buffer(2, need, &ws, st)) return rc;
  } else if (ws_bytes < need) {
    return fail(LNSKV_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed", ws_bytes, need);
  } else if ((reinterpret_cast<uintptr_t>(ws) & 15) != 0) {
    return fail(LNSKV_ERR_WORKSPACE, "workspace must be 16-byte aligned");
  }
  half8* xa = static_cast<half8*>(ws);
  const int n_tiles = (n_vec + 7) / 8;
  const int64_t n_ops = (int64_t)n_tiles * nsb * kWave;
  q4l_x_operands_kernel<<<(unsigned)((n_ops + kBlock - 1) / kBlock), kBlock, 0, st>>>(x_dev, x_stride, n_vec, nsb,
                                                                                      n_ops, xa);
  // up to 8 tiles (64 vectors) per launch
  for (int t0 = 0; t0 < n_tiles; t0 += kQ4lMaxTiles) {
    const int nt = std::min(n_tiles - t0, kQ4lMaxTiles);
    switch (nt) {  // exactly the pass's tiles: every operand load is in the workspace
      case 1: launch_q4l<1>(W, xa, y_dev, rows, bpr, n_vec, t0, y_stride, st); break;
      case 2: launch_q4l<2>(W, xa, y_dev, rows, bpr, n_vec, t0, y_stride, st); break;
      case 3: launch_q4l<3>(W, xa, y_dev, rows, bpr, n_vec, t0, y_stride, st); break;
      case 4: launch_q4l<4>(W, xa, y_dev, rows, bpr, n_vec, t0, y_stride, st); break;
      case 5: launch_q4l<5>(W, xa, y_dev, rows, bpr, n_vec, t0, y_stride, st); break;
      case 6: launch_q4l<6>(W, xa, y_dev, rows, bpr, n_vec, t0, y_stride, st); break;
      case 7: launch_q4l<7>(W, xa, y_dev, rows, bpr, n_vec, t0, y_stride, st); break;
      default: launch_q4l<8>(W, xa, y_dev, rows, bpr, n_vec, t0, y_stride, st); break;
    }
  }
  return hip_check("q4l gemv kernel launch");
}
