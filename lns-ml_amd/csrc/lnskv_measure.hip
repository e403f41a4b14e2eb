// Load ceiling of the decode's page pattern (measurement only; the reference
// has no counterpart).  Each (physical page, kv head) unit is the 16 rows of
// one kv head in a page of K and the same in V (256 bytes each for f16 d128 /
// f32 d64, 128 bytes plus the K and V scales for Q8A d128): the bytes a decode
// reads per page.  A wave walks its units with plain 16-byte loads and
// no arithmetic besides an XOR that keeps the loads alive, two units in
// flight (the next one issued as soon as one arrives).  Timed over the same
// units, in the same order and wave split, as a decode step, it gives the
// bandwidth the memory system delivers for that pattern with nothing else in
// the way.
#include <type_traits>

#include "lnskv_device.h"

namespace lnskv {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int N>
__device__ __forceinline__ void wait_loads() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// The loads of one unit (16 token rows of one kv head in K and in V), rows
// of ROW bytes (128: Q8A d128; 256: f16 d128, f32 d64, Q8A d256; 512: f16
// d256), kL = ROW / 16 lanes per row: lane (r, c) = (lane / kL, lane % kL)
// loads 16-byte chunk c of rows r, r + 64/kL, ... of K and of V (the 16
// rows once each), then, with SC (Q8A pages), one 4-byte scale: that of
// token lane % 16, from V for lanes with bit 4 set and from K otherwise --
// the bytes a decode reads per unit.
template <int ROW, bool SC>
struct Unit {
  static constexpr int kLanesPerRow = ROW / 16;
  static constexpr int kRowsPerLoad = kWave / kLanesPerRow;
  static constexpr int kLoadsPerPool = kPage / kRowsPerLoad;
  static constexpr int kLoads = 2 * kLoadsPerPool + (SC ? 1 : 0);
};

template <int ROW, bool SC>
__device__ __forceinline__ void load_unit(const uint8_t* k, const uint8_t* v, const float* ks, const float* vs,
                                          uint32_t page, int32_t kvh, uint32_t num_pages, int32_t n_kv,
                                          u32x4 (&b)[Unit<ROW, SC>::kLoads]) {
  using U = Unit<ROW, SC>;
  const int lane = (int)(threadIdx.x & (kWave - 1));
  // ids outside the pools read page 0 / kv head 0 (in bounds)
  const size_t pg = page < num_pages ? page : 0u;
  const size_t h = kvh >= 0 && kvh < n_kv ? (size_t)kvh : 0u;
  const size_t row_bytes = (size_t)n_kv * ROW;
  const size_t base = pg * kPage * row_bytes + h * ROW + (size_t)(lane / U::kLanesPerRow) * row_bytes +
                      (size_t)(lane % U::kLanesPerRow) * 16;
#pragma unroll
  for (int j = 0; j < U::kLoadsPerPool; ++j) {
    b[j] = *reinterpret_cast<const u32x4*>(k + base + (size_t)j * U::kRowsPerLoad * row_bytes);
    b[U::kLoadsPerPool + j] = *reinterpret_cast<const u32x4*>(v + base + (size_t)j * U::kRowsPerLoad * row_bytes);
  }
  if constexpr (SC) {
    const float* sp = (lane & 16) ? vs : ks;
    const float sc = sp[(pg * kPage + (size_t)(lane & 15)) * (size_t)n_kv + h];
    b[2 * U::kLoadsPerPool] = u32x4{__builtin_bit_cast(uint32_t, sc), 0u, 0u, 0u};
  }
}

template <int ROW, bool SC>
__device__ __forceinline__ void fold(u32x4& acc, const u32x4 (&b)[Unit<ROW, SC>::kLoads]) {
#pragma unroll
  for (int j = 0; j < Unit<ROW, SC>::kLoads; ++j) acc ^= b[j];
}

template <int ROW, bool SC>
__global__ __launch_bounds__(kWave) void read_units_kernel(const uint8_t* k, const uint8_t* v, const float* ks,
                                                           const float* vs, const uint32_t* unit_page,
                                                           const int32_t* unit_kvh, const int32_t* wave_start,
                                                           uint32_t num_pages, int32_t n_kv, uint32_t* sink) {
  constexpr int L = Unit<ROW, SC>::kLoads;
  const int w = blockIdx.x, lane = (int)(threadIdx.x & (kWave - 1));
  const int u0 = wave_start[w], u1 = wave_start[w + 1];
  u32x4 acc = {0u, 0u, 0u, 0u};
  if (u1 > u0) {
    u32x4 b0[L], b1[L];
    load_unit<ROW, SC>(k, v, ks, vs, unit_page[u0], unit_kvh[u0], num_pages, n_kv, b0);
    const int v1 = min(u0 + 1, u1 - 1);
    load_unit<ROW, SC>(k, v, ks, vs, unit_page[v1], unit_kvh[v1], num_pages, n_kv, b1);
    int u = u0;
    for (; u + 2 < u1; u += 2) {
      wait_loads<L>();
      fold<ROW, SC>(acc, b0);
      load_unit<ROW, SC>(k, v, ks, vs, unit_page[u + 2], unit_kvh[u + 2], num_pages, n_kv, b0);
      wait_loads<L>();
      fold<ROW, SC>(acc, b1);
      const int n1 = min(u + 3, u1 - 1);
      load_unit<ROW, SC>(k, v, ks, vs, unit_page[n1], unit_kvh[n1], num_pages, n_kv, b1);
    }
    // b1 holds unit u + 1 when it exists, else a stand-in copy of unit u
    wait_loads<0>();
    fold<ROW, SC>(acc, b0);
    if (u + 1 < u1) fold<ROW, SC>(acc, b1);
  }
  sink[(size_t)w * kWave + lane] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

// Plain streaming read of a contiguous buffer (the read ceiling): thread t
// of T loads 16-byte chunks t, t + T, t + 2T, ..., U of them issued before
// any is used, so each wave instruction reads 1 KiB contiguous and the grid
// sweeps the buffer front to back.  Nothing is written unless the XOR of
// what one thread read hits one value (so that the loads cannot be elided).
template <int U>
__global__ __launch_bounds__(256) void read_stream_kernel(const u32x4* __restrict__ p, size_t n16,
                                                          uint32_t* sink) {
  const size_t nt = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (size_t)(U - 1) * nt < n16; i += (size_t)U * nt) {
    u32x4 b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) b[u] = p[i + (size_t)u * nt];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= b[u];
  }
  for (; i < n16; i += nt) acc ^= p[i];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u) sink[0] = 1u;
}

}  // namespace
}  // namespace lnskv

using namespace lnskv;

extern "C" int lnskv_read_stream(const void* buf, size_t bytes, int32_t loads_in_flight, int32_t blocks_per_cu,
                                 uint32_t* sink, lnskv_stream_t stream) {
  clear_error();
  if (!buf || !sink) return fail(LNSKV_ERR_INVALID, "buffer and sink must be non-null");
  if (bytes == 0 || bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(buf) & 15) != 0)
    return fail(LNSKV_ERR_INVALID, "the buffer must be 16-byte aligned and a positive multiple of 16 bytes");
  if (blocks_per_cu < 1 || blocks_per_cu > 8)
    return fail(LNSKV_ERR_INVALID, "blocks_per_cu %d out of range [1, 8]", blocks_per_cu);
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return fail(LNSKV_ERR_HIP, "device compute-unit count unavailable");
  const unsigned grid = (unsigned)(cus * blocks_per_cu);
  const hipStream_t st = (hipStream_t)stream;
  const u32x4* p = static_cast<const u32x4*>(buf);
  const size_t n16 = bytes / 16;
  switch (loads_in_flight) {
    case 1: read_stream_kernel<1><<<grid, 256, 0, st>>>(p, n16, sink); break;
    case 2: read_stream_kernel<2><<<grid, 256, 0, st>>>(p, n16, sink); break;
    case 4: read_stream_kernel<4><<<grid, 256, 0, st>>>(p, n16, sink); break;
    case 8: read_stream_kernel<8><<<grid, 256, 0, st>>>(p, n16, sink); break;
    case 16: read_stream_kernel<16><<<grid, 256, 0, st>>>(p, n16, sink); break;
    default: return fail(LNSKV_ERR_INVALID, "loads_in_flight %d must be 1, 2, 4, 8 or 16", loads_in_flight);
  }
  return hip_check("read stream launch");
}

extern "C" int lnskv_read_units(const lnskv_pages* c, const uint32_t* unit_page, const int32_t* unit_kvh,
                                const int32_t* wave_start, int32_t n_waves, uint32_t* sink,
                                lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (!unit_page || !unit_kvh || !wave_start || !sink)
    return fail(LNSKV_ERR_INVALID, "unit lists, wave starts and sink must be non-null");
  if (n_waves <= 0 || n_waves > 65535) return fail(LNSKV_ERR_INVALID, "n_waves %d out of range [1, 65535]", n_waves);
  const size_t row = (size_t)c->head_dim * dtype_bytes(c->dtype);
  const bool q8 = c->dtype == LNSKV_DTYPE_Q8A;
  const hipStream_t st = (hipStream_t)stream;
  const uint8_t* kp = static_cast<const uint8_t*>(c->k_pages);
  const uint8_t* vp = static_cast<const uint8_t*>(c->v_pages);
  const unsigned grid = (unsigned)n_waves;
  const int32_t nkv = (int32_t)c->n_kv_heads;
  auto probe = [&](auto row_c, auto sc_c) {
    constexpr int R = decltype(row_c)::value;
    constexpr bool S = decltype(sc_c)::value;
    read_units_kernel<R, S><<<grid, kWave, 0, st>>>(kp, vp, S ? c->k_scales : nullptr, S ? c->v_scales : nullptr,
                                                    unit_page, unit_kvh, wave_start, c->num_pages, nkv, sink);
  };
  if (row == 128 && q8) probe(std::integral_constant<int, 128>{}, std::true_type{});
  else if (row == 256 && q8) probe(std::integral_constant<int, 256>{}, std::true_type{});
  else if (row == 256) probe(std::integral_constant<int, 256>{}, std::false_type{});
  else if (row == 512 && !q8) probe(std::integral_constant<int, 512>{}, std::false_type{});
  else
    return fail(LNSKV_ERR_UNSUPPORTED,
                "the load probe reads kv-head rows of 256 or 512 bytes (f16 d128/d256, f32 d64) or Q8A rows of "
                "128 or 256 bytes (d128/d256); got %zu bytes", row);
  return hip_check("load probe launch");
}
