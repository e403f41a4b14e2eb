// Load ceiling of the decode's page pattern (measurement only; the reference
// has no counterpart).  Each (physical page, kv head) unit is the 16 rows x
// 256 bytes of one kv head in a page of K and the same in V: the bytes a
// decode reads per page.  A wave walks its units with plain 16-byte loads and
// no arithmetic besides an XOR that keeps the loads alive, two units in
// flight (the next one issued as soon as one arrives).  Timed over the same
// units, in the same order and wave split, as a decode step, it gives the
// bandwidth the memory system delivers for that pattern with nothing else in
// the way.
#include "lnskv_device.h"

namespace lnskv {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSliceRow = 256;  // bytes of one kv head's row (head_dim x dtype bytes)

template <int N>
__device__ __forceinline__ void wait_loads() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Lane (r, c) = (lane / 16, lane % 16) loads 16-byte chunk c of rows
// r, r + 4, r + 8, r + 12 of the unit: 8 loads per unit (4 K, 4 V).
__device__ __forceinline__ void load_unit(const uint8_t* k, const uint8_t* v, uint32_t page, int32_t kvh,
                                          uint32_t num_pages, int32_t n_kv, uint32_t row_bytes, u32x4 (&b)[8]) {
  const int lane = (int)(threadIdx.x & (kWave - 1));
  // ids outside the pools read page 0 / kv head 0 (in bounds)
  const size_t pg = page < num_pages ? page : 0u;
  const size_t h = kvh >= 0 && kvh < n_kv ? (size_t)kvh : 0u;
  const size_t base = pg * kPage * row_bytes + h * kSliceRow + (size_t)(lane >> 4) * row_bytes + (size_t)(lane & 15) * 16;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    b[j] = *reinterpret_cast<const u32x4*>(k + base + (size_t)j * 4 * row_bytes);
    b[4 + j] = *reinterpret_cast<const u32x4*>(v + base + (size_t)j * 4 * row_bytes);
  }
}

__global__ __launch_bounds__(kWave) void read_units_kernel(const uint8_t* k, const uint8_t* v,
                                                           const uint32_t* unit_page, const int32_t* unit_kvh,
                                                           const int32_t* wave_start, uint32_t num_pages,
                                                           int32_t n_kv, uint32_t* sink) {
  const int w = blockIdx.x, lane = (int)(threadIdx.x & (kWave - 1));
  const int u0 = wave_start[w], u1 = wave_start[w + 1];
  const uint32_t row_bytes = (uint32_t)n_kv * kSliceRow;
  u32x4 acc = {0u, 0u, 0u, 0u};
  if (u1 > u0) {
    u32x4 b0[8], b1[8];
    load_unit(k, v, unit_page[u0], unit_kvh[u0], num_pages, n_kv, row_bytes, b0);
    const int v1 = min(u0 + 1, u1 - 1);
    load_unit(k, v, unit_page[v1], unit_kvh[v1], num_pages, n_kv, row_bytes, b1);
    int u = u0;
    for (; u + 2 < u1; u += 2) {
      wait_loads<8>();
#pragma unroll
      for (int j = 0; j < 8; ++j) acc ^= b0[j];
      load_unit(k, v, unit_page[u + 2], unit_kvh[u + 2], num_pages, n_kv, row_bytes, b0);
      wait_loads<8>();
#pragma unroll
      for (int j = 0; j < 8; ++j) acc ^= b1[j];
      const int n1 = min(u + 3, u1 - 1);
      load_unit(k, v, unit_page[n1], unit_kvh[n1], num_pages, n_kv, row_bytes, b1);
    }
    // b1 holds unit u + 1 when it exists, else a stand-in copy of unit u
    wait_loads<0>();
    const bool two = u + 1 < u1;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc ^= two ? b0[j] ^ b1[j] : b0[j];
  }
  sink[(size_t)w * kWave + lane] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace
}  // namespace lnskv

using namespace lnskv;

extern "C" int lnskv_read_units(const lnskv_pages* c, const uint32_t* unit_page, const int32_t* unit_kvh,
                                const int32_t* wave_start, int32_t n_waves, uint32_t* sink,
                                lnskv_stream_t stream) {
  clear_error();
  if (int rc = check_pages(c)) return rc;
  if (!unit_page || !unit_kvh || !wave_start || !sink)
    return fail(LNSKV_ERR_INVALID, "unit lists, wave starts and sink must be non-null");
  if (n_waves <= 0 || n_waves > 65535) return fail(LNSKV_ERR_INVALID, "n_waves %d out of range [1, 65535]", n_waves);
  if ((size_t)c->head_dim * dtype_bytes(c->dtype) != (size_t)kSliceRow)
    return fail(LNSKV_ERR_UNSUPPORTED, "the load probe reads 256-byte kv-head rows (head_dim x dtype bytes = %zu)",
                (size_t)c->head_dim * dtype_bytes(c->dtype));
  read_units_kernel<<<(unsigned)n_waves, kWave, 0, (hipStream_t)stream>>>(
      static_cast<const uint8_t*>(c->k_pages), static_cast<const uint8_t*>(c->v_pages), unit_page, unit_kvh,
      wave_start, c->num_pages, (int32_t)c->n_kv_heads, sink);
  return hip_check("load probe launch");
}
