// The reference engine's per-token loop driven from compiled C++ through the
// C ABI alone (include/lnskv.h): no Python in between, as a native engine
// would call it.  One sequence, Hq 32 / Hkv 8 / head_dim 128 on Q8A pages (the
// reference's paged type), a 40-token sliding window on a pool of
// lnskv_window_pages(40) pages, so that pages are evicted and reused:
//   per position pos: lnskv_step_pages (evict, then ensure: engine.rs:
//   2960-2990 with the exhaustion fixed), lnskv_block_tables_sync
//   (upload_block_table, engine.rs:2992-3005, writing only the entries that
//   changed: a patch when a page is mapped or evicted, nothing on the other
//   positions), lnskv_dispatch_attention_paged
//   (dispatch_attention_paged_q8a, lns-metal/src/lib.rs:1046-1094) with
//   p_start = lnskv_kv_p_start(pos, 40) (engine.rs:3007-3013), then the
//   o_proj: lnskv_q4l_gemv_accumulate adds W_o attn_out to the residual x
//   (gemv_accumulate_multirow_enc, engine.rs:3433-3446) over a 4096 x 4096
//   Q4_L matrix repacked once by lnskv_q4l_prepare (prepare_tensor,
//   lns-metal/src/lib.rs:1255-1320), its workspace zeroed once.
// Checked against a host restatement: the stored codes and scales bit for bit
// (lns_decode.metal:547-593: absmax / 127, round half away from zero, clamp
// 127; read back with lnskv_gather), every output row within 1e-5 of an f64
// softmax over the dequantized window, and at every tenth position W_o times
// that position's output within 2e-6 of sum |w x| of an f64 product over the
// decoded weights (the weight of nibble i of a device block: sign bit 3,
// magnitude m = bits 0-2, zero for m = 0, else the sub-block's f16 scale times
// 2^(m - 5)).  Prints one line and exits 0 when every check holds, 1
// otherwise.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

#include "lnskv.h"

namespace {

constexpr int kHq = 32, kHkv = 8, kD = 128, kWindow = 40, kPositions = 150;
constexpr int kDim = kHq * kD;         // W_o: kDim x kDim (model dim = Hq * head_dim)
constexpr int kBpr = kDim / 256;       // Q4_L blocks per row
constexpr int kOprojCheckEvery = 10;

// SplitMix64 -> values in [-2, 2)
struct Rng {
  uint64_t s;
  float next() {
    s += 0x9E3779B97F4A7C15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(z >> 40) / (float)(1u << 24) * 4.0f - 2.0f;
  }
};

// One kv head's row as the reference's kernel quantizes it.
void quantize(const float* x, int8_t* codes, float* scale) {
  float amax = 0.0f;
  for (int i = 0; i < kD; ++i) amax = std::max(amax, std::fabs(x[i]));
  const float sc = amax == 0.0f ? 1.0f : amax / 127.0f;
  for (int i = 0; i < kD; ++i) {
    const float r = std::round(x[i] / sc);
    codes[i] = (int8_t)std::max(-127.0f, std::min(127.0f, r));
  }
  *scale = sc;
}

// f16 bits -> float (normal numbers, subnormals, zero)
float half_to_float(uint16_t h) {
  const int e = (h >> 10) & 31, m = h & 1023;
  const float v = e == 0 ? std::ldexp((float)m, -24) : std::ldexp((float)(m | 1024), e - 25);
  return (h >> 15) ? -v : v;
}

// The weights of a rows x cols device-block matrix, [row][col].
std::vector<float> decode_q4l(const std::vector<uint8_t>& blocks, int rows, int cols) {
  const int bpr = cols / 256;
  std::vector<float> w((size_t)rows * cols);
  for (int r = 0; r < rows; ++r)
    for (int b = 0; b < bpr; ++b) {
      const uint8_t* blk = &blocks[((size_t)r * bpr + b) * LNSKV_Q4L_DEVICE_BYTES];
      for (int i = 0; i < 256; ++i) {
        const uint8_t byte = blk[16 + i / 2];
        const int nib = (i & 1) ? byte >> 4 : byte & 15, m = nib & 7;
        const float sc = half_to_float((uint16_t)(blk[2 * (i / 32)] | (blk[2 * (i / 32) + 1] << 8)));
        const float mag = m == 0 ? 0.0f : sc * std::ldexp(1.0f, m - 5);
        w[(size_t)r * cols + b * 256 + i] = (nib & 8) ? -mag : mag;
      }
    }
  return w;
}

bool ok(int rc, const char* what) {
  if (rc == LNSKV_OK) return true;
  std::printf("engine_loop FAILED: %s: status %d: %s\n", what, rc, lnskv_last_error());
  return false;
}

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::printf("engine_loop FAILED: %s: %s\n", what, hipGetErrorString(e));
  return false;
}

template <class T>
T* dev_alloc(size_t n) {
  void* p = nullptr;
  return hipMalloc(&p, n * sizeof(T)) == hipSuccess ? static_cast<T*>(p) : nullptr;
}

int run() {
  lnskv_pages c{};
  c.num_pages = (uint32_t)lnskv_window_pages(kWindow);
  c.n_kv_heads = kHkv;
  c.head_dim = kD;
  c.dtype = LNSKV_DTYPE_Q8A;
  if (!ok(lnskv_pages_alloc(&c), "lnskv_pages_alloc")) return 1;
  lnskv_page_pool* pool = nullptr;
  lnskv_block_tables* bt = nullptr;
  const int max_pages = kPositions / 16 + 1;
  if (!ok(lnskv_page_pool_create(c.num_pages, &pool), "lnskv_page_pool_create")) return 1;
  if (!ok(lnskv_block_tables_create(1, max_pages, &bt), "lnskv_block_tables_create")) return 1;

  uint32_t* table_dev = dev_alloc<uint32_t>(max_pages);
  float* q_dev = dev_alloc<float>(kHq * kD);
  float* k_dev = dev_alloc<float>(kHkv * kD);
  float* v_dev = dev_alloc<float>(kHkv * kD);
  float* out_dev = dev_alloc<float>(kHq * kD);
  int8_t* kc_dev = dev_alloc<int8_t>(kHkv * kD);
  int8_t* vc_dev = dev_alloc<int8_t>(kHkv * kD);
  float* ks_dev = dev_alloc<float>(kHkv);
  float* vs_dev = dev_alloc<float>(kHkv);
  if (!table_dev || !q_dev || !k_dev || !v_dev || !out_dev || !kc_dev || !vc_dev || !ks_dev || !vs_dev) {
    std::printf("engine_loop FAILED: hipMalloc\n");
    return 1;
  }

  // o_proj weights: random disk super-blocks (scale_global a positive f16 in
  // [2^-12, 2^-2), 8 local-scale nibbles, 256 weight nibbles), repacked once
  Rng wrng{11};
  std::vector<uint8_t> disk((size_t)kDim * kBpr * LNSKV_Q4L_DISK_BYTES);
  for (size_t blk = 0; blk < (size_t)kDim * kBpr; ++blk) {
    uint8_t* d = &disk[blk * LNSKV_Q4L_DISK_BYTES];
    for (int i = 0; i < LNSKV_Q4L_DISK_BYTES; ++i) d[i] = (uint8_t)((wrng.next() + 2.0f) * 64.0f);
    const uint16_t g = (uint16_t)(((3 + (int)((wrng.next() + 2.0f) * 2.5f)) << 10) | (d[1] & 3) << 8 | d[0]);
    d[0] = (uint8_t)(g & 255);
    d[1] = (uint8_t)(g >> 8);
  }
  std::vector<uint8_t> wblocks((size_t)kDim * kBpr * LNSKV_Q4L_DEVICE_BYTES);
  if (!ok(lnskv_q4l_prepare(disk.data(), disk.size(), kDim, kDim, wblocks.data()), "lnskv_q4l_prepare")) return 1;
  const std::vector<float> W = decode_q4l(wblocks, kDim, kDim);
  size_t ws_bytes = 0;
  if (!ok(lnskv_q4l_workspace_size(kDim, 1, &ws_bytes), "lnskv_q4l_workspace_size")) return 1;
  uint8_t* w_dev = dev_alloc<uint8_t>(wblocks.size());
  uint8_t* ws_dev = dev_alloc<uint8_t>(std::max<size_t>(ws_bytes, 16));
  float* x_dev = dev_alloc<float>(kDim);
  float* y_dev = dev_alloc<float>(kDim);
  if (!w_dev || !ws_dev || !x_dev || !y_dev) {
    std::printf("engine_loop FAILED: hipMalloc\n");
    return 1;
  }
  if (!hip_ok(hipMemcpy(w_dev, wblocks.data(), wblocks.size(), hipMemcpyHostToDevice), "W_o upload") ||
      !hip_ok(hipMemset(ws_dev, 0, std::max<size_t>(ws_bytes, 16)), "workspace zero") ||
      !hip_ok(hipMemset(x_dev, 0, kDim * 4), "x zero"))
    return 1;
  std::vector<float> y(kDim);
  double worst_oproj = 0.0;

  // every position's dequantized K and V, [pos][kvh][d]
  std::vector<double> kq((size_t)kPositions * kHkv * kD), vq((size_t)kPositions * kHkv * kD);
  std::vector<float> q(kHq * kD), k(kHkv * kD), v(kHkv * kD), out(kHq * kD);
  std::vector<int8_t> kc(kHkv * kD), vc(kHkv * kD), hk(kD), hv(kD);
  std::vector<float> ks(kHkv), vs(kHkv);
  Rng rng{7};
  const double scale = 1.0 / std::sqrt((double)kD);
  double worst = 0.0;
  for (int pos = 0; pos < kPositions; ++pos) {
    for (auto& x : q) x = rng.next();
    for (auto& x : k) x = rng.next();
    for (auto& x : v) x = rng.next() * 0.5f;
    if (!hip_ok(hipMemcpy(q_dev, q.data(), q.size() * 4, hipMemcpyHostToDevice), "q upload") ||
        !hip_ok(hipMemcpy(k_dev, k.data(), k.size() * 4, hipMemcpyHostToDevice), "k upload") ||
        !hip_ok(hipMemcpy(v_dev, v.data(), v.size() * 4, hipMemcpyHostToDevice), "v upload"))
      return 1;
    if (!ok(lnskv_step_pages(bt, pool, 0, 0, pos, kWindow), "lnskv_step_pages")) return 1;
    if (!ok(lnskv_block_tables_sync(bt, table_dev, nullptr), "lnskv_block_tables_sync")) return 1;
    const int p_start = lnskv_kv_p_start(pos, kWindow);
    if (!ok(lnskv_dispatch_attention_paged(q_dev, k_dev, v_dev, &c, table_dev, out_dev, (uint32_t)pos, kD, kHq,
                                           kHkv, (uint32_t)p_start, nullptr),
            "lnskv_dispatch_attention_paged"))
      return 1;

    // the stored row: codes and scales bit-exact
    if (!ok(lnskv_gather(&c, table_dev, pos, 1, kc_dev, vc_dev, ks_dev, vs_dev, nullptr), "lnskv_gather") ||
        !ok(lnskv_sync(nullptr), "lnskv_sync"))
      return 1;
    if (!hip_ok(hipMemcpy(kc.data(), kc_dev, kc.size(), hipMemcpyDeviceToHost), "codes") ||
        !hip_ok(hipMemcpy(vc.data(), vc_dev, vc.size(), hipMemcpyDeviceToHost), "codes") ||
        !hip_ok(hipMemcpy(ks.data(), ks_dev, ks.size() * 4, hipMemcpyDeviceToHost), "scales") ||
        !hip_ok(hipMemcpy(vs.data(), vs_dev, vs.size() * 4, hipMemcpyDeviceToHost), "scales") ||
        !hip_ok(hipMemcpy(out.data(), out_dev, out.size() * 4, hipMemcpyDeviceToHost), "out"))
      return 1;
    for (int h = 0; h < kHkv; ++h) {
      float sk = 0.0f, sv = 0.0f;
      quantize(&k[h * kD], hk.data(), &sk);
      quantize(&v[h * kD], hv.data(), &sv);
      if (!std::equal(hk.begin(), hk.end(), kc.begin() + h * kD) ||
          !std::equal(hv.begin(), hv.end(), vc.begin() + h * kD) || ks[h] != sk || vs[h] != sv) {
        std::printf("engine_loop FAILED: stored codes or scales differ at pos %d head %d\n", pos, h);
        return 1;
      }
      for (int i = 0; i < kD; ++i) {
        kq[((size_t)pos * kHkv + h) * kD + i] = (double)hk[i] * sk;
        vq[((size_t)pos * kHkv + h) * kD + i] = (double)hv[i] * sv;
      }
    }

    // f64 attention over [p_start, pos]; query head hq reads kv head hq / 4
    for (int hq = 0; hq < kHq; ++hq) {
      const int h = hq / (kHq / kHkv);
      std::vector<double> s;
      for (int t = p_start; t <= pos; ++t) {
        double dot = 0.0;
        for (int i = 0; i < kD; ++i) dot += (double)q[hq * kD + i] * kq[((size_t)t * kHkv + h) * kD + i];
        s.push_back(dot * scale);
      }
      const double m = *std::max_element(s.begin(), s.end());
      double l = 0.0;
      for (auto& x : s) l += (x = std::exp(x - m));
      double rmax = 1e-30, err = 0.0;
      for (int i = 0; i < kD; ++i) {
        double r = 0.0;
        for (int t = p_start; t <= pos; ++t) r += s[t - p_start] * vq[((size_t)t * kHkv + h) * kD + i];
        r /= l;
        rmax = std::max(rmax, std::fabs(r));
        err = std::max(err, std::fabs((double)out[hq * kD + i] - r));
      }
      worst = std::max(worst, err / rmax);
      if (err / rmax >= 1e-5) {
        std::printf("engine_loop FAILED: pos %d head %d row error %.3e\n", pos, hq, err / rmax);
        return 1;
      }
    }
    // o_proj: the residual x += W_o out, as the engine's step does; every
    // tenth position also W_o out alone, checked on the host
    if (!ok(lnskv_q4l_gemv_accumulate(w_dev, out_dev, x_dev, kDim, kDim, 1, kDim, kDim, ws_dev, ws_bytes, nullptr),
            "lnskv_q4l_gemv_accumulate"))
      return 1;
    if (pos % kOprojCheckEvery == 0) {
      if (!hip_ok(hipMemset(y_dev, 0, kDim * 4), "y zero") ||
          !ok(lnskv_q4l_gemv_accumulate(w_dev, out_dev, y_dev, kDim, kDim, 1, kDim, kDim, ws_dev, ws_bytes,
                                        nullptr),
              "lnskv_q4l_gemv_accumulate") ||
          !ok(lnskv_sync(nullptr), "lnskv_sync") ||
          !hip_ok(hipMemcpy(y.data(), y_dev, kDim * 4, hipMemcpyDeviceToHost), "y"))
        return 1;
      for (int r = 0; r < kDim; ++r) {
        double ref = 0.0, mag = 0.0;
        for (int c2 = 0; c2 < kDim; ++c2) {
          const double p = (double)W[(size_t)r * kDim + c2] * out[c2];
          ref += p;
          mag += std::fabs(p);
        }
        const double err = std::fabs((double)y[r] - ref) / (mag + 1e-30);
        worst_oproj = std::max(worst_oproj, err);
        if (err > 2e-6) {
          std::printf("engine_loop FAILED: o_proj at pos %d row %d: error %.3e of sum |w x|\n", pos, r, err);
          return 1;
        }
      }
    }
    // the window's pages only, never more than lnskv_window_pages(window)
    const uint32_t* row = lnskv_block_tables_host(bt);
    const int live = (int)std::count_if(row, row + max_pages, [](uint32_t p) { return p != LNSKV_NO_PAGE; });
    if (live > lnskv_window_pages(kWindow)) {
      std::printf("engine_loop FAILED: %d live pages at pos %d\n", live, pos);
      return 1;
    }
  }
  if (!ok(lnskv_sync(nullptr), "lnskv_sync")) return 1;
  std::printf("engine_loop ok: %d positions, window %d on a %u-page pool, max row error %.3e, o_proj max error "
              "%.3e of sum |w x|\n", kPositions, kWindow, c.num_pages, worst, worst_oproj);
  lnskv_block_tables_destroy(bt);
  lnskv_page_pool_destroy(pool);
  for (void* p : {(void*)table_dev, (void*)q_dev, (void*)k_dev, (void*)v_dev, (void*)out_dev, (void*)kc_dev,
                  (void*)vc_dev, (void*)ks_dev, (void*)vs_dev, (void*)w_dev, (void*)ws_dev, (void*)x_dev,
                  (void*)y_dev})
    (void)hipFree(p);
  return ok(lnskv_pages_free(&c), "lnskv_pages_free") ? 0 : 1;
}

}  // namespace

int main() { return run(); }
