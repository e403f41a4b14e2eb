// The reference engine's per-token loop driven from compiled C++ through the
// C ABI alone (include/lnskv.h): no Python in between, as a native engine
// would call it.  One sequence, Hq 32 / Hkv 8 / head_dim 128 on Q8A pages (the
// reference's paged type), a 40-token sliding window on a pool of
// lnskv_window_pages(40) pages, so that pages are evicted and reused:
//   per position pos: lnskv_step_pages (evict, then ensure: engine.rs:
//   2960-2990 with the exhaustion fixed), lnskv_block_tables_upload
//   (upload_block_table, engine.rs:2992-3005), lnskv_dispatch_attention_paged
//   (dispatch_attention_paged_q8a, lns-metal/src/lib.rs:1046-1094) with
//   p_start = lnskv_kv_p_start(pos, 40) (engine.rs:3007-3013).
// Checked against a host restatement: the stored codes and scales bit for bit
// (lns_decode.metal:547-593: absmax / 127, round half away from zero, clamp
// 127; read back with lnskv_gather) and every output row within 1e-5 of an
// f64 softmax over the dequantized window.  Prints one line and exits 0 when
// every check holds, 1 otherwise.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

#include "lnskv.h"

namespace {

constexpr int kHq = 32, kHkv = 8, kD = 128, kWindow = 40, kPositions = 150;

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
    if (!ok(lnskv_block_tables_upload(bt, table_dev, nullptr), "lnskv_block_tables_upload")) return 1;
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
    // the window's pages only, never more than lnskv_window_pages(window)
    const uint32_t* row = lnskv_block_tables_host(bt);
    const int live = (int)std::count_if(row, row + max_pages, [](uint32_t p) { return p != LNSKV_NO_PAGE; });
    if (live > lnskv_window_pages(kWindow)) {
      std::printf("engine_loop FAILED: %d live pages at pos %d\n", live, pos);
      return 1;
    }
  }
  std::printf("engine_loop ok: %d positions, window %d on a %u-page pool, max row error %.3e\n", kPositions,
              kWindow, c.num_pages, worst);
  lnskv_block_tables_destroy(bt);
  lnskv_page_pool_destroy(pool);
  for (void* p : {(void*)table_dev, (void*)q_dev, (void*)k_dev, (void*)v_dev, (void*)out_dev, (void*)kc_dev,
                  (void*)vc_dev, (void*)ks_dev, (void*)vs_dev})
    (void)hipFree(p);
  return ok(lnskv_pages_free(&c), "lnskv_pages_free") ? 0 : 1;
}

}  // namespace

int main() { return run(); }
