// Host-side page bookkeeping of liblnskv: the PagePool free list, batched block
// tables and the engine's page helpers, plus the error channel shared by every
// entry point.  Nothing here touches the GPU except lnskv_block_tables_upload.
//
// Mirrors lns-inference/src/engine.rs:
//   PagePool                      :20-44
//   kv_block_tables (u32::MAX)    :65
//   ensure_kv_page                :2960-2974
//   evict_kv_pages                :2976-2990
//   upload_block_table            :2992-3005
//   kv_p_start                    :3007-3013
//   clear_kv_cache (tables part)  :2923-2930
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <deque>
#include <limits>
#include <new>
#include <vector>

#include "lnskv_internal.h"

namespace lnskv {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int check_geometry(const lnskv_pages* c) {
  if (!c) return fail(LNSKV_ERR_INVALID, "page descriptor is NULL");
  if (c->dtype != LNSKV_DTYPE_F32 && c->dtype != LNSKV_DTYPE_F16 && c->dtype != LNSKV_DTYPE_Q8A)
    return fail(LNSKV_ERR_INVALID, "unknown dtype %d", c->dtype);
  if (c->head_dim != 64 && c->head_dim != 128 && c->head_dim != 256)
    return fail(LNSKV_ERR_UNSUPPORTED, "head_dim %u not supported (64, 128, 256)", c->head_dim);
  if (c->n_kv_heads == 0 || c->n_kv_heads > 256)
    return fail(LNSKV_ERR_INVALID, "n_kv_heads %u out of range [1, 256]", c->n_kv_heads);
  if (c->num_pages == 0 || c->num_pages >= (1u << 27))
    return fail(LNSKV_ERR_INVALID, "num_pages %u out of range [1, 2^27)", c->num_pages);
  return LNSKV_OK;
}

int check_pages(const lnskv_pages* c) {
  if (int rc = check_geometry(c)) return rc;
  if (!c->k_pages || !c->v_pages) return fail(LNSKV_ERR_INVALID, "K/V page pools are NULL");
  if (c->dtype == LNSKV_DTYPE_Q8A && (!c->k_scales || !c->v_scales))
    return fail(LNSKV_ERR_INVALID, "Q8A pools need k_scales and v_scales");
  return LNSKV_OK;
}

// f32 -> f16 bits, round to nearest even (overflow to infinity, NaN kept
// quiet), and back; host side of the Q4L repack.
uint16_t f32_to_f16_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // 65520 and up round to infinity
  if (ax < 0x38800000u) {                                    // below 2^-14: f16 subnormal or zero
    // units of 2^-24: shift the 24-bit significand right, rounding to even
    if (ax < 0x33000000u) return (uint16_t)sign;  // below 2^-25: rounds to zero (2^-25 itself ties to 0)
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e;  // value = m * 2^(e - 150) = m >> shift units of 2^-24
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((((ax >> 23) & 0xFFu) - 112u) << 10) | ((ax >> 13) & 0x3FFu);
  const uint32_t rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

float f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  float v;
  if (e == 0)
    v = std::ldexp((float)m, -24);
  else if (e == 31)
    v = m ? std::numeric_limits<float>::quiet_NaN() : std::numeric_limits<float>::infinity();
  else
    v = std::ldexp((float)(m | 0x400u), (int)e - 25);
  uint32_t bits;
  std::memcpy(&bits, &v, 4);
  bits |= sign;
  std::memcpy(&v, &bits, 4);
  return v;
}

}  // namespace lnskv

using lnskv::fail;

// ---------------------------------------------------------------------------
// PagePool (engine.rs:20-44).  The free list is a FIFO deque exactly as the
// reference's VecDeque<u32>: new/reset hold 0..capacity in order, alloc pops
// the front, free pushes the back.  The reference frees unconditionally; here
// a page carries a reference count so that copy-on-write forks can share it,
// and free returns it to the list when the count reaches zero.  With no
// retain calls the observable order is identical to the reference.
struct lnskv_page_pool {
  uint32_t capacity;
  std::deque<uint32_t> free_list;
  std::vector<uint32_t> refs;
};

extern "C" {

const char* lnskv_last_error(void) { return lnskv::g_last_error.c_str(); }
const char* lnskv_version(void) { return "lnskv 0.1.0 (gfx950)"; }

size_t lnskv_page_bytes(const lnskv_pages* c) {
  if (!c) return 0;
  return (size_t)LNSKV_PAGE_SIZE * c->n_kv_heads * c->head_dim * lnskv::dtype_bytes(c->dtype);
}

int lnskv_page_pool_create(uint32_t capacity, lnskv_page_pool** out) {
  if (!out) return fail(LNSKV_ERR_INVALID, "out is NULL");
  *out = nullptr;
  auto* p = new (std::nothrow) lnskv_page_pool();
  if (!p) return fail(LNSKV_ERR_NOMEM, "page pool allocation failed");
  p->capacity = capacity;
  try {
    p->refs.assign(capacity, 0);
  } catch (...) {
    delete p;
    return fail(LNSKV_ERR_NOMEM, "page pool of %u pages: allocation failed", capacity);
  }
  lnskv_page_pool_reset(p);
  *out = p;
  return LNSKV_OK;
}

void lnskv_page_pool_destroy(lnskv_page_pool* p) { delete p; }

void lnskv_page_pool_reset(lnskv_page_pool* p) {
  if (!p) return;
  p->free_list.clear();
  for (uint32_t i = 0; i < p->capacity; ++i) p->free_list.push_back(i);
  std::fill(p->refs.begin(), p->refs.end(), 0u);
}

int lnskv_page_pool_alloc(lnskv_page_pool* p, uint32_t* page_out) {
  if (!p || !page_out) return fail(LNSKV_ERR_INVALID, "pool or page_out is NULL");
  if (p->free_list.empty()) return fail(LNSKV_ERR_POOL_EXHAUSTED, "KV page pool exhausted");
  const uint32_t id = p->free_list.front();
  p->free_list.pop_front();
  p->refs[id] = 1;
  *page_out = id;
  return LNSKV_OK;
}

int lnskv_page_pool_free(lnskv_page_pool* p, uint32_t page) {
  if (!p) return fail(LNSKV_ERR_INVALID, "pool is NULL");
  if (page >= p->capacity) return fail(LNSKV_ERR_INVALID, "page %u outside pool of %u", page, p->capacity);
  if (p->refs[page] == 0) return fail(LNSKV_ERR_INVALID, "page %u is not allocated", page);
  if (--p->refs[page] == 0) p->free_list.push_back(page);
  return LNSKV_OK;
}

int lnskv_page_pool_retain(lnskv_page_pool* p, uint32_t page) {
  if (!p) return fail(LNSKV_ERR_INVALID, "pool is NULL");
  if (page >= p->capacity) return fail(LNSKV_ERR_INVALID, "page %u outside pool of %u", page, p->capacity);
  if (p->refs[page] == 0) return fail(LNSKV_ERR_INVALID, "page %u is not allocated", page);
  ++p->refs[page];
  return LNSKV_OK;
}

uint32_t lnskv_page_pool_num_free(const lnskv_page_pool* p) {
  return p ? (uint32_t)p->free_list.size() : 0;
}
uint32_t lnskv_page_pool_capacity(const lnskv_page_pool* p) { return p ? p->capacity : 0; }
uint32_t lnskv_page_pool_refcount(const lnskv_page_pool* p, uint32_t page) {
  return (p && page < p->capacity) ? p->refs[page] : 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Batched block tables: the reference keeps one growable Vec<u32> per layer for
// its single sequence (engine.rs:65) and copies it into a fixed 2 KB buffer
// (engine.rs:735-736).  Here a layer holds n_seq fixed-capacity rows, so a
// position past the row is an error instead of an overflow of the device copy.
struct lnskv_block_tables {
  int32_t n_seq;
  int32_t max_pages;
  std::vector<uint32_t> table;  // [n_seq][max_pages]
  std::vector<int32_t> len;     // logical pages in use per row
  // What lnskv_block_tables_sync still has to write: every entry (`all`), or
  // the flat indices in `changed` (each once, flagged in `mark`).
  bool all = true;
  std::vector<uint32_t> changed;
  std::vector<uint8_t> mark;
};

namespace {
bool row_ok(const lnskv_block_tables* t, int32_t seq) {
  return t && seq >= 0 && seq < t->n_seq;
}

// Sets entry lp of row seq, noting it for the next sync when its value changes.
void set_entry(lnskv_block_tables* t, int32_t seq, int32_t lp, uint32_t v) {
  const size_t i = (size_t)seq * (size_t)t->max_pages + (size_t)lp;
  if (t->table[i] == v) return;
  t->table[i] = v;
  if (!t->all && !t->mark[i]) {
    t->mark[i] = 1;
    t->changed.push_back((uint32_t)i);
  }
}
}  // namespace

extern "C" {

int lnskv_block_tables_create(int32_t n_seq, int32_t max_pages, lnskv_block_tables** out) {
  if (!out) return fail(LNSKV_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (n_seq <= 0 || max_pages <= 0)
    return fail(LNSKV_ERR_INVALID, "n_seq %d and max_pages %d must be positive", n_seq, max_pages);
  auto* t = new (std::nothrow) lnskv_block_tables();
  if (!t) return fail(LNSKV_ERR_NOMEM, "block table allocation failed");
  t->n_seq = n_seq;
  t->max_pages = max_pages;
  try {
    t->table.assign((size_t)n_seq * (size_t)max_pages, LNSKV_NO_PAGE);
    t->len.assign((size_t)n_seq, 0);
    t->mark.assign(t->table.size(), 0);
  } catch (...) {
    delete t;
    return fail(LNSKV_ERR_NOMEM, "block tables %d x %d: allocation failed", n_seq, max_pages);
  }
  *out = t;
  return LNSKV_OK;
}

void lnskv_block_tables_destroy(lnskv_block_tables* t) { delete t; }

const uint32_t* lnskv_block_tables_host(const lnskv_block_tables* t) {
  return t ? t->table.data() : nullptr;
}
int32_t lnskv_block_tables_stride(const lnskv_block_tables* t) { return t ? t->max_pages : 0; }
int32_t lnskv_block_tables_len(const lnskv_block_tables* t, int32_t seq) {
  return row_ok(t, seq) ? t->len[(size_t)seq] : 0;
}

void lnskv_block_tables_reset(lnskv_block_tables* t) {
  if (!t) return;
  std::fill(t->table.begin(), t->table.end(), LNSKV_NO_PAGE);
  std::fill(t->len.begin(), t->len.end(), 0);
  for (uint32_t i : t->changed) t->mark[i] = 0;
  t->changed.clear();
  t->all = true;
}

int lnskv_ensure_kv_page(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t layer,
                         int32_t seq, int32_t pos) {
  if (!row_ok(t, seq) || !pool) return fail(LNSKV_ERR_INVALID, "bad table/pool or seq %d", seq);
  if (pos < 0) return fail(LNSKV_ERR_INVALID, "negative position %d", pos);
  const int32_t lp = pos / LNSKV_PAGE_SIZE;
  uint32_t* row = t->table.data() + (size_t)seq * (size_t)t->max_pages;
  int32_t& len = t->len[(size_t)seq];
  if (lp < len && row[lp] != LNSKV_NO_PAGE) return LNSKV_OK;
  if (lp >= t->max_pages)
    return fail(LNSKV_ERR_INVALID, "position %d needs logical page %d; the table row holds %d",
                pos, lp, t->max_pages);
  while (len <= lp) set_entry(t, seq, len++, LNSKV_NO_PAGE);
  uint32_t phys;
  if (lnskv_page_pool_alloc(pool, &phys) != LNSKV_OK)
    return fail(LNSKV_ERR_POOL_EXHAUSTED, "KV page pool exhausted at layer %d (pos=%d)", layer, pos);
  set_entry(t, seq, lp, phys);
  return LNSKV_OK;
}

int32_t lnskv_kv_p_start(int32_t pos, int32_t window) {
  if (window > 0) return pos > window - 1 ? pos - (window - 1) : 0;
  return 0;
}

int lnskv_evict_kv_pages(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t seq, int32_t pos,
                         int32_t window) {
  if (!row_ok(t, seq) || !pool) return fail(LNSKV_ERR_INVALID, "bad table/pool or seq %d", seq);
  if (window <= 0) return LNSKV_OK;
  const int32_t evict_before = lnskv_kv_p_start(pos, window) / LNSKV_PAGE_SIZE;
  uint32_t* row = t->table.data() + (size_t)seq * (size_t)t->max_pages;
  const int32_t n = std::min(evict_before, t->len[(size_t)seq]);
  for (int32_t lp = 0; lp < n; ++lp) {
    if (row[lp] != LNSKV_NO_PAGE) {
      if (int rc = lnskv_page_pool_free(pool, row[lp])) return rc;
      set_entry(t, seq, lp, LNSKV_NO_PAGE);
    }
  }
  return LNSKV_OK;
}

// The engine sizes a sliding-window layer's pool at ceil(w/16) pages
// (engine.rs:726-730) and calls ensure_kv_page before evict_kv_pages
// (engine.rs:1601-1603, 3231-3232).  A window whose start is not page-aligned
// spans one page more than that, so the pool runs dry at the first position
// where it does.  lnskv_step_pages evicts first and then ensures, and
// lnskv_window_pages gives the page count that order needs.
int32_t lnskv_window_pages(int32_t window) {
  if (window <= 0) return 0;
  // [p, p + w - 1] touches pages p/16 .. (p + w - 1)/16: at most (w - 1 + 15)/16 + 1
  return (int32_t)(((int64_t)window + LNSKV_PAGE_SIZE - 2) / LNSKV_PAGE_SIZE + 1);
}

int lnskv_step_pages(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t layer, int32_t seq, int32_t pos,
                     int32_t window) {
  if (int rc = lnskv_evict_kv_pages(t, pool, seq, pos, window)) return rc;
  return lnskv_ensure_kv_page(t, pool, layer, seq, pos);
}

int lnskv_free_sequence(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t seq) {
  if (!row_ok(t, seq) || !pool) return fail(LNSKV_ERR_INVALID, "bad table/pool or seq %d", seq);
  uint32_t* row = t->table.data() + (size_t)seq * (size_t)t->max_pages;
  for (int32_t lp = 0; lp < t->len[(size_t)seq]; ++lp) {
    if (row[lp] != LNSKV_NO_PAGE) {
      if (int rc = lnskv_page_pool_free(pool, row[lp])) return rc;
      set_entry(t, seq, lp, LNSKV_NO_PAGE);
    }
  }
  t->len[(size_t)seq] = 0;
  return LNSKV_OK;
}

int lnskv_fork_sequence(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t parent,
                        int32_t child, int32_t n_tok, uint32_t* copy_src, uint32_t* copy_dst,
                        int32_t* n_copy) {
  if (!row_ok(t, parent) || !row_ok(t, child) || !pool || parent == child || !n_copy)
    return fail(LNSKV_ERR_INVALID, "bad fork arguments (parent %d, child %d)", parent, child);
  *n_copy = 0;
  if (t->len[(size_t)child] != 0) return fail(LNSKV_ERR_INVALID, "fork target row %d is not empty", child);
  const int32_t n_pages = (n_tok + LNSKV_PAGE_SIZE - 1) / LNSKV_PAGE_SIZE;
  if (n_tok < 0 || n_pages > t->len[(size_t)parent])
    return fail(LNSKV_ERR_INVALID, "fork of %d tokens exceeds parent row %d", n_tok, parent);
  const uint32_t* prow = t->table.data() + (size_t)parent * (size_t)t->max_pages;
  uint32_t* crow = t->table.data() + (size_t)child * (size_t)t->max_pages;
  const bool partial_tail = (n_tok % LNSKV_PAGE_SIZE) != 0;
  const int32_t n_shared = partial_tail ? n_pages - 1 : n_pages;
  uint32_t fresh = LNSKV_NO_PAGE;
  if (partial_tail) {
    if (prow[n_pages - 1] == LNSKV_NO_PAGE)
      return fail(LNSKV_ERR_INVALID, "parent row %d has no page at its tail", parent);
    if (lnskv_page_pool_alloc(pool, &fresh) != LNSKV_OK)
      return fail(LNSKV_ERR_POOL_EXHAUSTED, "KV page pool exhausted forking row %d", parent);
    if (!copy_src || !copy_dst) {
      lnskv_page_pool_free(pool, fresh);
      return fail(LNSKV_ERR_INVALID, "copy_src/copy_dst are NULL");
    }
  }
  for (int32_t lp = 0; lp < n_shared; ++lp) {
    if (prow[lp] != LNSKV_NO_PAGE) lnskv_page_pool_retain(pool, prow[lp]);
    set_entry(t, child, lp, prow[lp]);
  }
  if (partial_tail) {
    set_entry(t, child, n_pages - 1, fresh);
    *copy_src = prow[n_pages - 1];
    *copy_dst = fresh;
    *n_copy = 1;
  }
  t->len[(size_t)child] = n_pages;
  return LNSKV_OK;
}

int lnskv_block_tables_upload(const lnskv_block_tables* t, uint32_t* dst_dev, lnskv_stream_t stream) {
  if (!t || !dst_dev) return fail(LNSKV_ERR_INVALID, "table or destination is NULL");
  const size_t bytes = t->table.size() * sizeof(uint32_t);
  hipError_t e = hipMemcpyAsync(dst_dev, t->table.data(), bytes, hipMemcpyHostToDevice,
                                (hipStream_t)stream);
  if (e != hipSuccess) return fail(LNSKV_ERR_HIP, "block table upload: %s", hipGetErrorString(e));
  return LNSKV_OK;
}

int lnskv_block_tables_sync(lnskv_block_tables* t, uint32_t* dst_dev, lnskv_stream_t stream) {
  if (!t || !dst_dev) return fail(LNSKV_ERR_INVALID, "table or destination is NULL");
  const hipStream_t st = (hipStream_t)stream;
  const size_t n = t->changed.size();
  if (t->all) {
    hipError_t e = hipMemcpyAsync(dst_dev, t->table.data(), t->table.size() * sizeof(uint32_t),
                                  hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return fail(LNSKV_ERR_HIP, "block table upload: %s", hipGetErrorString(e));
  } else if (n == 0) {
    return LNSKV_OK;
  } else if (n <= LNSKV_TABLE_PATCH_MAX) {
    uint32_t val[LNSKV_TABLE_PATCH_MAX];
    for (size_t j = 0; j < n; ++j) val[j] = t->table[t->changed[j]];
    if (int rc = lnskv::table_patch(dst_dev, (int)n, t->changed.data(), val, stream)) return rc;
  } else {
    const auto mm = std::minmax_element(t->changed.begin(), t->changed.end());
    const size_t lo = *mm.first, hi = *mm.second;
    hipError_t e = hipMemcpyAsync(dst_dev + lo, t->table.data() + lo, (hi - lo + 1) * sizeof(uint32_t),
                                  hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return fail(LNSKV_ERR_HIP, "block table upload: %s", hipGetErrorString(e));
  }
  for (uint32_t i : t->changed) t->mark[i] = 0;
  t->changed.clear();
  t->all = false;
  return LNSKV_OK;
}

int lnskv_block_table_patch(uint32_t* dst_dev, int32_t n, const uint32_t* idx, const uint32_t* val,
                            lnskv_stream_t stream) {
  if (!dst_dev || !idx || !val) return fail(LNSKV_ERR_INVALID, "destination, indices and values must be non-null");
  return lnskv::table_patch(dst_dev, n, idx, val, stream);
}

int64_t lnskv_block_tables_changed(const lnskv_block_tables* t) {
  if (!t) return 0;
  return t->all ? (int64_t)t->table.size() : (int64_t)t->changed.size();
}

// RoPE tables (engine.rs:826-833 and 139-195), host only.
int32_t lnskv_rope_dim(int32_t head_dim, float partial_rotary_factor) {
  const int32_t rot = (int32_t)std::lround((double)((float)head_dim * partial_rotary_factor));
  return rot >= 2 && rot < head_dim ? rot : head_dim;
}

int lnskv_rope_inv_freqs(int32_t rotary_dim, float theta, int32_t mode, const float* params, float* out) {
  lnskv::clear_error();
  if (rotary_dim < 2 || rotary_dim % 2 != 0) return fail(LNSKV_ERR_INVALID, "rotary_dim %d must be even and >= 2", rotary_dim);
  if (!out) return fail(LNSKV_ERR_INVALID, "output is NULL");
  if (mode < LNSKV_ROPE_DEFAULT || mode > LNSKV_ROPE_YARN) return fail(LNSKV_ERR_INVALID, "rope mode %d", mode);
  const int n_params = mode == LNSKV_ROPE_DEFAULT || mode == LNSKV_ROPE_LINEAR ? 1 : 4;
  if (!params) return fail(LNSKV_ERR_INVALID, "rope mode %d needs %d parameters", mode, n_params);
  const float two_pi = 6.28318530717958647692f;
  for (int32_t i = 0; i < rotary_dim / 2; ++i) {
    // f32 throughout, as the reference computes it
    const float base = std::pow(theta, -(2.0f * (float)i) / (float)rotary_dim);
    float f = base;
    if (n_params == 1) {
      f = base / std::max(params[0], 1.0f);
    } else {
      // Llama3 {factor, original_max_pos, low, high}; YaRN {factor, original_max_pos, beta_fast, beta_slow}
      const float factor = params[0], orig = params[1];
      const float low = mode == LNSKV_ROPE_LLAMA3 ? params[2] : params[3];
      const float high = mode == LNSKV_ROPE_LLAMA3 ? params[3] : params[2];
      const float wavelen = two_pi / base;
      if (wavelen < orig / high) {
        f = base;
      } else if (wavelen > orig / low) {
        f = base / factor;
      } else {
        const float smooth = (orig / wavelen - low) / (high - low);
        f = base * ((1.0f - smooth) / factor + smooth);
      }
    }
    out[i] = f;
  }
  return LNSKV_OK;
}

// prepare_tensor's Q4L branch (lns-metal/src/lib.rs:1296-1315): per
// super-block, the 8 effective scales f16(scale_global * 2^(sl - 7)) (round
// to nearest even), then the 128 weight bytes unchanged.
int lnskv_q4l_prepare(const void* disk_blocks, size_t disk_bytes, int32_t rows, int32_t cols, void* out_blocks) {
  lnskv::clear_error();
  if (!disk_blocks || !out_blocks) return fail(LNSKV_ERR_INVALID, "disk and output blocks must be non-null");
  if (rows <= 0 || cols <= 0) return fail(LNSKV_ERR_INVALID, "rows %d and cols %d must be positive", rows, cols);
  const size_t n_blocks = (size_t)rows * (size_t)((cols + 255) / 256);
  if (disk_bytes < n_blocks * LNSKV_Q4L_DISK_BYTES)
    return fail(LNSKV_ERR_INVALID, "%zu bytes of Q4L blocks, %zu needed for %d x %d", disk_bytes,
                n_blocks * LNSKV_Q4L_DISK_BYTES, rows, cols);
  const uint8_t* src = static_cast<const uint8_t*>(disk_blocks);
  uint8_t* dst = static_cast<uint8_t*>(out_blocks);
  for (size_t b = 0; b < n_blocks; ++b, src += LNSKV_Q4L_DISK_BYTES, dst += LNSKV_Q4L_DEVICE_BYTES) {
    const float g = lnskv::f16_bits_to_f32((uint16_t)(src[0] | (src[1] << 8)));
    for (int i = 0; i < 8; ++i) {
      const int sl = (src[2 + i / 2] >> ((i % 2) * 4)) & 0xF;
      const uint16_t e = lnskv::f32_to_f16_bits(g * std::ldexp(1.0f, sl - 7));
      dst[2 * i] = (uint8_t)(e & 0xFF);
      dst[2 * i + 1] = (uint8_t)(e >> 8);
    }
    std::memcpy(dst + 16, src + 6, 128);
  }
  return LNSKV_OK;
}

}  // extern "C"
