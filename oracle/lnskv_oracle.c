/*
 * lnskv_oracle.c — CPU restatement of lns-ml's paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP library, never part of it.
 * Build: see oracle/Makefile (gcc -O3 -march=native -fopenmp, no fast-math,
 * -ffp-contract=off so every a*b+c rounds twice, as written).
 *
 * Pinning (what fixes each function independently of this file):
 *   orc_f32_to_f16      exhaustive sweep of all 2^32 f32 patterns against the
 *                       x86 F16C converter (orc_f16_check_range) and numpy
 *   orc_q8a_quantize    closed forms: zero head -> scale 1, q 0; amax element
 *                       -> +-127; ties round half away from zero; brute force
 *   orc_pool_*          FIFO closed forms (engine.rs:22-44)
 *   orc_append/gather/copy  identities: gather(append(x)) == cvt(x), copy then
 *                       gather equals the source, untouched pages unchanged
 *   orc_decode_*        f64 brute force vs closed forms (one token -> v, equal
 *                       keys -> mean(V), dominant score -> V_argmax), numpy
 *                       softmax on small cases, split-K == no split
 */
#include "lnskv_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* f32 -> f16, roundTiesToEven.  The reference's f16 cache write is the Metal
 * cast `(half)k_in[...]` (lns_decode.metal:284-287), an RNE conversion. */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {                       /* inf / nan */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* quiet NaN */
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
  if (ax >= 0x38800000u) {                       /* normal f16 range */
    uint32_t t = ax - (112u << 23);              /* rebias 127 -> 15 */
    t += 0x0fffu + ((t >> 13) & 1u);             /* round half to even */
    return (uint16_t)(sign | (t >> 13));
  }
  /* |f| < 2^-14: f16 subnormal, unit 2^-24 */
  const uint32_t e = ax >> 23;
  if (e < 102u) return (uint16_t)sign;           /* < 2^-25: rounds to zero */
  const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
  const uint32_t shift = 126u - e;               /* 14..24 */
  uint32_t qv = m >> shift;
  const uint32_t rem = m & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (qv & 1u))) qv++;
  return (uint16_t)(sign | qv);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  uint32_t x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else {                                     /* subnormal: m * 2^-24 */
      float v = (float)m * 5.9604644775390625e-08f;
      memcpy(&x, &v, 4);
      x |= sign;
    }
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e + 112u) << 23) | (m << 13);
  }
  float out;
  memcpy(&out, &x, 4);
  return out;
}

__attribute__((target("f16c"))) static uint16_t f16c_convert(float f) {
  return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
}

uint64_t orc_f16_check_range(uint64_t lo, uint64_t hi, int n_threads) {
  uint64_t bad = 0;
  if (n_threads < 1) n_threads = 1;
#pragma omp parallel for reduction(+ : bad) schedule(static) num_threads(n_threads)
  for (int64_t i = (int64_t)lo; i < (int64_t)hi; ++i) {
    uint32_t bits = (uint32_t)i;
    float f;
    memcpy(&f, &bits, 4);
    if (orc_f32_to_f16(f) != f16c_convert(f)) bad++;
  }
  return bad;
}

void orc_f32_to_f16_array(const float* x, size_t n, uint16_t* out, int n_threads) {
  if (n_threads < 1) n_threads = 1;
#pragma omp parallel for schedule(static) num_threads(n_threads)
  for (int64_t i = 0; i < (int64_t)n; ++i) out[i] = orc_f32_to_f16(x[i]);
}

void orc_f16_of_patterns(uint64_t lo, size_t n, uint16_t* out, int n_threads) {
  if (n_threads < 1) n_threads = 1;
#pragma omp parallel for schedule(static) num_threads(n_threads)
  for (int64_t i = 0; i < (int64_t)n; ++i) {
    const uint32_t bits = (uint32_t)(lo + (uint64_t)i);
    float f;
    memcpy(&f, &bits, 4);
    out[i] = orc_f32_to_f16(f);
  }
}

/* ------------------------------------------------------------------------ */
/* Q8A: per (slot, kv head) absmax scale, lns_decode.metal:547-570 (K) and
 * :572-593 (V): amax = max|x|; sc = amax == 0 ? 1 : amax / 127;
 * q = (char)clamp(round(x / sc), -127, 127) with round = half away from zero. */
void orc_q8a_quantize(const float* x, int d, int8_t* q, float* scale) {
  float amax = 0.0f;
  for (int i = 0; i < d; ++i) amax = fmaxf(amax, fabsf(x[i]));
  const float sc = amax == 0.0f ? 1.0f : amax / 127.0f;
  for (int i = 0; i < d; ++i) {
    float r = roundf(x[i] / sc);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    q[i] = (int8_t)r;
  }
  *scale = sc;
}

/* ------------------------------------------------------------------------ */
/* PagePool, engine.rs:20-44: a FIFO of physical page ids; new(cap) holds
 * 0..cap in order, alloc = pop_front, free_page = push_back, reset refills. */
struct orc_pool {
  uint32_t capacity;
  uint32_t* ring; /* capacity + 1 slots */
  uint32_t head, count;
};

orc_pool* orc_pool_new(uint32_t capacity) {
  orc_pool* p = (orc_pool*)calloc(1, sizeof(orc_pool));
  p->capacity = capacity;
  p->ring = (uint32_t*)malloc(sizeof(uint32_t) * ((size_t)capacity + 1));
  orc_pool_reset(p);
  return p;
}
void orc_pool_delete(orc_pool* p) {
  if (!p) return;
  free(p->ring);
  free(p);
}
void orc_pool_reset(orc_pool* p) {
  for (uint32_t i = 0; i < p->capacity; ++i) p->ring[i] = i;
  p->head = 0;
  p->count = p->capacity;
}
int orc_pool_alloc(orc_pool* p, uint32_t* out) {
  if (p->count == 0) return -1;
  *out = p->ring[p->head];
  p->head = (p->head + 1) % (p->capacity + 1);
  p->count--;
  return 0;
}
void orc_pool_free_page(orc_pool* p, uint32_t idx) {
  /* The reference pushes without checks; a ring of capacity+1 slots holds any
   * sequence of frees of pages that were allocated. */
  p->ring[(p->head + p->count) % (p->capacity + 1)] = idx;
  p->count++;
}
uint32_t orc_pool_num_free(const orc_pool* p) { return p->count; }

/* ensure_kv_page, engine.rs:2960-2974: lp = pos/16; grow the table with
 * u32::MAX; allocate only when the entry is missing. */
int orc_ensure_kv_page(orc_pool* p, uint32_t* bt, int* bt_len, int bt_cap, int pos) {
  const int lp = pos / ORC_PAGE_SIZE;
  if (lp < *bt_len && bt[lp] != ORC_NO_PAGE) return 0;
  if (lp >= bt_cap) return -2;
  while (*bt_len <= lp) bt[(*bt_len)++] = ORC_NO_PAGE;
  uint32_t phys;
  if (orc_pool_alloc(p, &phys) != 0) return -1;
  bt[lp] = phys;
  return 0;
}

/* evict_kv_pages, engine.rs:2976-2990: free logical pages [0, p_start/16). */
void orc_evict_kv_pages(orc_pool* p, uint32_t* bt, int bt_len, int pos, int window) {
  if (window == 0) return;
  const int p_start = pos > window - 1 ? pos - (window - 1) : 0;
  const int evict_before = p_start / ORC_PAGE_SIZE;
  const int n = evict_before < bt_len ? evict_before : bt_len;
  for (int lp = 0; lp < n; ++lp) {
    if (bt[lp] != ORC_NO_PAGE) {
      orc_pool_free_page(p, bt[lp]);
      bt[lp] = ORC_NO_PAGE;
    }
  }
}

/* kv_p_start, engine.rs:3007-3013 */
int orc_kv_p_start(int pos, int window) {
  if (window > 0) return pos > window - 1 ? pos - (window - 1) : 0;
  return 0;
}

/* ------------------------------------------------------------------------ */
static size_t elem_size(int dtype) { return dtype == ORC_F32 ? 4 : dtype == ORC_F16 ? 2 : 1; }

static int slot_of(const orc_pages* c, const uint32_t* bt_row, int pos, uint32_t* slot) {
  const uint32_t phys = bt_row[pos / ORC_PAGE_SIZE];
  if (phys == ORC_NO_PAGE || phys >= c->num_pages) return -1;
  *slot = phys * ORC_PAGE_SIZE + (uint32_t)(pos % ORC_PAGE_SIZE);
  return 0;
}

/* Write one head vector x[d] (f32) into slot/head of one pool. */
static void store_head(const orc_pages* c, int which_v, uint32_t slot, int h, const float* x) {
  const int d = (int)c->head_dim;
  const size_t off = ((size_t)slot * c->n_kv_heads + (size_t)h) * (size_t)d;
  void* base = which_v ? c->v_pages : c->k_pages;
  if (c->dtype == ORC_F32) {
    memcpy((float*)base + off, x, sizeof(float) * (size_t)d);      /* f32: plain copy */
  } else if (c->dtype == ORC_F16) {
    uint16_t* dst = (uint16_t*)base + off;
    for (int i = 0; i < d; ++i) dst[i] = orc_f32_to_f16(x[i]);    /* metal:284-287 */
  } else {
    float* sc = which_v ? c->v_scales : c->k_scales;               /* metal:547-593 */
    orc_q8a_quantize(x, d, (int8_t*)base + off, &sc[(size_t)slot * c->n_kv_heads + (size_t)h]);
  }
}

/* Slot math lns_decode.metal:541-545 (write_lp = pos/16, write_off = pos%16,
 * slot = block_table[write_lp]*16 + write_off); batched over tokens. */
int orc_append(const orc_pages* c, const float* k_new, const float* v_new,
               const int32_t* tok_seq, const int32_t* tok_pos, int n_tok,
               const uint32_t* bt, int bt_stride, int n_rows) {
  const int nkv = (int)c->n_kv_heads, d = (int)c->head_dim;
  int skipped = 0;
  for (int t = 0; t < n_tok; ++t) {
    if (tok_seq[t] < 0 || tok_seq[t] >= n_rows) {
      skipped++;
      continue;
    }
    const uint32_t* row = bt + (size_t)tok_seq[t] * (size_t)bt_stride;
    uint32_t slot;
    if (tok_pos[t] < 0 || tok_pos[t] / ORC_PAGE_SIZE >= bt_stride || slot_of(c, row, tok_pos[t], &slot)) {
      skipped++;
      continue;
    }
    for (int h = 0; h < nkv; ++h) {
      store_head(c, 0, slot, h, k_new + ((size_t)t * nkv + h) * d);
      store_head(c, 1, slot, h, v_new + ((size_t)t * nkv + h) * d);
    }
  }
  return skipped;
}

int orc_gather(const orc_pages* c, const uint32_t* bt_row, int start, int n_tok,
               void* k_out, void* v_out, float* ks_out, float* vs_out) {
  const size_t es = elem_size(c->dtype);
  const size_t row = (size_t)c->n_kv_heads * c->head_dim * es;
  int missing = 0;
  for (int t = 0; t < n_tok; ++t) {
    uint32_t slot;
    if (slot_of(c, bt_row, start + t, &slot)) {
      memset((char*)k_out + (size_t)t * row, 0, row);
      memset((char*)v_out + (size_t)t * row, 0, row);
      missing++;
      continue;
    }
    memcpy((char*)k_out + (size_t)t * row, (const char*)c->k_pages + (size_t)slot * row, row);
    memcpy((char*)v_out + (size_t)t * row, (const char*)c->v_pages + (size_t)slot * row, row);
    if (c->dtype == ORC_Q8A && ks_out && vs_out) {
      memcpy(ks_out + (size_t)t * c->n_kv_heads, c->k_scales + (size_t)slot * c->n_kv_heads,
             sizeof(float) * c->n_kv_heads);
      memcpy(vs_out + (size_t)t * c->n_kv_heads, c->v_scales + (size_t)slot * c->n_kv_heads,
             sizeof(float) * c->n_kv_heads);
    }
  }
  return missing;
}

void orc_page_copy(const orc_pages* c, const uint32_t* src, const uint32_t* dst, int n) {
  const size_t es = elem_size(c->dtype);
  const size_t page = (size_t)ORC_PAGE_SIZE * c->n_kv_heads * c->head_dim * es;
  const size_t spage = (size_t)ORC_PAGE_SIZE * c->n_kv_heads;
  for (int i = 0; i < n; ++i) {
    memcpy((char*)c->k_pages + (size_t)dst[i] * page, (const char*)c->k_pages + (size_t)src[i] * page, page);
    memcpy((char*)c->v_pages + (size_t)dst[i] * page, (const char*)c->v_pages + (size_t)src[i] * page, page);
    if (c->dtype == ORC_Q8A) {
      memcpy(c->k_scales + (size_t)dst[i] * spage, c->k_scales + (size_t)src[i] * spage, sizeof(float) * spage);
      memcpy(c->v_scales + (size_t)dst[i] * spage, c->v_scales + (size_t)src[i] * spage, sizeof(float) * spage);
    }
  }
}

double orc_stored_value(const orc_pages* c, int which_v, uint32_t slot, int h, int i) {
  const size_t off = ((size_t)slot * c->n_kv_heads + (size_t)h) * c->head_dim + (size_t)i;
  const void* base = which_v ? c->v_pages : c->k_pages;
  if (c->dtype == ORC_F32) return (double)((const float*)base)[off];
  if (c->dtype == ORC_F16) return (double)orc_f16_to_f32(((const uint16_t*)base)[off]);
  const float* sc = which_v ? c->v_scales : c->k_scales;
  return (double)((const int8_t*)base)[off] * (double)sc[(size_t)slot * c->n_kv_heads + (size_t)h];
}

/* ------------------------------------------------------------------------ */
/* Reference-order scan for query heads [h0, h0+nh) sharing kv head kvh:
 * lns_decode.metal:595-645.  m = -1e38, l = 0, acc = 0; per token p in the
 * window: dot = sum q_i*k_i; s = dot*scale; m' = max(m,s); alpha = exp(m-m');
 * beta = exp(s-m'); acc = alpha*acc + beta*v (Q8A: beta*vs*v8, :631-634);
 * l = alpha*l + beta; out = acc * (1/l).  Metal's simd_sum order is not
 * observable here; the dot is summed in index order. */
static void refscan_group(const orc_pages* c, const float* q, float* out, const uint32_t* bt_row,
                          int p0, int p1, int kvh, int h0, int nh, float scale, float* acc) {
  const int d = (int)c->head_dim, nkv = (int)c->n_kv_heads;
  for (int hh = 0; hh < nh; ++hh) {
    const int h = h0 + hh;
    const float* qh = q + (size_t)h * d;
    float m = -1e38f, l = 0.0f;
    for (int i = 0; i < d; ++i) acc[i] = 0.0f;
    for (int p = p0; p < p1; ++p) {
      uint32_t slot;
      if (slot_of(c, bt_row, p, &slot)) continue;
      const size_t off = ((size_t)slot * nkv + kvh) * d;
      float dot = 0.0f;
      float vs = 1.0f;
      if (c->dtype == ORC_F32) {
        const float* kh = (const float*)c->k_pages + off;
        for (int i = 0; i < d; ++i) dot += qh[i] * kh[i];
      } else if (c->dtype == ORC_F16) {
        const uint16_t* kh = (const uint16_t*)c->k_pages + off;
        for (int i = 0; i < d; ++i) dot += qh[i] * orc_f16_to_f32(kh[i]);
      } else {
        const int8_t* kh = (const int8_t*)c->k_pages + off;
        const float ks = c->k_scales[(size_t)slot * nkv + kvh];
        for (int i = 0; i < d; ++i) dot += qh[i] * ((float)kh[i] * ks);
        vs = c->v_scales[(size_t)slot * nkv + kvh];
      }
      const float score = dot * scale;
      const float m_new = fmaxf(m, score);
      const float alpha = expf(m - m_new);
      const float beta = expf(score - m_new);
      if (c->dtype == ORC_F32) {
        const float* vh = (const float*)c->v_pages + off;
        for (int i = 0; i < d; ++i) acc[i] = alpha * acc[i] + beta * vh[i];
      } else if (c->dtype == ORC_F16) {
        const uint16_t* vh = (const uint16_t*)c->v_pages + off;
        for (int i = 0; i < d; ++i) acc[i] = alpha * acc[i] + beta * orc_f16_to_f32(vh[i]);
      } else {
        const int8_t* vh = (const int8_t*)c->v_pages + off;
        const float beta_vs = beta * vs;
        for (int i = 0; i < d; ++i) acc[i] = alpha * acc[i] + beta_vs * (float)vh[i];
      }
      m = m_new;
      l = alpha * l + beta;
    }
    float* oh = out + (size_t)h * d;
    if (l > 0.0f) {
      const float l_inv = 1.0f / l;
      for (int i = 0; i < d; ++i) oh[i] = acc[i] * l_inv;
    } else {
      for (int i = 0; i < d; ++i) oh[i] = 0.0f; /* empty window */
    }
  }
}

void orc_decode_refscan(const orc_pages* c, const float* q, float* out,
                        const uint32_t* bt, int bt_stride, const int32_t* kv_len,
                        const int32_t* p_start, int n_seq, int n_heads, float scale,
                        int n_threads) {
  const int nkv = (int)c->n_kv_heads, d = (int)c->head_dim, rep = n_heads / nkv;
  if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(dynamic, 1)
    for (int w = 0; w < n_seq * nkv; ++w) {
      const int s = w / nkv, kvh = w % nkv;
      const int p0 = p_start ? p_start[s] : 0;
      refscan_group(c, q + (size_t)s * n_heads * d, out + (size_t)s * n_heads * d,
                    bt + (size_t)s * bt_stride, p0, kv_len[s], kvh, kvh * rep, rep, scale, acc);
    }
    free(acc);
  }
}

void orc_append_decode_refscan(const orc_pages* c, const float* q, const float* k_new,
                               const float* v_new, float* out, const uint32_t* bt,
                               int bt_stride, const int32_t* kv_len, const int32_t* p_start,
                               int n_seq, int n_heads, float scale, int n_threads) {
  const int nkv = (int)c->n_kv_heads, d = (int)c->head_dim, rep = n_heads / nkv;
  if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
  {
    float* acc = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for schedule(dynamic, 1)
    for (int w = 0; w < n_seq * nkv; ++w) {
      const int s = w / nkv, kvh = w % nkv;
      const uint32_t* row = bt + (size_t)s * bt_stride;
      uint32_t slot;
      /* engine.rs:3231-3233 then lns_decode.metal:541-593: append first */
      if (kv_len[s] > 0 && slot_of(c, row, kv_len[s] - 1, &slot) == 0) {
        store_head(c, 0, slot, kvh, k_new + ((size_t)s * nkv + kvh) * d);
        store_head(c, 1, slot, kvh, v_new + ((size_t)s * nkv + kvh) * d);
      }
      const int p0 = p_start ? p_start[s] : 0;
      refscan_group(c, q + (size_t)s * n_heads * d, out + (size_t)s * n_heads * d, row, p0,
                    kv_len[s], kvh, kvh * rep, rep, scale, acc);
    }
    free(acc);
  }
}

/* ------------------------------------------------------------------------ */
/* f64 ground truth: softmax(q.K^T * scale) . V over the exact stored values. */
static void f64_head(const orc_pages* c, const float* qh, double* oh, const uint32_t* bt_row,
                     int p0, int p1, int kvh, double scale, double* sc_buf) {
  const int d = (int)c->head_dim;
  double mx = -INFINITY;
  int n = 0;
  for (int p = p0; p < p1; ++p) {
    uint32_t slot;
    if (slot_of(c, bt_row, p, &slot)) { sc_buf[p - p0] = NAN; continue; }
    double dot = 0.0;
    for (int i = 0; i < d; ++i) dot += (double)qh[i] * orc_stored_value(c, 0, slot, kvh, i);
    sc_buf[p - p0] = dot * scale;
    if (sc_buf[p - p0] > mx) mx = sc_buf[p - p0];
    n++;
  }
  for (int i = 0; i < d; ++i) oh[i] = 0.0;
  if (n == 0) return;
  double den = 0.0;
  for (int p = p0; p < p1; ++p) {
    if (isnan(sc_buf[p - p0])) continue;
    uint32_t slot = 0;
    slot_of(c, bt_row, p, &slot);
    const double w = exp(sc_buf[p - p0] - mx);
    den += w;
    for (int i = 0; i < d; ++i) oh[i] += w * orc_stored_value(c, 1, slot, kvh, i);
  }
  for (int i = 0; i < d; ++i) oh[i] /= den;
}

void orc_decode_f64(const orc_pages* c, const float* q, double* out,
                    const uint32_t* bt, int bt_stride, const int32_t* kv_len,
                    const int32_t* p_start, int n_seq, int n_heads, double scale,
                    int n_threads) {
  const int nkv = (int)c->n_kv_heads, d = (int)c->head_dim, rep = n_heads / nkv;
  int max_len = 1;
  for (int s = 0; s < n_seq; ++s) if (kv_len[s] > max_len) max_len = kv_len[s];
  if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads)
  {
    double* buf = (double*)malloc(sizeof(double) * (size_t)max_len);
#pragma omp for schedule(dynamic, 1)
    for (int w = 0; w < n_seq * n_heads; ++w) {
      const int s = w / n_heads, h = w % n_heads;
      const int p0 = p_start ? p_start[s] : 0;
      f64_head(c, q + ((size_t)s * n_heads + h) * d, out + ((size_t)s * n_heads + h) * d,
               bt + (size_t)s * bt_stride, p0, kv_len[s], h / rep, scale, buf);
    }
    free(buf);
  }
}

void orc_decode_split_f64(const orc_pages* c, const float* q, double* out,
                          const uint32_t* bt, int bt_stride, const int32_t* kv_len,
                          const int32_t* p_start, int n_seq, int n_heads, double scale,
                          int split) {
  const int nkv = (int)c->n_kv_heads, d = (int)c->head_dim, rep = n_heads / nkv;
  double* acc = (double*)malloc(sizeof(double) * (size_t)d);
  double* tot = (double*)malloc(sizeof(double) * (size_t)d);
  for (int s = 0; s < n_seq; ++s) {
    const uint32_t* row = bt + (size_t)s * bt_stride;
    const int p0 = p_start ? p_start[s] : 0, p1 = kv_len[s];
    for (int h = 0; h < n_heads; ++h) {
      const float* qh = q + ((size_t)s * n_heads + h) * d;
      const int kvh = h / rep;
      /* per-partition (m_j, l_j, acc_j), combined with a running max M */
      double M = -INFINITY, L = 0.0;
      for (int i = 0; i < d; ++i) tot[i] = 0.0;
      for (int j0 = 0; j0 < p1; j0 += split) {
        const int a = j0 > p0 ? j0 : p0, b = j0 + split < p1 ? j0 + split : p1;
        if (a >= b) continue;
        double m = -INFINITY, l = 0.0;
        for (int i = 0; i < d; ++i) acc[i] = 0.0;
        for (int pass = 0; pass < 2; ++pass) {
          for (int p = a; p < b; ++p) {
            uint32_t slot;
            if (slot_of(c, row, p, &slot)) continue;
            double dot = 0.0;
            for (int i = 0; i < d; ++i) dot += (double)qh[i] * orc_stored_value(c, 0, slot, kvh, i);
            const double sc = dot * scale;
            if (pass == 0) { if (sc > m) m = sc; continue; }
            const double w = exp(sc - m);
            l += w;
            for (int i = 0; i < d; ++i) acc[i] += w * orc_stored_value(c, 1, slot, kvh, i);
          }
        }
        if (l == 0.0) continue;
        /* log-sum-exp combine of (m, l, acc) into (M, L, tot) */
        const double Mn = m > M ? m : M;
        const double a_old = isinf(M) ? 0.0 : exp(M - Mn), a_new = exp(m - Mn);
        for (int i = 0; i < d; ++i) tot[i] = a_old * tot[i] + a_new * acc[i];
        L = a_old * L + a_new * l;
        M = Mn;
      }
      double* oh = out + ((size_t)s * n_heads + h) * d;
      for (int i = 0; i < d; ++i) oh[i] = L > 0.0 ? tot[i] / L : 0.0;
    }
  }
  free(acc);
  free(tot);
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---- RoPE ------------------------------------------------------------------
 * compute_rope_inv_freqs, engine.rs:139-195: base_i = theta^(-2i/rotary_dim),
 * then the scaling mode's adjustment of each frequency. */
void orc_rope_inv_freqs(int rotary_dim, float theta, int mode, const float* params, float* out) {
  const int half = rotary_dim / 2;
  const float tau = 6.28318530717958647692f;
  for (int i = 0; i < half; ++i) {
    const float base = powf(theta, -(2.0f * (float)i) / (float)rotary_dim);
    float f = base;
    if (mode == ORC_ROPE_DEFAULT || mode == ORC_ROPE_LINEAR) {
      f = base / fmaxf(params[0], 1.0f);
    } else {  /* LLAMA3 {factor, original_max_pos, low, high}; YARN {factor, original_max_pos, beta_fast, beta_slow} */
      const float factor = params[0], omp = params[1];
      const float lo = mode == ORC_ROPE_LLAMA3 ? params[2] : params[3];  /* low_freq_factor / beta_slow */
      const float hi = mode == ORC_ROPE_LLAMA3 ? params[3] : params[2];  /* high_freq_factor / beta_fast */
      const float wavelen = tau / base;
      const float low_w = omp / lo, high_w = omp / hi;
      if (wavelen < high_w) {
        f = base;
      } else if (wavelen > low_w) {
        f = base / factor;
      } else {
        const float smooth = (omp / wavelen - lo) / (hi - lo);
        f = base * ((1.0f - smooth) / factor + smooth);
      }
    }
    out[i] = f;
  }
}

/* sin and cos of a RoPE angle (the f32 product pos * inv_freq[i], as
 * engine.rs:217 and lns_decode.metal:176 form it).  The reference takes them
 * from the platform's f32 sin_cos (engine.rs:218, Rust -> libm) or Metal's
 * fast sincos (lns_decode.metal:178), whose last bits differ between
 * platforms; this restatement fixes them as one rounding to f32 of an f64
 * evaluation: Cody-Waite reduction by pi/2 (pi/2 split into two 26-bit parts
 * and a 53-bit tail, derived from pi to 80 digits; k times a part is exact
 * for |k| < 2^27), then the Taylor series of sin to r^17 and of cos to r^18
 * on |r| <= pi/4, in Horner form with fused multiply-adds.  The library
 * evaluates the same steps in the same order.  Pinned against libm's double
 * sin/cos (tests/test_rope_oracle.py): within 4 ulp of f64, and its f32
 * roundings equal the f32 roundings of libm's double results. */
void orc_rope_sincos(float theta, float* s, float* c) {
  const double t = (double)theta;
  const double k = rint(t * 0x1.45f306dc9c883p-1);
  const double r = ((t - k * 0x1.921fb5p+0) - k * 0x1.110b46p-26) - k * 0x1.1a62633145c07p-54;
  const double z = r * r;
  double ps = 0x1.952c77030ad4ap-49;
  ps = fma(ps, z, -0x1.ae7f3e733b81fp-41);
  ps = fma(ps, z, 0x1.6124613a86d09p-33);
  ps = fma(ps, z, -0x1.ae64567f544e4p-26);
  ps = fma(ps, z, 0x1.71de3a556c734p-19);
  ps = fma(ps, z, -0x1.a01a01a01a01ap-13);
  ps = fma(ps, z, 0x1.1111111111111p-7);
  ps = fma(ps, z, -0x1.5555555555555p-3);
  const double sr = fma(r * z, ps, r);
  double pc = -0x1.6827863b97d97p-53;
  pc = fma(pc, z, 0x1.ae7f3e733b81fp-45);
  pc = fma(pc, z, -0x1.93974a8c07c9dp-37);
  pc = fma(pc, z, 0x1.1eed8eff8d898p-29);
  pc = fma(pc, z, -0x1.27e4fb7789f5cp-22);
  pc = fma(pc, z, 0x1.a01a01a01a01ap-16);
  pc = fma(pc, z, -0x1.6c16c16c16c17p-10);
  pc = fma(pc, z, 0x1.5555555555555p-5);
  pc = fma(pc, z, -0x1.0000000000000p-1);
  const double cr = fma(z, pc, 1.0);
  const int q = (int)((long long)k & 3);
  const double sv = q == 0 ? sr : (q == 1 ? cr : (q == 2 ? -sr : -cr));
  const double cv = q == 0 ? cr : (q == 1 ? -sr : (q == 2 ? -cr : sr));
  *s = (float)sv;
  *c = (float)cv;
}

/* apply_cpu_rope_with_freqs, engine.rs:200-229 (the same rotation as the
 * rope_with_freqs kernel, lns_decode.metal:158-191): the first rotary_dim
 * elements of a head are two halves (x0 = first[i], x1 = second[i]) rotated
 * by angle pos * inv_freqs[i]; the rest of the head is untouched. */
void orc_rope_apply(float* x, int n_rows, int heads, int head_dim, int rotary_dim, const float* inv_freqs,
                    int n_inv, const int32_t* pos) {
  int rd = rotary_dim < head_dim ? rotary_dim : head_dim;
  if (rd < 2) rd = 2;
  rd &= ~1;
  const int half = rd / 2;
  const int n = half < n_inv ? half : n_inv;
  for (int r = 0; r < n_rows; ++r) {
    for (int h = 0; h < heads; ++h) {
      float* v = x + ((size_t)r * heads + h) * head_dim;
      for (int i = 0; i < n; ++i) {
        const float angle = (float)pos[r] * inv_freqs[i];
        float sn, cs;
        orc_rope_sincos(angle, &sn, &cs);
        const float x0 = v[i], x1 = v[half + i];
        v[i] = x0 * cs - x1 * sn;
        v[half + i] = x0 * sn + x1 * cs;
      }
    }
  }
}

/* split_gated_query_interleaved, engine.rs:287-307 (the kernel form is
 * split_gated_query_kernel, lns_decode.metal:193-209): head h of row r starts
 * at (r * heads + h) * 2 * head_dim; its first head_dim values are q, the
 * next head_dim are gate logits, squashed by the f32 logistic function. */
void orc_split_gated_query(const float* in, float* q_out, float* gate_out, int n_rows, int heads, int head_dim) {
  for (size_t hh = 0; hh < (size_t)n_rows * heads; ++hh) {
    const float* src = in + hh * 2 * head_dim;
    for (int i = 0; i < head_dim; ++i) {
      q_out[hh * head_dim + i] = src[i];
      gate_out[hh * head_dim + i] = 1.0f / (1.0f + expf(-src[head_dim + i]));
    }
  }
}

/* prepare_tensor's Q4L branch, lns-metal/src/lib.rs:1296-1315. */
void orc_q4l_prepare(const uint8_t* disk, int n_blocks, uint8_t* dev) {
  for (int b = 0; b < n_blocks; ++b) {
    const uint8_t* src = disk + (size_t)b * 134;
    uint8_t* dst = dev + (size_t)b * 144;
    const uint16_t g_bits = (uint16_t)(src[0] | (src[1] << 8));
    const float g = orc_f16_to_f32(g_bits);
    for (int i = 0; i < 8; ++i) {
      const int sl = (src[2 + i / 2] >> ((i % 2) * 4)) & 0xF;
      const float ef = g * (float)ldexp(1.0, sl - 7); /* exact power-of-two product in f32 */
      const uint16_t eb = orc_f32_to_f16(ef); /* round to nearest even, as F16::from_f32 */
      dst[2 * i] = (uint8_t)(eb & 0xFF);
      dst[2 * i + 1] = (uint8_t)(eb >> 8);
    }
    memcpy(dst + 16, src + 6, 128);
  }
}

/* lns_decode_byte, lns_decode.metal:38-48, over one block. */
void orc_q4l_decode_block(const uint8_t* blk, float* w) {
  static const float lut[8] = {0.0f, 0.0625f, 0.125f, 0.25f, 0.5f, 1.0f, 2.0f, 4.0f};
  for (int i = 0; i < 256; ++i) {
    const float scale = orc_f16_to_f32((uint16_t)(blk[2 * (i / 32)] | (blk[2 * (i / 32) + 1] << 8)));
    const int nib = (blk[16 + i / 2] >> ((i % 2) * 4)) & 0xF;
    const float sgn = 1.0f - 2.0f * (float)((nib >> 3) & 1);
    w[i] = sgn * scale * lut[nib & 7];
  }
}

void orc_q4l_gemv_f64(const uint8_t* blocks, const float* x, int x_stride, const float* y_in, int y_stride,
                      double* y_out, int rows, int cols, int n_vec) {
  const int bpr = cols / 256;
  float w[256];
  for (int r = 0; r < rows; ++r) {
    for (int v = 0; v < n_vec; ++v) y_out[(size_t)v * y_stride + r] = (double)y_in[(size_t)v * y_stride + r];
    for (int b = 0; b < bpr; ++b) {
      orc_q4l_decode_block(blocks + ((size_t)r * bpr + b) * 144, w);
      for (int v = 0; v < n_vec; ++v) {
        double acc = 0.0;
        const float* xv = x + (size_t)v * x_stride + (size_t)b * 256;
        for (int i = 0; i < 256; ++i) acc += (double)w[i] * (double)xv[i];
        y_out[(size_t)v * y_stride + r] += acc;
      }
    }
  }
}

void orc_q4l_decode_matrix(const uint8_t* blocks, int rows, int cols, float* w) {
  const int bpr = cols / 256;
  for (int r = 0; r < rows; ++r)
    for (int b = 0; b < bpr; ++b)
      orc_q4l_decode_block(blocks + ((size_t)r * bpr + b) * 144, w + (size_t)r * cols + (size_t)b * 256);
}
