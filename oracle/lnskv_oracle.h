/*
 * lnskv_oracle.h — CPU restatement of lns-ml's paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against; it is never linked into, loaded by or called from the
 * product library (liblnskv.so).  Only the test suite, the smoke check and the
 * CPU-baseline leg of the benchmark may load it.
 *
 * Every function follows a named place in the reference (paths relative to the
 * lns-ml repository root):
 *   lns-metal/src/shaders/lns_decode.metal   kernels (append, Q8A, online softmax)
 *   lns-inference/src/engine.rs              PagePool, block tables, page helpers
 *
 * Page layout (shared with the HIP library): per layer, separate K and V pools
 *   pages[num_pages][16][n_kv_heads][head_dim]   (slot-major, engine.rs:731-734)
 *   Q8A scales[num_pages * 16][n_kv_heads]       (engine.rs:733-734)
 * A "slot" is phys_page * 16 + (pos % 16) (lns_decode.metal:541-545).
 */
#ifndef LNSKV_ORACLE_H
#define LNSKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_PAGE_SIZE 16
#define ORC_NO_PAGE 0xFFFFFFFFu

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8A = 2 };

/* ---- element conversions ------------------------------------------------ */
uint16_t orc_f32_to_f16(float x);           /* IEEE binary16 roundTiesToEven */
float orc_f16_to_f32(uint16_t h);           /* exact widening */
/* count of mismatches vs the x86 F16C converter over bit patterns [lo, hi) */
uint64_t orc_f16_check_range(uint64_t lo, uint64_t hi, int n_threads);
void orc_q8a_quantize(const float* x, int d, int8_t* q, float* scale);
void orc_f32_to_f16_array(const float* x, size_t n, uint16_t* out, int n_threads);
/* conversion of the bit patterns [lo, lo+n) reinterpreted as f32 */
void orc_f16_of_patterns(uint64_t lo, size_t n, uint16_t* out, int n_threads);

/* ---- PagePool (engine.rs:20-44) ----------------------------------------- */
typedef struct orc_pool orc_pool;
orc_pool* orc_pool_new(uint32_t capacity);
void orc_pool_delete(orc_pool* p);
int orc_pool_alloc(orc_pool* p, uint32_t* out);   /* 0 ok, -1 exhausted */
void orc_pool_free_page(orc_pool* p, uint32_t idx);
void orc_pool_reset(orc_pool* p);
uint32_t orc_pool_num_free(const orc_pool* p);

/* ---- page helpers for one block table (engine.rs:2958-3013) -------------- */
/* bt: row of capacity bt_cap, *bt_len logical pages in use.  Returns 0, or -1
 * when the pool is exhausted, -2 when the row is full. */
int orc_ensure_kv_page(orc_pool* p, uint32_t* bt, int* bt_len, int bt_cap, int pos);
void orc_evict_kv_pages(orc_pool* p, uint32_t* bt, int bt_len, int pos, int window);
int orc_kv_p_start(int pos, int window);

/* ---- append / gather / copy --------------------------------------------- */
typedef struct {
  void* k_pages;
  void* v_pages;
  float* k_scales;
  float* v_scales;
  uint32_t num_pages;
  uint32_t n_kv_heads;
  uint32_t head_dim;
  int32_t dtype;
} orc_pages;

/* Write token t's K/V ([n_tok][n_kv][d] f32) into slot
 * bt[tok_seq[t]][tok_pos[t]/16]*16 + tok_pos[t]%16.  Returns the number of
 * tokens skipped: sequence outside [0, n_rows), position outside the table
 * row, or page entry missing or outside the pool. */
int orc_append(const orc_pages* c, const float* k_new, const float* v_new,
               const int32_t* tok_seq, const int32_t* tok_pos, int n_tok,
               const uint32_t* bt, int bt_stride, int n_rows);
/* Copy tokens [start, start+n_tok) of one sequence into contiguous
 * [n_tok][n_kv][d] arrays in page dtype (+ [n_tok][n_kv] scales for Q8A). */
int orc_gather(const orc_pages* c, const uint32_t* bt_row, int start, int n_tok,
               void* k_out, void* v_out, float* ks_out, float* vs_out);
void orc_page_copy(const orc_pages* c, const uint32_t* src, const uint32_t* dst, int n);
/* value of stored element (page dtype -> f64, Q8A dequantized as q*scale) */
double orc_stored_value(const orc_pages* c, int which_v, uint32_t slot, int h, int i);

/* ---- decode attention ---------------------------------------------------- */
/* q [n_seq][n_heads][d] f32, out same.  Attends tokens [p_start[s], kv_len[s]).
 * p_start may be NULL (0).  Query head h uses kv head h / (n_heads/n_kv). */
void orc_decode_refscan(const orc_pages* c, const float* q, float* out,
                        const uint32_t* bt, int bt_stride, const int32_t* kv_len,
                        const int32_t* p_start, int n_seq, int n_heads, float scale,
                        int n_threads);
void orc_decode_f64(const orc_pages* c, const float* q, double* out,
                    const uint32_t* bt, int bt_stride, const int32_t* kv_len,
                    const int32_t* p_start, int n_seq, int n_heads, double scale,
                    int n_threads);
/* Split-K in f64: partitions of split tokens starting at token 0, each giving
 * (m, l, acc[d]); then out = sum e^(m_j-M) acc_j / sum e^(m_j-M) l_j. */
void orc_decode_split_f64(const orc_pages* c, const float* q, double* out,
                          const uint32_t* bt, int bt_stride, const int32_t* kv_len,
                          const int32_t* p_start, int n_seq, int n_heads, double scale,
                          int split);
/* One whole step as the reference performs it: append token kv_len[s]-1 of
 * every sequence, then the reference-order f32 scan.  Used for the timed CPU
 * baseline; OpenMP over (sequence, kv head). */
void orc_append_decode_refscan(const orc_pages* c, const float* q, const float* k_new,
                               const float* v_new, float* out, const uint32_t* bt,
                               int bt_stride, const int32_t* kv_len, const int32_t* p_start,
                               int n_seq, int n_heads, float scale, int n_threads);
int orc_max_threads(void);

/* ---- RoPE (engine.rs:137-229, lns_decode.metal:154-191) ----------------- */
enum { ORC_ROPE_DEFAULT = 0, ORC_ROPE_LINEAR = 1, ORC_ROPE_LLAMA3 = 2, ORC_ROPE_YARN = 3 };
/* compute_rope_inv_freqs (engine.rs:139-195): out[rotary_dim / 2].  params:
 * DEFAULT {scaling_factor}, LINEAR {factor}, LLAMA3 {factor, original_max_pos,
 * low_freq_factor, high_freq_factor}, YARN {factor, original_max_pos,
 * beta_fast, beta_slow}.  f32 arithmetic throughout, as the reference. */
void orc_rope_inv_freqs(int rotary_dim, float theta, int mode, const float* params, float* out);
/* sin and cos of the f32 angle theta: one f32 rounding of an f64 evaluation
 * (Cody-Waite by pi/2, Taylor series; see the definition). */
void orc_rope_sincos(float theta, float* s, float* c);
/* apply_cpu_rope_with_freqs (engine.rs:200-229) on x[n_rows][heads][head_dim]
 * in place; row r is at position pos[r]; angle_i = pos * inv_freqs[i]. */
void orc_rope_apply(float* x, int n_rows, int heads, int head_dim, int rotary_dim, const float* inv_freqs,
                    int n_inv, const int32_t* pos);

/* ---- gated query (engine.rs:287-307, lns_decode.metal:193-221) ---------- */
/* split_gated_query_interleaved (engine.rs:287-307): in[n_rows][heads][2*head_dim]
 * -> q_out[n_rows][heads][head_dim] (first halves) and gate_out (same shape)
 * = 1 / (1 + exp(-x)) of the second halves, in f32 as the reference. */
void orc_split_gated_query(const float* in, float* q_out, float* gate_out, int n_rows, int heads, int head_dim);

/* ---- o_proj over Q4_L weights (lns-core/src/quant/q4l.rs, lns-metal) ----- */
/* Disk super-block (Q4LSuperBlock, q4l.rs:136-158): 134 bytes = scale_global
 * (f16 bits, LE), 4 bytes of local-scale nibbles (sub-block i in nibble i,
 * low nibble first), 128 weight bytes (weight i in nibble i, low nibble
 * first; bit 3 sign, bits 0-2 magnitude m).  Device block (prepare_tensor,
 * lns-metal/src/lib.rs:1255-1320; block_q4_l, lns_decode.metal:12-15): 144
 * bytes = 8 f16 effective scales f16(f32(scale_global) * 2^(sl - 7)) (round to
 * nearest even), then the 128 weight bytes.  n_blocks super-blocks. */
void orc_q4l_prepare(const uint8_t* disk, int n_blocks, uint8_t* dev);
/* Weights of one device block as the kernel forms them (lns_decode_byte,
 * lns_decode.metal:38-48): w[i] = (1 - 2 s) * f32(scale[i / 32]) * LUT[m],
 * LUT = {0, 2^-4, ..., 2^2}. */
void orc_q4l_decode_block(const uint8_t* dev_block, float* w256);
/* q4l_gemv_accumulate_multirow (lns_decode.metal:1174-1225) for n_vec
 * vectors, in float64: y[b][r] = y_in[b][r] + sum_c W[r][c] x[b][c], W the
 * rows x cols device blocks (cols / 256 per row, cols a multiple of 256). */
void orc_q4l_gemv_f64(const uint8_t* dev_blocks, const float* x, int x_stride, const float* y_in,
                      int y_stride, double* y_out, int rows, int cols, int n_vec);
/* The kernel's weights of a rows x cols device matrix, w[rows][cols]. */
void orc_q4l_decode_matrix(const uint8_t* dev_blocks, int rows, int cols, float* w);

#ifdef __cplusplus
}
#endif
#endif
