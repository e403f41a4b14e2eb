/*
 * lnskv.h — C ABI of the MI355X (gfx950) paged KV-cache library.
 *
 * Replaces lns-ml's paged KV path:
 *   - the paged attention call on MetalContext (encode_/dispatch_/
 *     attention_paged_q8a[_enc], lns-metal/src/lib.rs:997-1094, 2085-2129)
 *     and its kernel flash_attention_paged_q8a
 *     (lns-metal/src/shaders/lns_decode.metal:498-646);
 *   - the engine's page bookkeeping: PagePool (lns-inference/src/engine.rs:20-44),
 *     ensure_kv_page / evict_kv_pages / upload_block_table / kv_p_start
 *     (engine.rs:2958-3013) and clear_kv_cache (engine.rs:2911-2934).
 *
 * Conventions
 *   - Every entry point returns 0 (LNSKV_OK) or a negative lnskv_status; the
 *     message of the last failure on the calling thread is lnskv_last_error().
 *     (The reference returns Result<(), String>; a binding maps status+message
 *     to that.)
 *   - Pointers named *_dev are device memory; everything else is host memory.
 *   - Device work is enqueued on the caller's HIP stream (hipStream_t passed as
 *     lnskv_stream_t; NULL = the null stream) and returns without waiting,
 *     except the lnskv_dispatch_* variants, which wait (the reference's
 *     dispatch_* commit-and-wait semantics, lib.rs:1091-1092).
 *   - Page layout, per layer: separate K and V pools
 *       pages[num_pages][16][n_kv_heads][head_dim]   (slot-major, engine.rs:731-734)
 *     Q8A adds f32 scales[num_pages*16][n_kv_heads] for K and for V.
 *     slot = block_table[pos/16]*16 + pos%16   (lns_decode.metal:541-545)
 *   - Block tables are u32 rows, LNSKV_NO_PAGE (u32::MAX) = unallocated
 *     (engine.rs:65).  Batched calls take [n_seq][bt_stride] row-major tables.
 *   - Query head h reads kv head h / (n_heads / n_kv_heads)  (lns_decode.metal:536-537).
 *   - Supported shapes: head_dim in {64, 128, 256}; n_heads a multiple of
 *     n_kv_heads with n_heads/n_kv_heads in {1, 2, 4, 8}.
 */
#ifndef LNSKV_H
#define LNSKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LNSKV_PAGE_SIZE 16           /* engine.rs:16 PAGE_SIZE, metal:516 PAGED_PAGE_SZ */
#define LNSKV_NO_PAGE 0xFFFFFFFFu    /* engine.rs:65 u32::MAX */

typedef void* lnskv_stream_t;        /* a hipStream_t */

typedef enum {
  LNSKV_DTYPE_F32 = 0,               /* plain copy on append */
  LNSKV_DTYPE_F16 = 1,               /* (half)x, round to nearest even (metal:284-287) */
  LNSKV_DTYPE_Q8A = 2                /* int8 + f32 absmax scale per (slot, head) (metal:547-593) */
} lnskv_dtype;

typedef enum {
  LNSKV_OK = 0,
  LNSKV_ERR_INVALID = -1,            /* bad argument or shape */
  LNSKV_ERR_NOMEM = -2,              /* host or device allocation failed */
  LNSKV_ERR_POOL_EXHAUSTED = -3,     /* engine.rs:2969-2971 "KV page pool exhausted ..." */
  LNSKV_ERR_HIP = -4,                /* a HIP runtime call failed */
  LNSKV_ERR_UNSUPPORTED = -5,        /* shape/dtype combination not built */
  LNSKV_ERR_WORKSPACE = -6           /* caller workspace smaller than required */
} lnskv_status;

/* One layer's paged K/V pools (device memory, owned by the caller or by an
 * lnskv_ctx).  Replaces the (k_cache, v_cache, k_scales, v_scales) buffer
 * quadruple of encode_attention_paged_q8a (lib.rs:997-1010). */
typedef struct lnskv_pages {
  void* k_pages;                     /* device, [num_pages][16][n_kv_heads][head_dim] */
  void* v_pages;                     /* device, same shape */
  float* k_scales;                   /* device, Q8A only: [num_pages*16][n_kv_heads] */
  float* v_scales;                   /* device, Q8A only */
  uint32_t num_pages;
  uint32_t n_kv_heads;
  uint32_t head_dim;
  int32_t dtype;                     /* lnskv_dtype */
} lnskv_pages;

const char* lnskv_last_error(void);
const char* lnskv_version(void);
/* bytes of one K (or V) page: 16 * n_kv_heads * head_dim * elem */
size_t lnskv_page_bytes(const lnskv_pages* c);

/* ---------------------------------------------------------------------------
 * Device pools.  lnskv_pages_alloc fills c->k_pages/v_pages (and scales for
 * Q8A) with zeroed device memory for the geometry already in *c; the caller
 * frees them with lnskv_pages_free.  Replaces the per-layer Metal buffer
 * allocation in InferenceEngine::new (engine.rs:717-773).
 * ------------------------------------------------------------------------- */
int lnskv_pages_alloc(lnskv_pages* c);
int lnskv_pages_free(lnskv_pages* c);

/* Zero every page and scale of the layer: clear_kv_cache's data part
 * (engine.rs:2912-2922).  Async on stream. */
int lnskv_clear(const lnskv_pages* c, lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * Append: token t's K and V (k_new_dev/v_new_dev [n_tok][n_kv_heads][head_dim],
 * f32) are converted to the page dtype and written to the slot of position
 * tok_pos_dev[t] in sequence tok_seq_dev[t] (row tok_seq_dev[t] of
 * block_tables_dev, which has n_rows rows of bt_stride entries).  Tokens may
 * straddle pages and any number of sequences.  A token whose sequence is
 * outside [0, n_rows), whose position is outside [0, 16*bt_stride), or whose
 * page entry is LNSKV_NO_PAGE or >= num_pages is not written.
 * Replaces the write half of flash_attention_paged_q8a (metal:541-593),
 * performed once per (token, kv head) instead of once per query head.
 * ------------------------------------------------------------------------- */
int lnskv_append(const lnskv_pages* c, const float* k_new_dev, const float* v_new_dev,
                 const int32_t* tok_seq_dev, const int32_t* tok_pos_dev, int32_t n_tok,
                 const uint32_t* block_tables_dev, int32_t bt_stride, int32_t n_rows,
                 lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * Single-query paged decode attention over a batch of sequences.
 *   q_dev [n_seq][n_heads][head_dim] f32 -> out_dev [n_seq][n_heads][head_dim] f32
 *   sequence s attends tokens [p_start_dev[s], kv_len_dev[s]) (p_start_dev may
 *   be NULL = 0; kv_len counts the newest token, so it is the reference's pos+1,
 *   and p_start is kv_p_start, engine.rs:3008-3013).
 *   out = softmax(scale * q.K^T) . V, by online softmax (metal:595-645).
 *   max_kv_len: host upper bound of kv_len over the batch (sizes the grid).
 *   A sequence whose kv_len exceeds max_kv_len or 16 * bt_stride is out of
 *   range: its output row is zero and the fused variants store nothing for
 *   it (as lnskv_append skips tokens outside the table).
 *   split_tokens: tokens per split-K partition (multiple of 16), or 0 to let
 *   the library schedule.  f16 and Q8A pages with head_dim 128 or 256 and at
 *   most 4096 sequences then run one of two schedules, each giving every
 *   workgroup an equal share of all the batch's pages: a small batch (at most
 *   16 pages per compute unit, bounded from max_kv_len) one kernel whose
 *   workgroups merge the pieces they share; a larger one stream-K (one wave
 *   per resident slot, then a merge kernel).  The environment variable
 *   LNSKV_DECODE_SCHEDULE=stream-k or =workgroup forces one of the two (the
 *   workspace query must see the same setting).  Q8A batches of more than
 *   4096 sequences run stream-K in launches of 4096 sequences.  Other shapes
 *   run split-K with a partition size chosen from the batch.
 *   workspace_dev/ws_bytes: 16-byte aligned device scratch of at least
 *   lnskv_decode_workspace_size(...) bytes (same n_seq, n_heads, max_kv_len
 *   and split_tokens, same current device), or NULL/0 to use a buffer the
 *   library keeps per device (calls that use it must not overlap in time; see
 *   lnskv_workspace_reserve for how it grows).  Its first
 *   LNSKV_WORKSPACE_HEADER_BYTES bytes must be zero before its first use
 *   (hipMemset once); every call leaves them zero again.  The rest holds the
 *   partial results of one call.  Calls that overlap in time need distinct
 *   workspaces.
 * Pages in the window whose table entry is LNSKV_NO_PAGE or >= num_pages are
 * skipped (contribute nothing).  An empty window gives a zero output row.
 * ------------------------------------------------------------------------- */
#define LNSKV_WORKSPACE_HEADER_BYTES 4096
int lnskv_decode_workspace_size(const lnskv_pages* c, int32_t n_seq, int32_t n_heads,
                                int32_t max_kv_len, int32_t split_tokens, size_t* bytes);
int lnskv_decode(const lnskv_pages* c, const float* q_dev, float* out_dev,
                 const uint32_t* block_tables_dev, int32_t bt_stride,
                 const int32_t* kv_len_dev, const int32_t* p_start_dev,
                 int32_t n_seq, int32_t n_heads, int32_t max_kv_len, float scale,
                 int32_t split_tokens, void* workspace_dev, size_t ws_bytes,
                 lnskv_stream_t stream);

/* Append + decode in one pass, the reference's per-layer step (engine.rs:
 * 3401-3422 -> metal:518-646): the newest token of every sequence, at
 * position kv_len_dev[s]-1, takes k_new_dev/v_new_dev[s] ([n_seq][n_kv][d]
 * f32), is written to its page, and is attended to with the stored (converted)
 * values.  Its page must already be allocated in the table (ensure_kv_page). */
int lnskv_append_decode(const lnskv_pages* c, const float* q_dev, const float* k_new_dev,
                        const float* v_new_dev, float* out_dev,
                        const uint32_t* block_tables_dev, int32_t bt_stride,
                        const int32_t* kv_len_dev, const int32_t* p_start_dev,
                        int32_t n_seq, int32_t n_heads, int32_t max_kv_len, float scale,
                        int32_t split_tokens, void* workspace_dev, size_t ws_bytes,
                        lnskv_stream_t stream);

/* lnskv_append_decode without a workspace argument, allocating nothing: no
 * counterpart in the reference.  It is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The partial results live in a static device array of
 * LNSKV_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a call
 * whose schedule needs more (lnskv_decode_workspace_size) returns
 * LNSKV_ERR_WORKSPACE before launching anything.  Every call on one GPU shares
 * that array: calls that overlap in time on one GPU race and give wrong
 * results.  Same kernels, same results bit for bit as lnskv_append_decode. */
#define LNSKV_NOALLOC_SCRATCH_BYTES ((size_t)24 << 20)
int lnskv_append_decode_noalloc(const lnskv_pages* c, const float* q_dev, const float* k_new_dev,
                                const float* v_new_dev, float* out_dev,
                                const uint32_t* block_tables_dev, int32_t bt_stride,
                                const int32_t* kv_len_dev, const int32_t* p_start_dev,
                                int32_t n_seq, int32_t n_heads, int32_t max_kv_len, float scale,
                                int32_t split_tokens, lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * RoPE fused into the append.  The reference rotates q and k in place with
 * rope_with_freqs (lns_decode.metal:154-191; angle_i = pos * inv_freqs[i], the
 * first rotary_dim elements of a head taken as two halves) just before
 * encode_attention_paged_q8a (engine.rs:1700-1720).  These entry points take q
 * and the new K before the rotation and apply it where the values are
 * converted and stored, so rotated K never goes back to memory as f32.  The
 * caller's q and k_new buffers are left as they are.
 * ------------------------------------------------------------------------- */
typedef enum lnskv_rope_mode {
  LNSKV_ROPE_DEFAULT = 0,  /* params {scaling_factor} */
  LNSKV_ROPE_LINEAR = 1,   /* params {factor} */
  LNSKV_ROPE_LLAMA3 = 2,   /* params {factor, original_max_pos, low_freq_factor, high_freq_factor} */
  LNSKV_ROPE_YARN = 3      /* params {factor, original_max_pos, beta_fast, beta_slow} */
} lnskv_rope_mode;

/* Rotary width the engine derives (engine.rs:826-833): round(head_dim *
 * partial_rotary_factor) when that lies in [2, head_dim), else head_dim. */
int32_t lnskv_rope_dim(int32_t head_dim, float partial_rotary_factor);

/* Host computation of the rotary_dim/2 inverse frequencies
 * (compute_rope_inv_freqs, engine.rs:139-195) into inv_freqs_host; upload
 * them once per model.  rotary_dim even and >= 2. */
int lnskv_rope_inv_freqs(int32_t rotary_dim, float theta, int32_t mode, const float* params,
                         float* inv_freqs_host);

typedef struct lnskv_rope {
  const float* inv_freqs_dev;  /* device, [rotary_dim / 2] f32 */
  int32_t rotary_dim;          /* even, 2 .. head_dim */
} lnskv_rope;

/* lnskv_append with K rotated first: token t's K (every kv head) turns by
 * position tok_pos_dev[t] before it is converted and stored; V is stored as
 * given.  f32/f16 pages with a rotary half that is a multiple of 8 (half/8 a
 * power of two) and 16-byte aligned inputs turn K inside the append; other
 * shapes (Q8A pages among them) first write the rotated K rows to
 * workspace_dev, which then needs lnskv_rope_append_workspace_size bytes
 * (16-byte aligned).  workspace_dev NULL: a buffer the library keeps per
 * device instead (calls that use it must not overlap in time). */
int lnskv_rope_append_workspace_size(const lnskv_pages* c, const lnskv_rope* rope, int32_t n_tok,
                                     size_t* bytes);
int lnskv_rope_append(const lnskv_pages* c, const lnskv_rope* rope, const float* k_new_dev,
                      const float* v_new_dev, const int32_t* tok_seq_dev, const int32_t* tok_pos_dev,
                      int32_t n_tok, const uint32_t* block_tables_dev, int32_t bt_stride, int32_t n_rows,
                      void* workspace_dev, size_t ws_bytes, lnskv_stream_t stream);

/* lnskv_append_decode with q_dev and k_new_dev before the rotation: both turn
 * by the new token's position kv_len_dev[s]-1, then the token is stored and
 * attended to as lnskv_append_decode does.  f16 pages with head_dim 128 and a
 * rotary width of 64 or 128 turn q and K inside the decode; other shapes (Q8A
 * pages among them) first write the rotated q and K rows into the workspace,
 * after the decode's partial results.  A caller's workspace therefore needs
 * lnskv_rope_decode_workspace_size bytes (it covers both cases); NULL uses the
 * library's per-device buffers (calls that use them must not overlap). */
int lnskv_rope_decode_workspace_size(const lnskv_pages* c, const lnskv_rope* rope, int32_t n_seq,
                                     int32_t n_heads, int32_t max_kv_len, int32_t split_tokens,
                                     size_t* bytes);
int lnskv_rope_append_decode(const lnskv_pages* c, const lnskv_rope* rope, const float* q_dev,
                             const float* k_new_dev, const float* v_new_dev, float* out_dev,
                             const uint32_t* block_tables_dev, int32_t bt_stride,
                             const int32_t* kv_len_dev, const int32_t* p_start_dev, int32_t n_seq,
                             int32_t n_heads, int32_t max_kv_len, float scale, int32_t split_tokens,
                             void* workspace_dev, size_t ws_bytes, lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * Chunked-prefill attention over pages.  The reference has none: it runs the
 * whole forward once per prompt token (engine.rs:2835-2855), each token
 * appended, then attending [p_start, pos] through the paged kernel.  This
 * computes, for a chunk of consecutive prompt tokens whose K/V are already in
 * the pages (lnskv_append first), every token's attention at once: query row
 * t attends positions [p_start, pos(t)] of its sequence -- what lnskv_decode
 * with kv_len = pos(t) + 1 gives that token alone.
 *   chunks_dev: n_chunks x {table row, first position, length, first token}
 *   (int32 x 4, 16-byte aligned): chunk i's tokens are q/out rows
 *   [first token, first token + length), at positions first position + 0,
 *   1, ...; chunks outside [0, n_rows) x [0, n_tok) are skipped.
 *   q_dev / out_dev: [n_tok][n_heads][head_dim] f32; p_start_dev: per table
 *   row (NULL = 0).  window > 0 (a sliding-window layer): query row t attends
 *   [max(p_start, pos(t) - window + 1), pos(t)], each prompt token its own
 *   kv_p_start as the reference's per-token loop gives it (engine.rs:
 *   3007-3013); window = 0: [p_start, pos(t)].  f16 or Q8A pages with
 *   head_dim 128 or 256 (Q8A: scale arrays under 2 GiB, num_pages * 16 * n_kv_heads
 *   < 2^29; LNSKV_ERR_UNSUPPORTED otherwise); Q8A codes are turned to
 *   f16 in LDS (code x 1, the row scale applied to the scores and to the
 *   probabilities), so the result is the dequantised pages' attention.
 * ------------------------------------------------------------------------- */
int lnskv_prefill_attention(const lnskv_pages* c, const float* q_dev, float* out_dev,
                            const int32_t* chunks_dev, int32_t n_chunks, int32_t n_tok,
                            const uint32_t* block_tables_dev, int32_t bt_stride, int32_t n_rows,
                            const int32_t* p_start_dev, int32_t window, int32_t n_heads, float scale,
                            lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * Gated attention (gated_query_attention models): the q projection holds, per
 * query head, head_dim q values then head_dim gate logits; the attention
 * output is multiplied by sigmoid(logits) before o_proj.
 * ---------------------------------------------------------------------------
 * lnskv_split_gated_query (split_gated_query_kernel, lns_decode.metal:193-209;
 * split_gated_query_interleaved, engine.rs:287-307): input_dev is
 * [n_rows][n_heads][2 * head_dim]; q_out_dev gets the first halves and
 * gate_out_dev 1 / (1 + exp(-x)) of the second, both [n_rows][n_heads][head_dim]
 * (the engine then norms and rotates q). */
int lnskv_split_gated_query(const float* input_dev, float* q_out_dev, float* gate_out_dev,
                            int32_t n_rows, int32_t n_heads, int32_t head_dim,
                            lnskv_stream_t stream);
/* lnskv_append_decode (rope NULL) or lnskv_rope_append_decode (rope non-NULL)
 * whose output row is multiplied, as it is stored, by gate_dev
 * ([n_seq][n_heads][head_dim], the gate_out above): the engine's
 * mul_inplace_enc after the attention (engine.rs:3424-3431,
 * mul_inplace_kernel lns_decode.metal:211-221) folded into the decode.  The
 * stored value is exactly out * gate of the ungated call (one f32 multiply);
 * an empty window still stores a zero row. */
int lnskv_gated_append_decode(const lnskv_pages* c, const lnskv_rope* rope, const float* gate_dev,
                              const float* q_dev, const float* k_new_dev, const float* v_new_dev,
                              float* out_dev, const uint32_t* block_tables_dev, int32_t bt_stride,
                              const int32_t* kv_len_dev, const int32_t* p_start_dev, int32_t n_seq,
                              int32_t n_heads, int32_t max_kv_len, float scale, int32_t split_tokens,
                              void* workspace_dev, size_t ws_bytes, lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * o_proj after the attention: x += W_o . attn_out over Q4_L weights
 * ---------------------------------------------------------------------------
 * Disk super-block (Q4LSuperBlock, lns-core/src/quant/q4l.rs:136-158), 134
 * bytes per 256 weights: scale_global (f16 bits), 8 local-scale nibbles (4
 * bytes), 128 weight bytes (weight i in nibble i, low nibble first; bit 3
 * sign, bits 0-2 magnitude m: 0 is zero, else 2^(m - 5)).  Device block
 * (block_q4_l, lns_decode.metal:12-15), 144 bytes: 8 f16 effective scales
 * f16(scale_global * 2^(scale_local - 7)), then the 128 weight bytes.  A
 * rows x cols matrix is rows x ceil(cols / 256) blocks, row-major. */
#define LNSKV_Q4L_DISK_BYTES 134
#define LNSKV_Q4L_DEVICE_BYTES 144
/* MetalContext::prepare_tensor, Q4L branch (lns-metal/src/lib.rs:1255-1320):
 * host repack of rows x ceil(cols/256) disk blocks into device blocks
 * (out_blocks: rows * ceil(cols/256) * 144 bytes of host memory); effective
 * scales rounded to nearest even, as F16::from_f32. */
int lnskv_q4l_prepare(const void* disk_blocks, size_t disk_bytes, int32_t rows, int32_t cols,
                      void* out_blocks);
/* q4l_gemv_accumulate_multirow (lns_decode.metal:1174-1225; the engine's
 * gemv_accumulate_multirow_enc for o_proj, engine.rs:3433-3446), batched:
 * y[v][r] += sum_c W[r][c] * x[v][c] for v < n_vec, x [n_vec][x_stride] and
 * y [n_vec][y_stride] f32 on the device, W the device blocks (16-byte
 * aligned).  cols a multiple of 256 (as the reference kernel's ncols >> 8),
 * |x| < 65504.  Products of f16 weight codes and f16 parts of x on the matrix
 * cores, f32 sums in a fixed order: the same bits on every call.
 * workspace_dev/ws_bytes: 16-byte aligned device scratch of at least
 * lnskv_q4l_workspace_size(cols, n_vec) bytes (0 when cols < 2048: no
 * workspace is read), or NULL/0 to use a buffer the library keeps per device.
 * A call none of whose launches splits its rows' blocks (enough row groups to
 * fill the GPU, e.g. rows >= 8192 for up to 16 vectors) reads no workspace and
 * may pass NULL without the library buffer being grown, under capture too.
 * It holds the partial sums of a launch that splits each row's blocks over
 * several workgroups, after LNSKV_WORKSPACE_HEADER_BYTES of arrival counts
 * that must be zero before the first use (hipMemset once); every call leaves
 * them zero.  Calls that share a workspace must not overlap in time. */
int lnskv_q4l_workspace_size(int32_t cols, int32_t n_vec, size_t* bytes);
int lnskv_q4l_gemv_accumulate(const void* blocks_dev, const float* x_dev, float* y_dev,
                              int32_t rows, int32_t cols, int32_t n_vec, int32_t x_stride,
                              int32_t y_stride, void* workspace_dev, size_t ws_bytes,
                              lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * The reference call itself, one sequence: append the token at `pos` (k_in,
 * v_in [n_kv_heads*head_dim] f32) into its page and attend over [p_start, pos]
 * with scale 1/sqrt(head_dim) (metal:539).  Arguments follow
 * MetalContext::encode_attention_paged_q8a (lib.rs:997-1013): q, k_in, v_in,
 * the cache buffers (here the descriptor c, whose dtype may be Q8A as in the
 * reference, or F16/F32), block_table, out, pos, head_dim, n_heads,
 * n_kv_heads, p_start.  head_dim and n_kv_heads must match c.
 * lnskv_dispatch_attention_paged additionally waits for completion
 * (dispatch_attention_paged_q8a, lib.rs:1046-1094).
 * ------------------------------------------------------------------------- */
int lnskv_attention_paged(const float* q_dev, const float* k_in_dev, const float* v_in_dev,
                          const lnskv_pages* c, const uint32_t* block_table_dev, float* out_dev,
                          uint32_t pos, uint32_t head_dim, uint32_t n_heads, uint32_t n_kv_heads,
                          uint32_t p_start, lnskv_stream_t stream);
int lnskv_dispatch_attention_paged(const float* q_dev, const float* k_in_dev,
                                   const float* v_in_dev, const lnskv_pages* c,
                                   const uint32_t* block_table_dev, float* out_dev, uint32_t pos,
                                   uint32_t head_dim, uint32_t n_heads, uint32_t n_kv_heads,
                                   uint32_t p_start, lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * Page copy (eviction churn, copy-on-write fork): page dst_dev[i] of K, V and
 * (Q8A) both scale arrays becomes a copy of page src_dev[i].  The reference has
 * no copy op; its free is PagePool::free_page (engine.rs:37-39).  Pairs whose
 * ids are >= num_pages are skipped.  dst pages must be distinct from every src.
 * ------------------------------------------------------------------------- */
int lnskv_page_copy(const lnskv_pages* c, const uint32_t* src_dev, const uint32_t* dst_dev,
                    int32_t n, lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * Block-table gather: tokens [start, start+n_tok) of one sequence (its table
 * row block_table_dev) copied into contiguous k_out_dev/v_out_dev
 * [n_tok][n_kv_heads][head_dim] in the page dtype, plus (Q8A, may be NULL)
 * ks_out_dev/vs_out_dev [n_tok][n_kv_heads].  The reference reads pages through
 * the table inside its scan (metal:606-612); this is that address math as an
 * export.  Tokens on missing pages come out as zeros.
 * ------------------------------------------------------------------------- */
int lnskv_gather(const lnskv_pages* c, const uint32_t* block_table_dev, int32_t start,
                 int32_t n_tok, void* k_out_dev, void* v_out_dev, float* ks_out_dev,
                 float* vs_out_dev, lnskv_stream_t stream);

/* Wait for all work queued on stream (the commit + wait_until_completed of
 * dispatch_*, lib.rs:1091-1092).  Also returns LNSKV_ERR_WORKSPACE when a
 * decode or Q4L GEMV call since the last lnskv_sync (on any stream of the
 * process) met an arrival count in its workspace header above what one call
 * can reach: that workspace's first LNSKV_WORKSPACE_HEADER_BYTES bytes were
 * not zeroed before its first use, and the cut segments' (decode) or split
 * rows' (Q4L) results of calls on it are wrong.  Such a count is left in
 * place, so every later call on that workspace is reported again.  A garbage
 * count that happens to lie within what a call can reach is not detected. */
int lnskv_sync(lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * The library's own device buffers (no counterpart in the reference, whose
 * Metal calls need none).  Entry points given a NULL workspace use a buffer
 * the library keeps per device: the decode workspace, the rotated RoPE rows,
 * the Q4L GEMV partial sums.  When one is too small a call allocates a larger one
 * (hipMalloc, no device synchronization) and keeps the old one alive, since
 * work queued earlier may still use it; while the call's stream is being
 * captured into a graph it fails with LNSKV_ERR_WORKSPACE instead.
 * lnskv_workspace_reserve grows them ahead of time (call it before capturing
 * a graph that passes NULL workspaces); lnskv_workspace_release waits for the
 * current device (hipDeviceSynchronize) and frees them all, outgrown ones
 * included.  Both act on the current device.
 * ------------------------------------------------------------------------- */
int lnskv_workspace_reserve(size_t decode_bytes, size_t rope_bytes, size_t q4l_bytes);
int lnskv_workspace_release(void);

/* ===========================================================================
 * Host-side page bookkeeping (no device memory; usable without a GPU).
 * ========================================================================= */

/* PagePool, engine.rs:20-44: FIFO free list of physical page ids.
 * create(cap) holds 0..cap in order; alloc = pop_front (LNSKV_ERR_POOL_EXHAUSTED
 * when empty); free = push_back; reset refills 0..cap.  Adds a reference count
 * per page for copy-on-write sharing (retain): free returns a page to the list
 * only when its count drops to zero.  Without retain this is exactly the
 * reference's behaviour. */
typedef struct lnskv_page_pool lnskv_page_pool;
int lnskv_page_pool_create(uint32_t capacity, lnskv_page_pool** out);
void lnskv_page_pool_destroy(lnskv_page_pool* p);
int lnskv_page_pool_alloc(lnskv_page_pool* p, uint32_t* page_out);
int lnskv_page_pool_free(lnskv_page_pool* p, uint32_t page);
int lnskv_page_pool_retain(lnskv_page_pool* p, uint32_t page);
void lnskv_page_pool_reset(lnskv_page_pool* p);
uint32_t lnskv_page_pool_num_free(const lnskv_page_pool* p);
uint32_t lnskv_page_pool_capacity(const lnskv_page_pool* p);
uint32_t lnskv_page_pool_refcount(const lnskv_page_pool* p, uint32_t page);

/* Batched block tables: n_seq rows of max_pages u32 entries (LNSKV_NO_PAGE
 * initialised) and a per-row logical length, the batched form of the engine's
 * kv_block_tables (engine.rs:65) for one layer.  Row-major with stride
 * max_pages, so lnskv_block_tables_host() can be uploaded as is. */
typedef struct lnskv_block_tables lnskv_block_tables;
int lnskv_block_tables_create(int32_t n_seq, int32_t max_pages, lnskv_block_tables** out);
void lnskv_block_tables_destroy(lnskv_block_tables* t);
const uint32_t* lnskv_block_tables_host(const lnskv_block_tables* t);
int32_t lnskv_block_tables_stride(const lnskv_block_tables* t);
int32_t lnskv_block_tables_len(const lnskv_block_tables* t, int32_t seq);
/* clear_kv_cache's table part (engine.rs:2923-2930): every row emptied and
 * filled with LNSKV_NO_PAGE (pages are not returned; reset the pool too). */
void lnskv_block_tables_reset(lnskv_block_tables* t);

/* ensure_kv_page (engine.rs:2960-2974): make sure logical page pos/16 of row
 * seq has a physical page, allocating from pool.  On exhaustion returns
 * LNSKV_ERR_POOL_EXHAUSTED with "KV page pool exhausted at layer {layer}
 * (pos={pos})"; a position past the row's capacity returns LNSKV_ERR_INVALID
 * (the reference's fixed 2 KB table would overflow, engine.rs:2999-3003). */
int lnskv_ensure_kv_page(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t layer,
                         int32_t seq, int32_t pos);
/* evict_kv_pages (engine.rs:2976-2990): with window > 0, free every logical
 * page of row seq that lies wholly before kv_p_start(pos, window). */
int lnskv_evict_kv_pages(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t seq,
                         int32_t pos, int32_t window);
/* kv_p_start (engine.rs:3007-3013): pos - window + 1 clamped at 0, or 0. */
int32_t lnskv_kv_p_start(int32_t pos, int32_t window);
/* The per-token page step of a sliding-window layer with the reference's
 * exhaustion fixed: evict_kv_pages(pos, window) first, then
 * ensure_kv_page(pos).  The reference calls them the other way round
 * (engine.rs:1601-1603, 3231-3232) on a pool of ceil(window/16) pages
 * (engine.rs:726-730), which runs dry as soon as a window starts mid-page.
 * With window <= 0 it is ensure_kv_page alone. */
int lnskv_step_pages(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t layer, int32_t seq,
                     int32_t pos, int32_t window);
/* Pages a pool needs per sequence so that lnskv_step_pages never exhausts it
 * for a window of `window` tokens: the most pages any window of that many
 * consecutive positions touches, (window + 14) / 16 + 1.  0 for window <= 0
 * (full attention: the context length decides). */
int32_t lnskv_window_pages(int32_t window);
/* Free every page of row seq (sequence finished or evicted) and empty it. */
int lnskv_free_sequence(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t seq);
/* Copy-on-write fork: row child becomes a view of the first n_tok tokens of
 * row parent.  Full pages are shared (refcount + 1); a partially filled tail
 * page gets a fresh page, and the (src, dst) pair the device must copy is
 * written to *copy_src / *copy_dst with *n_copy = 1 (else 0).  Row child must
 * be empty. */
int lnskv_fork_sequence(lnskv_block_tables* t, lnskv_page_pool* pool, int32_t parent,
                        int32_t child, int32_t n_tok, uint32_t* copy_src, uint32_t* copy_dst,
                        int32_t* n_copy);
/* upload_block_table (engine.rs:2992-3005): copy rows [0, n_seq) to the device
 * table (same stride), async on stream.  The runtime stages the host rows
 * before the call returns (it does not wait for earlier work on the stream),
 * so the host table may be changed as soon as the call returns. */
int lnskv_block_tables_upload(const lnskv_block_tables* t, uint32_t* dst_dev,
                              lnskv_stream_t stream);
/* upload_block_table for a device table that stays with its host table (the
 * engine's kv_block_table_bufs[l], engine.rs:735-736, refreshed every token at
 * engine.rs:1604 and 3233): writes only the entries that changed since the
 * last lnskv_block_tables_sync of t.  The first call, and the first after
 * lnskv_block_tables_reset, writes every entry.  A call with nothing changed
 * (a decoding sequence gets a new page once every 16 tokens) enqueues
 * nothing; up to LNSKV_TABLE_PATCH_MAX changed entries travel by value in the
 * arguments of one small kernel; more, as one copy of the span holding them.
 * dst_dev must be the device table the previous sync of t wrote, written by
 * nothing else since.  Async on stream; the host table may change as soon as
 * the call returns. */
#define LNSKV_TABLE_PATCH_MAX 64
int lnskv_block_tables_sync(lnskv_block_tables* t, uint32_t* dst_dev, lnskv_stream_t stream);
/* Entries the next lnskv_block_tables_sync of t will write (host only). */
int64_t lnskv_block_tables_changed(const lnskv_block_tables* t);
/* The patch under lnskv_block_tables_sync, for callers that keep their own
 * host tables: dst_dev[idx[j]] = val[j] for j < n, 1 <= n <=
 * LNSKV_TABLE_PATCH_MAX, the pairs copied into the kernel's arguments before
 * the call returns.  Async on stream. */
int lnskv_block_table_patch(uint32_t* dst_dev, int32_t n, const uint32_t* idx, const uint32_t* val,
                            lnskv_stream_t stream);

/* ---------------------------------------------------------------------------
 * Measurement (no counterpart in the reference)
 * ---------------------------------------------------------------------------
 * lnskv_read_units: loads, with plain 16-byte loads and no arithmetic, the K
 * and V rows of units (unit_page[u], unit_kvh[u]) -- the 16 rows one kv head
 * holds in one page, per pool, and for Q8A pages their 16 K and 16 V scales --
 * wave w taking units [wave_start[w], wave_start[w + 1]) with two units in
 * flight.  Given the units of a decode step in the decode's order and wave
 * split, its duration is the load ceiling of that step's page pattern.  Rows
 * (head_dim x dtype bytes) of 256 bytes (f16 d128, f32 d64) or 512 (f16
 * d256), Q8A rows of 128 (d128) or 256 bytes (d256); page ids >= num_pages
 * and kv heads outside [0, n_kv_heads) read page 0 / kv head 0.  wave_start
 * holds n_waves + 1 non-decreasing indices into the unit lists.
 * sink[w * 64 + lane] receives the XOR of the 32-bit words lane loaded for
 * wave w's units, each unit once: with L = row bytes / 16 lanes per row, lane
 * (r, c) = (lane / L, lane % L) loads 16-byte chunk c of rows r, r + 64/L,
 * ... (< 16) of K and of V, and for Q8A pages also the scale of token
 * lane % 16 (V for lanes with bit 4 set, K otherwise). */
int lnskv_read_units(const lnskv_pages* c, const uint32_t* unit_page, const int32_t* unit_kvh,
                     const int32_t* wave_start, int32_t n_waves, uint32_t* sink,
                     lnskv_stream_t stream);
/* lnskv_read_stream: the plain read ceiling.  Reads bytes (a positive multiple
 * of 16) of buf_dev (16-byte aligned) front to back with 16-byte loads,
 * loads_in_flight (1, 2, 4, 8 or 16) per thread issued before any is used,
 * blocks_per_cu (1..8) workgroups of 256 threads per compute unit, thread t of
 * T reading chunks t, t + T, ... (each wave instruction 1 KiB contiguous).
 * Nothing is written except by a thread whose XOR of the 32-bit words it read
 * is 0x9E3779B9: it stores 1 to sink_dev[0] (this keeps the loads from being
 * elided). */
int lnskv_read_stream(const void* buf_dev, size_t bytes, int32_t loads_in_flight, int32_t blocks_per_cu,
                      uint32_t* sink_dev, lnskv_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LNSKV_H */
