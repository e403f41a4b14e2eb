//! Raw bindings of liblnskv's C ABI (`include/lnskv.h`), one `extern "C"`
//! declaration per entry point of the header, in its order, with the header's
//! parameter names.  C types map as: `int` -> `c_int`, `int32_t` -> `i32`,
//! `uint32_t` -> `u32`, `size_t` -> `usize`, `float` -> `f32`, `T*` ->
//! `*mut T`, `const T*` -> `*const T`, `lnskv_stream_t` -> [`HipStream`].
//! Every pointer named `*_dev` is device memory.  The safe layer is in
//! `lib.rs`; nothing here checks anything.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

/// `LNSKV_PAGE_SIZE`: token slots per page (engine.rs:16 `PAGE_SIZE`).
pub const LNSKV_PAGE_SIZE: u32 = 16;
/// `LNSKV_NO_PAGE`: an unallocated block-table entry (engine.rs:65 `u32::MAX`).
pub const LNSKV_NO_PAGE: u32 = 0xFFFF_FFFF;
/// `LNSKV_WORKSPACE_HEADER_BYTES`: the leading bytes of a decode workspace
/// that must be zero before its first use.
pub const LNSKV_WORKSPACE_HEADER_BYTES: usize = 4096;
/// `LNSKV_NOALLOC_SCRATCH_BYTES`: the static scratch of `lnskv_append_decode_noalloc`.
pub const LNSKV_NOALLOC_SCRATCH_BYTES: usize = 24 << 20;
/// `LNSKV_Q4L_DISK_BYTES` / `LNSKV_Q4L_DEVICE_BYTES`: one Q4_L super-block on disk / on the device.
pub const LNSKV_Q4L_DISK_BYTES: usize = 134;
pub const LNSKV_Q4L_DEVICE_BYTES: usize = 144;
/// `LNSKV_TABLE_PATCH_MAX`: changed block-table entries one patch writes by value.
pub const LNSKV_TABLE_PATCH_MAX: usize = 64;

/// `lnskv_dtype`.
pub const LNSKV_DTYPE_F32: i32 = 0;
pub const LNSKV_DTYPE_F16: i32 = 1;
pub const LNSKV_DTYPE_Q8A: i32 = 2;

/// `lnskv_status`.
pub const LNSKV_OK: c_int = 0;
pub const LNSKV_ERR_INVALID: c_int = -1;
pub const LNSKV_ERR_NOMEM: c_int = -2;
pub const LNSKV_ERR_POOL_EXHAUSTED: c_int = -3;
pub const LNSKV_ERR_HIP: c_int = -4;
pub const LNSKV_ERR_UNSUPPORTED: c_int = -5;
pub const LNSKV_ERR_WORKSPACE: c_int = -6;

/// `lnskv_rope_mode`.
pub const LNSKV_ROPE_DEFAULT: i32 = 0;
pub const LNSKV_ROPE_LINEAR: i32 = 1;
pub const LNSKV_ROPE_LLAMA3: i32 = 2;
pub const LNSKV_ROPE_YARN: i32 = 3;

/// `lnskv_stream_t`: a `hipStream_t`; null is the null stream.
pub type HipStream = *mut c_void;

/// `lnskv_pages`: one layer's K/V pools (replaces the k_cache, v_cache,
/// k_scales, v_scales buffers of `encode_attention_paged_q8a`, lib.rs:997-1010).
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct LnskvPages {
    pub k_pages: *mut c_void,
    pub v_pages: *mut c_void,
    pub k_scales: *mut f32,
    pub v_scales: *mut f32,
    pub num_pages: u32,
    pub n_kv_heads: u32,
    pub head_dim: u32,
    pub dtype: i32,
}

/// `lnskv_rope`: device inverse frequencies and the rotary width.
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct LnskvRope {
    pub inv_freqs_dev: *const f32,
    pub rotary_dim: i32,
}

/// Opaque `lnskv_page_pool` (the C++ pool; the crate's own pool is `paging::PagePool`).
#[repr(C)]
pub struct LnskvPagePool {
    _private: [u8; 0],
}

/// Opaque `lnskv_block_tables`.
#[repr(C)]
pub struct LnskvBlockTables {
    _private: [u8; 0],
}

extern "C" {
    pub fn lnskv_last_error() -> *const c_char;
    pub fn lnskv_version() -> *const c_char;
    pub fn lnskv_page_bytes(c: *const LnskvPages) -> usize;
    pub fn lnskv_pages_alloc(c: *mut LnskvPages) -> c_int;
    pub fn lnskv_pages_free(c: *mut LnskvPages) -> c_int;
    pub fn lnskv_clear(c: *const LnskvPages, stream: HipStream) -> c_int;
    pub fn lnskv_append(
        c: *const LnskvPages,
        k_new_dev: *const f32,
        v_new_dev: *const f32,
        tok_seq_dev: *const i32,
        tok_pos_dev: *const i32,
        n_tok: i32,
        block_tables_dev: *const u32,
        bt_stride: i32,
        n_rows: i32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_decode_workspace_size(
        c: *const LnskvPages,
        n_seq: i32,
        n_heads: i32,
        max_kv_len: i32,
        split_tokens: i32,
        bytes: *mut usize,
    ) -> c_int;
    pub fn lnskv_decode(
        c: *const LnskvPages,
        q_dev: *const f32,
        out_dev: *mut f32,
        block_tables_dev: *const u32,
        bt_stride: i32,
        kv_len_dev: *const i32,
        p_start_dev: *const i32,
        n_seq: i32,
        n_heads: i32,
        max_kv_len: i32,
        scale: f32,
        split_tokens: i32,
        workspace_dev: *mut c_void,
        ws_bytes: usize,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_append_decode(
        c: *const LnskvPages,
        q_dev: *const f32,
        k_new_dev: *const f32,
        v_new_dev: *const f32,
        out_dev: *mut f32,
        block_tables_dev: *const u32,
        bt_stride: i32,
        kv_len_dev: *const i32,
        p_start_dev: *const i32,
        n_seq: i32,
        n_heads: i32,
        max_kv_len: i32,
        scale: f32,
        split_tokens: i32,
        workspace_dev: *mut c_void,
        ws_bytes: usize,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_append_decode_noalloc(
        c: *const LnskvPages,
        q_dev: *const f32,
        k_new_dev: *const f32,
        v_new_dev: *const f32,
        out_dev: *mut f32,
        block_tables_dev: *const u32,
        bt_stride: i32,
        kv_len_dev: *const i32,
        p_start_dev: *const i32,
        n_seq: i32,
        n_heads: i32,
        max_kv_len: i32,
        scale: f32,
        split_tokens: i32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_rope_dim(head_dim: i32, partial_rotary_factor: f32) -> i32;
    pub fn lnskv_rope_inv_freqs(
        rotary_dim: i32,
        theta: f32,
        mode: i32,
        params: *const f32,
        inv_freqs_host: *mut f32,
    ) -> c_int;
    pub fn lnskv_rope_append_workspace_size(
        c: *const LnskvPages,
        rope: *const LnskvRope,
        n_tok: i32,
        bytes: *mut usize,
    ) -> c_int;
    pub fn lnskv_rope_append(
        c: *const LnskvPages,
        rope: *const LnskvRope,
        k_new_dev: *const f32,
        v_new_dev: *const f32,
        tok_seq_dev: *const i32,
        tok_pos_dev: *const i32,
        n_tok: i32,
        block_tables_dev: *const u32,
        bt_stride: i32,
        n_rows: i32,
        workspace_dev: *mut c_void,
        ws_bytes: usize,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_rope_decode_workspace_size(
        c: *const LnskvPages,
        rope: *const LnskvRope,
        n_seq: i32,
        n_heads: i32,
        max_kv_len: i32,
        split_tokens: i32,
        bytes: *mut usize,
    ) -> c_int;
    pub fn lnskv_rope_append_decode(
        c: *const LnskvPages,
        rope: *const LnskvRope,
        q_dev: *const f32,
        k_new_dev: *const f32,
        v_new_dev: *const f32,
        out_dev: *mut f32,
        block_tables_dev: *const u32,
        bt_stride: i32,
        kv_len_dev: *const i32,
        p_start_dev: *const i32,
        n_seq: i32,
        n_heads: i32,
        max_kv_len: i32,
        scale: f32,
        split_tokens: i32,
        workspace_dev: *mut c_void,
        ws_bytes: usize,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_prefill_attention(
        c: *const LnskvPages,
        q_dev: *const f32,
        out_dev: *mut f32,
        chunks_dev: *const i32,
        n_chunks: i32,
        n_tok: i32,
        block_tables_dev: *const u32,
        bt_stride: i32,
        n_rows: i32,
        p_start_dev: *const i32,
        window: i32,
        n_heads: i32,
        scale: f32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_split_gated_query(
        input_dev: *const f32,
        q_out_dev: *mut f32,
        gate_out_dev: *mut f32,
        n_rows: i32,
        n_heads: i32,
        head_dim: i32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_gated_append_decode(
        c: *const LnskvPages,
        rope: *const LnskvRope,
        gate_dev: *const f32,
        q_dev: *const f32,
        k_new_dev: *const f32,
        v_new_dev: *const f32,
        out_dev: *mut f32,
        block_tables_dev: *const u32,
        bt_stride: i32,
        kv_len_dev: *const i32,
        p_start_dev: *const i32,
        n_seq: i32,
        n_heads: i32,
        max_kv_len: i32,
        scale: f32,
        split_tokens: i32,
        workspace_dev: *mut c_void,
        ws_bytes: usize,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_q4l_prepare(
        disk_blocks: *const c_void,
        disk_bytes: usize,
        rows: i32,
        cols: i32,
        out_blocks: *mut c_void,
    ) -> c_int;
    pub fn lnskv_q4l_workspace_size(cols: i32, n_vec: i32, bytes: *mut usize) -> c_int;
    pub fn lnskv_q4l_gemv_accumulate(
        blocks_dev: *const c_void,
        x_dev: *const f32,
        y_dev: *mut f32,
        rows: i32,
        cols: i32,
        n_vec: i32,
        x_stride: i32,
        y_stride: i32,
        workspace_dev: *mut c_void,
        ws_bytes: usize,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_attention_paged(
        q_dev: *const f32,
        k_in_dev: *const f32,
        v_in_dev: *const f32,
        c: *const LnskvPages,
        block_table_dev: *const u32,
        out_dev: *mut f32,
        pos: u32,
        head_dim: u32,
        n_heads: u32,
        n_kv_heads: u32,
        p_start: u32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_dispatch_attention_paged(
        q_dev: *const f32,
        k_in_dev: *const f32,
        v_in_dev: *const f32,
        c: *const LnskvPages,
        block_table_dev: *const u32,
        out_dev: *mut f32,
        pos: u32,
        head_dim: u32,
        n_heads: u32,
        n_kv_heads: u32,
        p_start: u32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_page_copy(
        c: *const LnskvPages,
        src_dev: *const u32,
        dst_dev: *const u32,
        n: i32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_gather(
        c: *const LnskvPages,
        block_table_dev: *const u32,
        start: i32,
        n_tok: i32,
        k_out_dev: *mut c_void,
        v_out_dev: *mut c_void,
        ks_out_dev: *mut f32,
        vs_out_dev: *mut f32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_sync(stream: HipStream) -> c_int;
    pub fn lnskv_workspace_reserve(decode_bytes: usize, rope_bytes: usize, q4l_bytes: usize) -> c_int;
    pub fn lnskv_workspace_release() -> c_int;
    pub fn lnskv_page_pool_create(capacity: u32, out: *mut *mut LnskvPagePool) -> c_int;
    pub fn lnskv_page_pool_destroy(p: *mut LnskvPagePool);
    pub fn lnskv_page_pool_alloc(p: *mut LnskvPagePool, page_out: *mut u32) -> c_int;
    pub fn lnskv_page_pool_free(p: *mut LnskvPagePool, page: u32) -> c_int;
    pub fn lnskv_page_pool_retain(p: *mut LnskvPagePool, page: u32) -> c_int;
    pub fn lnskv_page_pool_reset(p: *mut LnskvPagePool);
    pub fn lnskv_page_pool_num_free(p: *const LnskvPagePool) -> u32;
    pub fn lnskv_page_pool_capacity(p: *const LnskvPagePool) -> u32;
    pub fn lnskv_page_pool_refcount(p: *const LnskvPagePool, page: u32) -> u32;
    pub fn lnskv_block_tables_create(n_seq: i32, max_pages: i32, out: *mut *mut LnskvBlockTables) -> c_int;
    pub fn lnskv_block_tables_destroy(t: *mut LnskvBlockTables);
    pub fn lnskv_block_tables_host(t: *const LnskvBlockTables) -> *const u32;
    pub fn lnskv_block_tables_stride(t: *const LnskvBlockTables) -> i32;
    pub fn lnskv_block_tables_len(t: *const LnskvBlockTables, seq: i32) -> i32;
    pub fn lnskv_block_tables_reset(t: *mut LnskvBlockTables);
    pub fn lnskv_ensure_kv_page(
        t: *mut LnskvBlockTables,
        pool: *mut LnskvPagePool,
        layer: i32,
        seq: i32,
        pos: i32,
    ) -> c_int;
    pub fn lnskv_evict_kv_pages(
        t: *mut LnskvBlockTables,
        pool: *mut LnskvPagePool,
        seq: i32,
        pos: i32,
        window: i32,
    ) -> c_int;
    pub fn lnskv_kv_p_start(pos: i32, window: i32) -> i32;
    pub fn lnskv_step_pages(
        t: *mut LnskvBlockTables,
        pool: *mut LnskvPagePool,
        layer: i32,
        seq: i32,
        pos: i32,
        window: i32,
    ) -> c_int;
    pub fn lnskv_window_pages(window: i32) -> i32;
    pub fn lnskv_free_sequence(t: *mut LnskvBlockTables, pool: *mut LnskvPagePool, seq: i32) -> c_int;
    pub fn lnskv_fork_sequence(
        t: *mut LnskvBlockTables,
        pool: *mut LnskvPagePool,
        parent: i32,
        child: i32,
        n_tok: i32,
        copy_src: *mut u32,
        copy_dst: *mut u32,
        n_copy: *mut i32,
    ) -> c_int;
    pub fn lnskv_block_tables_upload(
        t: *const LnskvBlockTables,
        dst_dev: *mut u32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_block_tables_sync(t: *mut LnskvBlockTables, dst_dev: *mut u32, stream: HipStream) -> c_int;
    pub fn lnskv_block_tables_changed(t: *const LnskvBlockTables) -> i64;
    pub fn lnskv_block_table_patch(
        dst_dev: *mut u32,
        n: i32,
        idx: *const u32,
        val: *const u32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_read_units(
        c: *const LnskvPages,
        unit_page: *const u32,
        unit_kvh: *const i32,
        wave_start: *const i32,
        n_waves: i32,
        sink: *mut u32,
        stream: HipStream,
    ) -> c_int;
    pub fn lnskv_read_stream(
        buf_dev: *const c_void,
        bytes: usize,
        loads_in_flight: i32,
        blocks_per_cu: i32,
        sink_dev: *mut u32,
        stream: HipStream,
    ) -> c_int;
}
