//! lns-kv-hip: lns-inference's paged KV cache on MI355X (gfx950).
//!
//! The drop-in for the engine's Metal paged path:
//! - [`KvLayer`] holds one layer's K/V pools (the engine's `paged_kv_data` /
//!   `paged_kv_scales` buffers, `engine.rs:62-63, 717-773`) in the
//!   reference's page layout `[page][16][n_kv][head_dim]`, Q8A by default;
//! - [`KvLayer::attention_paged`] replaces `attention_paged_q8a_enc` /
//!   `encode_attention_paged_q8a` (`lns-metal/src/lib.rs:997-1043,
//!   2085-2129`) with the same arguments in the same order, and
//!   [`KvLayer::dispatch_attention_paged`] the waiting `dispatch_` form
//!   (`:1046-1094`);
//! - [`KvPaging`] is one layer's `PagePool` + block table + device table
//!   (`engine.rs:20-44, 65-66, 2958-3013`), host code in Rust
//!   ([`paging`]), with the sliding-window exhaustion fixed;
//! - [`KvLayer::append_decode`] is the batched serving form (one call per
//!   layer for every decoding sequence);
//! - [`Q4lMatrix`] is a Q4_L weight matrix on the device (`prepare_tensor`,
//!   `lns-metal/src/lib.rs:1255-1320`) and [`Q4lMatrix::gemv_accumulate`] the
//!   o_proj after the attention (`gemv_accumulate_multirow_enc`,
//!   `engine.rs:3433-3446`) for every decoding sequence in one call.
//!
//! Errors are the reference's `Result<(), String>`; library failures carry
//! liblnskv's message (for pool exhaustion, the engine's own text).  Device
//! work is asynchronous on the given HIP stream (null: the null stream), as
//! the reference's encoder calls are on its command buffer.

pub mod hip;
pub mod paging;
pub mod sys;

use std::ffi::CStr;
use std::os::raw::{c_int, c_void};
use std::ptr;

pub use hip::{stream_synchronize, DeviceBuffer};
pub use paging::{flatten_tables, kv_p_start, window_pages, BlockTable, PagePool, NO_PAGE, PAGE_SIZE};
pub use sys::HipStream;

/// liblnskv status -> the reference's `Result<(), String>`.
pub fn check(rc: c_int) -> Result<(), String> {
    if rc == sys::LNSKV_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(sys::lnskv_last_error()) };
    Err(msg.to_string_lossy().into_owned())
}

/// liblnskv's build string (names the gfx target).
pub fn version() -> String {
    unsafe { CStr::from_ptr(sys::lnskv_version()) }.to_string_lossy().into_owned()
}

/// Page element type: Q8A is the reference's (`lns_decode.metal:547-593`).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum KvDtype {
    F32,
    F16,
    Q8A,
}

impl KvDtype {
    pub fn raw(self) -> i32 {
        match self {
            KvDtype::F32 => sys::LNSKV_DTYPE_F32,
            KvDtype::F16 => sys::LNSKV_DTYPE_F16,
            KvDtype::Q8A => sys::LNSKV_DTYPE_Q8A,
        }
    }
}

/// One layer's paged K/V pools on the device, freed on drop.
pub struct KvLayer {
    pages: sys::LnskvPages,
}

unsafe impl Send for KvLayer {}

/// Device pointers of one batched append + decode step (`lnskv_append_decode`).
#[derive(Clone, Copy, Debug)]
pub struct DecodeBatch {
    /// `[n_seq][n_heads][head_dim]` f32
    pub q: *const f32,
    /// `[n_seq][n_kv][head_dim]` f32: the new token of every sequence
    pub k_new: *const f32,
    pub v_new: *const f32,
    /// `[n_seq][n_heads][head_dim]` f32
    pub out: *mut f32,
    /// `[n_seq][bt_stride]` u32, `NO_PAGE` where unmapped
    pub block_tables: *const u32,
    pub bt_stride: usize,
    /// `[n_seq]` i32, including the new token (the reference's `pos + 1`)
    pub kv_len: *const i32,
    /// `[n_seq]` i32 window starts, or null for 0
    pub p_start: *const i32,
    pub n_seq: usize,
    pub n_heads: usize,
    pub max_kv_len: usize,
    pub scale: f32,
    /// 0: the library schedules (stream-K on the matrix cores for f16/Q8A, d=128)
    pub split_tokens: usize,
}

fn i32_of(x: usize, what: &str) -> Result<i32, String> {
    i32::try_from(x).map_err(|_| format!("{what} = {x} does not fit in i32"))
}

fn u32_of(x: usize, what: &str) -> Result<u32, String> {
    u32::try_from(x).map_err(|_| format!("{what} = {x} does not fit in u32"))
}

impl KvLayer {
    /// Zeroed pools of `num_pages` pages (`lnskv_pages_alloc`).
    pub fn new(num_pages: u32, n_kv_heads: u32, head_dim: u32, dtype: KvDtype) -> Result<Self, String> {
        let mut pages = sys::LnskvPages {
            k_pages: ptr::null_mut(),
            v_pages: ptr::null_mut(),
            k_scales: ptr::null_mut(),
            v_scales: ptr::null_mut(),
            num_pages,
            n_kv_heads,
            head_dim,
            dtype: dtype.raw(),
        };
        check(unsafe { sys::lnskv_pages_alloc(&mut pages) })?;
        Ok(Self { pages })
    }

    /// The descriptor the C ABI takes.
    pub fn desc(&self) -> &sys::LnskvPages {
        &self.pages
    }

    /// `clear_kv_cache`'s data part (`engine.rs:2912-2922`).
    pub fn clear(&self, stream: HipStream) -> Result<(), String> {
        check(unsafe { sys::lnskv_clear(&self.pages, stream) })
    }

    /// `attention_paged_q8a_enc(enc, q, k, v, k_cache, v_cache, k_scales,
    /// v_scales, block_table, out, pos, head_dim, n_heads, n_kv_heads,
    /// p_start)` (`lns-metal/src/lib.rs:2085-2129`): append the token at
    /// `pos` (`k_in`, `v_in`: `[n_kv * head_dim]` f32 on the device) into its
    /// page and attend `[p_start, pos]` with scale `1/sqrt(head_dim)`; `out`
    /// gets `[n_heads][head_dim]` f32.  The page of `pos` must be mapped in
    /// `block_table_dev` (`KvPaging::step` first, as the engine's order has it).
    #[allow(clippy::too_many_arguments)]
    pub fn attention_paged(
        &self,
        q: *const f32,
        k_in: *const f32,
        v_in: *const f32,
        block_table_dev: *const u32,
        out: *mut f32,
        pos: usize,
        head_dim: usize,
        n_heads: usize,
        n_kv_heads: usize,
        p_start: usize,
        stream: HipStream,
    ) -> Result<(), String> {
        check(unsafe {
            sys::lnskv_attention_paged(
                q,
                k_in,
                v_in,
                &self.pages,
                block_table_dev,
                out,
                u32_of(pos, "pos")?,
                u32_of(head_dim, "head_dim")?,
                u32_of(n_heads, "n_heads")?,
                u32_of(n_kv_heads, "n_kv_heads")?,
                u32_of(p_start, "p_start")?,
                stream,
            )
        })
    }

    /// `dispatch_attention_paged_q8a` (`lib.rs:1046-1094`): as
    /// [`attention_paged`](Self::attention_paged), then waits for completion.
    #[allow(clippy::too_many_arguments)]
    pub fn dispatch_attention_paged(
        &self,
        q: *const f32,
        k_in: *const f32,
        v_in: *const f32,
        block_table_dev: *const u32,
        out: *mut f32,
        pos: usize,
        head_dim: usize,
        n_heads: usize,
        n_kv_heads: usize,
        p_start: usize,
        stream: HipStream,
    ) -> Result<(), String> {
        check(unsafe {
            sys::lnskv_dispatch_attention_paged(
                q,
                k_in,
                v_in,
                &self.pages,
                block_table_dev,
                out,
                u32_of(pos, "pos")?,
                u32_of(head_dim, "head_dim")?,
                u32_of(n_heads, "n_heads")?,
                u32_of(n_kv_heads, "n_kv_heads")?,
                u32_of(p_start, "p_start")?,
                stream,
            )
        })
    }

    /// Bytes of device workspace [`append_decode`](Self::append_decode) needs
    /// for this batch shape.
    pub fn decode_workspace_size(
        &self,
        n_seq: usize,
        n_heads: usize,
        max_kv_len: usize,
        split_tokens: usize,
    ) -> Result<usize, String> {
        let mut bytes = 0usize;
        check(unsafe {
            sys::lnskv_decode_workspace_size(
                &self.pages,
                i32_of(n_seq, "n_seq")?,
                i32_of(n_heads, "n_heads")?,
                i32_of(max_kv_len, "max_kv_len")?,
                i32_of(split_tokens, "split_tokens")?,
                &mut bytes,
            )
        })?;
        Ok(bytes)
    }

    /// Every sequence's new token appended and attended in one call
    /// (`lnskv_append_decode`).  `workspace`: a device buffer of at least
    /// `decode_workspace_size` bytes (per stream) made by
    /// [`DeviceBuffer::zeroed`] (its first `LNSKV_WORKSPACE_HEADER_BYTES`
    /// must be zero; every call leaves them so), or `None` for the library's
    /// per-device buffer (calls must then not overlap).
    pub fn append_decode(
        &self,
        b: &DecodeBatch,
        workspace: Option<&mut DeviceBuffer<u8>>,
        stream: HipStream,
    ) -> Result<(), String> {
        let (ws, ws_bytes) = match workspace {
            Some(w) => (w.as_mut_ptr() as *mut c_void, w.len()),
            None => (ptr::null_mut(), 0),
        };
        check(unsafe {
            sys::lnskv_append_decode(
                &self.pages,
                b.q,
                b.k_new,
                b.v_new,
                b.out,
                b.block_tables,
                i32_of(b.bt_stride, "bt_stride")?,
                b.kv_len,
                b.p_start,
                i32_of(b.n_seq, "n_seq")?,
                i32_of(b.n_heads, "n_heads")?,
                i32_of(b.max_kv_len, "max_kv_len")?,
                b.scale,
                i32_of(b.split_tokens, "split_tokens")?,
                ws,
                ws_bytes,
                stream,
            )
        })
    }

    /// Pages `dst_dev[i] <- src_dev[i]` for K, V and the Q8A scales
    /// (copy-on-write forks: the `(src, dst)` pairs [`BlockTable::fork`] returns).
    pub fn page_copy(&self, src_dev: *const u32, dst_dev: *const u32, n: usize, stream: HipStream) -> Result<(), String> {
        check(unsafe { sys::lnskv_page_copy(&self.pages, src_dev, dst_dev, i32_of(n, "n")?, stream) })
    }

    /// Tokens `[start, start + n_tok)` of one sequence copied out of the pages
    /// (`k_out`/`v_out`: `[n_tok][n_kv][head_dim]` in the page type; Q8A scales
    /// `[n_tok][n_kv]` f32, or null).
    #[allow(clippy::too_many_arguments)]
    pub fn gather(
        &self,
        block_table_dev: *const u32,
        start: usize,
        n_tok: usize,
        k_out: *mut c_void,
        v_out: *mut c_void,
        ks_out: *mut f32,
        vs_out: *mut f32,
        stream: HipStream,
    ) -> Result<(), String> {
        check(unsafe {
            sys::lnskv_gather(
                &self.pages,
                block_table_dev,
                i32_of(start, "start")?,
                i32_of(n_tok, "n_tok")?,
                k_out,
                v_out,
                ks_out,
                vs_out,
                stream,
            )
        })
    }
}

impl Drop for KvLayer {
    fn drop(&mut self) {
        unsafe {
            let _ = sys::lnskv_pages_free(&mut self.pages);
        }
    }
}

/// One layer's page bookkeeping for one sequence: the engine's
/// `kv_page_pools[l]`, `kv_block_tables[l]` and `kv_block_table_bufs[l]`
/// (`engine.rs:64-66`), with the device table sized to the table's capacity.
pub struct KvPaging {
    pub layer: usize,
    pub pool: PagePool,
    pub table: BlockTable,
    table_dev: DeviceBuffer<u32>,
    // the entries the device table holds (what the last upload wrote); None
    // until the first upload
    on_device: Option<Vec<u32>>,
}

impl KvPaging {
    /// A pool of `capacity` pages (for a sliding window of `w` tokens,
    /// `window_pages(w)` is enough) and a table of `max_pages` entries.
    pub fn new(layer: usize, capacity: usize, max_pages: usize) -> Result<Self, String> {
        Ok(Self {
            layer,
            pool: PagePool::new(capacity),
            table: BlockTable::new(max_pages),
            table_dev: DeviceBuffer::new(max_pages)?,
            on_device: None,
        })
    }

    /// The step before the attention at `pos` (`engine.rs:3218-3233`): evict
    /// what left the window, map the page of `pos`, upload the table on the
    /// stream the attention is then enqueued on.
    pub fn step(&mut self, pos: usize, window: usize, stream: HipStream) -> Result<(), String> {
        self.table.step_pages(&mut self.pool, self.layer, pos, window)?;
        self.upload(stream)
    }

    /// `upload_block_table` (`engine.rs:2992-3005`): the table's entries into
    /// the device table, ordered on `stream` after the work already queued
    /// there (a previous step's attention still reading the table finishes
    /// first); the host rows are staged before the call returns.
    /// Only the entries that differ from what the device table holds are
    /// written: none on most tokens (a new page comes every 16), up to
    /// `LNSKV_TABLE_PATCH_MAX` by value through `lnskv_block_table_patch`
    /// (no staging copy), the whole row otherwise.
    pub fn upload(&mut self, stream: HipStream) -> Result<(), String> {
        let now = self.table.as_slice();
        if let Some(dev) = &self.on_device {
            let mut idx: Vec<u32> = Vec::new();
            let mut val: Vec<u32> = Vec::new();
            for (i, &v) in now.iter().enumerate() {
                if dev.get(i) != Some(&v) {
                    idx.push(i as u32);
                    val.push(v);
                }
            }
            if idx.is_empty() {
                return Ok(());
            }
            if idx.len() <= sys::LNSKV_TABLE_PATCH_MAX {
                let dst = self.table_dev.as_mut_ptr();
                check(unsafe {
                    sys::lnskv_block_table_patch(dst, idx.len() as i32, idx.as_ptr(), val.as_ptr(), stream)
                })?;
                self.on_device = Some(now.to_vec());
                return Ok(());
            }
        }
        self.table_dev.copy_from_async(now, stream)?;
        self.on_device = Some(now.to_vec());
        Ok(())
    }

    /// The device table `attention_paged` reads.
    pub fn table_dev(&self) -> *const u32 {
        self.table_dev.as_ptr()
    }

    /// `clear_kv_cache`'s table and pool part (`engine.rs:2923-2930`).
    pub fn reset(&mut self) {
        self.pool.reset();
        self.table = BlockTable::new(self.table.max_pages());
        self.on_device = None;
    }
}

/// One Q4_L weight matrix on the device: the disk super-blocks
/// (`LNSKV_Q4L_DISK_BYTES` per 256 weights, row-major) repacked by
/// `lnskv_q4l_prepare` into device blocks and uploaded once, as
/// `prepare_tensor(.., QuantType::Q4L)` does (`lns-metal/src/lib.rs:1255-1320`),
/// plus the GEMV's workspace.
pub struct Q4lMatrix {
    pub rows: usize,
    pub cols: usize,
    blocks: DeviceBuffer<u8>,
    workspace: DeviceBuffer<u8>,
    ws_vectors: usize,
}

impl Q4lMatrix {
    pub fn prepare(disk: &[u8], rows: usize, cols: usize) -> Result<Self, String> {
        let n_blocks = rows * ((cols + 255) / 256);
        let mut host = vec![0u8; n_blocks * sys::LNSKV_Q4L_DEVICE_BYTES];
        check(unsafe {
            sys::lnskv_q4l_prepare(
                disk.as_ptr() as *const c_void,
                disk.len(),
                rows as i32,
                cols as i32,
                host.as_mut_ptr() as *mut c_void,
            )
        })?;
        Ok(Self {
            rows,
            cols,
            blocks: DeviceBuffer::from_slice(&host)?,
            workspace: DeviceBuffer::new(0)?,
            ws_vectors: 0,
        })
    }

    /// `gemv_accumulate_multirow_enc(enc, o_proj, attn_out, x, dim, attn_dim)`
    /// (`engine.rs:3433-3446`) for `n_vec` sequences at once: x[v] += W
    /// attn_out[v], with attn_out `[n_vec][cols]` and x `[n_vec][rows]` f32 on
    /// the device.  The workspace grows to the largest `n_vec` seen; its
    /// arrival counts start at zero and every call leaves them zero, so calls
    /// on one matrix must not overlap in time.
    pub fn gemv_accumulate(
        &mut self,
        attn_out_dev: *const f32,
        x_dev: *mut f32,
        n_vec: usize,
        stream: HipStream,
    ) -> Result<(), String> {
        if n_vec > self.ws_vectors {
            let mut bytes: usize = 0;
            check(unsafe { sys::lnskv_q4l_workspace_size(self.cols as i32, n_vec as i32, &mut bytes) })?;
            self.workspace = DeviceBuffer::zeroed(bytes.max(16))?;
            self.ws_vectors = n_vec;
        }
        check(unsafe {
            sys::lnskv_q4l_gemv_accumulate(
                self.blocks.as_ptr() as *const c_void,
                attn_out_dev,
                x_dev,
                self.rows as i32,
                self.cols as i32,
                n_vec as i32,
                self.cols as i32,
                self.rows as i32,
                self.workspace.as_mut_ptr() as *mut c_void,
                self.workspace.len(),
                stream,
            )
        })
    }
}
