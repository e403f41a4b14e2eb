//! Host-side page bookkeeping in Rust: the engine's `PagePool` and its
//! per-sequence block-table helpers, rewritten for a drop-in.
//!
//! Follows `lns-inference/src/engine.rs`:
//! - `PagePool` (`:20-44`): a FIFO free list of physical page ids, `new(cap)`
//!   holding `0..cap` in order, `alloc` = `pop_front`, `free_page` =
//!   `push_back`, `reset` refills `0..cap`;
//! - the block table `Vec<u32>` per layer (`:65`, `u32::MAX` = no page) and
//!   its helpers `ensure_kv_page` (`:2960-2974`), `evict_kv_pages`
//!   (`:2976-2990`), `upload_block_table` (`:2992-3005`) and `kv_p_start`
//!   (`:3007-3013`).
//!
//! Three things differ, each on purpose:
//! - every page carries a reference count, so that copy-on-write forks can
//!   share full pages; `free_page` returns a page to the free list when its
//!   count reaches zero (without `retain` the order is the reference's);
//! - a table has a fixed capacity and a position past it is an error, where
//!   the engine's upload would overflow its fixed 2 KB device buffer;
//! - [`BlockTable::step_pages`] evicts before it ensures.  The engine calls
//!   them the other way round (`:1601-1603`, `:3231-3232`) on a pool of
//!   `ceil(w/16)` pages (`:726-730`), which runs dry as soon as a window
//!   starts mid-page; [`window_pages`] gives the pool size the fixed order
//!   needs.

use std::collections::VecDeque;

/// Token slots per page (`engine.rs:16`).
pub const PAGE_SIZE: usize = 16;
/// An unallocated block-table entry (`engine.rs:65`).
pub const NO_PAGE: u32 = u32::MAX;

/// FIFO free list of physical page ids with a reference count per page.
#[derive(Debug, Clone)]
pub struct PagePool {
    capacity: usize,
    free: VecDeque<u32>,
    refs: Vec<u32>,
}

impl PagePool {
    /// `PagePool::new` (`engine.rs:27-32`): pages `0..capacity`, all free.
    pub fn new(capacity: usize) -> Self {
        assert!(capacity <= u32::MAX as usize, "page ids are u32");
        Self { capacity, free: (0..capacity as u32).collect(), refs: vec![0; capacity] }
    }

    /// `alloc` (`engine.rs:33-35`): the front of the free list, or `None`
    /// when the pool is exhausted.
    pub fn alloc(&mut self) -> Option<u32> {
        let p = self.free.pop_front()?;
        self.refs[p as usize] = 1;
        Some(p)
    }

    /// `free_page` (`engine.rs:36-38`): drops one reference; the page goes to
    /// the back of the free list when none is left.
    pub fn free_page(&mut self, idx: u32) -> Result<(), String> {
        let i = idx as usize;
        if i >= self.capacity {
            return Err(format!("page {idx} is outside the pool of {} pages", self.capacity));
        }
        if self.refs[i] == 0 {
            return Err(format!("page {idx} is not allocated"));
        }
        self.refs[i] -= 1;
        if self.refs[i] == 0 {
            self.free.push_back(idx);
        }
        Ok(())
    }

    /// One more holder of an allocated page (a copy-on-write share).
    pub fn retain(&mut self, idx: u32) -> Result<(), String> {
        let i = idx as usize;
        if i >= self.capacity || self.refs[i] == 0 {
            return Err(format!("page {idx} is not allocated"));
        }
        self.refs[i] += 1;
        Ok(())
    }

    /// `reset` (`engine.rs:39-42`): every page free again, in order.
    pub fn reset(&mut self) {
        self.free.clear();
        self.free.extend(0..self.capacity as u32);
        self.refs.iter_mut().for_each(|r| *r = 0);
    }

    pub fn capacity(&self) -> usize {
        self.capacity
    }

    pub fn num_free(&self) -> usize {
        self.free.len()
    }

    pub fn refcount(&self, idx: u32) -> u32 {
        self.refs.get(idx as usize).copied().unwrap_or(0)
    }
}

/// `kv_p_start` (`engine.rs:3007-3013`): the first position a sliding window
/// of `window` tokens attends at `pos` (0 for `window == 0`, full attention).
pub fn kv_p_start(pos: usize, window: usize) -> usize {
    if window > 0 {
        pos.saturating_sub(window - 1)
    } else {
        0
    }
}

/// Pages per sequence that [`BlockTable::step_pages`] needs for a sliding
/// window: the most pages any `window` consecutive positions touch,
/// `(window + 14) / 16 + 1`; 0 for full attention (`window == 0`).
pub fn window_pages(window: usize) -> usize {
    if window == 0 {
        0
    } else {
        (window + PAGE_SIZE - 2) / PAGE_SIZE + 1
    }
}

/// One sequence's block table in one layer: logical page `pos / 16` to
/// physical page, `NO_PAGE` where none is mapped, at most `max_pages` entries.
#[derive(Debug, Clone)]
pub struct BlockTable {
    pages: Vec<u32>,
    max_pages: usize,
}

impl BlockTable {
    pub fn new(max_pages: usize) -> Self {
        Self { pages: Vec::new(), max_pages }
    }

    /// The mapped entries, logical page order (what `upload` copies).
    pub fn as_slice(&self) -> &[u32] {
        &self.pages
    }

    pub fn max_pages(&self) -> usize {
        self.max_pages
    }

    /// `ensure_kv_page` (`engine.rs:2960-2974`): map the logical page of `pos`,
    /// allocating it from `pool` on first touch.  Exhaustion gives the
    /// reference's message; a position past the table's capacity is an error.
    pub fn ensure_kv_page(&mut self, pool: &mut PagePool, layer: usize, pos: usize) -> Result<(), String> {
        let lp = pos / PAGE_SIZE;
        if lp < self.pages.len() && self.pages[lp] != NO_PAGE {
            return Ok(());
        }
        if lp >= self.max_pages {
            return Err(format!(
                "position {pos} needs logical page {lp}; the table holds {} pages",
                self.max_pages
            ));
        }
        while self.pages.len() <= lp {
            self.pages.push(NO_PAGE);
        }
        let phys = pool
            .alloc()
            .ok_or_else(|| format!("KV page pool exhausted at layer {layer} (pos={pos})"))?;
        self.pages[lp] = phys;
        Ok(())
    }

    /// `evict_kv_pages` (`engine.rs:2976-2990`): with `window > 0`, return to
    /// the pool every logical page that lies wholly before `kv_p_start(pos)`.
    pub fn evict_kv_pages(&mut self, pool: &mut PagePool, pos: usize, window: usize) -> Result<(), String> {
        if window == 0 {
            return Ok(());
        }
        let evict_before = kv_p_start(pos, window) / PAGE_SIZE;
        let n = evict_before.min(self.pages.len());
        for lp in 0..n {
            let phys = self.pages[lp];
            if phys != NO_PAGE {
                pool.free_page(phys)?;
                self.pages[lp] = NO_PAGE;
            }
        }
        Ok(())
    }

    /// The per-token page step with the exhaustion fixed: evict, then ensure.
    /// A pool of `window_pages(window)` pages per sequence never runs dry.
    pub fn step_pages(&mut self, pool: &mut PagePool, layer: usize, pos: usize, window: usize) -> Result<(), String> {
        self.evict_kv_pages(pool, pos, window)?;
        self.ensure_kv_page(pool, layer, pos)
    }

    /// Every mapped page back to the pool (the sequence ended or was evicted).
    pub fn free_all(&mut self, pool: &mut PagePool) -> Result<(), String> {
        for p in self.pages.iter_mut() {
            if *p != NO_PAGE {
                pool.free_page(*p)?;
                *p = NO_PAGE;
            }
        }
        self.pages.clear();
        Ok(())
    }

    /// Copy-on-write fork of the first `n_tok` tokens: full pages are shared
    /// (one more reference each); a partly filled last page gets a fresh
    /// page, and `(src, dst)` is the page the device must copy
    /// (`lnskv_page_copy`).
    pub fn fork(&self, pool: &mut PagePool, n_tok: usize) -> Result<(BlockTable, Option<(u32, u32)>), String> {
        let n_pages = (n_tok + PAGE_SIZE - 1) / PAGE_SIZE;
        if n_pages > self.pages.len() {
            return Err(format!("fork of {n_tok} tokens: the parent maps {} pages", self.pages.len()));
        }
        let full = n_tok / PAGE_SIZE;
        let mut child = BlockTable::new(self.max_pages);
        for lp in 0..full {
            let p = self.pages[lp];
            if p != NO_PAGE {
                pool.retain(p)?;
            }
            child.pages.push(p);
        }
        let mut copy = None;
        if n_pages > full {
            let src = self.pages[full];
            if src == NO_PAGE {
                child.pages.push(NO_PAGE);
            } else {
                let dst = match pool.alloc() {
                    Some(d) => d,
                    None => {
                        child.free_all(pool)?;
                        return Err(format!("KV page pool exhausted forking {n_tok} tokens"));
                    }
                };
                child.pages.push(dst);
                copy = Some((src, dst));
            }
        }
        Ok((child, copy))
    }
}

/// The batched form a serving loop uploads once per layer and step:
/// `rows.len()` sequences, each row padded with `NO_PAGE` to `stride`
/// entries, row-major (`[n_seq][stride]`, what `lnskv_append_decode` reads).
pub fn flatten_tables(rows: &[BlockTable], stride: usize, out: &mut Vec<u32>) -> Result<(), String> {
    out.clear();
    out.reserve(rows.len() * stride);
    for (s, r) in rows.iter().enumerate() {
        if r.pages.len() > stride {
            return Err(format!("row {s} maps {} pages, more than the stride {stride}", r.pages.len()));
        }
        out.extend_from_slice(&r.pages);
        out.extend(std::iter::repeat(NO_PAGE).take(stride - r.pages.len()));
    }
    Ok(())
}

#[cfg(test)]
mod tests {
    use super::*;

    #[test]
    fn pool_is_fifo_like_the_reference() {
        let mut p = PagePool::new(4);
        assert_eq!((p.alloc(), p.alloc()), (Some(0), Some(1)));
        p.free_page(0).unwrap();
        assert_eq!((p.alloc(), p.alloc(), p.alloc()), (Some(2), Some(3), Some(0)));
        assert_eq!(p.alloc(), None);
        p.reset();
        assert_eq!((p.num_free(), p.alloc()), (4, Some(0)));
        assert!(p.free_page(9).is_err() && p.free_page(1).is_err());
    }

    #[test]
    fn exhaustion_message_is_the_reference_text() {
        let (mut p, mut t) = (PagePool::new(1), BlockTable::new(8));
        t.ensure_kv_page(&mut p, 5, 0).unwrap();
        let e = t.ensure_kv_page(&mut p, 5, 16).unwrap_err();
        assert_eq!(e, "KV page pool exhausted at layer 5 (pos=16)");
    }

    #[test]
    fn table_capacity_is_an_error_not_an_overflow() {
        let (mut p, mut t) = (PagePool::new(8), BlockTable::new(2));
        t.ensure_kv_page(&mut p, 0, 31).unwrap();
        assert!(t.ensure_kv_page(&mut p, 0, 32).is_err());
        assert_eq!(t.as_slice().len(), 2);
    }

    #[test]
    fn reference_order_exhausts_a_window_sized_pool() {
        // ensure before evict on ceil(w/16) pages fails at pos = w
        let w = 64;
        let (mut p, mut t) = (PagePool::new(w / 16), BlockTable::new(64));
        for pos in 0..w {
            t.ensure_kv_page(&mut p, 0, pos).unwrap();
            t.evict_kv_pages(&mut p, pos, w).unwrap();
        }
        assert!(t.ensure_kv_page(&mut p, 0, w).is_err());
    }

    #[test]
    fn step_pages_never_exhausts_window_pages() {
        for &w in &[1usize, 2, 15, 16, 17, 31, 32, 33, 64, 100, 4096] {
            let need = window_pages(w);
            let (mut p, mut t) = (PagePool::new(need), BlockTable::new(10_000 / 16 + 1));
            let mut most = 0;
            for pos in 0..10_000 {
                t.step_pages(&mut p, 0, pos, w).unwrap();
                let (lo, hi) = (kv_p_start(pos, w) / 16, pos / 16);
                let live: Vec<usize> =
                    t.as_slice().iter().enumerate().filter(|&(_, &x)| x != NO_PAGE).map(|(i, _)| i).collect();
                assert_eq!(live, (lo..=hi).collect::<Vec<_>>(), "w {w} pos {pos}");
                most = most.max(live.len());
            }
            assert_eq!(most, need, "w {w}");
            let (mut small, mut t2) = (PagePool::new(need - 1), BlockTable::new(10_000 / 16 + 1));
            assert!((0..10_000).any(|pos| t2.step_pages(&mut small, 0, pos, w).is_err()), "w {w}");
        }
    }

    #[test]
    fn fork_shares_full_pages_and_copies_the_tail() {
        let (mut p, mut t) = (PagePool::new(8), BlockTable::new(8));
        for pos in 0..40 {
            t.ensure_kv_page(&mut p, 0, pos).unwrap();
        }
        let (mut child, copy) = t.fork(&mut p, 40).unwrap();
        assert_eq!(&child.as_slice()[..2], &t.as_slice()[..2]);
        assert_eq!(copy, Some((t.as_slice()[2], child.as_slice()[2])));
        assert_eq!((p.refcount(t.as_slice()[0]), p.refcount(t.as_slice()[2])), (2, 1));
        child.free_all(&mut p).unwrap();
        t.free_all(&mut p).unwrap();
        assert_eq!(p.num_free(), 8);
    }

    #[test]
    fn flattened_rows_are_padded() {
        let (mut p, mut a, mut b) = (PagePool::new(8), BlockTable::new(4), BlockTable::new(4));
        a.ensure_kv_page(&mut p, 0, 20).unwrap();
        b.ensure_kv_page(&mut p, 0, 0).unwrap();
        let mut out = Vec::new();
        flatten_tables(&[a, b], 3, &mut out).unwrap();
        assert_eq!(out, vec![NO_PAGE, 0, NO_PAGE, 1, NO_PAGE, NO_PAGE]);
    }
}
