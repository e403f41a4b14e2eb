"""Host side of the five workloads (no GPU): seeded tables and lengths, page
ownership, and the algorithmic byte counts the roofline uses."""
import numpy as np
import pytest

from lnskv import NO_PAGE, PAGE_SIZE
from lnskv.configs import SplitMix64, make


def test_splitmix64_known_values():
    # SplitMix64 reference sequence for state 0 (Vigna's splitmix64.c)
    r = SplitMix64(0, 0)
    r.state = 0
    assert [r.next_u64() for _ in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_tables_cover_every_token_and_pages_are_owned_once(name):
    w = make(name)
    t = w.tables
    for s in range(w.n_seq):
        n = (int(w.kv_len[s]) + PAGE_SIZE - 1) // PAGE_SIZE
        assert (t[s, :n] != NO_PAGE).all() and (t[s, :n] < w.num_pages).all()
        assert (t[s, n:] == NO_PAGE).all()
    live = t[t != NO_PAGE]
    _, counts = np.unique(live, return_counts=True)
    assert counts.max() == (2 if name == "c5" else 1)


def test_c1_shape():
    w = make("c1")
    assert (w.n_heads, w.n_kv, w.head_dim, w.num_pages) == (32, 4, 64, 64)
    assert w.ctx_len.tolist() == [512] and w.tables[0, :33].size == 33
    assert len(set(w.tables[0, :33].tolist())) == 33


def test_c2_lengths_and_bytes():
    w = make("c2")
    assert w.n_seq == 32 and w.ctx_len.min() >= 512 and w.ctx_len.max() <= 4096
    b = w.algorithmic_bytes()
    # ~303.6 MB expected for the mean context; recomputed from the seeded draw
    per_tok = 2 * 8 * 128 * 2
    assert b["kv_read"] == int(w.kv_len.sum()) * per_tok
    assert 200e6 < b["total"] < 400e6


def test_c2_page_types_share_the_draw_and_count_their_bytes():
    """make("c2", dtype=...) keeps lengths and tables; K+V bytes per token
    are 2*Hkv*d*e_kv, plus 2*Hkv*4 of scales for Q8A (int8 codes)."""
    f16 = make("c2")
    for dtype, e, extra in ((0, 4, 0), (2, 1, 2 * 8 * 4)):
        w = make("c2", dtype=dtype)
        assert w.dtype == dtype
        assert np.array_equal(w.kv_len, f16.kv_len) and np.array_equal(w.tables, f16.tables)
        b = w.algorithmic_bytes()
        per_tok = 2 * 8 * 128 * e + extra
        assert b["kv_read"] == int(w.kv_len.sum()) * per_tok
        assert b["append"] == 32 * (2 * 8 * 128 * 4 + per_tok)


def test_c3_c4_shapes():
    w3 = make("c3")
    assert w3.split == 512 and (w3.kv_len == 32769).all() and w3.num_pages == 4 * 2049
    w4 = make("c4")
    assert w4.n_new.tolist().count(256) == 16 and int(w4.decode.sum()) == 48
    cs, cp = w4.chunk_tokens()
    assert len(cs) == 16 * 256
    assert any(int(c) % 16 != 0 for c in w4.ctx_len[:16])  # chunks start mid-page


def test_c5_churn_structure():
    w = make("c5")
    t = w.tables
    assert w.n_seq == 136 and 0 < len(w.copies) <= 8
    for src, dst in w.copies:
        assert dst not in t[:128]
        assert src in t[:128]
    # freed pages were handed to the new sequences (FIFO: after the spare ones)
    new_pages = t[w.info["freed_rows"]]
    reused = np.intersect1d(new_pages[new_pages != NO_PAGE], w.info["freed_pages"])
    assert len(reused) > 0
