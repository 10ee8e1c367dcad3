"""The host page-table controller (include/granite4_kv_pool.h) against the
behaviour the reference's own tests fix: test_kv_pool.cc (layout offsets,
sizing, allocation, prefix sharing, LRU retention and eviction, row tables)
and test_kv_pool_controller.cc (session slots, prefill reuse, commit,
resident sessions). The cases restate those tests' setups and expected
values (page ids included: the free list hands out the highest id first);
the code under test is this library's own. Host-only: no GPU.

The small pool of the reference's tests: 2 layers x 2 KV heads x head_dim 4
(32 bytes per token), 4 tokens per page, a 512-byte budget = 4 pages."""
import numpy as np
import pytest

from pkg import layerops

L = layerops()


def small_pool():
    return L.PagedKV(2, 2, 4, 4, 512)


def small_ctrl():
    return L.KvPoolController(2, 2, 4, 4, 512)


def toks(start, n):
    return list(range(start, start + n))


def rows_valid(rows, n, pool_pages, tpp):
    """A position -> row table: in range, no row claimed twice, and each
    page's rows consecutive in token order."""
    rows = list(rows[:n])
    if any(r < 0 or r >= pool_pages * tpp for r in rows) or len(set(rows)) != n:
        return False
    return all(rows[i] + 1 == rows[i + 1] for i in range(n - 1) if (i + 1) % tpp)


# ----------------------------------------------------------------- PagedKV

def test_layout_offsets():
    off = lambda *a: L.kv_layout_offset(2, 2, 4, 4, *a)  # noqa: E731
    assert off(0, 0, 0, 0, 0) == 0
    assert off(0, 0, 0, 0, 1) == 1      # dim stride
    assert off(0, 0, 0, 1, 0) == 4      # head stride
    assert off(0, 0, 1, 0, 0) == 8      # K -> V
    assert off(0, 1, 0, 0, 0) == 16     # layer stride
    assert off(1, 0, 0, 0, 0) == 32     # token stride
    assert off(2, 1, 1, 1, 3) == 2 * 32 + 16 + 8 + 4 + 3
    for bad in [(4, 0, 0, 0, 0), (0, 2, 0, 0, 0), (0, 0, 2, 0, 0), (0, 0, 0, 2, 0),
                (0, 0, 0, 0, 4)]:
        assert off(*bad) == L.NO_INDEX


def test_pool_sizing():
    p = small_pool()
    assert p.page_bytes() == 128 and p.pool_pages() == 4 and p.capacity_tokens() == 16
    assert p.free_pages() == 4 and p.used_pages() == 0
    # Granite 4.2 8B: 40 layers x 8 KV heads x 128 = 81920 bytes per token
    budget = 10 * 2 ** 30
    g = L.PagedKV(40, 8, 128, 16, budget)
    assert g.page_bytes() == 16 * 81920
    assert g.pool_pages() == budget // (16 * 81920)
    assert g.capacity_tokens() == g.pool_pages() * 16


def test_alloc_and_locate():
    p = small_pool()
    s = p.create_sequence()
    assert s == 0
    t = toks(0, 10)
    assert p.reserve(s, 10, t) and p.sequence_tokens(s) == 10
    assert p.free_pages() == 1
    for i in range(10):
        page, local = p.locate(s, i)
        assert local == i % 4
        assert page == p.locate(s, i - i % 4)[0]
    assert p.locate(s, 10) == (L.NO_INDEX, L.NO_INDEX)
    assert p.reserve(s, 11, toks(0, 11)) and p.free_pages() == 1  # fills the partial page
    assert not p.reserve(s, 17, toks(0, 17))                       # beyond capacity
    assert p.sequence_tokens(s) == 11
    assert p.block_table(s) == [3, 2, 1]  # highest page id first


def test_prefix_reuse():
    p = small_pool()
    a = p.create_sequence()
    shared = toks(100, 16)
    assert p.reserve(a, 16, shared)
    assert all(p.mark_written(a, i) for i in range(4))
    assert p.cached_pages() == 4 and p.free_pages() == 0
    b = p.create_sequence()
    assert p.match_prefix(b, shared) == 16
    assert p.sequence_tokens(b) == 16 and p.free_pages() == 0 and p.shared_pages() == 4
    assert p.locate(b, 5) == (2, 1)  # A's second page is page 2
    c = p.create_sequence()
    assert p.match_prefix(c, toks(500, 16)) == 0 and p.sequence_tokens(c) == 0
    p.release(a)
    p.release(b)
    assert p.free_pages() == 0 and p.retained_pages() == 4


def test_lru_eviction():
    p = small_pool()
    a = p.create_sequence()
    p.reserve(a, 16, toks(700, 16))
    for i in range(4):
        p.mark_written(a, i)  # pages 3, 2, 1, 0 in that order
    p.release(a)
    assert p.retained_pages() == 4
    b = p.create_sequence()
    assert p.reserve(b, 4, toks(900, 4))
    assert p.evicted_pages() == 1 and p.free_pages() == 0 and p.used_pages() == 4
    assert p.retained_pages() == 3 and p.cached_pages() == 3
    assert p.locate(b, 3) == (3, 3)  # the least recently marked page (3) was evicted


def test_eviction_respects_live_refs():
    p = L.PagedKV(2, 2, 4, 4, 256)
    assert p.pool_pages() == 2
    a, b = p.create_sequence(), p.create_sequence()
    p.reserve(a, 4, toks(0, 4))
    p.mark_written(a, 0)
    p.reserve(b, 4, toks(10, 4))
    p.mark_written(b, 0)
    assert p.free_pages() == 0
    c = p.create_sequence()
    assert c == -1  # live sequences are bounded by the page count
    p.release(b)
    c = p.create_sequence()
    # b's page is retained (evictable), a's is live: one page, not two
    assert not p.reserve(c, 8, toks(20, 8))
    assert p.evicted_pages() == 0 and p.retained_pages() == 1  # a failed reserve changes nothing
    assert p.ref_count(p.locate(a, 0)[0]) == 1
    assert p.sequence_tokens(c) == 0
    assert p.reserve(c, 4, toks(20, 4)) and p.evicted_pages() == 1


def test_block_table_and_row_table():
    p = small_pool()
    s = p.create_sequence()
    p.reserve(s, 8, toks(0, 8))
    bt = p.block_table(s)
    assert len(bt) == 2 and p.locate(s, 0)[0] == bt[0] and p.locate(s, 4)[0] == bt[1]
    assert p.locate(s, 7)[1] == 3
    rt = p.row_table(s, 8)
    assert list(rt) == [bt[i // 4] * 4 + i % 4 for i in range(8)]
    assert p.row_table(s, 9) is None and p.row_table(-1, 1) is None
    # shared + private: one cached page then two private ones
    p.mark_written(s, 0)
    r = p.create_sequence()
    t = toks(0, 4) + toks(50, 8)
    assert p.match_prefix(r, t) == 4
    assert p.reserve(r, 12, t)
    rbt = p.block_table(r)
    assert len(rbt) == 3 and rbt[0] == bt[0]
    rr = p.row_table(r, 12)
    assert list(rr) == [rbt[i // 4] * 4 + i % 4 for i in range(12)]
    assert rr[0] != rr[4]
    p.release(s)
    assert p.block_table(s) == [] and p.block_table(-1) == [] and p.block_table(999) == []


def test_release_frees_uncached_and_retains_cached():
    p = small_pool()
    a = p.create_sequence()
    p.reserve(a, 8, toks(0, 8))
    p.mark_written(a, 0)
    p.mark_written(a, 1)
    assert p.cached_pages() == 2 and p.free_pages() == 2
    p.release(a)
    assert p.retained_pages() == 2 and p.free_pages() == 2
    b = p.create_sequence()
    p.reserve(b, 4, toks(1, 4))
    assert p.free_pages() == 1
    p.release(b)
    assert p.free_pages() == 2 and p.retained_pages() == 2


def test_clear_and_sequence_bound():
    p = small_pool()
    a = p.create_sequence()
    p.reserve(a, 8, toks(0, 8))
    p.mark_written(a, 0)
    p.clear()
    assert p.free_pages() == 4 and p.cached_pages() == 0 and p.live_sequences() == 0
    assert p.evicted_pages() == 0
    ids = [p.create_sequence() for _ in range(4)]
    assert all(i >= 0 for i in ids) and p.create_sequence() == -1
    p.release(ids[0])
    assert p.create_sequence() >= 0


def test_truncate_keeps_cached_pages_whole():
    p = small_pool()
    s = p.create_sequence()
    t = toks(0, 14)
    p.reserve(s, 14, t)
    p.mark_written(s, 0)
    p.mark_written(s, 1)
    p.truncate_sequence(s, 6)  # keeps 2 pages; page 1 is cached, so it stays whole
    assert len(p.block_table(s)) == 2 and p.sequence_tokens(s) == 8
    assert p.free_pages() == 2
    q = p.create_sequence()
    p.reserve(q, 7, toks(40, 7))
    p.truncate_sequence(q, 5)  # private tail page cut to one token
    assert p.sequence_tokens(q) == 5 and len(p.block_table(q)) == 2
    assert p.reserve(q, 8, toks(40, 4) + [77, 78, 79, 80])
    assert p.mark_written(q, 1)  # the regrown page is complete again


def test_truncate_inside_cached_tail_without_drop():
    """No page dropped: the count is min(filled, n) as in the reference
    (kv_pool.cc:319-321), even when the tail page is cached. Growing back
    over the cached page's own tokens is allowed; other tokens would
    overwrite shared rows and are refused with nothing changed."""
    p = small_pool()
    s = p.create_sequence()
    t = toks(0, 8)
    assert p.reserve(s, 8, t)
    assert p.mark_written(s, 0) and p.mark_written(s, 1)
    p.truncate_sequence(s, 6)
    assert p.sequence_tokens(s) == 6 and len(p.block_table(s)) == 2
    free = p.free_pages()
    assert not p.reserve(s, 8, t[:6] + [901, 902])
    assert p.sequence_tokens(s) == 6 and p.free_pages() == free
    assert p.reserve(s, 10, t + [5, 6])  # the page's own ids, then a new page
    assert p.sequence_tokens(s) == 10 and len(p.block_table(s)) == 3
    assert p.page_in_cache(p.block_table(s)[1])


# --------------------------------------------------------- KvPoolController

def test_slot_capacity():
    c = small_ctrl()
    assert c.max_slots() == 4
    assert [c.new_slot() for _ in range(4)] == [0, 1, 2, 3]
    assert c.new_slot() == -1
    c.release_slot(0)
    assert c.new_slot() == 0
    assert c.new_slot() == -1  # the recycled slot is in use again


def test_prefill_fresh_and_rows():
    c = small_ctrl()
    a = c.new_slot()
    ok, reused = c.prefill(a, toks(100, 10))
    assert ok and reused == 0 and c.committed(a) == 10 and c.free_pages() == 1
    assert rows_valid(c.row_table(a, 10), 10, c.pool_pages(), c.tokens_per_page())


def test_concurrent_and_sequential_prefix_reuse():
    c = small_ctrl()
    a, b = c.new_slot(), c.new_slot()
    assert c.prefill(a, toks(100, 16)) == (True, 0)
    assert c.prefill(b, toks(100, 16)) == (True, 16)
    assert c.committed(b) == 16 and c.shared_pages() == 4 and c.used_pages() == 4
    assert c.free_pages() == 0
    c2 = small_ctrl()
    a = c2.new_slot()
    c2.prefill(a, toks(100, 16))
    c2.release_slot(a)
    assert c2.retained_pages() == 4
    b = c2.new_slot()
    assert c2.prefill(b, toks(100, 16)) == (True, 16)
    assert c2.retained_pages() == 0


def test_partial_prefix_reuse():
    c = small_ctrl()
    a, b = c.new_slot(), c.new_slot()
    c.prefill(a, toks(100, 12))
    ok, reused = c.prefill(b, toks(100, 12) + [999, 998])
    assert ok and reused == 12 and c.committed(b) == 14 and c.free_pages() == 0


def test_commit_extends_stably_and_noop():
    c = small_ctrl()
    a = c.new_slot()
    t = toks(100, 6)
    c.prefill(a, t)
    assert c.committed(a) == 6 and c.cached_pages() == 1
    before = c.row_table(a, 6)
    t += [200, 201]
    c.commit(a, t)
    assert c.committed(a) == 8 and c.cached_pages() == 2
    after = c.row_table(a, 8)
    assert rows_valid(after, 8, c.pool_pages(), c.tokens_per_page())
    assert list(after[:6]) == list(before)
    c2 = small_ctrl()
    b = c2.new_slot()
    c2.prefill(b, toks(0, 4))
    c2.commit(b, toks(0, 4))
    assert c2.committed(b) == 4 and c2.free_pages() == 3


def test_prefill_over_capacity_and_eviction_under_pressure():
    c = small_ctrl()
    a = c.new_slot()
    assert c.prefill(a, toks(0, 17)) == (False, 0)
    assert c.committed(a) == 0 and c.free_pages() == 4
    c = small_ctrl()
    a = c.new_slot()
    c.prefill(a, toks(100, 16))
    c.release_slot(a)
    b = c.new_slot()
    assert c.prefill(b, toks(500, 16)) == (True, 0)
    assert c.evicted_pages() == 4 and c.used_pages() == 4


def test_shared_arena_device_contract():
    """Shared prompt prefix -> identical arena rows; no row claimed by two
    different logical positions of the two sessions."""
    c = L.KvPoolController(2, 2, 4, 4, 128 * 8)
    a, b = c.new_slot(), c.new_slot()
    pa = toks(100, 13)
    pb = toks(100, 8) + toks(700, 7)
    c.prefill(a, pa)
    ok, reused = c.prefill(b, pb)
    assert ok and reused == 8
    ra, rb = c.row_table(a, 13), c.row_table(b, 15)
    arena = c.pool_pages() * c.tokens_per_page()
    assert all(0 <= r < arena for r in list(ra) + list(rb))
    assert list(ra[:8]) == list(rb[:8])
    owner = {}
    for who, rows, t in (("a", ra, pa), ("b", rb, pb)):
        for i, r in enumerate(rows):
            key = (t[i], i)
            assert owner.setdefault(int(r), key) == key
    assert len(set(ra) | set(rb)) == 13 + 15 - 8


def test_release_slot_retains_cache_and_shutdown():
    c = small_ctrl()
    a = c.new_slot()
    c.prefill(a, toks(0, 8))
    c.release_slot(a)
    assert c.committed(a) == 0 and c.retained_pages() == 2
    a = c.new_slot()
    assert c.prefill(a, toks(0, 8)) == (True, 8) and c.committed(a) == 8
    c.shutdown()
    assert c.pool_pages() == 4 and c.free_pages() == 4 and c.cached_pages() == 0
    assert c.committed(a) == 0


def test_resident_sessions():
    c = small_ctrl()
    a, b = c.open_slot(), c.open_slot()
    assert a >= 0 and b >= 0 and a != b
    assert c.ensure(a, 8) and c.ensure(b, 8) and c.free_pages() == 0
    ra, rb = c.row_table(a, 8), c.row_table(b, 8)
    assert not set(ra) & set(rb)
    assert not c.ensure(a, 12) and c.committed(a) == 8
    assert list(c.row_table(a, 8)) == list(ra)
    c.trim(b, 4)
    assert c.free_pages() == 1
    assert c.ensure(a, 12)
    ra3 = c.row_table(a, 12)
    assert list(ra3[:8]) == list(ra) and rows_valid(ra3, 12, 4, 4)
    assert list(c.row_table(b, 4)) == list(rb[:4])
    c = small_ctrl()
    a = c.open_slot()
    assert c.pages_missing(a, 10) == 3 and c.ensure(a, 10) and c.slot_pages(a) == 3
    assert c.pages_missing(a, 12) == 0 and c.pages_missing(a, 13) == 1
    c.trim(a, 5)
    assert c.slot_pages(a) == 2 and c.committed(a) == 5
    assert c.ensure(a, 9)
    c.drop(a)
    assert c.slot_pages(a) == 0 and c.free_pages() == 4 and c.cached_pages() == 0


def test_row_tables_match_the_row_table_helper():
    """The controller's tables equal granite4_row_table over its block table
    (the helper the kernels' d_pt tests use)."""
    p = L.PagedKV(2, 2, 4, 16, 128 * 16 * 64)
    s = p.create_sequence()
    t = toks(3, 200)
    assert p.reserve(s, 200, t)
    bt = np.array(p.block_table(s), np.int32)
    want = np.empty(200, np.int32)
    L.lib.granite4_row_table(bt.ctypes.data, 200, 16, want.ctypes.data)
    np.testing.assert_array_equal(p.row_table(s, 200), want)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_workload_invariants(seed):
    """Random prefill / commit / release / trim traffic over a 64-page pool:
    the allocation invariant (free + held pages = pool), sharing never hands
    one row to two different token prefixes, and row tables stay valid."""
    rng = np.random.default_rng(seed)
    c = L.KvPoolController(2, 2, 4, 16, 128 * 16 * 64)
    prompts = [list(rng.integers(0, 50, 16 * int(rng.integers(1, 4)))) for _ in range(5)]
    live = {}
    for _ in range(400):
        op = rng.integers(0, 4)
        if op == 0:
            s = c.new_slot()
            if s < 0:
                continue
            base = prompts[int(rng.integers(0, len(prompts)))]
            t = base + list(rng.integers(0, 50, int(rng.integers(0, 20))))
            ok, _ = c.prefill(s, t)
            if ok:
                live[s] = t
            else:
                c.release_slot(s)
        elif op == 1 and live:
            s = list(live)[int(rng.integers(0, len(live)))]
            live[s] = live[s] + list(rng.integers(0, 50, int(rng.integers(1, 10))))
            c.commit(s, live[s])
            live[s] = live[s][:c.committed(s)]
        elif op == 2 and live:
            s = list(live)[int(rng.integers(0, len(live)))]
            c.release_slot(s)
            del live[s]
        assert c.free_pages() + c.used_pages() == c.pool_pages()
        owner = {}
        for s, t in live.items():
            n = c.committed(s)
            rows = c.row_table(s, n)
            assert rows_valid(rows, n, c.pool_pages(), c.tokens_per_page())
            for i, r in enumerate(rows):
                key = tuple(t[: i + 1])
                assert owner.setdefault(int(r), key) == key
