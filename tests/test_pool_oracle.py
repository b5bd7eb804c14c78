"""Pins for the integer restatement of the page pool, caches, decode-batch
metadata and scheduler (oracle/pool_oracle.py).

Expected values are derived by hand from the reference's code paths (cited
per test), plus invariants checked over random traces. A planted mistake in
a copy of the allocator (popping new slabs after old free pages instead of
before) is shown to fail the slab-growth known answer.
"""
import numpy as np
import pytest

from oracle.pool_oracle import PoolOracle, CacheOracle, decode_batch_metadata, BatcherOracle

PAGE = 1000   # page bytes used in the hand examples


def test_sizing_follows_reference_formulas():
    # minitorch/paged_kv_cache.py:52-60: pps = min(pps, budget // page_bytes),
    # max_slabs = budget // slab_bytes, max_pages = max_slabs * pps
    p = PoolOracle(page_bytes=PAGE, max_bytes=10_500, pages_per_slab=4)
    assert (p.pages_per_slab, p.slab_bytes, p.max_slabs, p.max_pages) == (4, 4000, 2, 8)
    p = PoolOracle(page_bytes=PAGE, max_bytes=2_999, pages_per_slab=4)
    assert (p.pages_per_slab, p.max_slabs, p.max_pages) == (2, 1, 2)
    with pytest.raises(ValueError):
        PoolOracle(page_bytes=PAGE, max_bytes=999)


def test_fresh_pool_yields_ascending_ids():
    p = PoolOracle(page_bytes=PAGE, max_bytes=100 * PAGE, pages_per_slab=4)
    o = object()
    assert [p.acquire(1, o)[0] for _ in range(6)] == [0, 1, 2, 3, 4, 5]
    assert p.slabs == 2 and p.free == [7, 6]


def test_new_slab_goes_on_top_of_older_free_pages():
    # paged_kv_cache.py:78-89: the while loop extends the free list with a
    # reversed new slab before popping, so new pages come out first.
    p = PoolOracle(page_bytes=PAGE, max_bytes=100 * PAGE, pages_per_slab=4)
    a = object()
    assert p.acquire(3, a) == [0, 1, 2]
    assert p.acquire(1, a) == [3]           # enough free pages: no new slab
    p2 = PoolOracle(page_bytes=PAGE, max_bytes=100 * PAGE, pages_per_slab=4)
    assert p2.acquire(3, a) == [0, 1, 2]
    assert p2.acquire(5, a) == [4, 5, 6, 7, 3]
    assert p2.free == []
    # a fresh pool asked for 6 opens two slabs before popping: 4..7 come first
    p3 = PoolOracle(page_bytes=PAGE, max_bytes=100 * PAGE, pages_per_slab=4)
    assert p3.acquire(6, a) == [4, 5, 6, 7, 0, 1]
    assert p3.free == [3, 2]


def _planted_acquire(pool, count):
    # wrong order: pop old free pages first, then open slabs
    pages = []
    while len(pages) < count:
        if not pool.free:
            start = pool.slabs * pool.pages_per_slab
            pool.slabs += 1
            pool.free.extend(reversed(range(start, start + pool.pages_per_slab)))
        pages.append(pool.free.pop())
    return pages


def test_planted_slab_order_mistake_is_caught():
    p = PoolOracle(page_bytes=PAGE, max_bytes=100 * PAGE, pages_per_slab=4)
    p.acquire(3, object())
    assert _planted_acquire(p, 5) != [4, 5, 6, 7, 3]


def test_release_is_lifo_in_given_order():
    p = PoolOracle(page_bytes=PAGE, max_bytes=100 * PAGE, pages_per_slab=4)
    a = object()
    pages = p.acquire(4, a)
    p.release([pages[2], pages[0]], a)
    assert p.acquire(2, a) == [pages[0], pages[2]]
    assert p.page_reuses == 2 and p.page_acquires == 6 and p.page_releases == 2
    with pytest.raises(ValueError):
        p.release([pages[1], pages[1]], a)
    with pytest.raises(ValueError):
        p.release([pages[1]], object())
    with pytest.raises(MemoryError):
        p.acquire(97, a)


def test_cache_prepare_distributes_one_acquire_over_rows():
    # paged_kv_cache.py:171-186: one acquire for all rows, sliced row by row
    p = PoolOracle(page_bytes=PAGE, max_bytes=100 * PAGE, page_size=16, pages_per_slab=4)
    c = CacheOracle(p, batch_size=3, capacity=100)
    c.prepare_append(20)                    # 2 pages per row: one acquire of 6
    assert c.pages == [[4, 5], [6, 7], [0, 1]]
    assert p.free == [3, 2]
    c.commit_append()
    c.prepare_append(13)                    # 33 tokens -> 3 pages per row: acquire(3)
    assert c.pages == [[4, 5, 8], [6, 7, 9], [0, 1, 10]]
    assert p.free == [3, 2, 11]
    c.abort_append()                        # releases only the new pages
    assert c.pages == [[4, 5], [6, 7], [0, 1]]
    assert p.free == [3, 2, 11, 8, 9, 10]
    assert c.table()[0][:3] == [4, 5, -1]
    c.close()
    assert not p.leased and p.page_releases == 9
    assert p.free[-6:] == [4, 5, 6, 7, 0, 1]


def test_decode_metadata_hand_example():
    # paged_decode.py:17-54: offsets = lengths, columns = max ceil((len+1)/P),
    # each cache prepare_append(1) in batch order, table padded with -1.
    p = PoolOracle(page_bytes=PAGE, max_bytes=100 * PAGE, page_size=16, pages_per_slab=4)
    caches = []
    for n in (16, 5, 32):
        c = CacheOracle(p, 1, 100)
        c.prepare_append(n)
        c.commit_append()
        caches.append(c)
    # pages: c0 [0], c1 [1], c2 [2, 3]; free list after slab growth: []
    offsets, columns, table = decode_batch_metadata(caches)
    assert offsets == [16, 5, 32] and columns == 3
    # c0 needs a page (16 % 16 == 0): slab 1 opens, pops 4; c2 needs one: pops 5
    assert table == [[0, 4, -1], [1, -1, -1], [2, 3, 5]]
    assert p.free == [7, 6]


def test_invariants_over_random_traces():
    rng = np.random.default_rng(0)
    p = PoolOracle(page_bytes=PAGE, max_bytes=60 * PAGE, page_size=8, pages_per_slab=7)
    owners = [object() for _ in range(5)]
    held = {id(o): [] for o in owners}
    for _ in range(2000):
        o = owners[int(rng.integers(5))]
        if rng.random() < 0.5:
            try:
                held[id(o)] += p.acquire(int(rng.integers(0, 8)), o)
            except MemoryError:
                pass
        elif held[id(o)]:
            k = int(rng.integers(1, len(held[id(o)]) + 1))
            p.release(held[id(o)][:k], o)
            del held[id(o)][:k]
        free, leased = set(p.free), set(p.leased)
        assert not free & leased
        assert len(free) == len(p.free)
        assert free | leased == set(range(p.slabs * p.pages_per_slab))
        assert p.page_acquires - p.page_releases == len(p.leased)


def test_batcher_head_of_line_blocking_and_budget_exemption():
    # continuous_batching.py:155-176
    p = PoolOracle(page_bytes=PAGE, max_bytes=10 * PAGE, page_size=16, pages_per_slab=4)   # 8 pages
    b = BatcherOracle(p, lambda rid, i: 7, max_batch_size=4, max_prefills_per_step=3,
                      prefill_token_budget=100)
    b.submit('a', [1] * 80, 1 + 16)        # capacity 96 -> 6 pages
    b.submit('b', [1] * 30, 4)             # 3 pages: 6 + 3 > 8 blocks b and everything behind it
    b.submit('c', [1] * 2, 2)
    b.step()
    assert b.steps[-1]['prefill_request_ids'] == ['a']
    assert b.steps[-1]['logical_reserved_pages'] == 6
    # 'a' decodes; b still blocked at the head of the queue
    b.step()
    assert b.steps[-1]['decode_request_ids'] == ['a'] and b.steps[-1]['prefill_request_ids'] == []
    while b.requests['a'].state != 'completed':
        b.step()
    # the step that completed 'a' admitted 'b' and 'c' (32 tokens, within budget)
    assert b.steps[-1]['prefill_request_ids'] == ['b', 'c']


def test_batcher_first_prefill_exempt_from_token_budget():
    p = PoolOracle(page_bytes=PAGE, max_bytes=200 * PAGE, page_size=16, pages_per_slab=4)
    b = BatcherOracle(p, lambda rid, i: 7, max_batch_size=8, max_prefills_per_step=4,
                      prefill_token_budget=50)
    b.submit('big', [1] * 300, 2)
    b.submit('small', [1] * 10, 2)
    b.step()
    assert b.steps[-1]['prefill_request_ids'] == ['big']     # 300 > 50 alone is fine; 'small' waits
    b.step()
    assert b.steps[-1]['decode_request_ids'] == ['big'] and b.steps[-1]['prefill_request_ids'] == ['small']


def test_batcher_cancel_and_finish_return_pages():
    p = PoolOracle(page_bytes=PAGE, max_bytes=200 * PAGE, page_size=16, pages_per_slab=4)
    b = BatcherOracle(p, lambda rid, i: 3 if rid == 'e' and i == 2 else 7, max_batch_size=2)
    b.submit('q', [1] * 20, 5)
    b.submit('e', [1] * 20, 9, eos=3)
    b.submit('z', [1] * 5, 5)
    b.step()
    assert b.cancel('z') and b.requests['z'].state == 'cancelled'
    assert not b.cancel('z')
    b.step()
    b.step()
    b.step()
    assert b.requests['e'].finish_reason == 'eos' and b.requests['e'].output == [7, 7, 3]
    b.cancel('q')
    assert not p.leased and b.reserved_pages == 0
    r = b.submit('huge', [1] * 1000, 24)   # reserves 64 pages > the 200-page budget? no: fits
    assert r.state == 'queued'
    p_small = PoolOracle(page_bytes=PAGE, max_bytes=4 * PAGE, page_size=16, pages_per_slab=4)
    b2 = BatcherOracle(p_small, lambda rid, i: 0)
    assert b2.submit('x', [1] * 100, 1).state == 'rejected'
