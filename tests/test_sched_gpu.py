"""Device page allocator and decode metadata vs the integer restatement of the
reference (oracle/pool_oracle.py): page IDs, block tables, offsets, free list
order and counters must be bit-exact on seeded traces."""
import numpy as np
import pytest

from minitorch_amd.amp import autocast
from minitorch_amd.paged_kv_cache import KVPagePool, PagedKVCache
from minitorch_amd.paged_decode import PagedDecodeBatch
from minitorch_amd.runtime import DeviceTensor, RawDeviceBuffer, runtime, P, I
from oracle.pool_oracle import PoolOracle, CacheOracle, decode_batch_metadata

pytestmark = pytest.mark.gpu


class _Attn:
    def __init__(self, h, d):
        self.n_head, self.attn_hidden_dim, self.attention_impl = h, d, 'flash'


class _Layer:
    def __init__(self, h, d):
        self.attention = _Attn(h, d)


class StubModel:
    """Layout-only model: enough for pools, caches and decode batches."""

    def __init__(self, layers=1, heads=2, dim=64, n_positions=1024, n_vocab=100):
        self._layers = tuple(_Layer(heads, dim) for _ in range(layers))
        self.n_positions, self.n_vocab, self.training = n_positions, n_vocab, False

    def transformer_layers(self):
        return self._layers

    def weights_version(self):
        return 0


def pool_pair(model, **kw):
    pool = KVPagePool(model, **kw)
    oracle = PoolOracle(page_bytes=pool.page_bytes, page_size=pool.page_size,
                        max_bytes=kw.get('max_bytes', 256 * 1024 ** 2),
                        pages_per_slab=kw.get('pages_per_slab', 4))
    assert (pool.pages_per_slab, pool.max_slabs, pool.max_pages) == \
        (oracle.pages_per_slab, oracle.max_slabs, oracle.max_pages)
    return pool, oracle


def assert_same_pool(pool, oracle):
    stats, ostats = pool.memory_stats(), oracle.memory_stats()
    for key, value in ostats.items():
        assert stats[key] == value, (key, stats[key], value)
    assert pool.free_stack() == oracle.free, 'free list differs'
    h = pool.header()
    assert h['error'] == 0
    assert (h['top'], h['slabs_opened'], h['leased'], h['acquires'], h['releases'], h['reuses']) == \
        (len(oracle.free), oracle.slabs, len(oracle.leased), oracle.page_acquires,
         oracle.page_releases, oracle.page_reuses)
    assert pool.num_slabs == oracle.slabs
    # slab table: opened slabs point into the pool, the rest are null
    table = pool.slab_table.download(np.uint64, pool.max_slabs)
    expect = [pool.kv.ptr + s * pool.slab_bytes if s < oracle.slabs else 0 for s in range(pool.max_slabs)]
    assert table.tolist() == expect


def test_fresh_pool_and_slab_growth_order():
    model = StubModel()
    pool, oracle = pool_pair(model, page_size=16, max_bytes=64 * 32768, pages_per_slab=4)
    a, b = object(), object()
    assert pool.acquire(1, a) == oracle.acquire(1, a) == [0]
    assert pool.acquire(2, b) == oracle.acquire(2, b) == [1, 2]
    assert_same_pool(pool, oracle)
    # 3 is free; asking for 5 opens slab 1 on top first: 4,5,6,7 then 3
    assert pool.acquire(5, a) == oracle.acquire(5, a) == [4, 5, 6, 7, 3]
    assert_same_pool(pool, oracle)
    pool.release([1, 2], b)
    oracle.release([1, 2], b)
    # free list [1, 2] is short of 3: slab 2 opens on top, 8, 9, 10 are popped
    assert pool.acquire(3, b) == oracle.acquire(3, b) == [8, 9, 10]
    assert_same_pool(pool, oracle)


def test_random_api_trace_matches_oracle():
    rng = np.random.default_rng(0)
    model = StubModel()
    pool, oracle = pool_pair(model, page_size=16, max_bytes=97 * 32768, pages_per_slab=5)
    owners = [object() for _ in range(4)]
    held = {id(o): [] for o in owners}
    for step in range(200):
        o = owners[int(rng.integers(4))]
        if rng.random() < 0.55:
            count = int(rng.integers(0, 9))
            try:
                expect = oracle.acquire(count, o)
            except MemoryError:
                with pytest.raises(MemoryError):
                    pool.acquire(count, o)
                continue
            got = pool.acquire(count, o)
            assert got == expect, step
            held[id(o)].extend(got)
        elif held[id(o)]:
            mine = held[id(o)]
            k = int(rng.integers(1, len(mine) + 1))
            pick = [mine.pop(int(rng.integers(len(mine)))) for _ in range(k)]
            pool.release(pick, o)
            oracle.release(pick, o)
        if step % 25 == 0:
            assert_same_pool(pool, oracle)
    assert_same_pool(pool, oracle)
    with pytest.raises(ValueError):
        pool.release([10 ** 6], owners[0])


@pytest.mark.parametrize('batch_size', [1, 3])
def test_cache_transactions_match_oracle(batch_size):
    rng = np.random.default_rng(batch_size)
    model = StubModel(n_positions=512)
    pool, oracle = pool_pair(model, page_size=8, max_bytes=300 * 16384, pages_per_slab=7)
    caches = []
    for trial in range(12):
        cap = int(rng.integers(20, 400))
        c = PagedKVCache(model, batch_size, cap, page_size=8, page_pool=pool)
        oc = CacheOracle(oracle, batch_size, cap)
        caches.append((c, oc))
        for _ in range(int(rng.integers(1, 5))):
            n = int(rng.integers(1, 40))
            if c.length + n > cap:
                break
            try:
                oc.prepare_append(n)
            except MemoryError:
                with pytest.raises(MemoryError):
                    c.prepare_append(n)
                c.close()
                oc.close()
                break
            c.prepare_append(n)
            if rng.random() < 0.2:
                c.abort_append()
                oc.abort_append()
                c.close()
                oc.close()
                break
            c._written_layers.update(range(len(c.layout)))
            c.commit_append()
            oc.commit_append()
            assert c.pages() == oc.pages
        if rng.random() < 0.4:
            c.close()
            oc.close()
        assert_same_pool(pool, oracle)
    for c, oc in caches:
        c.close()
        oc.close()
    assert_same_pool(pool, oracle)
    assert pool.used_pages == 0


def _decode_round(model, pool, oracle, pairs, rng):
    """One decode step for every (cache, oracle cache) pair, with attention
    run on random Q/K/V so the transaction commits."""
    caches = [c for c, _ in pairs]
    b = len(caches)
    h, d = model._layers[0].attention.n_head, model._layers[0].attention.attn_hidden_dim
    idx = DeviceTensor.from_numpy(np.zeros((b, 1), np.float32))
    batch = PagedDecodeBatch(model, idx, caches)
    offsets, columns, table = decode_batch_metadata([oc for _, oc in pairs])
    with batch:
        batch.prepare()
        runtime().synchronize()
        assert batch.columns == columns
        assert batch.device_offsets.download(np.int32, b).tolist() == offsets
        assert batch.position_ids.to_numpy().reshape(-1).tolist() == [float(o) for o in offsets]
        cu = np.concatenate([[0], np.cumsum(np.array(offsets) + 1)]).tolist()
        assert batch.cu_seqlens.download(np.int32, b + 1).tolist() == cu
        assert batch.table.download(np.int32, b * columns).reshape(b, columns).tolist() == table
        for layer in range(len(model._layers)):
            q, k, v = (DeviceTensor.from_numpy(rng.standard_normal((b, h, 1, d)).astype(np.float32))
                       for _ in range(3))
            batch.decode_attention(layer, q, k, v)
        batch.commit()
    for _, oc in pairs:
        oc.commit_append()


def test_decode_batches_match_oracle_over_many_steps():
    rng = np.random.default_rng(1)
    model = StubModel(layers=2, heads=2, dim=64, n_positions=256)
    pool, oracle = pool_pair(model, page_size=16, max_bytes=220 * 32768, pages_per_slab=6)
    live = []
    for step in range(60):
        # admit: a new request with a prefill
        if len(live) < 9 and rng.random() < 0.5:
            cap = int(rng.integers(40, 256))
            n = int(rng.integers(1, min(cap, 120)))
            c = PagedKVCache(model, 1, cap, page_size=16, page_pool=pool)
            oc = CacheOracle(oracle, 1, cap)
            try:
                oc.prepare_append(n)
            except MemoryError:
                with pytest.raises(MemoryError):
                    c.prepare_append(n)
                c.close()
                continue
            c.prepare_append(n)
            c._written_layers.update(range(len(c.layout)))
            c.commit_append()
            oc.commit_append()
            live.append((c, oc))
        # finish requests at capacity, and some at random, in list order
        keep = []
        for c, oc in live:
            if c.length + 1 >= c.capacity or rng.random() < 0.08:
                c.close()
                oc.close()
            else:
                keep.append((c, oc))
        live = keep
        if live:
            order = list(rng.permutation(len(live)))
            _decode_round(model, pool, oracle, [live[i] for i in order], rng)
            for c, oc in live:
                assert c.pages() == oc.pages
        assert_same_pool(pool, oracle)
    for c, oc in live:
        c.close()
        oc.close()
    assert_same_pool(pool, oracle)


def test_decode_batch_of_2143_rows_matches_oracle():
    # Past the rows whose slot and page count the metadata kernel keeps in
    # LDS (2048), with a table of 2143 x 8 entries (several unrolled passes
    # of 1024 threads x 8): pages, table and free list bit-exact.
    rng = np.random.default_rng(7)
    model = StubModel(layers=1, heads=1, dim=64, n_positions=128)
    pool, oracle = pool_pair(model, page_size=16, max_bytes=24000 * 2 * 64 * 16 * 4, pages_per_slab=64)
    pairs = []
    for _ in range(2500):
        n = int(rng.integers(1, 60))
        c = PagedKVCache(model, 1, 128, page_size=16, page_pool=pool)
        oc = CacheOracle(oracle, 1, 128)
        c.prepare_append(n)
        oc.prepare_append(n)
        c._written_layers.update(range(len(c.layout)))
        c.commit_append()
        oc.commit_append()
        pairs.append((c, oc))
    # free every seventh request so the step pops reused pages and opens slabs
    live = []
    for i, (c, oc) in enumerate(pairs):
        if i % 7 == 3:
            c.close()
            oc.close()
        else:
            live.append((c, oc))
    assert len(live) == 2143
    order = list(rng.permutation(len(live)))
    live = [live[i] for i in order]
    for _ in range(2):
        _decode_round(model, pool, oracle, live, rng)
        for c, oc in live:
            assert c.pages() == oc.pages
        assert_same_pool(pool, oracle)
    for c, oc in live:
        c.close()
        oc.close()
    assert_same_pool(pool, oracle)


@pytest.mark.parametrize('rows,capacity', [(700, 256), (1500, 128), (300, 1024), (1024, 256)])
def test_decode_batch_table_paths_match_oracle(rows, capacity):
    # The metadata kernel holds the whole table in registers when rows x
    # columns <= 16384 (700 x 16, 1500 x 8 over two 1024-row passes, 1024 x 16)
    # and re-reads the page lists otherwise (300 x 64): pages, table and free
    # list bit-exact over two steps that pop reused pages and open slabs.
    rng = np.random.default_rng([11, rows])
    model = StubModel(layers=1, heads=1, dim=64, n_positions=capacity)
    pool, oracle = pool_pair(model, page_size=16, max_bytes=(rows * capacity // 16 + 64) * 2 * 64 * 16 * 4,
                             pages_per_slab=32)
    pairs = []
    for _ in range(rows + rows // 5 + 8):
        n = int(rng.integers(1, capacity - 4))
        c = PagedKVCache(model, 1, capacity, page_size=16, page_pool=pool)
        oc = CacheOracle(oracle, 1, capacity)
        c.prepare_append(n)
        oc.prepare_append(n)
        c._written_layers.update(range(len(c.layout)))
        c.commit_append()
        oc.commit_append()
        pairs.append((c, oc))
    # close every seventh request, then all past the first `rows` left
    live = []
    for i, (c, oc) in enumerate(pairs):
        if i % 7 == 3 or len(live) == rows:
            c.close()
            oc.close()
        else:
            live.append((c, oc))
    assert len(live) == rows
    order = list(rng.permutation(len(live)))
    live = [live[i] for i in order]
    for _ in range(2):
        _decode_round(model, pool, oracle, live, rng)
        for c, oc in live:
            assert c.pages() == oc.pages
        assert_same_pool(pool, oracle)
    for c, oc in live:
        c.close()
        oc.close()
    assert_same_pool(pool, oracle)


@pytest.mark.parametrize('fused', [False, True])
def test_decode_budget_exhaustion_aborts_like_reference(fused):
    # fused: the metadata launch also embeds the rows (mt_sched_decode_prepare_embed),
    # as the sync-free step issues it; the abort must leave the same pool
    model = StubModel(layers=1, heads=1, dim=64, n_positions=128)
    page_bytes = 2 * 1 * 1 * 64 * 16 * 4
    pool, oracle = pool_pair(model, page_size=16, max_bytes=6 * page_bytes, pages_per_slab=2)
    pairs = []
    for n in (16, 32, 16, 15):      # 1 + 2 + 1 + 1 = 5 pages of 6
        c = PagedKVCache(model, 1, 100, page_size=16, page_pool=pool)
        oc = CacheOracle(oracle, 1, 100)
        c.prepare_append(n)
        oc.prepare_append(n)
        c._written_layers.add(0)
        c.commit_append()
        oc.commit_append()
        pairs.append((c, oc))
    # rows 0, 1, 2 sit on page boundaries and need a page each: only one is left
    idx = None if fused else DeviceTensor.from_numpy(np.zeros((4, 1), np.float32))
    wte = DeviceTensor.from_numpy(np.ones((8, 64), np.float32))
    wpe = DeviceTensor.from_numpy(np.ones((128, 64), np.float32))
    x = DeviceTensor((4, 64), 'float32')
    with pytest.raises(MemoryError):
        with PagedDecodeBatch(model, idx, [c for c, _ in pairs]) as batch:
            batch.prepare(embed=(x.ptr, wte.ptr, wpe.ptr, 8, 128, 64) if fused else None)
    with pytest.raises(MemoryError):
        decode_batch_metadata_with_abort([oc for _, oc in pairs])
    runtime().synchronize()
    assert_same_pool(pool, oracle)
    assert [c.valid for c, _ in pairs] == [False, False, True, True]
    for c, oc in pairs:
        c.close()
        oc.close()
    assert_same_pool(pool, oracle)


def decode_batch_metadata_with_abort(caches):
    """Reference PagedDecodeBatch.prepare + __exit__ on failure
    (minitorch/paged_decode.py:44-46,88-90)."""
    prepared = []
    try:
        for c in caches:
            prepared.append(c)
            c.prepare_append(1)
    except Exception:
        for c in prepared:
            c.abort_append()
        raise


def test_low_precision_pool_dtype_and_bytes():
    model = StubModel(layers=3, heads=4, dim=64)
    with autocast('bfloat16'):
        pool = KVPagePool(model, page_size=32, max_bytes=10 * 1024 ** 2, pages_per_slab=3)
    assert pool.dtype == 'bfloat16'
    assert pool.page_bytes == 2 * 3 * 4 * 64 * 32 * 2
    assert pool.memory_stats()['kv_pool_reserved_bytes'] == 0
    pool.close()


def test_acquire_lists_skips_entries_beyond_columns_or_budget():
    # mt_pool_acquire_lists reads its page counts from device memory, so the
    # kernel checks them itself: an entry that would write past its slot's
    # columns, or pop beyond the free budget, is skipped and sets bit 1 of the
    # header's error word; valid entries around it still run. (Each bad count
    # exceeds its limit by one, so that even an unguarded pop stays inside the
    # pool state.)
    model = StubModel(n_positions=128)           # 8 columns of 16 tokens
    pool = KVPagePool(model, page_size=16, max_bytes=64 * 16384, pages_per_slab=4)   # 64 pages
    caches = [PagedKVCache(model, 1, 128, page_size=16, page_pool=pool) for _ in range(3)]
    slots = [c.slot for c in caches]
    before = pool.header()

    def run(counts):
        lists = DeviceTensor.from_numpy(np.array(slots + counts, np.int32), 'int32')
        pool._call('mt_pool_acquire_lists', [P, P, I, P], lists.ptr, lists.ptr + 4 * len(slots), len(slots),
                   pool._scratch.ptr)
        runtime().synchronize()
        return pool.header()

    h = run([0, pool.max_cols + 1, 0])          # one more than a slot's columns
    assert h['error'] == 2 and (h['top'], h['leased'], h['acquires']) == (before['top'], 0, 0)
    assert pool.slot_pages.download(np.int32).tolist() == [-1] * (pool.max_slots * pool.max_cols)
    h = run([2, pool.max_pages - 1, 3])         # the middle entry exceeds what the first leaves free
    assert h['error'] == 2 and h['leased'] == 5 and h['acquires'] == 5
    table = pool.slot_pages.download(np.int32).reshape(pool.max_slots, pool.max_cols)
    assert table[slots[0], :2].tolist() == [0, 1] and table[slots[1]].tolist() == [-1] * pool.max_cols
    # the third pop finds 2 free pages (slab 0's 3, 2), opens slab 1 on top
    assert table[slots[2], :3].tolist() == [4, 5, 6]
    # leave the pool consistent for close(): the host mirrors never saw these pops
    pool._call('mt_pool_release_rows', [P, I, I, I], pool.slots_ptr(slots[0]), 1, 0, 1)
    pool._call('mt_pool_release_rows', [P, I, I, I], pool.slots_ptr(slots[2]), 1, 0, 1)
    runtime().synchronize()
    assert pool.header()['leased'] == 0
    for c in caches:
        c.close()
    pool.close()


def _pool_with_rows(seed, rows, n_positions=512):
    model = StubModel(layers=1, heads=2, dim=64, n_positions=n_positions)
    pool = KVPagePool(model, page_size=16, max_bytes=(rows * n_positions // 16 + 64) * 2 * 2 * 64 * 16 * 4,
                      pages_per_slab=8)
    rng = np.random.default_rng(seed)
    caches = []
    for _ in range(rows):
        c = PagedKVCache(model, 1, n_positions, page_size=16, page_pool=pool)
        c.prepare_append(int(rng.integers(1, n_positions - 40)))
        c._written_layers.update(range(len(c.layout)))
        c.commit_append()
        caches.append(c)
    return model, pool, caches


@pytest.mark.parametrize('rows,n_pos', [(1, 512), (2, 512), (37, 512), (128, 512), (37, 200)])
def test_fused_prepare_embed_equals_prepare_then_embed(rows, n_pos):
    # mt_sched_decode_prepare_embed against mt_sched_decode_prepare followed by
    # mt_embed_tokens on two identically built pools: the step's metadata,
    # the pool state and the embeddings bit for bit, including a NaN token, an
    # id past the vocabulary and (n_pos 200) positions past the position table
    # (NaN rows)
    from minitorch_amd import paged_ops
    vocab, dim = 300, 64
    rng = np.random.default_rng([3, rows])
    wte = DeviceTensor.from_numpy(rng.standard_normal((vocab, dim)).astype(np.float32))
    wpe = DeviceTensor.from_numpy(rng.standard_normal((512, dim)).astype(np.float32))
    tokens = rng.integers(0, vocab, 4096).astype(np.float32)
    tokens[[0, 5]] = [np.nan, vocab + 3]
    worlds = []
    for fused in (True, False):
        model, pool, caches = _pool_with_rows(rows, rows)
        pool.slot_tokens.upload(np.resize(tokens, pool.max_slots))
        x = DeviceTensor((rows, dim), 'float32')
        batch = PagedDecodeBatch(model, None, caches)
        batch.prepare(graph=True)
        if fused:
            batch.prepare_device(embed=(x.ptr, wte.ptr, wpe.ptr, vocab, n_pos, dim))
        else:
            batch.prepare_device()
            paged_ops.embed_tokens(x.ptr, wte.ptr, wpe.ptr, None, batch.position_ids.ptr, rows, vocab, n_pos, dim,
                                   slot_tokens=pool.slot_tokens.ptr, slots=batch.device_slots.ptr,
                                   num_slots=pool.max_slots)
        runtime().synchronize()
        worlds.append(dict(
            x=x.to_numpy().view(np.uint32),
            table=batch.table.download(np.int32, rows * batch.columns),
            offsets=batch.device_offsets.download(np.int32, rows),
            cu=batch.cu_seqlens.download(np.int32, rows + 1),
            pos=batch.position_ids.to_numpy().view(np.uint32),
            free=pool.free_stack(), header=pool.header()))
    a, b = worlds
    for key in a:
        if isinstance(a[key], np.ndarray):
            assert np.array_equal(a[key], b[key]), key
        else:
            assert a[key] == b[key], key
    if n_pos < 512:
        # rows at or past the position table are NaN, the others are not all NaN
        nan_rows = np.isnan(a['x'].view(np.float32)).all(axis=1)
        assert nan_rows.any() and not nan_rows.all()


@pytest.mark.parametrize('dtype', ['float32', 'bfloat16', 'float16'])
@pytest.mark.parametrize('rows', [1, 3, 64])
def test_argmax_commit_equals_feedback_then_add_length(rows, dtype):
    # mt_row_argmax_commit against mt_row_argmax_feedback followed by
    # mt_sched_add_length: the ids, the slot tokens and every slot's committed
    # length (rows in a shuffled slot order)
    from minitorch_amd import paged_ops
    rng = np.random.default_rng([4, rows])
    width = 50257
    logits = DeviceTensor.from_numpy(rng.standard_normal((rows, 1, width)).astype(np.float32), dtype)
    results = []
    for fused in (True, False):
        model, pool, caches = _pool_with_rows(rows + 11, rows)
        order = rng.permutation(rows) if fused else order_used
        order_used = order
        slots = RawDeviceBuffer(4 * rows)
        slots.upload(np.array([caches[i].slot for i in order], np.int32))
        ids = DeviceTensor((rows, 1), 'float32')
        if fused:
            paged_ops.row_argmax_commit(ids.ptr, pool.slot_tokens.ptr, slots.ptr, pool.max_slots, pool.slot_len_ptr,
                                        1, logits.ptr, rows, width, dtype)
        else:
            paged_ops.row_argmax_feedback(ids.ptr, pool.slot_tokens.ptr, slots.ptr, pool.max_slots, logits.ptr,
                                          rows, width, dtype)
            pool._call('mt_sched_add_length', [P, I, I], slots.ptr, rows, 1)
        runtime().synchronize()
        results.append((ids.to_numpy().ravel(), pool.slot_tokens.download(np.float32, pool.max_slots),
                        pool.state.download(np.int32, pool.max_slots, pool._offsets[5])))
    (i1, t1, l1), (i2, t2, l2) = results
    assert np.array_equal(i1, i2)
    assert np.array_equal(t1.view(np.uint32), t2.view(np.uint32))
    assert np.array_equal(l1, l2)
    ref = np.argmax(logits.to_numpy()[:, 0], axis=1)
    assert np.array_equal(i1.astype(int), ref)
