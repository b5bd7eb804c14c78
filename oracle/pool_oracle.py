"""Integer-exact restatement of the reference's page pool, paged caches, decode
batch metadata and continuous-batching scheduler. TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module, as the checker for the device-side page
allocator and scheduler metadata. It holds no device memory: a "cache" is its
page lists and length, and the model is replaced by a token function.

Followed line by line:
* KVPagePool: sizing (minitorch/paged_kv_cache.py:41-61), acquire with slab
  growth pushing a new slab's page IDs reversed on top of the free list and
  LIFO pops (:71-94), release appending in the given order (:96-103),
  memory_stats (:105-112);
* PagedKVCache page lists: prepare_append distributing one acquire over rows
  (:171-189), abort releasing only the new pages (:228-234), close releasing
  every row's pages row by row (:125-131);
* PagedDecodeBatch.prepare: offsets, columns and the [B, columns] table
  (minitorch/paged_decode.py:17-54);
* ContinuousBatcher: submit (minitorch/continuous_batching.py:84-106),
  decode-before-admit step with FIFO head-of-line blocking, the
  prefill_token_budget exemption of the first prefill, reserved-page
  accounting, finish on length/EOS and cancel (:108-188).

Pinned by hand-derived known answers and invariants in tests/test_pool_oracle.py.
"""
from collections import deque
import math


class PoolOracle:
    def __init__(self, *, page_bytes, page_size=16, max_bytes=256 * 1024 ** 2, pages_per_slab=4):
        if page_size not in (8, 16, 32):
            raise ValueError('page_size must be 8, 16 or 32')
        if min(max_bytes, pages_per_slab) < 1:
            raise ValueError('Positive KV budget and pages_per_slab required')
        if max_bytes < page_bytes:
            raise ValueError('KV budget must hold at least one page')
        self.page_size = page_size
        self.page_bytes = page_bytes
        self.pages_per_slab = min(pages_per_slab, max_bytes // page_bytes)
        self.slab_bytes = self.pages_per_slab * page_bytes
        self.max_slabs = max_bytes // self.slab_bytes
        self.max_pages = self.max_slabs * self.pages_per_slab
        self.slabs = 0
        self.free = []
        self.leased = {}
        self.issued = set()
        self.page_acquires = self.page_releases = self.page_reuses = 0

    def acquire(self, count, owner):
        if count < 0:
            raise ValueError('invalid page count')
        if count > self.max_pages - len(self.leased):
            raise MemoryError('KV page budget exhausted')
        while len(self.free) < count:
            start = self.slabs * self.pages_per_slab
            self.slabs += 1
            self.free.extend(reversed(range(start, start + self.pages_per_slab)))
        pages = [self.free.pop() for _ in range(count)]
        self.page_acquires += count
        self.page_reuses += sum(p in self.issued for p in pages)
        self.issued.update(pages)
        self.leased.update((p, owner) for p in pages)
        return pages

    def release(self, pages, owner):
        pages = list(pages)
        if len(set(pages)) != len(pages) or any(self.leased.get(p, None) is not owner for p in pages):
            raise ValueError('Invalid page ownership or duplicate release')
        for p in pages:
            del self.leased[p]
            self.free.append(p)
        self.page_releases += len(pages)

    def memory_stats(self):
        reserved = self.slabs * self.slab_bytes
        assigned = len(self.leased) * self.page_bytes
        return dict(kv_pool_reserved_bytes=reserved, kv_pool_assigned_bytes=assigned,
                    kv_pool_free_bytes=reserved - assigned,
                    kv_pool_used_pages=len(self.leased), kv_pool_free_pages=len(self.free),
                    kv_pool_max_pages=self.max_pages, kv_pool_page_acquires=self.page_acquires,
                    kv_pool_page_releases=self.page_releases, kv_pool_page_reuses=self.page_reuses)


class CacheOracle:
    """Page lists and committed length of one paged cache (batch rows)."""

    def __init__(self, pool, batch_size=1, capacity=1024):
        self.pool = pool
        self.batch_size = batch_size
        self.capacity = capacity
        self.table_columns = (capacity + pool.page_size - 1) // pool.page_size
        self.pages = [[] for _ in range(batch_size)]
        self.length = 0
        self.pending = None
        self.new_pages = []
        self.previous = None
        self.closed = False

    def prepare_append(self, tokens):
        if self.pending is not None or self.closed:
            raise ValueError('append already pending')
        if tokens < 1 or self.length + tokens > self.capacity:
            raise ValueError('Invalid append size or cache capacity exceeded')
        self.pending = tokens
        self.previous = [len(r) for r in self.pages]
        required = (self.length + tokens + self.pool.page_size - 1) // self.pool.page_size
        count = sum(required - len(r) for r in self.pages)
        try:
            self.new_pages = self.pool.acquire(count, self)
        except Exception:
            self.abort_append()
            raise
        cursor = 0
        for row in self.pages:
            extra = required - len(row)
            row.extend(self.new_pages[cursor:cursor + extra])
            cursor += extra

    def commit_append(self):
        self.length += self.pending
        self.pending = None
        self.new_pages = []
        self.previous = None

    def abort_append(self):
        if self.new_pages:
            self.pool.release(self.new_pages, self)
            for row, count in zip(self.pages, self.previous):
                del row[count:]
        self.new_pages = []
        self.previous = None
        self.pending = None

    def table(self):
        t = [[-1] * self.table_columns for _ in range(self.batch_size)]
        for b, row in enumerate(self.pages):
            t[b][:len(row)] = row
        return t

    def close(self):
        if self.closed:
            return
        self.abort_append()
        owned = [p for row in self.pages for p in row]
        if owned:
            self.pool.release(owned, self)
        for row in self.pages:
            row.clear()
        self.closed = True


def decode_batch_metadata(caches):
    """PagedDecodeBatch metadata for batch-1 caches in batch order:
    (offsets, columns, table [B][columns]) after every cache's prepare_append(1)
    (minitorch/paged_decode.py:17-54). Mutates the caches' page lists."""
    page_size = caches[0].pool.page_size
    offsets = [c.length for c in caches]
    columns = max((c.length + 1 + page_size - 1) // page_size for c in caches)
    for c in caches:
        c.prepare_append(1)
    table = [[-1] * columns for _ in caches]
    for i, c in enumerate(caches):
        table[i][:len(c.pages[0])] = c.pages[0]
    return offsets, columns, table


class RequestOracle:
    def __init__(self, request_id, prompt, max_new_tokens, eos, capacity, reserved_pages):
        self.request_id = request_id
        self.prompt = tuple(prompt)
        self.max_new_tokens = max_new_tokens
        self.eos = eos
        self.capacity = capacity
        self.reserved_pages = reserved_pages
        self.state = 'queued'
        self.finish_reason = None
        self.output = []
        self.cache = None

    @property
    def done(self):
        return self.state in ('completed', 'cancelled', 'rejected', 'failed')


class BatcherOracle:
    """Scheduling decisions and page IDs of ContinuousBatcher with a token
    function ``next_token(request_id, position_index)`` in place of the model."""

    def __init__(self, pool, next_token, *, max_batch_size=4, max_prefills_per_step=1,
                 prefill_token_budget=512, n_positions=1024):
        self.pool = pool
        self.next_token = next_token
        self.max_batch_size = max_batch_size
        self.max_prefills_per_step = max_prefills_per_step
        self.prefill_token_budget = prefill_token_budget
        self.n_positions = n_positions
        self.requests, self.active, self.pending = {}, {}, deque()
        self.reserved_pages = 0
        self.peak_used_pages = 0
        self.iteration = 0
        self.steps = []

    def submit(self, request_id, prompt, max_new_tokens=32, eos=None):
        capacity = len(prompt) + max_new_tokens - 1
        if capacity > self.n_positions:
            raise ValueError('Prompt plus output exceeds model position capacity')
        r = RequestOracle(request_id, prompt, max_new_tokens, eos, capacity,
                          math.ceil(capacity / self.pool.page_size))
        self.requests[request_id] = r
        if r.reserved_pages > self.pool.max_pages:
            r.state, r.finish_reason = 'rejected', 'kv_budget'
        else:
            self.pending.append(r)
        return r

    def _finish(self, r, state, reason):
        if r.request_id in self.active:
            del self.active[r.request_id]
            self.reserved_pages -= r.reserved_pages
        if r.cache is not None:
            r.cache.close()
            r.cache = None
        r.state, r.finish_reason = state, reason

    def cancel(self, request_id):
        r = self.requests[request_id]
        if r.done:
            return False
        if r.state == 'queued':
            self.pending.remove(r)
        self._finish(r, 'cancelled', 'cancelled')
        return True

    def _emit(self, r, token):
        r.output.append(int(token))
        reason = ('eos' if token == r.eos else
                  'length' if len(r.output) >= r.max_new_tokens else None)
        if reason is not None:
            self._finish(r, 'completed', reason)
        return (r.request_id, int(token), reason)

    def step(self):
        events, decode_ids, prefill_ids = [], list(self.active), []
        prefill_tokens = 0
        decode_tables = None
        if decode_ids:
            batch = [self.active[rid] for rid in decode_ids]
            offsets, columns, table = decode_batch_metadata([r.cache for r in batch])
            decode_tables = (offsets, columns, table)
            for r in batch:
                r.cache.commit_append()
            self.peak_used_pages = max(self.peak_used_pages, len(self.pool.leased))
            tokens = [self.next_token(r.request_id, len(r.output)) for r in batch]
            events.extend(self._emit(r, t) for r, t in zip(batch, tokens))
        while self.pending and len(self.active) < self.max_batch_size and len(prefill_ids) < self.max_prefills_per_step:
            r = self.pending[0]
            if self.reserved_pages + r.reserved_pages > self.pool.max_pages:
                break
            if prefill_ids and prefill_tokens + len(r.prompt) > self.prefill_token_budget:
                break
            self.pending.popleft()
            self.active[r.request_id] = r
            self.reserved_pages += r.reserved_pages
            r.state = 'active'
            r.cache = CacheOracle(self.pool, 1, r.capacity)
            r.cache.prepare_append(len(r.prompt))
            r.cache.commit_append()
            self.peak_used_pages = max(self.peak_used_pages, len(self.pool.leased))
            events.append(self._emit(r, self.next_token(r.request_id, 0)))
            prefill_ids.append(r.request_id)
            prefill_tokens += len(r.prompt)
        self.steps.append(dict(iteration=self.iteration, decode_request_ids=decode_ids,
                               prefill_request_ids=prefill_ids, decode_tables=decode_tables,
                               logical_reserved_pages=self.reserved_pages,
                               peak_used_pages=self.peak_used_pages, **self.pool.memory_stats()))
        self.iteration += 1
        return events

    @property
    def has_work(self):
        return bool(self.active or self.pending)
