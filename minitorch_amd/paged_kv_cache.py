"""Paged KV pool and per-request paged caches (reference minitorch/paged_kv_cache.py).

Same public surface and page-ID sequence as the reference, MI355X-first inside:

* ``KVPagePool`` reserves its whole KV budget at construction as one device
  allocation (288 GB of HBM makes the reference's lazily cudaMalloc'ed slabs
  unnecessary) and opens slabs *logically* in the reference's order, so page
  IDs, ``len(pool._slabs)`` and the reserved-bytes statistic match it.
* The free list, page ownership, per-row page lists, lengths and the slab
  table live in a device state blob handled by ``sched_kernels.so``
  (``include/mt_sched.h``); caches and decode batches change them with kernels,
  never by reading them back. The host mirrors only what the reference's
  checks need without device reads: counts of free/leased pages, opened slabs,
  per-row page counts, and whether each free-list entry was issued before
  (for ``kv_pool_page_reuses``).
* A cache's block table is its rows of the pool's slot table (row stride
  ``pool.max_cols``), so adding a page never re-uploads a table.
"""
import ctypes as ct
import math
import weakref
import numpy as np

from .amp import autocast_dtype
from .dtypes import itemsize
from .kv_cache import CacheBase
from .runtime import RawDeviceBuffer, DeviceTensor, library, call, runtime, P, I, Z
from . import paged_ops

U64 = ct.c_ulonglong


def sched_library():
    return library('sched_kernels')


class _DeviceView:
    """A byte range inside a RawDeviceBuffer (``.ptr``, ``.nbytes``)."""

    def __init__(self, buffer, offset, nbytes):
        self._buffer, self._offset, self.nbytes = buffer, offset, nbytes

    @property
    def ptr(self):
        return self._buffer.ptr + self._offset

    def download(self, dtype, count=None):
        if count is None:
            count = self.nbytes // np.dtype(dtype).itemsize
        return self._buffer.download(dtype, count, self._offset)

    def close(self):
        pass


class KVPagePool:
    """Page budget, device page allocator and slot table shared by paged caches.

    Each slab is [layers, 2, pages_per_slab, heads, page_size, head_dim]
    (reference minitorch/paged_kv_cache.py:27-69).
    """

    def __init__(self, model, *, page_size=16, max_bytes=256 * 1024 ** 2, pages_per_slab=4,
                 max_slots=None):
        if getattr(model, 'training', False):
            raise ValueError('Page pool requires device storage and model.eval()')
        layers = model.transformer_layers()
        layout = tuple((l.attention.n_head, l.attention.attn_hidden_dim) for l in layers)
        if not layout or len(set(layout)) != 1 or any(d > 128 for _, d in layout):
            raise ValueError('Page pool requires uniform head layout and head_dim<=128')
        if type(page_size) is not int or page_size not in (8, 16, 32):
            raise ValueError('page_size must be 8, 16 or 32')
        if type(max_bytes) is not int or type(pages_per_slab) is not int or min(max_bytes, pages_per_slab) < 1:
            raise ValueError('Positive KV budget and pages_per_slab required')
        self.model = weakref.ref(model)
        self.layout = layout
        self.layers = len(layout)
        self.heads, self.dim = layout[0]
        self.dtype = autocast_dtype() or 'float32'
        self.page_size = page_size
        self.page_bytes = 2 * self.layers * self.heads * self.dim * page_size * itemsize(self.dtype)
        if max_bytes < self.page_bytes:
            raise ValueError('KV budget must hold at least one page')
        self.pages_per_slab = min(pages_per_slab, max_bytes // self.page_bytes)
        self.slab_bytes = self.pages_per_slab * self.page_bytes
        self.max_slabs = max_bytes // self.slab_bytes
        self.max_pages = self.max_slabs * self.pages_per_slab
        if self.max_pages > 2 ** 31 - 1:
            raise ValueError('Page IDs must fit int32')
        self.max_bytes = max_bytes
        self.max_cols = (model.n_positions + page_size - 1) // page_size
        self.max_slots = int(max_slots) if max_slots else max(1, min(self.max_pages, 1 << 16))
        self.kv = RawDeviceBuffer(self.max_slabs * self.slab_bytes)
        offsets = (ct.c_size_t * 9)()
        call(sched_library(), 'mt_pool_layout', [I, I, I, I, ct.POINTER(ct.c_size_t)],
             self.max_pages, self.max_slabs, self.max_slots, self.max_cols, offsets)
        self._offsets = list(offsets)
        self.state = RawDeviceBuffer(self._offsets[8])
        self.slab_table = _DeviceView(self.state, self._offsets[4], self.max_slabs * 8)
        self.slot_pages = _DeviceView(self.state, self._offsets[7], self.max_slots * self.max_cols * 4)
        self.slot_ids = RawDeviceBuffer(4 * self.max_slots)
        self.slot_ids.upload(np.arange(self.max_slots, dtype=np.int32))
        self._call('mt_pool_init', [])
        self._scratch = RawDeviceBuffer(4 * self.max_pages)
        # host mirrors
        self._slabs = []                 # one entry per opened slab (base address)
        self._free_issued = []           # free stack bottom..top: was the page issued before?
        self._leased_count = 0
        self.page_acquires = self.page_releases = self.page_reuses = 0
        self._slot_used = bytearray(self.max_slots)
        self._slot_tokens = None
        self._owner_ids = {}
        self._next_owner = self.max_slots
        self.closed = False

    # ------------------------------------------------------------ device ---
    def _geometry(self):
        return (self.state.ptr, self.max_pages, self.max_slabs, self.max_slots, self.max_cols,
                self.pages_per_slab, self.kv.ptr, self.slab_bytes)

    _GEOMETRY_TYPES = [P, I, I, I, I, I, U64, U64]

    def _call(self, name, types, *args):
        call(sched_library(), name, self._GEOMETRY_TYPES + types, *self._geometry(), *args)

    @property
    def slot_len_ptr(self):
        """Device address of the per-slot committed lengths (int32[max_slots])."""
        return self.state.ptr + self._offsets[5]

    def slots_ptr(self, first):
        return self.slot_ids.ptr + 4 * first

    def header(self):
        """Device header: top, slabs_opened, leased, error, acquires, releases, reuses."""
        raw = self.state.download(np.uint8, 40, self._offsets[0])
        ints = raw[:16].view(np.int32)
        longs = raw[16:].view(np.int64)
        return dict(top=int(ints[0]), slabs_opened=int(ints[1]), leased=int(ints[2]),
                    error=int(ints[3]), acquires=int(longs[0]), releases=int(longs[1]),
                    reuses=int(longs[2]))

    def free_stack(self):
        """Device free list bottom..top (for tests and introspection)."""
        top = self.header()['top']
        return self.state.download(np.int32, top, self._offsets[1]).tolist()

    # ------------------------------------------------------ host mirrors ---
    def _open_slab(self):
        index = len(self._slabs)
        self._slabs.append(self.kv.ptr + index * self.slab_bytes)
        self._free_issued.extend([False] * self.pages_per_slab)

    def _mirror_bulk_pop(self, count):
        while len(self._free_issued) < count:
            self._open_slab()
        popped = self._free_issued[len(self._free_issued) - count:]
        del self._free_issued[len(self._free_issued) - count:]
        self.page_reuses += sum(popped)
        self.page_acquires += count
        self._leased_count += count

    def _mirror_sequential_pops(self, pops):
        for _ in range(pops):
            if not self._free_issued:
                self._open_slab()
            self.page_reuses += self._free_issued.pop()
        self.page_acquires += pops
        self._leased_count += pops

    def _mirror_release(self, n):
        self._free_issued.extend([True] * n)
        self._leased_count -= n
        self.page_releases += n

    def _check_budget(self, count):
        if count > self.max_pages - self._leased_count:
            raise MemoryError('KV page budget exhausted')

    @property
    def num_slabs(self):
        return len(self._slabs)

    @property
    def used_pages(self):
        return self._leased_count

    # ------------------------------------- several one-row caches at once ---
    def close_caches(self, caches):
        """``close()`` of one-row caches of this pool, in order, with one
        release launch: pages are pushed cache by cache in page order, as
        consecutive ``close()`` calls push them."""
        caches = [c for c in caches if not c.closed]
        if len(caches) < 2 or any(c.pool is not self or c.batch_size != 1 or c._owns_pool for c in caches):
            for c in caches:
                c.close()
            return
        for c in caches:
            c.abort_append()
        slots = DeviceTensor.from_numpy(np.array([c.slot for c in caches], np.int32), 'int32')
        self._call('mt_pool_release_rows', [P, I, I, I], slots.ptr, len(caches), 0, 1)
        for c in caches:
            counts = self._row_counts.pop(c.slot, None) or []
            self._mirror_release(sum(counts))
            for i in range(len(counts)):
                counts[i] = 0
            self._free_slots(c.slot, 1)
            c._release.detach()
            c.closed, c.valid, c.length = True, False, 0

    def append_lists(self, caches, tokens):
        """Host int32 lists for ``prepare_appends`` and ``commit_appends`` of
        one-row caches before their appends: the caches' slots, the pages each
        append takes, the tokens."""
        slots = [c.slot for c in caches]
        counts = [(c.length + int(n) + c.page_size - 1) // c.page_size - c._counts[0] for c, n in zip(caches, tokens)]
        return slots + counts + [int(n) for n in tokens]

    def prepare_appends(self, caches, tokens, device_lists):
        """``prepare_append(tokens[i])`` of one-row caches of this pool, in
        order, with one launch (``mt_pool_acquire_lists``): the same pages as
        consecutive calls. ``device_lists``: device address of
        ``append_lists(caches, tokens)`` (int32), uploaded by the caller. When
        the appends together exceed the page budget nothing is prepared and
        MemoryError is raised (consecutive calls would have prepared the
        caches before the one that fails)."""
        lists = self.append_lists(caches, tokens)
        n = len(caches)
        counts = lists[n:2 * n]
        if sum(counts) > self.max_pages - self._leased_count:
            raise MemoryError('KV page budget exhausted')
        prepared = []
        try:
            for c, t in zip(caches, tokens):
                CacheBase.prepare_append(c, int(t))
                prepared.append(c)
                c._previous_counts = list(c._counts)
        except Exception:
            for c in prepared:
                c.abort_append()
            raise
        if sum(counts):
            self._call('mt_pool_acquire_lists', [P, P, I, P], device_lists, device_lists + 4 * n, n,
                       self._scratch.ptr)
        for c, k in zip(caches, counts):
            if k:
                self._mirror_bulk_pop(k)
                c._counts[0] += k
            c._new_count = k

    def commit_appends(self, caches, device_lists):
        """``commit_append()`` of prepared one-row caches with one length
        launch (``mt_sched_add_lengths``); ``device_lists`` as
        ``prepare_appends`` takes it, followed by the tokens."""
        n = len(caches)
        for c in caches:
            c.commit_append(device=False)
        self._call('mt_sched_add_lengths', [P, P, I], device_lists, device_lists + 8 * n, n)

    # ------------------------------------------------------------ slots ---
    def _alloc_slots(self, n):
        first = self._slot_used.find(b'\x00' * n)
        if first < 0:
            raise MemoryError('Page pool has no free cache slots')
        self._slot_used[first:first + n] = b'\x01' * n
        return first

    def _free_slots(self, first, n):
        self._slot_used[first:first + n] = b'\x00' * n

    @property
    def slot_tokens(self):
        """Device fp32 array [max_slots]: the last token of each cache slot's
        request, written by the greedy selection of a prefill or decode step
        and read by the next decode step (device-side token feedback). Starts
        as NaN (an unset token embeds as a NaN row)."""
        if self._slot_tokens is None:
            self._slot_tokens = RawDeviceBuffer(4 * self.max_slots)
            self._slot_tokens.fill_words(0x7FC00000)
        return self._slot_tokens

    def _owner_id(self, owner):
        key = id(owner)
        if key not in self._owner_ids:
            self._owner_ids[key] = (self._next_owner, weakref.ref(owner) if _weakrefable(owner) else owner)
            self._next_owner += 1
        return self._owner_ids[key][0]

    # ------------------------------------------------------------- API ----
    def acquire(self, count, owner):
        """Lease ``count`` pages to ``owner`` and return their IDs (reference
        minitorch/paged_kv_cache.py:71-94). Reads the IDs back from the device."""
        if self.closed or type(count) is not int or count < 0:
            raise ValueError('Closed pool or invalid page count')
        self._check_budget(count)
        if count == 0:
            return []
        self._call('mt_pool_pop', [I, I, P], count, self._owner_id(owner), self._scratch.ptr)
        self._mirror_bulk_pop(count)
        return self._scratch.download(np.int32, count).tolist()

    def release(self, pages, owner):
        """Return pages leased to ``owner`` (reference minitorch/paged_kv_cache.py:96-103)."""
        pages = [int(p) for p in pages]
        if self.closed or len(set(pages)) != len(pages):
            raise ValueError('Invalid page ownership or duplicate release')
        if not pages:
            self.page_releases += 0
            return
        oid = self._owner_ids.get(id(owner), (None,))[0]
        owners = self.state.download(np.int32, self.max_pages, self._offsets[3])
        if oid is None or any(not 0 <= p < self.max_pages or owners[p] != oid for p in pages):
            raise ValueError('Invalid page ownership or duplicate release')
        self._scratch.upload(np.array(pages, np.int32))
        self._call('mt_pool_push', [P, I, I], self._scratch.ptr, len(pages), oid)
        self._mirror_release(len(pages))

    def memory_stats(self):
        """The reference's keys (minitorch/paged_kv_cache.py:105-117):
        ``kv_pool_reserved_bytes`` counts the slabs opened so far, as the
        reference's lazily allocated slabs would hold them. This pool holds
        its whole budget in one device allocation from construction, which
        ``kv_pool_physical_bytes`` reports (0 once closed)."""
        reserved = len(self._slabs) * self.slab_bytes
        assigned = self._leased_count * self.page_bytes
        return dict(kv_pool_reserved_bytes=reserved, kv_pool_assigned_bytes=assigned,
                    kv_pool_physical_bytes=0 if self.closed else self.kv.nbytes,
                    kv_pool_free_bytes=reserved - assigned,
                    kv_pool_metadata_bytes=0 if self.closed else self.state.nbytes,
                    kv_pool_used_pages=self._leased_count, kv_pool_free_pages=len(self._free_issued),
                    kv_pool_max_pages=self.max_pages, kv_pool_page_acquires=self.page_acquires,
                    kv_pool_page_releases=self.page_releases, kv_pool_page_reuses=self.page_reuses)

    def close(self):
        if self.closed:
            return
        if self._leased_count:
            raise ValueError('Cannot close page pool while caches own pages')
        ws = getattr(self, '_decode_workspace', None)
        if ws is not None:
            ws.release_graphs()      # captured decode steps hold this pool's addresses
        self._slabs.clear()
        self._free_issued.clear()
        for buffer in (self.kv, self.state, self.slot_ids, self._scratch, self._slot_tokens):
            if buffer is not None:
                buffer.close()
        self.closed = True


def _weakrefable(obj):
    try:
        weakref.ref(obj)
        return True
    except TypeError:
        return False


def _release_cache(pool, first, rows, owns_pool):
    """Finalizer: return every row's pages and the slots (reference
    minitorch/paged_kv_cache.py:125-131)."""
    if pool.closed:
        return
    counts = getattr(pool, '_row_counts', {}).pop(first, None) or []
    # release every row's pages, row by row, and zero the rows' lengths
    pool._call('mt_pool_release_rows', [P, I, I, I], pool.slots_ptr(first), rows, 0, 1)
    pool._mirror_release(sum(counts))
    for i in range(len(counts)):
        counts[i] = 0
    pool._free_slots(first, rows)
    if owns_pool:
        pool.close()


class PagedKVCache(CacheBase):
    """Per-request paged KV cache with the reference's transaction API
    (minitorch/paged_kv_cache.py:134-263). Rows are consecutive pool slots."""

    def __init__(self, model, batch_size=1, capacity=None, *, page_size=16, page_pool=None,
                 kv_budget_bytes=256 * 1024 ** 2, pages_per_slab=4, paged_prefill_impl='flash'):
        if paged_prefill_impl not in ('flash', 'paged_reference'):
            raise ValueError('Choose flash or paged_reference prefill')
        self.paged_prefill_impl = paged_prefill_impl
        super().__init__(model, batch_size, capacity)
        self._owns_pool = page_pool is None
        pool = page_pool if page_pool is not None else KVPagePool(
            model, page_size=page_size, max_bytes=kv_budget_bytes, pages_per_slab=pages_per_slab)
        if (pool.closed or pool.model() is not model or pool.layout != self.layout
                or pool.dtype != self.dtype or pool.page_size != page_size):
            if self._owns_pool:
                pool.close()
            raise ValueError('Page pool/model/backend/layout/precision/page_size mismatch')
        self.pool = pool
        self.page_size = page_size
        self.table_columns = (self.capacity + page_size - 1) // page_size
        if self.batch_size * self.table_columns > 2 ** 31 - 1:
            if self._owns_pool:
                pool.close()
            raise ValueError('Page table is too large')
        try:
            self.slot = pool._alloc_slots(batch_size)
        except MemoryError:
            if self._owns_pool:
                pool.close()
            raise
        if not hasattr(pool, '_row_counts'):
            pool._row_counts = {}
        self._counts = [0] * batch_size         # pages per row (host mirror)
        pool._row_counts[self.slot] = self._counts
        self._previous_counts = None
        self._new_count = 0
        self._release = weakref.finalize(self, _release_cache, pool, self.slot, batch_size, self._owns_pool)

    # The block table is this cache's rows of the pool slot table.
    @property
    def block_table(self):
        return _DeviceView(self.pool.state, self.pool._offsets[7] + 4 * self.slot * self.pool.max_cols,
                           4 * self.batch_size * self.pool.max_cols)

    @property
    def slots_ptr(self):
        return self.pool.slots_ptr(self.slot)

    def pages(self):
        """Page IDs per row (reads the device slot table)."""
        raw = self.block_table.download(np.int32).reshape(self.batch_size, self.pool.max_cols)
        return [row[:n].tolist() for row, n in zip(raw, self._counts)]

    def validate(self, model, idx, prefill):
        super().validate(model, idx, prefill)
        if self.pool.closed:
            raise ValueError('Page pool is closed')

    def prepare_append(self, tokens):
        super().prepare_append(tokens)
        self._previous_counts = list(self._counts)
        required = (self.length + tokens + self.page_size - 1) // self.page_size
        per_row = required - self._counts[0]
        count = per_row * self.batch_size
        try:
            self.pool._check_budget(count)
            if count:
                self.pool._call('mt_pool_acquire_rows', [P, I, I, P], self.slots_ptr,
                                self.batch_size, per_row, self.pool._scratch.ptr)
                self.pool._mirror_bulk_pop(count)
                for i in range(self.batch_size):
                    self._counts[i] += per_row
            self._new_count = count
        except Exception:
            self.abort_append()
            raise

    def _prepare_decode_row(self, got_page):
        """Host half of prepare_append(1) when the device decode-batch kernel
        has already taken the row's page (PagedDecodeBatch)."""
        CacheBase.prepare_append(self, 1)
        self._previous_counts = list(self._counts)
        if got_page:
            self._counts[0] += 1
            self._new_count = 1
        else:
            self._new_count = 0

    def _common(self, layer):
        pool = self.pool
        return dict(page_size=self.page_size, pages_per_slab=pool.pages_per_slab,
                    num_slabs=pool.num_slabs, columns=pool.max_cols, layer=layer,
                    layers=len(self.layout), dtype=self.dtype)

    def _attention(self, layer, q, k, v, *, prefill):
        self._check_attention(layer, q, k, v)
        b, h, n, d = q.shape
        common = self._common(layer)
        paged_ops.paged_append(k.ptr, v.ptr, self.pool.slab_table.ptr, self.block_table.ptr,
                               b=b, h=h, n=n, d=d, offset=self.length, **common)
        out = DeviceTensor(q.shape, self.dtype)
        paged_ops.paged_attention(out.ptr, q.ptr, self.pool.slab_table.ptr, self.block_table.ptr,
                                  b=b, h=h, nq=n, nk=self.length + n, d=d, offset=self.length,
                                  **common)
        self.last_attention_path = ('paged_reference_prefill' if prefill and self.paged_prefill_impl == 'paged_reference'
                                    else 'paged_prefill' if prefill else 'paged_decode')
        self._written_layers.add(layer)
        return out

    def commit_append(self, *, device=True):
        tokens = self._pending_tokens
        super().commit_append()
        if device:
            self.pool._call('mt_sched_add_length', [P, I, I], self.slots_ptr, self.batch_size, tokens)
        self._new_count = 0
        self._previous_counts = None

    def abort_append(self, *, device=True):
        if self._new_count and self._previous_counts is not None:
            keep = self._previous_counts[0]
            if device:
                self.pool._call('mt_pool_release_rows', [P, I, I, I], self.slots_ptr,
                                self.batch_size, keep, 0)
            self.pool._mirror_release(self._new_count)
            self._counts[:] = self._previous_counts
        self._new_count = 0
        self._previous_counts = None
        super().abort_append()

    @property
    def nbytes(self):
        return sum(self._counts) * self.pool.page_bytes

    def memory_stats(self):
        capacity = self.nbytes
        live = self.batch_size * self.length * self.pool.page_bytes // self.page_size
        result = dict(kv_live_bytes=live, kv_capacity_bytes=capacity, kv_unused_bytes=capacity - live,
                      kv_slot_utilization=live / capacity if capacity else None,
                      kv_metadata_bytes=0 if self.closed else 4 * self.batch_size * self.pool.max_cols,
                      kv_allocator_slack_bytes=0)
        result.update(self.pool.memory_stats())
        return result

    def reset(self):
        if self.closed:
            raise ValueError('Cannot reset a closed cache')
        self.abort_append()
        self.pool._call('mt_pool_release_rows', [P, I, I, I], self.slots_ptr, self.batch_size, 0, 1)
        self.pool._mirror_release(sum(self._counts))
        for i in range(self.batch_size):
            self._counts[i] = 0
        super().reset()

    def close(self):
        if self.closed:
            return
        self.abort_append()
        self._release()
        self.closed, self.valid, self.length = True, False, 0
