"""Transactional ragged decode over independent paged caches (reference
minitorch/paged_decode.py:10-93).

The reference builds the [B, columns] block table, the offsets and the
position IDs on the host and uploads them (plus two cudaMallocs) every step.
Here ``prepare()`` uploads only the batch's slot IDs (asynchronously, from
pinned memory) and one kernel, ``mt_sched_decode_prepare``, takes each row's
new page from the device free list and writes the table, offsets, positions
and cu_seqlens into a workspace the pool keeps. ``decode_attention`` then runs
the fused append + attention kernel per layer on that metadata.
"""
import numpy as np

from .paged_kv_cache import PagedKVCache, _DeviceView
from .runtime import RawDeviceBuffer, PinnedHostBuffer, DeviceTensor, runtime, P, I
from . import paged_ops


# Rows a graph-mode workspace is sized for (more when a batch is larger).
GRAPH_ROWS = 256


def _padded_work_list(work, items, merges, b, cap, split_tokens):
    """A decode work list padded to the fixed length of a captured step:
    b x ceil(cap / split) (row, split) entries, then b merge rows when a row
    can span several splits; padding entries are -1 (skipped by the kernels)."""
    nsplit_max = -(-cap // split_tokens)
    items_pad, merges_pad = b * nsplit_max, (b if nsplit_max > 1 else 0)
    out = np.full(2 * items_pad + merges_pad, -1, np.int32)
    out[:2 * items] = work[:2 * items]
    out[2 * items_pad:2 * items_pad + merges] = work[2 * items:2 * items + merges]
    return out, items_pad, merges_pad


class _DecodeWorkspace:
    """Per-pool device buffers for decode metadata, grown on demand, and the
    captured decode steps (graphs) that use them: a graph holds their device
    addresses, so every graph is released when a buffer is reallocated."""

    def __init__(self):
        self.rows = self.cols = self.work = 0
        self.buffer = None
        self.stagings = None
        self.partials = None
        self.partial_bytes = 0
        self.graphs = {}          # batch size -> captured step
        self.eager_steps = {}     # batch size -> eager steps run in graph mode
        self.uncapturable = set()  # batch sizes whose capture failed: eager from then on

    def release_graphs(self):
        for step in self.graphs.values():
            step.close()
        self.graphs.clear()

    def ensure(self, rows, cols, work):
        if rows <= self.rows and cols <= self.cols and work <= self.work and self.buffer is not None:
            return
        self.release_graphs()
        self.rows, self.cols, self.work = max(rows, self.rows), max(cols, self.cols), max(work, self.work)
        r, c = self.rows, self.cols
        # slots | work list | offsets | positions | cu_seqlens | new_page | table
        self.sizes = [4 * r, 4 * self.work, 4 * r, 4 * r, 4 * (r + 1), 4 * r, 4 * r * c]
        self.offsets = np.cumsum([0] + [(s + 255) // 256 * 256 for s in self.sizes]).tolist()
        self.buffer = RawDeviceBuffer(int(self.offsets[-1]))
        # slots and the work list go up in one copy, from two staging buffers
        # used in turn, so that a step can be prepared while the previous
        # step's upload is still queued
        self.stagings = [PinnedHostBuffer(int(self.offsets[2])) for _ in range(2)]
        self.turn = 0
        self.uploaded = None  # the slots and work list the device buffer holds

    def upload(self, payload):
        """Upload the slots and work list, unless the buffer already holds
        exactly these (a steady batch: every row grows by one token, so the
        longest-first order changes only when a row joins, leaves or reaches
        another split). Only this method writes that part of the buffer."""
        if self.uploaded is not None and np.array_equal(self.uploaded, payload):
            return
        self.staging.upload_async(self.ptr(0), payload)
        self.uploaded = payload.copy()

    @property
    def staging(self):
        self.turn ^= 1
        return self.stagings[self.turn]

    def ensure_partials(self, nbytes):
        if nbytes > self.partial_bytes:
            self.release_graphs()
            self.partials = RawDeviceBuffer(nbytes)
            self.partial_bytes = nbytes
        return self.partials.ptr if nbytes else None

    def ptr(self, index):
        return self.buffer.ptr + int(self.offsets[index])


class PagedDecodeBatch:
    """Batched projections plus per-row paged attention on the default stream.

    Owns only transient metadata; the child caches keep their pages and
    committed lengths. A failed execution aborts every participating cache.
    """

    def __init__(self, model, idx, caches):
        self.caches = tuple(caches)
        if not self.caches or len({id(c) for c in self.caches}) != len(self.caches):
            raise ValueError('Decode batch needs nonempty, unique caches')
        if any(not isinstance(c, PagedKVCache) for c in self.caches):
            raise ValueError('Batched decode requires paged caches')
        self.pool = self.caches[0].pool
        self.dtype, self.layout = self.pool.dtype, self.pool.layout
        self.batch_size = len(self.caches)
        # idx None: the token IDs are the caches' last tokens kept on the
        # device (token feedback of the sync-free decode loop).
        if idx is not None and (not isinstance(idx, DeviceTensor) or idx.shape != (self.batch_size, 1)
                                or idx.dtype != 'float32'):
            raise ValueError('Expected FP32 token IDs [request_count,1] on model backend')
        for cache in self.caches:
            cache._validate_model(model)
            if (cache.pool is not self.pool or self.pool.closed or cache.batch_size != 1 or
                    cache._pending_tokens is not None or not 0 < cache.length < cache.capacity):
                raise ValueError('Decode caches must share a live pool, have batch=1 and remaining capacity')
        self.offsets = np.array([c.length for c in self.caches], np.int32)
        self.columns = max((c.length + 1 + self.pool.page_size - 1) // self.pool.page_size for c in self.caches)
        self.table = self.device_offsets = self.position_ids = self.cu_seqlens = self.work = None
        self._prepared, self._written_layers = [], set()
        self._committed = False
        self._device_prepared = False
        self._graph = False
        self.last_attention_path = 'paged_batch_decode'

    def _workspace(self, work_len, rows=None):
        ws = getattr(self.pool, '_decode_workspace', None)
        if ws is None:
            ws = self.pool._decode_workspace = _DecodeWorkspace()
        ws.ensure(rows or self.batch_size, self.columns, work_len)
        return ws

    def prepare(self, *, graph=False, embed=None):
        """Upload the batch's slots and work list, then build the step's
        metadata on the device (with ``embed``, and the rows' embeddings: see
        ``prepare_device``) and update the host mirrors.

        With ``graph`` the metadata takes the fixed shapes a captured step
        replays with: the table is [B, pool.max_cols] (the split length
        follows from it), the work list is padded to B x (most splits a row
        can have) entries, plus B merge rows when rows can split, with -1
        rows that the kernels skip, the page budget is read from the pool
        header on the device, and the workspace is sized for ``GRAPH_ROWS``
        rows so that batches up to that size share it. The device half is
        then left to ``prepare_device``, which the caller issues inside the
        capture (or before replaying one)."""
        if self._prepared or self._committed:
            raise ValueError('Decode batch already executed')
        pool, b = self.pool, self.batch_size
        self._graph = graph
        if graph:
            self.columns = pool.max_cols
        heads = max(h for h, _ in self.layout)
        # Work list: every (row, split) longest first, balanced over the
        # compute units; the kernel writes each row to its own output row.
        self.split_tokens = paged_ops.split_tokens_for(page_size=pool.page_size, columns=self.columns)
        work, self.work_items, self.merge_rows = paged_ops.decode_work_list(
            self.offsets + 1, heads, self.split_tokens, runtime().compute_units())
        rows = None
        if graph:
            rows = max(b, GRAPH_ROWS)
            work, self.work_items, self.merge_rows = _padded_work_list(
                work, self.work_items, self.merge_rows, b, self.columns * pool.page_size, self.split_tokens)
            reserve = len(_padded_work_list(work[:0], 0, 0, rows, self.columns * pool.page_size,
                                            self.split_tokens)[0])
        ws = self._workspace(reserve if graph else len(work), rows)
        slots = np.array([c.slot for c in self.caches], np.int32)
        needs = (self.offsets % pool.page_size) == 0
        avail = pool.max_pages - pool._leased_count
        upload = np.zeros(int(ws.offsets[2]) // 4, np.int32)
        upload[:b] = slots
        w0 = int(ws.offsets[1]) // 4
        upload[w0:w0 + len(work)] = work
        ws.upload(upload[:w0 + len(work)])
        self._ws = ws
        self._limit = -1 if graph else avail
        if not graph:
            self.prepare_device(embed)
        self.table = _DeviceView(ws.buffer, int(ws.offsets[6]), 4 * b * self.columns)
        self.device_slots = _DeviceView(ws.buffer, int(ws.offsets[0]), 4 * b)
        self.device_offsets = _DeviceView(ws.buffer, int(ws.offsets[2]), 4 * b)
        self.cu_seqlens = _DeviceView(ws.buffer, int(ws.offsets[4]), 4 * (b + 1))
        self.work = _DeviceView(ws.buffer, int(ws.offsets[1]), 4 * len(work))
        self.position_ids = DeviceTensor((b, 1), 'float32', buffer=ws.buffer, byte_offset=int(ws.offsets[3]))
        # Host half, row by row like the reference (paged_decode.py:44-46):
        # the row whose page would exceed the budget raises MemoryError (in
        # graph mode before any device work of the step).
        pops = 0
        for cache, need in zip(self.caches, needs):
            self._prepared.append(cache)
            if need and pops >= avail:
                CacheBase_prepare_failed(cache)
                raise MemoryError('KV page budget exhausted')
            cache._prepare_decode_row(bool(need))
            if need:
                pool._mirror_sequential_pops(1)
                pops += 1

    def prepare_device(self, embed=None):
        """``mt_sched_decode_prepare``: each row's new page from the device
        free list, and the table, offsets, positions and cu_seqlens. With
        ``embed`` = (x, wte, wpe, vocab, n_positions, dim) the same launch also
        writes the rows' token embeddings into ``x`` from the pool's per-slot
        last tokens (``mt_sched_decode_prepare_embed``)."""
        ws, pool = self._ws, self.pool
        args = (ws.ptr(0), self.batch_size, self.columns, pool.page_size, self._limit, ws.ptr(6), ws.ptr(2),
                ws.ptr(3), ws.ptr(4), ws.ptr(5))
        if embed is None:
            pool._call('mt_sched_decode_prepare', [P, I, I, I, I, P, P, P, P, P], *args)
        else:
            x, wte, wpe, vocab, n_positions, dim = embed
            pool._call('mt_sched_decode_prepare_embed', [P, I, I, I, I, P, P, P, P, P, P, P, P, P, I, I, I, I],
                       *args, x, wte, wpe, pool.slot_tokens.ptr, pool.max_slots, vocab, n_positions, dim)
        self._device_prepared = True

    def decode_attention(self, layer, q, k, v):
        if self.table is None or layer in self._written_layers or not 0 <= layer < len(self.layout):
            raise ValueError('Invalid decode batch layer/transaction')
        h, d = self.layout[layer]
        if any(not isinstance(t, DeviceTensor) or t.shape != (self.batch_size, h, 1, d) or t.dtype != self.dtype
               for t in (q, k, v)):
            raise ValueError('Invalid batched decode Q/K/V')
        out = DeviceTensor(q.shape, self.dtype)
        pool = self.pool
        partial_bytes = paged_ops.decode_workspace_bytes(b=self.batch_size, h=h, page_size=pool.page_size,
                                                         columns=self.columns, split_tokens=self.split_tokens)
        partials = self._ws.ensure_partials(partial_bytes)
        paged_ops.paged_decode_split(out.ptr, q.ptr, k.ptr, v.ptr, pool.slab_table.ptr, self.table.ptr,
                                     self.device_offsets.ptr, b=self.batch_size, h=h, d=d,
                                     page_size=pool.page_size, pages_per_slab=pool.pages_per_slab,
                                     num_slabs=pool.num_slabs, columns=self.columns, layer=layer,
                                     layers=len(self.layout), dtype=self.dtype,
                                     split_tokens=self.split_tokens, work=self.work.ptr,
                                     work_items=self.work_items, merge_rows=self.merge_rows,
                                     workspace=partials, workspace_bytes=partial_bytes)
        self._written_layers.add(layer)
        for cache in self.caches:
            cache._written_layers.add(layer)
            cache.last_attention_path = self.last_attention_path
        return out

    def attention_metadata(self):
        """The batch's paged metadata for every layer at once (``mt_decode_attention``
        of include/mt_model.h), for the native decoder loop; the split partials
        are sized for the widest layer."""
        from .model import DecodeAttentionStruct
        if self.table is None or self._written_layers:
            raise ValueError('Invalid decode batch layer/transaction')
        pool = self.pool
        heads = max(h for h, _ in self.layout)
        partial_bytes = paged_ops.decode_workspace_bytes(b=self.batch_size, h=heads, page_size=pool.page_size,
                                                         columns=self.columns, split_tokens=self.split_tokens)
        if self._graph:
            # sized for the workspace's rows, so that batch sizes share it
            partial_bytes = paged_ops.decode_workspace_bytes(b=self._ws.rows, h=heads, page_size=pool.page_size,
                                                             columns=self.columns, split_tokens=self.split_tokens)
        partials = self._ws.ensure_partials(partial_bytes)
        # A captured step must see pages of slabs opened after the capture:
        # it bounds page IDs by the whole budget's slabs (all allocated).
        slabs = pool.max_slabs if self._graph else pool.num_slabs
        return DecodeAttentionStruct(pool.slab_table.ptr, self.table.ptr, self.device_offsets.ptr,
                                     pool.page_size, pool.pages_per_slab, slabs, self.columns,
                                     len(self.layout), self.split_tokens, self.work.ptr, self.work_items,
                                     self.merge_rows, partials, partial_bytes)

    def mark_layers_written(self):
        """Record that every layer's K/V was appended (by the native decoder loop)."""
        for layer in range(len(self.layout)):
            self._written_layers.add(layer)
            for cache in self.caches:
                cache._written_layers.add(layer)
                cache.last_attention_path = self.last_attention_path

    def commit_device(self):
        """``mt_sched_add_length``: every row's committed length + 1 on the device."""
        self.pool._call('mt_sched_add_length', [P, I, I], self._ws.ptr(0), self.batch_size, 1)

    def commit(self, *, device=True):
        """Commit every cache; ``device=False`` when the device half (every
        row's length + 1) ran already: in the greedy selection
        (``mt_row_argmax_commit``) of a sync-free or captured step."""
        if len(self._written_layers) != len(self.layout):
            raise ValueError('Cannot commit incomplete decode batch')
        if any(c._pending_tokens != 1 or len(c._written_layers) != len(c.layout) for c in self.caches):
            raise ValueError('Decode transaction modified during execution')
        if device:
            self.commit_device()
        for cache in self.caches:
            cache.commit_append(device=False)
        self._committed = True

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc, tb):
        if not self._committed:
            if self._device_prepared:
                self.pool._call('mt_sched_decode_abort', [P, I, P], self._ws.ptr(0), self.batch_size,
                                self._ws.ptr(5))
            for cache in self._prepared:
                cache.abort_append(device=False)
        self.position_ids = None


def CacheBase_prepare_failed(cache):
    """State of a cache whose prepare_append(1) failed on the budget: the
    reference's prepare_append aborts itself (paged_kv_cache.py:187-189)."""
    from .kv_cache import CacheBase
    CacheBase.prepare_append(cache, 1)
    cache._previous_counts = list(cache._counts)
    cache._new_count = 0
