"""Seeded synthetic inputs for the op-level paged decode configurations.

A case is the state just before one decode step: a page pool image holding
the committed K/V of every request, an int32 block table [B, columns] whose
physical pages come from a seeded shuffle of the pool (taken in request
order), committed lengths ``offsets = L - 1``, and the step's Q/K/V
[B, H, 1, D]. Values are N(0, 1) from ``numpy.random.default_rng(seed)``.

The pool is one contiguous device allocation split into slabs of
``pages_per_slab`` pages, each slab laid out [layers][2][pps][H][P][D]
(reference src/paged_attention_kernel.cu:2), so the host image is an array
[num_slabs, layers, 2, pps, H, P, D].
"""
from dataclasses import dataclass
import numpy as np
from .dtypes import encode_host, storage_numpy_dtype, itemsize, normalize_dtype
from .runtime import DeviceTensor, RawDeviceBuffer, runtime


@dataclass
class PagedDecodeCase:
    batch: int
    heads: int
    dim: int
    page_size: int
    pages_per_slab: int
    num_slabs: int
    layers: int
    layer: int
    dtype: str
    lengths: np.ndarray      # int64 [B], keys attended including the new token
    table: np.ndarray        # int32 [B, columns]
    image: np.ndarray        # storage dtype [num_slabs, layers, 2, pps, H, P, D]
    q: np.ndarray            # storage dtype [B, H, 1, D]
    k: np.ndarray
    v: np.ndarray

    @property
    def offsets(self):
        return (self.lengths - 1).astype(np.int32)

    @property
    def columns(self):
        return self.table.shape[1]

    @property
    def page_bytes(self):
        return 2 * self.layers * self.heads * self.dim * self.page_size * itemsize(self.dtype)

    @property
    def slab_bytes(self):
        return self.page_bytes * self.pages_per_slab


def _normal(rng, shape, dtype):
    return encode_host(rng.standard_normal(shape, dtype=np.float32), dtype).reshape(shape)


def make_decode_case(seed, *, batch, heads, dim, page_size, lengths, pool_pages,
                     pages_per_slab, dtype, layers=1, layer=0, columns=None):
    """Build a case; ``lengths`` are the per-request key counts L_i (>= 1)."""
    dtype = normalize_dtype(dtype)
    rng = np.random.default_rng(seed)
    lengths = np.asarray(lengths, np.int64)
    pages_needed = (lengths + page_size - 1) // page_size
    if pages_needed.sum() > pool_pages:
        raise ValueError('Pool too small for the requested contexts')
    if pool_pages % pages_per_slab:
        raise ValueError('pool_pages must be a multiple of pages_per_slab')
    num_slabs = pool_pages // pages_per_slab
    columns = int(pages_needed.max()) if columns is None else columns
    perm = rng.permutation(pool_pages).astype(np.int32)
    table = np.full((batch, columns), -1, np.int32)
    cursor = 0
    for b in range(batch):
        n = int(pages_needed[b])
        table[b, :n] = perm[cursor:cursor + n]
        cursor += n
    q = _normal(rng, (batch, heads, 1, dim), dtype)
    k = _normal(rng, (batch, heads, 1, dim), dtype)
    v = _normal(rng, (batch, heads, 1, dim), dtype)
    image = np.zeros((num_slabs, layers, 2, pages_per_slab, heads, page_size, dim),
                     storage_numpy_dtype(dtype))
    used = table[table >= 0]
    block = _normal(rng, (used.size, layers, 2, heads, page_size, dim), dtype)
    image[used // pages_per_slab, :, :, used % pages_per_slab] = block
    return PagedDecodeCase(batch, heads, dim, page_size, pages_per_slab, num_slabs, layers, layer,
                           dtype, lengths, table, image, q, k, v)


def config1_case(seed=0):
    """Config 1: B=4, L={7,33,64,120}, H=12, D=64, P=16, fp32, 64-page pool."""
    return make_decode_case(seed, batch=4, heads=12, dim=64, page_size=16,
                            lengths=[7, 33, 64, 120], pool_pages=64, pages_per_slab=4,
                            dtype='float32')


def config2_lengths(seed=0, batch=64):
    return np.random.default_rng([seed, 2]).integers(128, 1025, size=batch)


def config2_case(seed=0, batch=64, dtype='float16'):
    """Config 2: B=64, L ~ U{128..1024}, H=12, D=64, P=16, fp16, 8192-page pool."""
    return make_decode_case(seed, batch=batch, heads=12, dim=64, page_size=16,
                            lengths=config2_lengths(seed, batch), pool_pages=8192,
                            pages_per_slab=64, dtype=dtype, columns=64)


def config5_lengths(seed=0, batch=512):
    rng = np.random.default_rng([seed, 5])
    return np.clip(np.round(np.exp(rng.normal(np.log(256.0), 1.2, size=batch))), 1, 8192).astype(np.int64)


class DevicePagedCase:
    """A case resident on the device: one pool allocation, slab table, block
    table, offsets, Q/K/V and the output."""

    def __init__(self, case):
        self.case = case
        c = case
        self.pool = RawDeviceBuffer(c.num_slabs * c.slab_bytes)
        self.pool.upload(c.image)
        base = self.pool.ptr
        self.slab_table = RawDeviceBuffer(8 * c.num_slabs)
        self.slab_table.upload(np.array([base + s * c.slab_bytes for s in range(c.num_slabs)], np.uint64))
        self.block_table = RawDeviceBuffer(c.table.nbytes)
        self.block_table.upload(c.table)
        self.offsets = RawDeviceBuffer(4 * c.batch)
        self.offsets.upload(c.offsets)
        self.q = DeviceTensor(c.q.shape, c.dtype)
        self.k = DeviceTensor(c.k.shape, c.dtype)
        self.v = DeviceTensor(c.v.shape, c.dtype)
        for t, a in ((self.q, c.q), (self.k, c.k), (self.v, c.v)):
            runtime().h2d(t.ptr, a)
        self.out = DeviceTensor(c.q.shape, c.dtype)

    def reset_pool(self):
        self.pool.upload(self.case.image)

    def pool_image(self):
        c = self.case
        raw = self.pool.download(storage_numpy_dtype(c.dtype))
        return raw.reshape(c.image.shape)

    def kwargs(self):
        c = self.case
        return dict(b=c.batch, h=c.heads, d=c.dim, page_size=c.page_size,
                    pages_per_slab=c.pages_per_slab, num_slabs=c.num_slabs, columns=c.columns,
                    layer=c.layer, layers=c.layers, dtype=c.dtype)


class DeviceRaggedCase:
    """A large op-level case built on the device (config 5 sizes): pool pages
    filled with a deterministic hash of (seed, index) in [-2, 2) instead of
    N(0, 1) host data, block table from a seeded shuffle of the pool, Q/K/V
    filled the same way. Used for timing; parity uses host-built cases."""

    def __init__(self, seed, *, batch, heads, dim, page_size, lengths, dtype, pages_per_slab=64,
                 slack_pages=64):
        from .dtypes import dtype_code
        rt = runtime()
        self.dtype = normalize_dtype(dtype)
        self.batch, self.heads, self.dim, self.page_size = batch, heads, dim, page_size
        self.lengths = np.asarray(lengths, np.int64)
        pages_needed = (self.lengths + page_size - 1) // page_size
        pool_pages = int(pages_needed.sum()) + slack_pages
        pool_pages = (pool_pages + pages_per_slab - 1) // pages_per_slab * pages_per_slab
        self.pages_per_slab, self.num_slabs = pages_per_slab, pool_pages // pages_per_slab
        self.layers, self.layer = 1, 0
        self.page_bytes = 2 * heads * dim * page_size * itemsize(self.dtype)
        self.slab_bytes = self.page_bytes * pages_per_slab
        self.columns = int(pages_needed.max())
        rng = np.random.default_rng([seed, 5, page_size])
        perm = rng.permutation(pool_pages).astype(np.int32)
        table = np.full((batch, self.columns), -1, np.int32)
        cursor = 0
        for b in range(batch):
            n = int(pages_needed[b])
            table[b, :n] = perm[cursor:cursor + n]
            cursor += n
        self.table_host = table
        self.pool = RawDeviceBuffer(self.num_slabs * self.slab_bytes)
        code = dtype_code(self.dtype)
        rt.check(rt.lib.mt_fill_random(self.pool.ptr, self.num_slabs * self.slab_bytes // itemsize(self.dtype),
                                       seed, code))
        self.slab_table = RawDeviceBuffer(8 * self.num_slabs)
        self.slab_table.upload(np.array([self.pool.ptr + s * self.slab_bytes for s in range(self.num_slabs)],
                                        np.uint64))
        self.block_table = RawDeviceBuffer(table.nbytes)
        self.block_table.upload(table)
        self.offsets = RawDeviceBuffer(4 * batch)
        self.offsets.upload((self.lengths - 1).astype(np.int32))
        shape = (batch, heads, 1, dim)
        self.q, self.k, self.v, self.out = (DeviceTensor(shape, self.dtype) for _ in range(4))
        for i, t in enumerate((self.q, self.k, self.v)):
            rt.check(rt.lib.mt_fill_random(t.ptr, t.size, seed + 1 + i, code))

    def kwargs(self):
        return dict(b=self.batch, h=self.heads, d=self.dim, page_size=self.page_size,
                    pages_per_slab=self.pages_per_slab, num_slabs=self.num_slabs, columns=self.columns,
                    layer=self.layer, layers=self.layers, dtype=self.dtype)
