"""mt_paged_decode_batch_noalloc against mt_paged_decode_batch through the C-ABI.

The no-allocation entry keeps its split partials in a fixed device array of
the library instead of the library's growable workspace; it runs the same
kernels, so outputs and the appended pool must be bit-identical to the
reference entry's. Contexts longer than 1024 tokens make the split path (and
so the array) active. Two calls run back to back, the second on a smaller
input, so that a stale partial left by the first would show.
"""
import ctypes as ct

import numpy as np
import pytest

from minitorch_amd.dtypes import dtype_code
from minitorch_amd.runtime import library, runtime, P, I
from minitorch_amd.workloads import make_decode_case, DevicePagedCase
from oracle import paged_oracle as po
from tolerances import assert_attention_close

pytestmark = pytest.mark.gpu
CODES = {'float32': po.F32, 'float16': po.F16, 'bfloat16': po.BF16}
SCRATCH_BYTES = 32 << 20      # MT_PAGED_NOALLOC_SCRATCH_BYTES


def _entry(name):
    f = getattr(library('paged_attention_kernel'), name)
    f.argtypes, f.restype = [P] * 7 + [I] * 10, I
    return f


def _call(name, dev):
    c = dev.case
    return _entry(name)(dev.out.ptr, dev.q.ptr, dev.k.ptr, dev.v.ptr, dev.slab_table.ptr,
                        dev.block_table.ptr, dev.offsets.ptr, c.batch, c.heads, c.dim, c.page_size,
                        c.pages_per_slab, c.num_slabs, c.columns, c.layer, c.layers, dtype_code(c.dtype))


def _case(seed, batch, heads, dim, dtype, max_len, page_size=16):
    rng = np.random.default_rng([seed, 77])
    lengths = rng.integers(1, max_len + 1, size=batch)
    lengths[0] = max_len                     # at least one row with several splits
    lengths[-1] = 1                          # and one with only the new token
    pages = int(((lengths + page_size - 1) // page_size).sum())
    pps = 16
    pool = (pages + 64 + pps - 1) // pps * pps
    columns = (max_len + page_size - 1) // page_size
    return make_decode_case(seed, batch=batch, heads=heads, dim=dim, page_size=page_size, lengths=lengths,
                            pool_pages=pool, pages_per_slab=pps, dtype=dtype, columns=columns)


def _compare(case):
    print(f'noalloc vs batch: B={case.batch} H={case.heads} D={case.dim} {case.dtype} '
          f'Lmax={case.lengths.max()} columns={case.columns}', flush=True)
    ref_dev, dev = DevicePagedCase(case), DevicePagedCase(case)
    assert _call('mt_paged_decode_batch', ref_dev) == 0
    assert _call('mt_paged_decode_batch_noalloc', dev) == 0
    runtime().synchronize()
    want, got = ref_dev.out.to_numpy(), dev.out.to_numpy()
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), 'output differs from mt_paged_decode_batch'
    assert np.array_equal(dev.pool_image().view(np.uint8), ref_dev.pool_image().view(np.uint8)), \
        'appended pool differs from mt_paged_decode_batch'
    image = case.image.copy()
    ref = po.image_decode_batch(image, CODES[case.dtype], case.table, case.columns, case.q, case.k, case.v,
                                case.offsets, case.layer)
    assert_attention_close(got, ref, case.dtype, context='noalloc')


def test_noalloc_matches_decode_batch_on_consecutive_calls():
    # first call: 3 splits of 1024 tokens in the longest rows; second call:
    # fewer rows, heads and splits, another dtype, through the same array
    _compare(_case(1, batch=24, heads=12, dim=64, dtype='float16', max_len=3000))
    _compare(_case(2, batch=5, heads=4, dim=64, dtype='bfloat16', max_len=1500))
    # and a table that needs no split at all, then fp32 / d 128 with splits
    _compare(_case(3, batch=7, heads=3, dim=64, dtype='float16', max_len=1000))
    _compare(_case(4, batch=3, heads=2, dim=128, dtype='float32', max_len=2100))


def test_noalloc_rejects_partials_beyond_its_array():
    # b*h = 32768 rows, 2 splits of d' = 128 partials: 34 MB > 32 MiB, refused
    # on the host before any launch. The arguments are real device buffers of
    # the call's shapes, laid out so that even a launch would stay in bounds:
    # every offset is 0 (one key, no row needs a split, so no partial is
    # written), every table entry is -1 and every slab null (nothing is read
    # from or appended to a page).
    from minitorch_amd.runtime import RawDeviceBuffer
    f = _entry('mt_paged_decode_batch_noalloc')
    b, h, d, psize, columns, slabs = 1024, 32, 128, 16, 128, 64
    assert b * h * 2 * (128 + 2) * 4 > SCRATCH_BYTES
    rows = [RawDeviceBuffer(b * h * d * 2) for _ in range(4)]        # out, q, k, v: fp16 [b, h, 1, d]
    for t in rows:
        t.fill_words(0)
    slab_table = RawDeviceBuffer(8 * slabs)
    slab_table.fill_words(0)
    table = RawDeviceBuffer(4 * b * columns)
    table.fill_words(0xFFFFFFFF)
    offsets = RawDeviceBuffer(4 * b)
    offsets.fill_words(0)
    args = [t.ptr for t in rows] + [slab_table.ptr, table.ptr, offsets.ptr]
    assert f(*args, b, h, d, psize, 16, slabs, columns, 0, 1, 1) == 1
    # half the rows fit: the same buffers are accepted
    assert (b // 2) * h * 2 * (128 + 2) * 4 <= SCRATCH_BYTES
    assert f(*args, b // 2, h, d, psize, 16, slabs, columns, 0, 1, 1) == 0
    runtime().synchronize()
    # each row's one key is the new token, whose page is missing: a NaN row
    out = rows[0].download(np.float16, (b // 2) * h * d)
    assert np.all(np.isnan(out))
