"""GPU parity of causal paged prefill attention (``mt_paged_attention``)
against the float64 oracle.

For fp16/bf16 with head_dim 64 or 128 and at least 16 queries the library
runs the matrix-core prefill kernel; the other shapes run the per-query
kernel. Both follow reference paged_forward with offsets == nullptr
(src/paged_attention_kernel.cu:35-85): nk = offset + nq, query qi attends
keys kj <= offset + qi, and a missing page gives NaN for every query that
attends it. Page sizes are 8, 16 and 32 (the entry point rejects others). Tolerances are in tests/tolerances.py.
"""
import numpy as np
import pytest

from minitorch_amd import paged_ops
from minitorch_amd.runtime import DeviceTensor, RawDeviceBuffer, runtime
from minitorch_amd.workloads import make_decode_case, DevicePagedCase
from oracle import paged_oracle as po
from tolerances import assert_attention_close

pytestmark = pytest.mark.gpu
CODES = {'float32': po.F32, 'float16': po.F16, 'bfloat16': po.BF16}


def prefill_case(seed, *, batch, heads, dim, page_size, nk, dtype, layers=1, layer=0,
                 pages_per_slab=4, spare_pages=0):
    pages = -(-nk // page_size) * batch + spare_pages
    pool = -(-pages // pages_per_slab) * pages_per_slab
    return make_decode_case(seed, batch=batch, heads=heads, dim=dim, page_size=page_size,
                            lengths=[nk] * batch, pool_pages=pool, pages_per_slab=pages_per_slab,
                            dtype=dtype, layers=layers, layer=layer)


def run_prefill(case, nq, nk, offset, seed=0, dev=None, present=None):
    rng = np.random.default_rng(seed)
    dt = case.dtype
    q = po.encode(rng.standard_normal((case.batch, case.heads, nq, case.dim), dtype=np.float32),
                  CODES[dt])
    dev = dev or DevicePagedCase(case)
    qd = DeviceTensor(q.shape, dt)
    runtime().h2d(qd.ptr, q)
    out = DeviceTensor(q.shape, dt)
    paged_ops.paged_attention(out.ptr, qd.ptr, dev.slab_table.ptr, dev.block_table.ptr,
                              b=case.batch, h=case.heads, nq=nq, nk=nk, d=case.dim,
                              page_size=case.page_size, pages_per_slab=case.pages_per_slab,
                              num_slabs=case.num_slabs, columns=case.columns, layer=case.layer,
                              layers=case.layers, offset=offset, dtype=dt)
    runtime().synchronize()
    ref = po.image_paged_attention(case.image, CODES[dt], case.table, case.columns, q, case.layer,
                                   offset, nk, present=present)
    got = out.to_numpy()
    assert_attention_close(got, ref, dt, context=f'{dt} nq={nq} nk={nk} off={offset}')
    return got, ref


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
@pytest.mark.parametrize('dim', [64, 128])
@pytest.mark.parametrize('nq,offset', [(16, 0), (64, 0), (100, 0), (200, 37), (130, 300)])
def test_prefill_shapes(dtype, dim, nq, offset):
    case = prefill_case(20 + nq + offset, batch=2, heads=3, dim=dim, page_size=16,
                        nk=offset + nq, dtype=dtype)
    run_prefill(case, nq, offset + nq, offset, seed=nq)


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
@pytest.mark.parametrize('page_size', [8, 32])
def test_prefill_page_sizes(dtype, page_size):
    nq, offset = 90, 45
    case = prefill_case(30 + page_size, batch=2, heads=2, dim=64, page_size=page_size,
                        nk=offset + nq, dtype=dtype, pages_per_slab=8)
    run_prefill(case, nq, offset + nq, offset, seed=page_size)


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
def test_prefill_window_crossing(dtype):
    # page_size 8 and more than 512 pages: the page bases are resolved in
    # windows of 512 pages (4096 keys).
    nq, offset = 96, 4100
    case = prefill_case(42, batch=1, heads=2, dim=64, page_size=8, nk=offset + nq, dtype=dtype,
                        pages_per_slab=16)
    run_prefill(case, nq, offset + nq, offset, seed=4)


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
def test_prefill_more_slabs_than_lds_holds(dtype):
    # one page per slab and 525 pages: the slab table (> 512 entries) is read
    # from global memory instead of LDS, across two windows of page bases.
    nq, offset = 96, 4100
    case = prefill_case(45, batch=1, heads=2, dim=64, page_size=8, nk=offset + nq, dtype=dtype,
                        pages_per_slab=1)
    assert case.num_slabs > 512
    run_prefill(case, nq, offset + nq, offset, seed=7)


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
def test_prefill_multi_layer(dtype):
    case = prefill_case(43, batch=2, heads=2, dim=128, page_size=16, nk=150, dtype=dtype,
                        layers=3, layer=1, pages_per_slab=5)
    run_prefill(case, 150, 150, 0, seed=5)


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
def test_prefill_missing_pages(dtype):
    # A hole at page 2 (keys 32..47) of request 0 and an out-of-pool page at
    # page 6 (keys 96..111) of request 1: queries attending them are NaN,
    # earlier queries are not.
    nq, offset = 120, 0
    case = prefill_case(44, batch=2, heads=2, dim=64, page_size=16, nk=nq, dtype=dtype)
    case.table[0, 2] = -1
    case.table[1, 6] = 10 ** 6
    got, ref = run_prefill(case, nq, nq, offset, seed=6)
    assert np.isnan(ref[0, :, 32:]).all() and not np.isnan(ref[0, :, :32]).any()
    assert np.isnan(ref[1, :, 96:]).all() and not np.isnan(ref[1, :, :96]).any()


def test_prefill_null_slab():
    case = prefill_case(45, batch=2, heads=2, dim=64, page_size=16, nk=100, dtype='float16')
    dev = DevicePagedCase(case)
    phys = int(case.table[1, 3])
    slabs = np.array([dev.pool.ptr + s * case.slab_bytes for s in range(case.num_slabs)], np.uint64)
    slabs[phys // case.pages_per_slab] = 0
    dev.slab_table.upload(slabs)
    present = np.ones(case.num_slabs, bool)
    present[phys // case.pages_per_slab] = False
    got, ref = run_prefill(case, 100, 100, 0, seed=7, dev=dev, present=present)
    assert np.isnan(ref).any() and not np.isnan(ref).all()


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
def test_prefill_large_scores(dtype):
    # Scaled inputs push the scores far apart, so the running max moves and
    # most weights underflow; the rescaling has to stay exact.
    nq = 70
    case = prefill_case(46, batch=1, heads=2, dim=64, page_size=16, nk=nq, dtype=dtype)
    f = po.decode(case.image, CODES[dtype]) * 6.0
    case.image[...] = po.encode(f.astype(np.float32), CODES[dtype])
    run_prefill(case, nq, nq, 0, seed=8)


def test_prefill_matches_per_query_kernel_below_threshold():
    # 15 queries run the per-query kernel, 16 the matrix-core kernel; both
    # against the oracle on the same pages.
    case = prefill_case(47, batch=2, heads=2, dim=64, page_size=16, nk=60, dtype='float16')
    dev = DevicePagedCase(case)
    run_prefill(case, 15, 59, 44, seed=9, dev=dev)
    run_prefill(case, 16, 60, 44, seed=9, dev=dev)


@pytest.mark.parametrize('dtype', ['float32', 'float16', 'bfloat16'])
@pytest.mark.parametrize('n', [5, 70])
def test_paged_prefill_token_major_equals_append_then_attention(dtype, n):
    # mt_paged_prefill reads q/k/v as column blocks of a fused [b, n, 3*h*d]
    # projection and writes [b, n, h*d]; it must equal mt_paged_append +
    # mt_paged_attention on head-split copies bit for bit (same kernels), and
    # the oracle within tolerance.
    b, h, d, offset = 2, 3, 64, 21
    case = prefill_case(50 + n, batch=b, heads=h, dim=d, page_size=16, nk=offset + n, dtype=dtype)
    rng = np.random.default_rng(n)
    qkv = po.encode(rng.standard_normal((b, n, 3 * h * d), dtype=np.float32), CODES[dtype])
    heads = lambda blk: np.ascontiguousarray(qkv[:, :, blk * h * d:(blk + 1) * h * d]
                                             .reshape(b, n, h, d).transpose(0, 2, 1, 3))
    q, k, v = heads(0), heads(1), heads(2)
    common = dict(page_size=16, pages_per_slab=case.pages_per_slab, num_slabs=case.num_slabs,
                  columns=case.columns, layer=0, layers=1, dtype=dtype)
    one, two = DevicePagedCase(case), DevicePagedCase(case)
    fused = DeviceTensor(qkv.shape, dtype)
    runtime().h2d(fused.ptr, qkv)
    item = 4 if dtype == 'float32' else 2
    out1 = DeviceTensor((b, n, h * d), dtype)
    paged_ops.paged_prefill(out1.ptr, fused.ptr, fused.ptr + h * d * item, fused.ptr + 2 * h * d * item,
                            one.slab_table.ptr, one.block_table.ptr, b=b, h=h, n=n, d=d, offset=offset,
                            qkv_stride=3 * h * d, out_stride=h * d, **common)
    qd, kd, vd = (DeviceTensor(x.shape, dtype) for x in (q, k, v))
    for t, x in ((qd, q), (kd, k), (vd, v)):
        runtime().h2d(t.ptr, x)
    out2 = DeviceTensor(q.shape, dtype)
    paged_ops.paged_append(kd.ptr, vd.ptr, two.slab_table.ptr, two.block_table.ptr, b=b, h=h, n=n, d=d,
                           offset=offset, **common)
    paged_ops.paged_attention(out2.ptr, qd.ptr, two.slab_table.ptr, two.block_table.ptr, b=b, h=h, nq=n,
                              nk=offset + n, d=d, offset=offset, **common)
    runtime().synchronize()
    assert np.array_equal(one.pool_image().view(np.uint8), two.pool_image().view(np.uint8))
    got1 = out1.raw_numpy().reshape(b, n, h, d).transpose(0, 2, 1, 3)
    got2 = out2.raw_numpy()
    assert np.array_equal(got1.view(np.uint8), got2.view(np.uint8))
    image = case.image.copy()
    po.image_append(image, case.table, case.columns, k, v, 0, offset=offset)
    ref = po.image_paged_attention(image, CODES[dtype], case.table, case.columns, q, 0, offset, offset + n)
    assert_attention_close(out2.to_numpy(), ref, dtype)


def run_ragged(dtype, d, tokens, offsets, *, page_size=16, h=3, seed=0, pps=4):
    """mt_paged_prefill_ragged over prompts of `tokens` rows at `offsets`
    against the oracle: each prompt's K/V appended to its own pages (whole
    pool image bit for bit) and its causal attention (tolerances of
    tests/tolerances.py)."""
    r = len(tokens)
    lengths = [o + n for o, n in zip(offsets, tokens)]
    pages = sum(-(-length // page_size) for length in lengths) + 3
    case = make_decode_case(seed, batch=r, heads=h, dim=d, page_size=page_size, lengths=lengths,
                            pool_pages=-(-pages // pps) * pps, pages_per_slab=pps, dtype=dtype)
    total, hd = sum(tokens), h * d
    rng = np.random.default_rng(seed)
    qkv = po.encode(rng.standard_normal((total, 3 * hd), dtype=np.float32), CODES[dtype])
    dev = DevicePagedCase(case)
    fused = DeviceTensor(qkv.shape, dtype)
    runtime().h2d(fused.ptr, qkv)
    out = DeviceTensor((total, hd), dtype)
    item = 4 if dtype == 'float32' else 2
    tables = [dev.block_table.ptr + 4 * i * case.columns for i in range(r)]
    paged_ops.paged_prefill_ragged(out.ptr, fused.ptr, fused.ptr + hd * item, fused.ptr + 2 * hd * item,
                                   dev.slab_table.ptr, tables, tokens, offsets, h=h, d=d, page_size=page_size,
                                   pages_per_slab=pps, num_slabs=case.num_slabs, columns=case.columns,
                                   layer=0, layers=1, dtype=dtype, qkv_stride=3 * hd, out_stride=hd)
    runtime().synchronize()
    image = case.image.copy()
    got = out.to_numpy()
    first = 0
    for i, (n, off) in enumerate(zip(tokens, offsets)):
        rows = qkv[first:first + n]
        heads = lambda blk: np.ascontiguousarray(rows[:, blk * hd:(blk + 1) * hd].reshape(1, n, h, d)
                                                 .transpose(0, 2, 1, 3))
        table = case.table[i:i + 1]
        po.image_append(image, table, case.columns, heads(1), heads(2), 0, offset=off)
        ref = po.image_paged_attention(image, CODES[dtype], table, case.columns, heads(0), 0, off, off + n)
        mine = got[first:first + n].reshape(1, n, h, d).transpose(0, 2, 1, 3)
        assert_attention_close(mine, ref, dtype, context=f'prompt {i} n={n} offset={off}')
        first += n
    assert np.array_equal(dev.pool_image().view(np.uint8), image.view(np.uint8)), 'append differs'


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
@pytest.mark.parametrize('dim', [64, 128])
def test_prefill_ragged_prompts(dtype, dim):
    # one launch: prompts of 1..130 tokens, tiles cut at 64, some at an offset
    run_ragged(dtype, dim, [1, 5, 16, 63, 64, 65, 130], [0, 7, 0, 100, 0, 33, 0], seed=dim)


@pytest.mark.parametrize('page_size', [8, 32])
def test_prefill_ragged_page_sizes(page_size):
    run_ragged('bfloat16', 64, [40, 9, 77], [3, 0, 50], page_size=page_size, seed=page_size)


def test_prefill_ragged_more_prompts_than_one_launch_takes():
    # 20 prompts: two launches of at most 16 prompts each
    rng = np.random.default_rng(3)
    tokens = [int(n) for n in rng.integers(1, 90, 20)]
    run_ragged('float16', 64, tokens, [int(o) for o in rng.integers(0, 40, 20)], h=2, seed=3)


def test_prefill_ragged_fp32_takes_the_per_prompt_path():
    run_ragged('float32', 64, [17, 3, 40], [0, 12, 5], h=2, seed=4)


def test_prefill_ragged_prompt_longer_than_one_launch_describes():
    # a prompt of more than 256 query tiles (16400 tokens) is prefilled on its
    # own; the result equals one mt_paged_prefill call per prompt bit for bit
    tokens, offsets, h, d, page = [20, 16400, 33], [5, 0, 0], 1, 64, 32
    lengths = [o + n for o, n in zip(offsets, tokens)]
    pages = sum(-(-x // page) for x in lengths) + 4
    case = make_decode_case(61, batch=3, heads=h, dim=d, page_size=page, lengths=lengths,
                            pool_pages=-(-pages // 8) * 8, pages_per_slab=8, dtype='bfloat16')
    total, hd = sum(tokens), h * d
    qkv = po.encode(np.random.default_rng(61).standard_normal((total, 3 * hd), dtype=np.float32), po.BF16)
    outs, images = [], []
    for ragged in (True, False):
        dev = DevicePagedCase(case)
        fused = DeviceTensor(qkv.shape, 'bfloat16')
        runtime().h2d(fused.ptr, qkv)
        out = DeviceTensor((total, hd), 'bfloat16')
        common = dict(h=h, d=d, page_size=page, pages_per_slab=8, num_slabs=case.num_slabs,
                      columns=case.columns, layer=0, layers=1, dtype='bfloat16', qkv_stride=3 * hd, out_stride=hd)
        tables = [dev.block_table.ptr + 4 * i * case.columns for i in range(3)]
        if ragged:
            paged_ops.paged_prefill_ragged(out.ptr, fused.ptr, fused.ptr + 2 * hd, fused.ptr + 4 * hd,
                                           dev.slab_table.ptr, tables, tokens, offsets, **common)
        else:
            row = 0
            for i, (n, off) in enumerate(zip(tokens, offsets)):
                base = fused.ptr + row * 3 * hd * 2
                paged_ops.paged_prefill(out.ptr + row * hd * 2, base, base + 2 * hd, base + 4 * hd,
                                        dev.slab_table.ptr, tables[i], b=1, n=n, offset=off, **common)
                row += n
        runtime().synchronize()
        outs.append(out.raw_numpy())
        images.append(dev.pool_image())
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(images[0].view(np.uint8), images[1].view(np.uint8))


@pytest.mark.parametrize('entry', ['prefill', 'ragged'])
def test_fused_append_with_missing_page_equals_append_then_attention(entry):
    # The matrix-core prefill reads the new keys from the K/V rows and writes
    # them to their pages itself. A missing page (table hole, out-of-pool
    # page) must still be skipped by the write and read as NaN, exactly as
    # mt_paged_append followed by mt_paged_attention does: bitwise equal
    # outputs (NaN rows included) and pool images.
    b, h, d, n, offset, page = 2, 2, 64, 70, 9, 16
    case = prefill_case(71, batch=b, heads=h, dim=d, page_size=page, nk=offset + n, dtype='bfloat16')
    case.table[0, 2] = -1          # keys 32..47 of request 0 (new tokens)
    case.table[1, 4] = 10 ** 6     # keys 64..78 of request 1
    rng = np.random.default_rng(71)
    qkv = po.encode(rng.standard_normal((b, n, 3 * h * d), dtype=np.float32), po.BF16)
    heads = lambda blk: np.ascontiguousarray(qkv[:, :, blk * h * d:(blk + 1) * h * d]
                                             .reshape(b, n, h, d).transpose(0, 2, 1, 3))
    q, k, v = heads(0), heads(1), heads(2)
    common = dict(page_size=page, pages_per_slab=case.pages_per_slab, num_slabs=case.num_slabs,
                  columns=case.columns, layer=0, layers=1, dtype='bfloat16')
    one, two = DevicePagedCase(case), DevicePagedCase(case)
    fused = DeviceTensor(qkv.shape, 'bfloat16')
    runtime().h2d(fused.ptr, qkv)
    out1 = DeviceTensor((b, n, h * d), 'bfloat16')
    if entry == 'prefill':
        paged_ops.paged_prefill(out1.ptr, fused.ptr, fused.ptr + h * d * 2, fused.ptr + 2 * h * d * 2,
                                one.slab_table.ptr, one.block_table.ptr, b=b, h=h, n=n, d=d, offset=offset,
                                qkv_stride=3 * h * d, out_stride=h * d, **common)
    else:
        tables = [one.block_table.ptr + 4 * i * case.columns for i in range(b)]
        paged_ops.paged_prefill_ragged(out1.ptr, fused.ptr, fused.ptr + h * d * 2, fused.ptr + 2 * h * d * 2,
                                       one.slab_table.ptr, tables, [n] * b, [offset] * b, h=h, d=d,
                                       qkv_stride=3 * h * d, out_stride=h * d, **common)
    qd, kd, vd = (DeviceTensor(x.shape, 'bfloat16') for x in (q, k, v))
    for t, x in ((qd, q), (kd, k), (vd, v)):
        runtime().h2d(t.ptr, x)
    out2 = DeviceTensor(q.shape, 'bfloat16')
    paged_ops.paged_append(kd.ptr, vd.ptr, two.slab_table.ptr, two.block_table.ptr, b=b, h=h, n=n, d=d,
                           offset=offset, **common)
    paged_ops.paged_attention(out2.ptr, qd.ptr, two.slab_table.ptr, two.block_table.ptr, b=b, h=h, nq=n,
                              nk=offset + n, d=d, offset=offset, **common)
    runtime().synchronize()
    assert np.array_equal(one.pool_image().view(np.uint8), two.pool_image().view(np.uint8))
    got1 = out1.raw_numpy().reshape(b, n, h, d).transpose(0, 2, 1, 3)
    got2 = out2.raw_numpy()
    assert np.array_equal(got1, got2)
    assert np.isnan(out2.to_numpy()).any()   # the holes are attended


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
@pytest.mark.parametrize('dim', [64, 128])
@pytest.mark.parametrize('nq,offset,page_size', [(1024, 0, 16), (700, 333, 32), (300, 2000, 8)])
def test_prefill_long_single_prompt_key_splits(dtype, dim, nq, offset, page_size):
    # One request of a few heads with a long context: its query tiles leave
    # most compute units idle, so their keys are split over workgroups and
    # merged (log-sum-exp). Against the oracle, through both entries: causal
    # attention over appended pages, and the fused append + attention.
    case = prefill_case(80 + nq, batch=1, heads=2, dim=dim, page_size=page_size, nk=offset + nq, dtype=dtype,
                        pages_per_slab=8)
    run_prefill(case, nq, offset + nq, offset, seed=nq)
    run_fused_single(case, nq, offset, seed=nq)


def run_fused_single(case, n, offset, seed=0):
    """mt_paged_prefill of one request on token-major fused QKV rows (the
    kernel appends the K/V itself) against the oracle's append + attention:
    pool image bit for bit, attention within tolerance."""
    dtype, h, d = case.dtype, case.heads, case.dim
    hd = h * d
    rng = np.random.default_rng(seed)
    qkv = po.encode(rng.standard_normal((1, n, 3 * hd), dtype=np.float32), CODES[dtype])
    dev = DevicePagedCase(case)
    fused = DeviceTensor(qkv.shape, dtype)
    runtime().h2d(fused.ptr, qkv)
    out = DeviceTensor((1, n, hd), dtype)
    item = 4 if dtype == 'float32' else 2
    paged_ops.paged_prefill(out.ptr, fused.ptr, fused.ptr + hd * item, fused.ptr + 2 * hd * item,
                            dev.slab_table.ptr, dev.block_table.ptr, b=1, h=h, n=n, d=d, page_size=case.page_size,
                            pages_per_slab=case.pages_per_slab, num_slabs=case.num_slabs, columns=case.columns,
                            layer=case.layer, layers=case.layers, offset=offset, dtype=dtype,
                            qkv_stride=3 * hd, out_stride=hd)
    runtime().synchronize()
    heads = lambda blk: np.ascontiguousarray(qkv[:, :, blk * hd:(blk + 1) * hd].reshape(1, n, h, d)
                                             .transpose(0, 2, 1, 3))
    image = case.image.copy()
    po.image_append(image, case.table, case.columns, heads(1), heads(2), case.layer, offset=offset)
    ref = po.image_paged_attention(image, CODES[dtype], case.table, case.columns, heads(0), case.layer,
                                   offset, offset + n)
    got = out.to_numpy().reshape(1, n, h, d).transpose(0, 2, 1, 3)
    assert_attention_close(got, ref, dtype, context=f'fused n={n} offset={offset}')
    assert np.array_equal(dev.pool_image().view(np.uint8), image.view(np.uint8)), 'append differs'


def test_prefill_key_splits_with_missing_pages():
    # holes inside the split key range: the queries that attend them are NaN,
    # the others are not (the merge keeps a NaN denominator)
    nq, offset = 900, 50
    case = prefill_case(91, batch=1, heads=2, dim=64, page_size=16, nk=offset + nq, dtype='bfloat16',
                        pages_per_slab=8)
    case.table[0, 10] = -1          # keys 160..175
    case.table[0, 40] = 10 ** 6     # keys 640..655
    got, ref = run_prefill(case, nq, offset + nq, offset, seed=9)
    assert np.isnan(ref[0, :, 160 - offset:]).all() and not np.isnan(ref[0, :, :160 - offset]).any()


def key_split_launches():
    import ctypes as ct
    f = paged_ops.paged_library().mt_paged_prefill_key_splits
    f.argtypes, f.restype = [ct.POINTER(ct.c_longlong)], ct.c_int
    n = ct.c_longlong()
    assert f(ct.byref(n)) == 0
    return n.value


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
@pytest.mark.parametrize('heads,dim', [(12, 64), (16, 64), (12, 128), (16, 128)])
def test_prefill_key_split_at_model_head_counts(heads, dim, dtype):
    # The shapes the split is for: a 1024-token prompt of DistilGPT-2 (12
    # heads; 16 tiles x 12 heads, B = 4 key blocks per split) and GPT-2-medium
    # (16 heads; 256 workgroups, an odd B = 5), at head_dim 64 and 128, through
    # mt_paged_attention (pages) and mt_paged_prefill (fused append); each
    # must take the key-split path, checked with the library's counter.
    nq = 1024
    case = prefill_case(90 + heads + dim, batch=1, heads=heads, dim=dim, page_size=16, nk=nq, dtype=dtype,
                        pages_per_slab=8)
    before = key_split_launches()
    run_prefill(case, nq, nq, 0, seed=heads + dim)
    assert key_split_launches() == before + 1, 'mt_paged_attention did not split the keys'
    run_fused_single(case, nq, 0, seed=heads + dim)
    assert key_split_launches() == before + 2, 'mt_paged_prefill did not split the keys'


def test_prefill_above_the_split_limit_stays_unsplit():
    # 25 heads x 16 query tiles = 400 workgroups > 256 compute units: the
    # prompt already fills the GPU, so it runs unsplit (and still matches)
    nq, heads = 1024, 25
    case = prefill_case(97, batch=1, heads=heads, dim=64, page_size=16, nk=nq, dtype='bfloat16', pages_per_slab=8)
    before = key_split_launches()
    run_prefill(case, nq, nq, 0, seed=97)
    run_fused_single(case, nq, 0, seed=97)
    assert key_split_launches() == before


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
@pytest.mark.parametrize('dim', [64, 128])
def test_prefill_ragged_key_splits(dtype, dim):
    # A replacement batch of config-4 shape (16 heads): one long prompt among
    # short ones. The long prompt's last tiles span more key blocks than their
    # share of the launch, so their keys are split over workgroups and merged;
    # every prompt against the oracle and the pool image bit for bit.
    tokens, offsets = [1000, 60, 130, 5, 300], [0, 0, 20, 7, 0]
    before = key_split_launches()
    run_ragged(dtype, dim, tokens, offsets, h=16, seed=dim + 1)
    assert key_split_launches() == before + 1, 'the ragged launch did not split the keys'


def test_prefill_ragged_short_prompts_stay_unsplit():
    before = key_split_launches()
    run_ragged('bfloat16', 64, [1, 5, 16, 63, 64, 65, 130], [0, 7, 0, 100, 0, 33, 0], h=16, seed=5)
    assert key_split_launches() == before
