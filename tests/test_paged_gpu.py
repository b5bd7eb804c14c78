"""GPU parity of the paged append / decode attention C-ABI against the oracle.

Every call goes through ``cuda_kernels/paged_attention_kernel.so``. Inputs are
seeded (numpy default_rng); tolerances are in tests/tolerances.py. The KV
append is checked bit-exact on the whole pool image.
"""
import numpy as np
import pytest

from minitorch_amd import paged_ops
from minitorch_amd.runtime import RawDeviceBuffer, DeviceTensor, runtime
from minitorch_amd.workloads import (make_decode_case, config1_case, config2_case,
                                     config5_lengths, DevicePagedCase)
from oracle import paged_oracle as po
from tolerances import assert_attention_close

pytestmark = pytest.mark.gpu
CODES = {'float32': po.F32, 'float16': po.F16, 'bfloat16': po.BF16}


def run_decode(dev, entry='batch', **extra):
    c = dev.case
    args = (dev.out.ptr, dev.q.ptr, dev.k.ptr, dev.v.ptr, dev.slab_table.ptr, dev.block_table.ptr,
            dev.offsets.ptr)
    if entry == 'batch':
        paged_ops.paged_decode_batch(*args, **dev.kwargs())
    else:
        ws_bytes = paged_ops.decode_workspace_bytes(b=c.batch, h=c.heads, page_size=c.page_size,
                                                    columns=c.columns,
                                                    split_tokens=extra.get('split_tokens', 0))
        ws = None
        if ws_bytes:
            ws = RawDeviceBuffer(ws_bytes)
            ws.fill_words(0)
        paged_ops.paged_decode_split(*args, **dev.kwargs(), workspace=ws.ptr if ws else None,
                                     workspace_bytes=ws_bytes, **extra)
    runtime().synchronize()
    return dev.out.to_numpy()


def oracle_decode(case, rows=None, present=None):
    image = case.image.copy()
    ref = po.image_decode_batch(image, CODES[case.dtype], case.table, case.columns, case.q, case.k,
                                case.v, case.offsets, case.layer, present=present, rows=rows)
    return ref, image


def check_case(case, entry='batch', rows=None, check_image=True, **extra):
    dev = DevicePagedCase(case)
    out = run_decode(dev, entry, **extra)
    ref, image = oracle_decode(case, rows=rows)
    if rows is not None:
        sel = tuple(np.array(rows).T)
        out, ref = out[sel], ref[sel]
    assert_attention_close(out, ref, case.dtype, context=f'{case.dtype} B={case.batch}')
    if check_image:
        assert np.array_equal(dev.pool_image().view(np.uint8), image.view(np.uint8)), 'append differs'
    return dev, out


def test_config1_fp32_full():
    check_case(config1_case(0))


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
def test_config1_shape_low_precision(dtype):
    case = make_decode_case(1, batch=4, heads=12, dim=64, page_size=16, lengths=[7, 33, 64, 120],
                            pool_pages=64, pages_per_slab=4, dtype=dtype)
    check_case(case)


def test_config2_full_fp16():
    check_case(config2_case(0))


@pytest.mark.parametrize('page_size', [8, 16, 32])
@pytest.mark.parametrize('dtype', ['float32', 'float16', 'bfloat16'])
def test_page_sizes_and_boundaries(page_size, dtype):
    # contexts on page and split boundaries: 1, P, P+1, 255..257, 512, 513, 1000
    lengths = [1, page_size, page_size + 1, 255, 256, 257, 512, 513, 1000]
    case = make_decode_case(2, batch=len(lengths), heads=3, dim=64, page_size=page_size,
                            lengths=lengths, pool_pages=512, pages_per_slab=8, dtype=dtype)
    check_case(case)


@pytest.mark.parametrize('dim', [128, 48, 80, 32])
@pytest.mark.parametrize('dtype', ['float32', 'bfloat16'])
def test_head_dims(dim, dtype):
    case = make_decode_case(3, batch=5, heads=2, dim=dim, page_size=16,
                            lengths=[1, 17, 100, 300, 700], pool_pages=96, pages_per_slab=4,
                            dtype=dtype)
    check_case(case)


def test_multi_layer_slab_addressing():
    case = make_decode_case(4, batch=3, heads=4, dim=64, page_size=16, lengths=[5, 40, 300],
                            pool_pages=48, pages_per_slab=3, dtype='float16', layers=3, layer=2)
    check_case(case)


@pytest.mark.parametrize('pool_pages', [512, 513, 700])
def test_slab_table_sizes(pool_pages):
    # one page per slab: up to 512 slabs the decode stages the slab table in
    # LDS, above it reads the table from global memory; both must agree.
    case = make_decode_case(13, batch=5, heads=3, dim=64, page_size=16, lengths=[1, 17, 200, 513, 90],
                            pool_pages=pool_pages, pages_per_slab=1, dtype='float16')
    assert case.table.max() >= min(pool_pages, 512) - 64  # pages spread over the whole pool
    check_case(case)


def test_missing_pages_give_nan_rows():
    case = make_decode_case(5, batch=4, heads=2, dim=64, page_size=16, lengths=[40, 40, 300, 20],
                            pool_pages=64, pages_per_slab=4, dtype='float32')
    case.table[0, 1] = -1          # hole inside the context -> NaN
    case.table[1, 2] = -1          # the new token's page missing -> NaN, no write
    case.table[2, 5] = 10 ** 6     # out-of-pool physical page -> NaN
    check_case(case)


def test_null_slab_reads_nan():
    case = make_decode_case(6, batch=2, heads=2, dim=64, page_size=16, lengths=[60, 33],
                            pool_pages=16, pages_per_slab=4, dtype='float32')
    dev = DevicePagedCase(case)
    # null out the slab of request 0's second page
    phys = int(case.table[0, 1])
    slabs = np.array([dev.pool.ptr + s * case.slab_bytes for s in range(case.num_slabs)], np.uint64)
    slabs[phys // case.pages_per_slab] = 0
    dev.slab_table.upload(slabs)
    out = run_decode(dev)
    present = np.ones(case.num_slabs, bool)
    present[phys // case.pages_per_slab] = False
    ref, image = oracle_decode(case, present=present)
    assert_attention_close(out, ref, 'float32')
    assert np.array_equal(dev.pool_image().view(np.uint8), image.view(np.uint8))


@pytest.mark.parametrize('split_tokens', [64, 128, 256, 1024])
@pytest.mark.parametrize('unroll', [1, 2, 4])
@pytest.mark.parametrize('waves', [2, 4, 8])
def test_split_entry_equals_oracle(split_tokens, unroll, waves):
    case = make_decode_case(7, batch=6, heads=3, dim=64, page_size=16,
                            lengths=[1, 64, 65, 500, 1024, 777], pool_pages=256, pages_per_slab=8,
                            dtype='float16')
    check_case(case, entry='split', split_tokens=split_tokens, unroll=unroll, waves=waves)


@pytest.mark.parametrize('dtype,dim,split_tokens', [('bfloat16', 128, 1024), ('float16', 64, 2048),
                                                     ('float32', 128, 512)])
def test_two_wave_workgroups_equal_oracle(dtype, dim, split_tokens):
    # 2-wave workgroups (a wave resolves the pages of up to 64 steps, so
    # splits above 1024 tokens fall back to 4 waves: the 2048 case)
    case = make_decode_case(15, batch=5, heads=4, dim=dim, page_size=16, lengths=[3, 1024, 1500, 700, 2048],
                            pool_pages=640, pages_per_slab=16, dtype=dtype)
    check_case(case, entry='split', split_tokens=split_tokens, waves=2)


def run_work_list(dev, lengths, split_tokens, waves=0, compute_units=8, reverse=False):
    c = dev.case
    work, items, merges = paged_ops.decode_work_list(lengths, c.heads, split_tokens, compute_units)
    if reverse:
        pairs = work[:2 * items].reshape(-1, 2)[::-1]
        work = np.concatenate([pairs.ravel(), work[2 * items:]]).astype(np.int32)
    buf = RawDeviceBuffer(4 * max(1, len(work)))
    buf.upload(work)
    ws_bytes = paged_ops.decode_workspace_bytes(b=c.batch, h=c.heads, page_size=c.page_size,
                                                columns=c.columns, split_tokens=split_tokens)
    ws = RawDeviceBuffer(max(4, ws_bytes))
    paged_ops.paged_decode_split(dev.out.ptr, dev.q.ptr, dev.k.ptr, dev.v.ptr, dev.slab_table.ptr,
                                 dev.block_table.ptr, dev.offsets.ptr, **dev.kwargs(),
                                 split_tokens=split_tokens, waves=waves, work=buf.ptr, work_items=items,
                                 merge_rows=merges, workspace=ws.ptr if ws_bytes else None,
                                 workspace_bytes=ws_bytes)
    runtime().synchronize()
    return dev.out.to_numpy()


@pytest.mark.parametrize('page_size', [8, 16, 32])
@pytest.mark.parametrize('waves', [2, 4, 8])
def test_work_list_equals_oracle_and_grid(page_size, waves):
    # rows of 0..3 splits visited longest first: same bits as the full grid
    lengths = [300, 5, 1024, 77, 16, 640, 1, 2100]
    case = make_decode_case(12, batch=8, heads=2, dim=64, page_size=page_size, lengths=lengths,
                            pool_pages=1024, pages_per_slab=16, dtype='bfloat16')
    dev = DevicePagedCase(case)
    listed = run_work_list(dev, lengths, 1024, waves)
    ref, image = oracle_decode(case)
    assert_attention_close(listed, ref, 'bfloat16')
    assert np.array_equal(dev.pool_image().view(np.uint8), image.view(np.uint8)), 'append differs'
    plain = run_decode(DevicePagedCase(case), entry='split', waves=waves, split_tokens=1024)
    assert np.array_equal(listed.view(np.uint16), plain.view(np.uint16))
    again = run_work_list(DevicePagedCase(case), lengths, 1024, waves, reverse=True)
    assert np.array_equal(listed.view(np.uint16), again.view(np.uint16))


def test_work_list_ragged_splits_fp16():
    # many split rows and a 256-token split: every (row, split) pair listed
    rng = np.random.default_rng(21)
    lengths = rng.integers(1, 1500, size=24)
    lengths[[3, 9]] = [1, 256]
    case = make_decode_case(14, batch=24, heads=4, dim=64, page_size=16, lengths=lengths,
                            pool_pages=4096, pages_per_slab=32, dtype='float16')
    dev = DevicePagedCase(case)
    out = run_work_list(dev, lengths, 256)
    ref, image = oracle_decode(case)
    assert_attention_close(out, ref, 'float16')
    assert np.array_equal(dev.pool_image().view(np.uint8), image.view(np.uint8)), 'append differs'


@pytest.mark.parametrize('dtype', ['float32', 'bfloat16'])
def test_qkv_row_stride_reads_fused_projection_blocks(dtype):
    # q, k, v as the three column blocks of one [B, 3*H*D] buffer: same bits
    # as contiguous inputs
    lengths = [3, 70, 512, 1025, 40]
    case = make_decode_case(15, batch=5, heads=4, dim=64, page_size=16, lengths=lengths,
                            pool_pages=256, pages_per_slab=8, dtype=dtype)
    plain = run_decode(DevicePagedCase(case), entry='split', split_tokens=512)
    dev = DevicePagedCase(case)
    hd = case.heads * case.dim
    fused = np.concatenate([a.reshape(case.batch, hd) for a in (case.q, case.k, case.v)], axis=1)
    qkv = DeviceTensor((case.batch, 3 * hd), dtype)
    runtime().h2d(qkv.ptr, np.ascontiguousarray(fused))
    item = 4 if dtype == 'float32' else 2
    ws_bytes = paged_ops.decode_workspace_bytes(b=case.batch, h=case.heads, page_size=16,
                                                columns=case.columns, split_tokens=512)
    ws = RawDeviceBuffer(ws_bytes)
    paged_ops.paged_decode_split(dev.out.ptr, qkv.ptr, qkv.ptr + hd * item, qkv.ptr + 2 * hd * item,
                                 dev.slab_table.ptr, dev.block_table.ptr, dev.offsets.ptr, **dev.kwargs(),
                                 split_tokens=512, qkv_stride=3 * hd, workspace=ws.ptr,
                                 workspace_bytes=ws_bytes)
    runtime().synchronize()
    strided = dev.out.to_numpy()
    view = np.uint32 if dtype == 'float32' else np.uint16
    assert np.array_equal(strided.view(view), plain.view(view))
    ref, image = oracle_decode(case)
    assert np.array_equal(dev.pool_image().view(np.uint8), image.view(np.uint8)), 'append differs'


def test_repeat_calls_are_deterministic():
    case = config2_case(1, batch=16)
    dev = DevicePagedCase(case)
    first = run_decode(dev)
    for _ in range(3):
        dev.reset_pool()
        again = run_decode(dev)
        assert np.array_equal(first.view(np.uint16), again.view(np.uint16))


def test_config5_ragged_bf16_sampled_rows():
    # Config 5 shape (H=25, bf16, lognormal contexts up to 8192) at B=96 with
    # the longest contexts forced in, checked on a seeded sample of rows.
    lengths = config5_lengths(0, 96)
    lengths[:4] = [8192, 4097, 1025, 1]
    for page_size in (16, 32):
        pages = int(((lengths + page_size - 1) // page_size).sum()) + 64
        pages = (pages + 63) // 64 * 64
        case = make_decode_case(8, batch=96, heads=25, dim=64, page_size=page_size,
                                lengths=lengths, pool_pages=pages, pages_per_slab=64,
                                dtype='bfloat16')
        rng = np.random.default_rng(9)
        rows = [(b, int(rng.integers(25))) for b in range(96)]
        check_case(case, rows=rows)


@pytest.mark.parametrize('page_size', [16, 32])
def test_config5_full_size_bench_case(page_size):
    # The exact case `bench.py --config 5` times: B=512, H=25, bf16, contexts
    # lognormal(ln 256, 1.2) clipped to [1, 8192], the hash-filled device pool,
    # the library's split length and the longest-first work list. Every row
    # is checked against the C oracle and the whole pool image bit for bit.
    full_size_against_c_oracle(config5_lengths(0, 512), 25, page_size, expect_merges=True)


def test_config4_attention_shape_full_size():
    # The decode attention of a config-4 step (128 rows, 16 heads, bf16,
    # contexts lognormal median 256 clipped to [16, 1024], page 16), as the
    # end-to-end loop launches it once per layer.
    from minitorch_amd.e2e import config4_lengths
    full_size_against_c_oracle(config4_lengths(np.random.default_rng([0, 4]), 128), 16, 16, expect_merges=False)


def full_size_against_c_oracle(lengths, heads, page_size, expect_merges):
    import ctypes as ct
    from minitorch_amd.workloads import DeviceRaggedCase
    from minitorch_amd.dtypes import decode_host
    from oracle import c_oracle
    lib = c_oracle.library()
    rt = runtime()
    b = len(lengths)
    case = DeviceRaggedCase(0, batch=b, heads=heads, dim=64, page_size=page_size, lengths=lengths,
                            dtype='bfloat16')
    kw = case.kwargs()
    image = case.pool.download(np.uint16)
    q, k, v = (t.raw_numpy() for t in (case.q, case.k, case.v))
    split = paged_ops.split_tokens_for(page_size=page_size, columns=case.columns)
    ws_bytes = paged_ops.decode_workspace_bytes(b=b, h=heads, page_size=page_size, columns=case.columns,
                                                split_tokens=split)
    ws = RawDeviceBuffer(max(ws_bytes, 4))
    work, items, merges = paged_ops.decode_work_list(case.lengths, heads, split, rt.compute_units())
    assert (merges > 0) == expect_merges  # the split reduction runs for config 5
    order = RawDeviceBuffer(4 * len(work))
    order.upload(work)
    paged_ops.paged_decode_split(case.out.ptr, case.q.ptr, case.k.ptr, case.v.ptr, case.slab_table.ptr,
                                 case.block_table.ptr, case.offsets.ptr, **kw, split_tokens=split,
                                 work=order.ptr, work_items=items, merge_rows=merges,
                                 workspace=ws.ptr, workspace_bytes=ws_bytes)
    runtime().synchronize()
    got = case.out.to_numpy()
    after = case.pool.download(np.uint16)

    slabs = np.array([image.ctypes.data + s * case.slab_bytes for s in range(case.num_slabs)], np.uint64)
    table = np.ascontiguousarray(case.table_host, np.int32)
    offsets = (case.lengths - 1).astype(np.int32)
    out = np.zeros_like(q)
    status = lib.oracle_paged_decode_batch(out.ctypes.data, q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                           slabs.ctypes.data, table.ctypes.data, offsets.ctypes.data,
                                           b, heads, 64, page_size, case.pages_per_slab, case.num_slabs,
                                           case.columns, 0, 1, c_oracle.CODES['bfloat16'], 0)
    assert status == 0
    ref = decode_host(out, 'bfloat16').reshape(got.shape)
    assert_attention_close(got, ref, 'bfloat16', context=f'B={b} H={heads} P={page_size}', ref_rounded=True)
    assert np.array_equal(after, image), 'append differs from the oracle'


@pytest.mark.parametrize('dtype', ['float32', 'float16', 'bfloat16'])
def test_multi_token_append_and_causal_attention(dtype):
    # Prefill-style use (reference minitorch/paged_kv_cache.py:205-221):
    # append n tokens at a common offset, then causal attention for nq = n.
    rng = np.random.default_rng(10)
    b, h, d, page_size, n, offset = 2, 3, 64, 16, 37, 20
    case = make_decode_case(11, batch=b, heads=h, dim=d, page_size=page_size,
                            lengths=[offset + n, offset + n], pool_pages=16, pages_per_slab=4,
                            dtype=dtype)
    dev = DevicePagedCase(case)
    k = po.encode(rng.standard_normal((b, h, n, d), dtype=np.float32), CODES[dtype])
    v = po.encode(rng.standard_normal((b, h, n, d), dtype=np.float32), CODES[dtype])
    q = po.encode(rng.standard_normal((b, h, n, d), dtype=np.float32), CODES[dtype])
    kd, vd, qd = (DeviceTensor(x.shape, dtype) for x in (k, v, q))
    for t, x in ((kd, k), (vd, v), (qd, q)):
        runtime().h2d(t.ptr, x)
    out = DeviceTensor(q.shape, dtype)
    common = dict(page_size=page_size, pages_per_slab=case.pages_per_slab,
                  num_slabs=case.num_slabs, columns=case.columns, layer=0, layers=1, dtype=dtype)
    paged_ops.paged_append(kd.ptr, vd.ptr, dev.slab_table.ptr, dev.block_table.ptr, b=b, h=h, n=n,
                           d=d, offset=offset, **common)
    paged_ops.paged_attention(out.ptr, qd.ptr, dev.slab_table.ptr, dev.block_table.ptr, b=b, h=h,
                              nq=n, nk=offset + n, d=d, offset=offset, **common)
    runtime().synchronize()
    image = case.image.copy()
    po.image_append(image, case.table, case.columns, k, v, 0, offset=offset)
    assert np.array_equal(dev.pool_image().view(np.uint8), image.view(np.uint8))
    ref = po.image_paged_attention(image, CODES[dtype], case.table, case.columns, q, 0, offset,
                                   offset + n)
    assert_attention_close(out.to_numpy(), ref, dtype)


@pytest.mark.parametrize('batch,columns', [(4, 64), (200, 64), (256, 64), (257, 64), (700, 64),
                                           (2100, 64), (5, 160), (300, 160)])
def test_decode_batch_device_ranked_order(batch, columns):
    # Without a host work list mt_paged_decode_batch visits the rows longest
    # first: b <= 256 rows of one split are ranked inside every workgroup;
    # larger batches and tables that may split (160 columns: 2560 tokens, up
    # to three splits) get a work list from order_kernel and a grid that
    # strides over it; 2100 rows take batch order. Many equal lengths (ties
    # go by row), an empty row (offset -1: zero output, no append) and a row
    # past its table (NaN output, no append) keep every order a permutation:
    # every (row, head) is written once, equal to the oracle, and the pool
    # image matches bit for bit.
    import dataclasses
    rng = np.random.default_rng([17, batch, columns])
    choices = [1, 16, 17, 64, 200, 1024] + ([1025, 2048, 2049, 2560] if columns > 64 else [])
    lengths = rng.choice(choices, size=batch)
    case = make_decode_case(17, batch=batch, heads=3, dim=64, page_size=16, lengths=lengths,
                            pool_pages=int(((lengths + 15) // 16).sum()) // 8 * 8 + 8, pages_per_slab=8,
                            dtype='float16', columns=columns)
    lengths = case.lengths.copy()
    lengths[1] = 0                          # offset -1
    lengths[batch - 2] = columns * 16 + 5   # beyond the table
    case = dataclasses.replace(case, lengths=lengths)
    dev, out = check_case(case)
    assert np.all(out[1] == 0) and np.all(np.isnan(out[batch - 2]))


def _device_order(lengths, *, heads, page_size, columns, split_tokens=0, compute_units=0):
    b = len(lengths)
    S = paged_ops.split_tokens_for(page_size=page_size, columns=columns, requested=split_tokens)
    nsplit = -(-columns * page_size // S)
    offsets = RawDeviceBuffer(4 * b)
    offsets.upload(np.asarray(lengths, np.int64).astype(np.int32) - 1)
    cap = 2 * b * nsplit + b
    lst = RawDeviceBuffer(4 * cap)
    lst.fill_words(0x7EEEEEEE)
    cnt = RawDeviceBuffer(8)
    paged_ops.paged_decode_order(offsets.ptr, b=b, h=heads, page_size=page_size, columns=columns,
                                 list_out=lst.ptr, count_out=cnt.ptr, split_tokens=split_tokens,
                                 compute_units=compute_units)
    runtime().synchronize()
    w, m = (int(x) for x in cnt.download(np.int32, 2))
    return lst.download(np.int32, cap), w, m, S


@pytest.mark.parametrize('batch,heads,page_size,columns,split,cus', [
    (1, 12, 16, 64, 0, 256), (64, 12, 16, 64, 0, 256), (300, 12, 16, 64, 0, 256),
    (512, 25, 16, 512, 0, 256), (512, 25, 32, 256, 0, 256), (160, 25, 16, 200, 256, 100),
    (2048, 7, 8, 300, 0, 256), (999, 16, 16, 64, 512, 37), (33, 300, 16, 128, 64, 256)])
def test_device_order_equals_host_work_list(batch, heads, page_size, columns, split, cus):
    # order_kernel's list equals paged_ops.decode_work_list (the numpy/Python
    # restatement of the scheduling order) element for element: ties of equal
    # lengths, lengths on split boundaries, one-token rows, full tables, more
    # heads than compute units (passes of one entry)
    rng = np.random.default_rng([5, batch, columns])
    cap_tokens = columns * page_size
    S = paged_ops.split_tokens_for(page_size=page_size, columns=columns, requested=split)
    pool = np.unique(np.clip([1, 2, S - 1, S, S + 1, 2 * S, cap_tokens, cap_tokens - 1, 100, 257], 1, cap_tokens))
    lengths = np.where(rng.random(batch) < 0.5, rng.choice(pool, batch), rng.integers(1, cap_tokens + 1, batch))
    got, w, m, S2 = _device_order(lengths, heads=heads, page_size=page_size, columns=columns,
                                  split_tokens=split, compute_units=cus)
    assert S2 == S
    ref, items, merges = paged_ops.decode_work_list(lengths.tolist(), heads, S, cus)
    assert (w, m) == (items, merges)
    assert np.array_equal(got[:2 * w + m], ref)


def test_device_order_empty_and_past_table_rows():
    # offset -1 (no key) and a row past its table each get one pair, split 0;
    # every (row, split) of the others appears exactly once
    lengths = np.array([0, 3000, 5, 1024 * 4 + 1, 2049, 1])  # columns 256 x 16 = 4096 tokens
    got, w, m, S = _device_order(lengths, heads=4, page_size=16, columns=256)
    pairs = got[:2 * w].reshape(-1, 2)
    want = {(0, 0), (3, 0), (2, 0), (5, 0)} | {(1, s) for s in range(3)} | {(4, s) for s in range(3)}
    assert sorted(map(tuple, pairs.tolist())) == sorted(want)
    assert list(got[2 * w:2 * w + m]) == [1, 4]


def test_many_residency_rounds_back_to_back():
    # config 5's shape class at a size the oracle checks quickly: far more
    # items than one residency round, rows split over up to three context
    # splits; eight launches in a row give the same bits each time
    rng = np.random.default_rng(31)
    lengths = np.clip(np.round(np.exp(rng.normal(np.log(256.0), 1.2, size=160))), 1, 3000).astype(np.int64)
    case = make_decode_case(31, batch=160, heads=25, dim=64, page_size=16, lengths=lengths,
                            pool_pages=int(((lengths + 15) // 16).sum() + 32) // 32 * 32, pages_per_slab=32,
                            dtype='bfloat16')
    dev, first = check_case(case, check_image=True)
    for _ in range(7):
        again = run_decode(dev)
        assert np.array_equal(first.view(np.uint16), again.view(np.uint16))
