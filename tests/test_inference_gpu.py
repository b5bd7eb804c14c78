"""Embedding gather, greedy argmax and last-position copy on the GPU vs the
oracle (exact)."""
import numpy as np
import pytest

from minitorch_amd import paged_ops
from minitorch_amd.kv_cache import greedy_token, last_position
from minitorch_amd.runtime import DeviceTensor, runtime
from oracle import paged_oracle as po

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('dim', [768, 1024, 30])
def test_embedding_gather_valid_and_invalid_ids(dim):
    rng = np.random.default_rng(dim)
    vocab = 501
    w = rng.standard_normal((vocab, dim)).astype(np.float32)
    ids = rng.integers(0, vocab, 40).astype(np.float32)
    ids[:7] = [np.nan, np.inf, -1, vocab, 3.5, -0.0, vocab - 1]
    wd, idd = DeviceTensor.from_numpy(w), DeviceTensor.from_numpy(ids)
    out = DeviceTensor((ids.size, dim))
    paged_ops.embedding_gather(out.ptr, wd.ptr, idd.ptr, ids.size, vocab, dim)
    got = out.to_numpy()
    ref = po.embedding_gather(w, ids)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.nan_to_num(got), np.nan_to_num(ref))


@pytest.mark.parametrize('dtype', ['float32', 'float16', 'bfloat16'])
@pytest.mark.parametrize('width', [1, 7, 50257, 4096])
def test_row_argmax_first_max_and_nan(dtype, width):
    rng = np.random.default_rng(width)
    rows = 9
    x = rng.standard_normal((rows, 1, width)).astype(np.float32)
    if width > 8:
        x[1, 0, [5, width - 3]] = 100.0          # tie: first index wins
        x[2, 0, [width // 2, 3]] = np.nan        # NaN wins, first NaN
        x[3, 0, :] = -np.inf                     # all -inf: index 0
        x[4, 0, :] = 2.0                         # all equal: index 0
        x[5, 0, -1] = np.inf
        x[6, 0, :] = -1.0
        x[6, 0, [3, 7]] = [-0.0, 0.0]            # -0 == +0: the first (index 3) wins
        x[7, 0, :] = -np.inf
        x[7, 0, [width - 2, 4]] = [np.nan, -5.0] # a NaN beats every number, even at a later index
    stored = po.encode(x, {'float32': 0, 'float16': 1, 'bfloat16': 2}[dtype])
    t = DeviceTensor(x.shape, dtype)
    runtime().h2d(t.ptr, stored)
    got = greedy_token(t).to_numpy()[:, 0]
    ref = po.row_argmax(po.decode(stored, {'float32': 0, 'float16': 1, 'bfloat16': 2}[dtype]))[:, 0]
    assert got.tolist() == ref.tolist()


def test_row_argmax_unaligned_rows():
    # width 50257 (odd) makes each fp16 row start at a different alignment
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 1, 50257)).astype(np.float16)
    for r in range(16):
        x[r, 0, (r * 3137) % 50257] = 50.0
    t = DeviceTensor(x.shape, 'float16')
    runtime().h2d(t.ptr, x)
    assert greedy_token(t).to_numpy()[:, 0].tolist() == np.argmax(x[:, 0].astype(np.float32), -1).tolist()


@pytest.mark.parametrize('rows', [1, 2, 3, 64, 128, 200, 256])
def test_row_argmax_row_counts_and_element_positions(rows):
    # GPT-2's 50257-wide bf16 logits at 1..256 rows (odd width: every row
    # starts at another 16-byte phase, so head, vectors and tail all occur);
    # each row's maximum sits in its head, a vector or its tail, sometimes
    # tied with an earlier or later equal value (first index wins) or beaten
    # by a NaN
    rng = np.random.default_rng([9, rows])
    width = 50257
    x = rng.standard_normal((rows, 1, width)).astype(np.float32)
    spots = [0, 1, 6, 7, 8, 15, 100, width // 2, width - 9, width - 2, width - 1]
    for r in range(rows):
        j = spots[r % len(spots)]
        x[r, 0, j] = 60.0
        if r % 3 == 1:
            x[r, 0, (j + 12345) % width] = 60.0   # a tie
        if r % 7 == 5:
            x[r, 0, (j * 7 + 3) % width] = np.nan
    stored = po.encode(x, 2)
    t = DeviceTensor(x.shape, 'bfloat16')
    runtime().h2d(t.ptr, stored)
    got = greedy_token(t).to_numpy()[:, 0]
    ref = po.row_argmax(po.decode(stored, 2))[:, 0]
    assert got.tolist() == ref.tolist()


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
@pytest.mark.parametrize('width', [9, 50257, 65536, 65537])
def test_row_argmax_16bit_bit_patterns(dtype, width):
    # 16-bit rows written as raw bits: NaNs of either sign and any payload,
    # signed zeros and infinities, at head, vector and tail positions; the
    # expected index is numpy.argmax of the decoded values (any NaN wins, the
    # first one; -0 == +0)
    code = {'float16': 1, 'bfloat16': 2}[dtype]
    inf, qnan = (0x7c00, 0x7e00) if dtype == 'float16' else (0x7f80, 0x7fc0)
    neg = 0x8000
    rng = np.random.default_rng([width, code])
    rows = 12
    # finite negatives below -1 everywhere (magnitude bits of 2.0 .. 4.0)
    lo, hi = (0x4000, 0x4400) if dtype == 'float16' else (0x4000, 0x4080)
    bits = (neg | rng.integers(lo, hi, (rows, width))).astype(np.uint16)
    last = width - 1
    mid = width // 2
    cases = [
        {3: neg | inf + 1},                              # negative NaN with a payload
        {mid: neg | qnan, 5: inf},                       # negative NaN beats +inf at a lower index
        {last: inf | 0x1ff, 0: neg},                     # positive NaN in the tail beats -0
        {4: neg, last: 0},                               # -0 first, +0 later: -0's index
        {last - 1: 0, 2: neg},                           # +0 later, -0 first
        {mid: 0, mid + 1: neg},                          # +0 first
        {1: neg | inf},                                  # only -inf and finite negatives: largest finite
        {0: inf, last: inf},                             # +inf tie: first
        {last: neg},                                     # -0 alone in the tail
        {min(7, last): 0x3c00 if dtype == 'float16' else 0x3f80},  # 1.0 at the head/vector boundary
        {},                                              # all finite negatives
        {mid: neg | inf + 1, 6: neg | qnan},             # two negative NaNs: the first
    ]
    for r, spots in enumerate(cases):
        for j, b in spots.items():
            bits[r, min(j, last)] = b
    if dtype == 'float16':
        values = bits.view(np.float16).astype(np.float32)
        stored = bits.view(np.float16)
    else:
        values = po.decode(bits, code)
        stored = bits
    t = DeviceTensor((rows, 1, width), dtype)
    runtime().h2d(t.ptr, np.ascontiguousarray(stored.reshape(rows, 1, width)))
    got = greedy_token(t).to_numpy()[:, 0]
    assert got.tolist() == np.argmax(values, axis=-1).astype(np.float32).tolist()


@pytest.mark.parametrize('dtype,width', [('float16', 200003), ('float32', 50257), ('float32', 70001)])
def test_row_argmax_rows_longer_than_one_round_trip(dtype, width):
    # rows longer than the 128 KiB one workgroup loads per round trip: the
    # maximum in the first, a middle and the last round, with a tie across rounds
    rng = np.random.default_rng(width)
    x = rng.standard_normal((5, 1, width)).astype(np.float32)
    per_round = 131072 // (4 if dtype == 'float32' else 2)   # elements per round trip
    for r, j in enumerate([3, width // 2, width - 1, per_round + 1, per_round - 1]):
        x[r, 0, j] = 70.0
    x[4, 0, width - 5] = 70.0
    code = {'float32': 0, 'float16': 1}[dtype]
    stored = po.encode(x, code)
    t = DeviceTensor(x.shape, dtype)
    runtime().h2d(t.ptr, stored)
    got = greedy_token(t).to_numpy()[:, 0]
    ref = po.row_argmax(po.decode(stored, code))[:, 0]
    assert got.tolist() == ref.tolist()


@pytest.mark.parametrize('dtype', ['float32', 'bfloat16'])
def test_last_position(dtype):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 5, 70)).astype(np.float32)
    t = DeviceTensor.from_numpy(x, dtype)
    got = last_position(t).raw_numpy()
    ref = po.last_row(t.raw_numpy())
    assert np.array_equal(got, ref)


@pytest.mark.parametrize('dtype', ['float32', 'float16', 'bfloat16'])
def test_row_argmax_feedback_scatters_to_slots_and_gather_reads_them(dtype):
    # Token feedback of the sync-free decode loop: the argmax of row r is also
    # stored in slot_tokens[slots[r]] (slots outside the table are skipped),
    # and the gather reads slot_tokens[slots[r]] back (NaN outside the table).
    from minitorch_amd import paged_ops
    from minitorch_amd.runtime import RawDeviceBuffer
    code = {'float32': 0, 'float16': 1, 'bfloat16': 2}[dtype]
    rng = np.random.default_rng(21)
    rows, width, num_slots = 6, 50257, 40
    x = rng.standard_normal((rows, 1, width)).astype(np.float32)
    stored = po.encode(x, code)
    t = DeviceTensor(x.shape, dtype)
    runtime().h2d(t.ptr, stored)
    slots = np.array([3, 17, -1, 39, 40, 5], np.int32)
    slot_dev = RawDeviceBuffer(4 * rows)
    slot_dev.upload(slots)
    table = RawDeviceBuffer(4 * num_slots)
    table.upload(np.full(num_slots, 7.0, np.float32))
    ids = DeviceTensor((rows, 1), 'float32')
    paged_ops.row_argmax_feedback(ids.ptr, table.ptr, slot_dev.ptr, num_slots, t.ptr, rows, width, dtype)
    got = ids.to_numpy()[:, 0]
    ref = po.row_argmax(po.decode(stored, code))[:, 0]
    assert got.tolist() == ref.tolist()
    expect = np.full(num_slots, 7.0, np.float32)
    for r, s in enumerate(slots):
        if 0 <= s < num_slots:
            expect[s] = ref[r]
    assert np.array_equal(table.download(np.float32), expect)
    back = DeviceTensor((rows, 1), 'float32')
    paged_ops.gather_slot_tokens(back.ptr, table.ptr, slot_dev.ptr, num_slots, rows)
    want = np.array([expect[s] if 0 <= s < num_slots else np.nan for s in slots], np.float32)
    assert np.array_equal(back.to_numpy()[:, 0], want, equal_nan=True)


def test_embed_tokens_equals_two_gathers_and_sum():
    # mt_embed_tokens against the oracle gathers (NaN rows for invalid token
    # ids or positions) and their sum, bit for bit; ids given directly and
    # through the slot table of the token feedback.
    from minitorch_amd import paged_ops
    from minitorch_amd.runtime import RawDeviceBuffer
    rng = np.random.default_rng(31)
    vocab, npos, dim, rows = 50, 20, 64, 9
    wte = rng.standard_normal((vocab, dim)).astype(np.float32)
    wpe = rng.standard_normal((npos, dim)).astype(np.float32)
    ids = np.array([0, 49, 7, -1, 50, 2.5, np.nan, 3, 4], np.float32)
    pos = np.array([0, 19, 5, 1, 2, 3, 4, 20, -0.0], np.float32)
    ref = po.embedding_gather(wte, ids) + po.embedding_gather(wpe, pos)
    W, Pt = DeviceTensor.from_numpy(wte), DeviceTensor.from_numpy(wpe)
    I, Q = DeviceTensor.from_numpy(ids), DeviceTensor.from_numpy(pos)
    x = DeviceTensor((rows, dim), 'float32')
    paged_ops.embed_tokens(x.ptr, W.ptr, Pt.ptr, I.ptr, Q.ptr, rows, vocab, npos, dim)
    assert np.array_equal(x.to_numpy(), ref, equal_nan=True)
    # the same ids through slots (one slot outside the table -> NaN row)
    num_slots = 16
    slots = np.array([5, 0, 15, 3, 9, 1, 2, 16, 8], np.int32)
    table = np.full(num_slots, 11.0, np.float32)
    for r, s in enumerate(slots):
        if s < num_slots:
            table[s] = ids[r]
    T = DeviceTensor.from_numpy(table)
    S = RawDeviceBuffer(4 * rows)
    S.upload(slots)
    x2 = DeviceTensor((rows, dim), 'float32')
    paged_ops.embed_tokens(x2.ptr, W.ptr, Pt.ptr, None, Q.ptr, rows, vocab, npos, dim, slot_tokens=T.ptr,
                           slots=S.ptr, num_slots=num_slots)
    want = ref.copy()
    want[7] = np.nan
    assert np.array_equal(x2.to_numpy(), want, equal_nan=True)
