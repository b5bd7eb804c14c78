"""Pins for the paged-attention oracle (oracle/paged_oracle.py, oracle/paged_oracle.c).

The reference ships no golden vectors for this path, so each oracle function
is pinned by what the mathematics fixes: exact rounding on every bf16
boundary, the C-order index of the slab array, closed forms of attention
(one key, identical keys, a dominant key), invariance under physical page
permutation and page size, brute-force loops on tiny inputs, the LSE merge of
splits, and agreement of the independent C restatement. Planted mistakes in
copies of the oracle show that the checks catch a dropped scale, a swapped
index and a wrong tie rule.
"""
import math

import numpy as np
import pytest

from oracle import paged_oracle as po
from oracle import c_oracle
from minitorch_amd.workloads import make_decode_case, config1_case

CODES = {'float32': po.F32, 'float16': po.F16, 'bfloat16': po.BF16}


# ------------------------------------------------------------------ bf16 ----
def _bf16_grid():
    bits = np.arange(0, 0x7f80, dtype=np.uint32)          # finite non-negative bf16
    return (bits << 16).view(np.float32)


def test_bf16_rounds_to_nearest_even_on_every_boundary():
    v = _bf16_grid()
    lo, hi = v[:-1], v[1:]
    mid = ((lo.astype(np.float64) + hi) / 2).astype(np.float32)    # exact in fp32
    assert np.array_equal((mid.astype(np.float64) * 2), lo.astype(np.float64) + hi)
    lo_bits = (lo.view(np.uint32) >> 16).astype(np.uint16)
    hi_bits = (hi.view(np.uint32) >> 16).astype(np.uint16)
    even = np.where(lo_bits % 2 == 0, lo_bits, hi_bits)
    assert np.array_equal(po.bf16_encode(mid), even)
    assert np.array_equal(po.bf16_encode(np.nextafter(mid, np.float32(np.inf))), hi_bits)
    assert np.array_equal(po.bf16_encode(np.nextafter(mid, np.float32(-np.inf))), lo_bits)
    assert np.array_equal(po.bf16_encode(-mid), even | np.uint16(0x8000))
    assert np.array_equal(po.bf16_encode(lo), lo_bits)          # representable values are exact


def test_bf16_specials():
    x = np.array([np.nan, np.inf, -np.inf, 3.4e38, -0.0], np.float32)
    e = po.bf16_encode(x)
    d = po.bf16_decode(e)
    assert np.isnan(d[0]) and (e[0] & 0x40)                     # quiet NaN
    assert d[1] == np.inf and d[2] == -np.inf and d[3] == np.inf
    assert e[4] == 0x8000


# -------------------------------------------------------------- indexing ----
def test_element_index_is_c_order_of_the_slab_array():
    layers, pps, h, p, d = 3, 5, 4, 8, 6
    shape = (layers, 2, pps, h, p, d)
    for idx in np.ndindex(*shape):
        layer, kind, slot, head, pos, col = idx
        got = po.element_index(layer, kind, slot, head, pos + 2 * p, col, h, d, p, pps)
        assert got == np.ravel_multi_index(idx, shape)


def _planted_index(layer, kind, slot, head, position, col, heads, dim, page_size, pages_per_slab):
    # slot and head swapped: a plausible transposition
    i = (((layer * 2 + kind) * heads + head) * pages_per_slab + slot) * page_size * dim
    return i + (position % page_size) * dim + col


def test_planted_index_transposition_is_caught():
    layers, pps, h, p, d = 2, 3, 4, 8, 2
    shape = (layers, 2, pps, h, p, d)
    bad = sum(_planted_index(*idx[:4], idx[4], idx[5], h, d, p, pps) != np.ravel_multi_index(idx, shape)
              for idx in np.ndindex(*shape))
    assert bad > 0


# ---------------------------------------------------------------- append ----
def _slabpool_from_image(case):
    c = case
    pool = po.SlabPool(c.layers, c.heads, c.dim, c.page_size, c.pages_per_slab, c.num_slabs, CODES[c.dtype])
    pool.slabs = [c.image[s].reshape(-1).copy() for s in range(c.num_slabs)]
    return pool


@pytest.mark.parametrize('dtype', ['float32', 'bfloat16'])
def test_append_forms_agree_and_leave_other_slots(dtype):
    case = make_decode_case(0, batch=3, heads=2, dim=8, page_size=8, lengths=[3, 9, 17],
                            pool_pages=12, pages_per_slab=3, dtype=dtype, layers=2, layer=1)
    case.table[1, 1] = -1                           # request 1's new token has no page
    pool = _slabpool_from_image(case)
    image = case.image.copy()
    po.paged_append(pool, case.table, case.columns, case.k, case.v, case.layer, offsets=case.offsets)
    po.image_append(image, case.table, case.columns, case.k, case.v, case.layer, offsets=case.offsets)
    flat = np.stack([s.reshape(image.shape[1:]) for s in pool.slabs])
    assert np.array_equal(flat.view(np.uint8), image.view(np.uint8))
    changed = np.argwhere(np.any(image != case.image, axis=-1))
    # exactly rows of (request 0, 2) x 2 heads x (K, V) changed (request 1 skipped)
    assert len(changed) <= 2 * 2 * 2
    for b in (0, 2):
        pos = int(case.offsets[b])
        page = int(case.table[b, pos // 8])
        for kind, src in ((0, case.k), (1, case.v)):
            assert np.array_equal(image[page // 3, 1, kind, page % 3, :, pos % 8], src[b, :, 0])


def test_gather_forms_agree_with_missing_pages():
    case = make_decode_case(1, batch=2, heads=3, dim=4, page_size=8, lengths=[20, 30],
                            pool_pages=12, pages_per_slab=4, dtype='float32')
    case.table[0, 1] = -1
    case.table[1, 2] = 999
    pool = _slabpool_from_image(case)
    for b in range(2):
        for h in range(3):
            k1, v1 = po.gather(pool, case.table[b], case.columns, 0, h, int(case.lengths[b]))
            k2, v2 = po.image_gather(case.image, po.F32, case.table[b], case.columns, 0, h, int(case.lengths[b]))
            assert np.array_equal(np.isnan(k1), np.isnan(k2)) and np.array_equal(np.nan_to_num(k1), np.nan_to_num(k2))
            assert np.array_equal(np.nan_to_num(v1), np.nan_to_num(v2))
    k, _ = po.image_gather(case.image, po.F32, case.table[0], case.columns, 0, 0, 20)
    assert np.isnan(k[8:16]).all() and not np.isnan(k[:8]).any()


# ------------------------------------------------------------- attention ----
def brute_force_attention(q, keys, vals):
    d = len(q)
    scores = []
    for kj in keys:
        s = 0.0
        for a, b in zip(q, kj):
            s += float(a) * float(b)
        scores.append(s / math.sqrt(d))
    m = max(scores)
    w = [math.exp(s - m) for s in scores]
    total = sum(w)
    return [sum(w[j] * float(vals[j][c]) for j in range(len(w))) / total for c in range(d)]


def test_attention_closed_forms():
    rng = np.random.default_rng(0)
    q = rng.standard_normal(64)
    v = rng.standard_normal((5, 64))
    assert np.allclose(po.attention_fp64(q, v[:1] * 0 + 1.0, v[:1]), v[0], rtol=0, atol=0)
    same = np.tile(rng.standard_normal(64), (5, 1))
    assert np.allclose(po.attention_fp64(q, same, v), v.mean(0), rtol=1e-14, atol=1e-14)
    keys = rng.standard_normal((5, 64)) * 0.01
    keys[3] = q * 100                            # dominant score
    assert np.allclose(po.attention_fp64(q, keys, v), v[3], atol=1e-12)
    assert np.all(po.attention_fp64(q, np.zeros((0, 64)), np.zeros((0, 64))) == 0)
    keys[1, 0] = np.nan
    assert np.isnan(po.attention_fp64(q, keys, v)).all()


def test_attention_matches_brute_force_on_tiny_inputs():
    rng = np.random.default_rng(1)
    for n in (1, 2, 7, 33):
        q = rng.standard_normal(8)
        keys = rng.standard_normal((n, 8))
        vals = rng.standard_normal((n, 8))
        assert np.allclose(po.attention_fp64(q, keys, vals), brute_force_attention(q, keys, vals),
                           rtol=1e-12, atol=1e-12)


def _planted_attention_no_scale(q, keys, vals):
    s = keys @ q
    p = np.exp(s - s.max())
    return p @ vals / p.sum()


def test_planted_missing_scale_is_caught():
    rng = np.random.default_rng(2)
    q, keys, vals = rng.standard_normal(64), rng.standard_normal((30, 64)), rng.standard_normal((30, 64))
    assert not np.allclose(_planted_attention_no_scale(q, keys, vals), brute_force_attention(q, keys, vals),
                           rtol=1e-6, atol=1e-6)


def test_fp32_reference_order_agrees_with_fp64():
    rng = np.random.default_rng(3)
    for n in (1, 31, 32, 33, 100, 1024):
        q = rng.standard_normal(64).astype(np.float32)
        keys = rng.standard_normal((n, 64)).astype(np.float32)
        vals = rng.standard_normal((n, 64)).astype(np.float32)
        a = po.attention_fp32_reference_order(q, keys, vals)
        b = po.attention_fp64(q, keys, vals)
        assert np.abs(a - b).max() <= 2e-6 * np.abs(b).max()
    keys[5] = np.nan
    assert np.isnan(po.attention_fp32_reference_order(q, keys, vals)).all()


def test_split_lse_merge_equals_unsplit():
    rng = np.random.default_rng(4)
    q = rng.standard_normal(64)
    keys, vals = rng.standard_normal((700, 64)), rng.standard_normal((700, 64))
    whole = po.attention_fp64(q, keys, vals)
    for cuts in ([256, 512], [1, 2, 3], [699]):
        edges = [0] + cuts + [700]
        parts = [po.split_partial(q, keys[a:b], vals[a:b]) for a, b in zip(edges, edges[1:])]
        assert np.allclose(po.lse_merge(parts), whole, rtol=1e-12, atol=1e-12)


def test_decode_invariant_under_page_permutation_and_page_size():
    lengths = [5, 40, 77]
    outs = []
    for seed, page_size in ((0, 16), (1, 16), (2, 32), (3, 8)):
        case = make_decode_case(seed, batch=3, heads=2, dim=16, page_size=page_size, lengths=lengths,
                                pool_pages=64, pages_per_slab=4, dtype='float32')
        # same logical K/V/Q for every case: rebuild the image from one fixed set
        rng = np.random.default_rng(99)
        q = rng.standard_normal((3, 2, 1, 16)).astype(np.float32)
        k = rng.standard_normal((3, 2, 1, 16)).astype(np.float32)
        v = rng.standard_normal((3, 2, 1, 16)).astype(np.float32)
        kv = rng.standard_normal((3, 2, 2, 77, 16)).astype(np.float32)   # [b, kind, h, pos, d]
        image = np.zeros_like(case.image)
        for b in range(3):
            for pos in range(lengths[b] - 1):
                page = int(case.table[b, pos // page_size])
                for kind in range(2):
                    image[page // 4, 0, kind, page % 4, :, pos % page_size] = kv[b, kind, :, pos]
        outs.append(po.image_decode_batch(image, po.F32, case.table, case.columns, q, k, v,
                                          case.offsets, 0))
    for o in outs[1:]:
        assert np.allclose(o, outs[0], rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------- C restatement --
@pytest.fixture(scope='module')
def clib():
    c_oracle.build()
    return c_oracle.library()


@pytest.mark.parametrize('dtype', ['float32', 'float16', 'bfloat16'])
def test_c_oracle_agrees_with_numpy_oracle(clib, dtype):
    case = make_decode_case(5, batch=5, heads=3, dim=64, page_size=16, lengths=[1, 16, 17, 100, 300],
                            pool_pages=64, pages_per_slab=4, dtype=dtype)
    case.table[3, 2] = -1
    host = c_oracle.HostCase(case)
    out = po.decode(host.run(clib, 4), CODES[dtype])
    image = case.image.copy()
    ref = po.image_decode_batch(image, CODES[dtype], case.table, case.columns, case.q, case.k, case.v,
                                case.offsets, 0)
    assert np.array_equal(host.image.view(np.uint8), image.view(np.uint8))
    assert np.array_equal(np.isnan(out), np.isnan(ref[..., :]))
    tol = 1e-5 if dtype == 'float32' else 1e-2
    assert np.nanmax(np.abs(out - ref)) <= tol


def test_c_oracle_config1(clib):
    case = config1_case(0)
    host = c_oracle.HostCase(case)
    out = host.run(clib, 2)
    ref = po.image_decode_batch(case.image.copy(), po.F32, case.table, case.columns, case.q, case.k,
                                case.v, case.offsets, 0)
    assert np.abs(out - ref).max() <= 1e-5 * np.abs(ref).max()


# ------------------------------------------------------------- token I/O ----
def test_embedding_gather_rules():
    w = np.arange(12, dtype=np.float32).reshape(4, 3)
    ids = np.array([0, 3, 2.0, -1, 4, 1.5, np.nan, np.inf], np.float32)
    out = po.embedding_gather(w, ids)
    assert np.array_equal(out[:3], w[[0, 3, 2]])
    assert np.isnan(out[3:]).all()


def _argmax_loop(row):
    best, index = None, None
    for j, v in enumerate(row):
        if index is None or (np.isnan(v) and not np.isnan(best)) or (not np.isnan(best) and not np.isnan(v) and v > best):
            best, index = v, j
    return index


def test_row_argmax_rules_against_explicit_loop():
    rng = np.random.default_rng(6)
    rows = rng.integers(-3, 4, (50, 1, 17)).astype(np.float32)
    rows[5, 0, [2, 9]] = np.nan
    rows[6, 0, :] = -np.inf
    rows[7, 0, 4] = np.inf
    got = po.row_argmax(rows)[:, 0]
    assert got.tolist() == [float(_argmax_loop(r[0])) for r in rows]


def test_planted_last_max_tie_rule_is_caught():
    row = np.array([1, 5, 5, 2], np.float32)
    last = len(row) - 1 - int(np.argmax(row[::-1]))
    assert last != _argmax_loop(row) == 1


@pytest.mark.parametrize('dtype', ['float32', 'float16', 'bfloat16'])
def test_c_oracle_causal_attention_agrees_with_numpy_oracle(clib, dtype):
    # oracle_paged_attention (the C restatement of mt_paged_attention) against
    # the numpy fp64 oracle: causal masks at an offset, a hole in the pages
    # (queries that reach it are NaN), two requests, page size 8.
    nq, offset = 37, 20
    case = make_decode_case(7, batch=2, heads=3, dim=64, page_size=8, lengths=[offset + nq] * 2,
                            pool_pages=32, pages_per_slab=4, dtype=dtype)
    case.table[1, 4] = -1                      # keys 32..39 of request 1 missing
    q = po.encode(np.random.default_rng(7).standard_normal((2, 3, nq, 64)).astype(np.float32), CODES[dtype])
    got = po.decode(c_oracle.paged_attention(clib, case, q, nq, offset + nq, offset, threads=4), CODES[dtype])
    ref = po.image_paged_attention(case.image, CODES[dtype], case.table, case.columns, q, 0, offset, offset + nq)
    assert np.isnan(ref[1, :, 12:]).all() and not np.isnan(ref[1, :, :12]).any()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    tol = 1e-5 * np.nanmax(np.abs(ref)) if dtype == 'float32' else 1e-2
    assert np.nanmax(np.abs(got - ref)) <= tol
