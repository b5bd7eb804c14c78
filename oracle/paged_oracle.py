"""CPU oracle for the paged decode path. TEST INFRASTRUCTURE ONLY.

Only tests, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker. The product path never calls
it.

This restates the reference's algorithm in numpy:

* element addressing of a paged slab (reference src/paged_attention_kernel.cu:7-21);
* the KV append through the block table (src/paged_attention_kernel.cu:23-33);
* paged attention for one new token per request and for nq >= 1 causal
  queries, both textbook in float64 (``attention_fp64``) and in the
  reference kernel's own fp32 order (``attention_fp32_reference_order``,
  src/paged_attention_kernel.cu:35-85): 32-key tiles, sequential dot over
  head_dim, ``s *= rsqrt(D)``, online softmax with ``alpha = isfinite(m) ?
  exp(m - m') : 0``, sequential P.V accumulation, and
  ``out = l > 0 ? acc / l : (isnan(l) ? NaN : 0)``;
* the split-context log-sum-exp merge (no reference counterpart; the closed
  form m = max m_i, o = sum e^(m_i - m) l_i o_i / sum e^(m_i - m) l_i);
* embedding gather with the NaN-on-invalid-id rule (src/inference_kernels.cu:7-14),
  greedy argmax with numpy's first-maximum / NaN-wins rule
  (src/inference_kernels.cu:32-55, minitorch/kv_cache.py:39-53) and the
  last-position copy (src/inference_kernels.cu:28-30);
* bf16 host encoding with round-to-nearest-even and quiet NaNs
  (minitorch/dtypes.py:37-51).

How each function is pinned is stated in its docstring; the checks live in
tests/test_oracle.py.
"""
import math
import numpy as np

F32, F16, BF16 = 0, 1, 2
DTYPE_NAMES = {F32: 'float32', F16: 'float16', BF16: 'bfloat16'}


# ----------------------------------------------------------------- dtypes ---
def bf16_encode(values):
    """float32 -> bf16 bit patterns (uint16), RNE, NaN kept quiet.

    Restates minitorch/dtypes.py:37-46. Pinned by exhaustive comparison with
    exact rational rounding on every bf16 boundary in tests/test_oracle.py.
    """
    bits = np.ascontiguousarray(values, dtype=np.float32).reshape(-1).view(np.uint32)
    rounded = ((bits + np.uint32(0x7fff) + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = ((bits & 0x7f800000) == 0x7f800000) & ((bits & 0x007fffff) != 0)
    out = np.where(nan, (bits >> 16).astype(np.uint16) | np.uint16(0x40), rounded)
    return out.astype(np.uint16).reshape(np.shape(values))


def bf16_decode(bits):
    """bf16 bit patterns -> float32 (minitorch/dtypes.py:49-51)."""
    return (np.asarray(bits).astype(np.uint32) << 16).view(np.float32)


def encode(values, dtype):
    """Host array of the storage type for ``dtype`` (float32/float16/bf16 bits)."""
    if dtype == F32:
        return np.ascontiguousarray(values, dtype=np.float32)
    if dtype == F16:
        return np.ascontiguousarray(values, dtype=np.float16)
    return bf16_encode(values)


def decode(stored, dtype):
    """Storage array -> float32 values."""
    if dtype == BF16:
        return bf16_decode(stored)
    return np.asarray(stored).astype(np.float32)


def storage_dtype(dtype):
    return {F32: np.float32, F16: np.float16, BF16: np.uint16}[dtype]


# ------------------------------------------------------------- addressing ---
def element_index(layer, kind, slot, head, position, col, heads, dim, page_size, pages_per_slab):
    """Element offset inside a slab (reference src/paged_attention_kernel.cu:18-19).

    Pinned by tests that scatter with this index and find each value at the
    C-order position of a [layers,2,pps,H,P,D] array.
    """
    i = (((layer * 2 + kind) * pages_per_slab + slot) * heads + head) * page_size * dim
    return i + (position % page_size) * dim + col


class SlabPool:
    """Host image of the device slabs: ``slabs[s]`` is a flat storage array.

    ``present[s]`` False models a null slab address in the uint64 slab table.
    """

    def __init__(self, layers, heads, dim, page_size, pages_per_slab, num_slabs, dtype,
                 fill=None, present=None):
        self.layers, self.heads, self.dim = layers, heads, dim
        self.page_size, self.pages_per_slab, self.num_slabs = page_size, pages_per_slab, num_slabs
        self.dtype = dtype
        self.slab_elems = layers * 2 * pages_per_slab * heads * page_size * dim
        self.slabs = []
        for s in range(num_slabs):
            if fill is None:
                self.slabs.append(np.zeros(self.slab_elems, storage_dtype(dtype)))
            else:
                self.slabs.append(encode(fill(s, self.slab_elems), dtype).reshape(-1))
        self.present = [True] * num_slabs if present is None else list(present)

    def copy(self):
        other = SlabPool.__new__(SlabPool)
        other.__dict__.update(self.__dict__)
        other.slabs = [s.copy() for s in self.slabs]
        other.present = list(self.present)
        return other

    def page_slot(self, table_row, columns, position):
        """(slab, slot) for a position, or None for a missing page
        (src/paged_attention_kernel.cu:11-16)."""
        logical = position // self.page_size
        if logical < 0 or logical >= columns:
            return None
        physical = int(table_row[logical])
        if physical < 0 or physical >= self.num_slabs * self.pages_per_slab:
            return None
        slab = physical // self.pages_per_slab
        if not self.present[slab]:
            return None
        return slab, physical % self.pages_per_slab

    def row_values(self, table_row, columns, layer, kind, head, position):
        """K or V row (float32, length dim) at a position; NaN for a missing page."""
        where = self.page_slot(table_row, columns, position)
        if where is None:
            return np.full(self.dim, np.nan, np.float32)
        slab, slot = where
        i = element_index(layer, kind, slot, head, position, 0, self.heads, self.dim,
                          self.page_size, self.pages_per_slab)
        return decode(self.slabs[slab][i:i + self.dim], self.dtype)


# ----------------------------------------------------------------- append ---
def paged_append(pool, table, columns, k, v, layer, offsets=None, offset=0):
    """Scatter K/V [B,H,n,D] (storage dtype) into the pool at offset(+pos).

    Restates src/paged_attention_kernel.cu:23-33: rows whose page is missing
    are skipped. ``offsets`` gives a per-request offset (decode), else the
    common ``offset``. Pinned by the closed-form index test and the
    untouched-slot invariant.
    """
    b, h, n, d = k.shape
    table = np.asarray(table).reshape(b, columns)
    for bi in range(b):
        base = int(offsets[bi]) if offsets is not None else offset
        for hi in range(h):
            for pos in range(n):
                position = base + pos
                where = pool.page_slot(table[bi], columns, position)
                if where is None:
                    continue
                slab, slot = where
                for kind, src in ((0, k), (1, v)):
                    i = element_index(layer, kind, slot, hi, position, 0, h, d, pool.page_size,
                                      pool.pages_per_slab)
                    pool.slabs[slab][i:i + d] = src[bi, hi, pos]


def gather(pool, table_row, columns, layer, head, length):
    """K and V [length, D] float32 of one (request, head), NaN rows for missing pages."""
    keys = np.stack([pool.row_values(table_row, columns, layer, 0, head, j) for j in range(length)]) \
        if length else np.zeros((0, pool.dim), np.float32)
    vals = np.stack([pool.row_values(table_row, columns, layer, 1, head, j) for j in range(length)]) \
        if length else np.zeros((0, pool.dim), np.float32)
    return keys, vals


# -------------------------------------------------------------- attention ---
def attention_fp64(q, keys, vals):
    """Textbook softmax(q.K^T / sqrt(D)) . V in float64 for one query.

    A NaN key or value poisons the result (NaN row), zero keys give a zero
    row, matching the reference's output rule (src/paged_attention_kernel.cu:84).
    Pinned by closed forms in tests/test_oracle.py (L = 1 gives v0, identical
    keys give the mean of V, a one-hot dominant score gives that row of V).
    """
    q = np.asarray(q, np.float64)
    keys = np.asarray(keys, np.float64)
    vals = np.asarray(vals, np.float64)
    if keys.shape[0] == 0:
        return np.zeros(q.shape[-1])
    s = keys @ q / math.sqrt(q.shape[-1])
    if np.isnan(s).any():
        # A NaN score makes the softmax denominator NaN: the whole row is NaN.
        return np.full(q.shape[-1], np.nan)
    s = s - s.max()
    p = np.exp(s)
    return (p @ vals) / p.sum()


def attention_fp32_reference_order(q, keys, vals, tile=32):
    """The reference kernel's fp32 arithmetic order for one query.

    Restates src/paged_attention_kernel.cu:44-84 for nq = 1 (one warp owns the
    query): per 32-key tile, s_j = (sum_d q_d k_jd) * rsqrt(D) with the dot
    accumulated sequentially over d; next_m = max(m, max_j s_j) with NaN
    ignored (fmaxf); alpha = isfinite(m) ? exp(m - next_m) : 0;
    p_j = exp(s_j - next_m); l = alpha l + sum p; acc = alpha acc + sum_j p_j v_j
    (j in tile order); out = l > 0 ? acc / l : (isnan(l) ? NaN : 0).
    The warp reductions (fa_max/fa_sum butterflies) are replaced by numpy
    reductions, so sums may round differently in the last bit. Pinned against
    ``attention_fp64`` (agreement to 1e-6 relative on random inputs).
    """
    f = np.float32
    q = np.asarray(q, f)
    keys = np.asarray(keys, f)
    vals = np.asarray(vals, f)
    n, d = keys.shape
    scale = f(1.0) / f(math.sqrt(d))
    m, l = f(-np.inf), f(0)
    acc = np.zeros(d, f)
    with np.errstate(invalid='ignore', over='ignore'):
        for start in range(0, n, tile):
            kt = keys[start:start + tile]
            vt = vals[start:start + tile]
            s = np.zeros(kt.shape[0], f)
            for c in range(d):
                s = (s + q[c] * kt[:, c]).astype(f)
            s = (s * scale).astype(f)
            finite = s[~np.isnan(s)]
            tile_max = finite.max() if finite.size else f(-np.inf)
            next_m = f(max(m, tile_max)) if not np.isnan(tile_max) else m
            alpha = f(np.exp(f(m - next_m))) if np.isfinite(m) else f(0)
            p = np.exp((s - next_m).astype(f)).astype(f)
            l = f(alpha * l + p.sum(dtype=f))
            update = np.zeros(d, f)
            for j in range(kt.shape[0]):
                update = (update + p[j] * vt[j]).astype(f)
            acc = (alpha * acc + update).astype(f)
            m = next_m
        if l > 0:
            return (acc / l).astype(f)
        return np.full(d, np.nan if np.isnan(l) else 0, f)


def lse_merge(parts):
    """Merge split partials [(m, l, acc[D])] (natural-log units) into one output.

    Closed form: M = max m_i, out = sum e^(m_i-M) acc_i / sum e^(m_i-M) l_i.
    Pinned in tests by split == unsplit on random inputs.
    """
    ms = np.array([p[0] for p in parts], np.float64)
    M = ms.max()
    w = np.where(np.isneginf(ms), 0.0, np.exp(ms - M))
    l = sum(wi * p[1] for wi, p in zip(w, parts))
    acc = sum(wi * np.asarray(p[2], np.float64) for wi, p in zip(w, parts))
    return acc / l


def split_partial(q, keys, vals):
    """(m, l, acc) of a key range in natural-log units, float64."""
    d = q.shape[-1]
    if keys.shape[0] == 0:
        return (-np.inf, 0.0, np.zeros(d))
    s = np.asarray(keys, np.float64) @ np.asarray(q, np.float64) / math.sqrt(d)
    m = s.max()
    p = np.exp(s - m)
    return (m, p.sum(), p @ np.asarray(vals, np.float64))


def decode_batch(pool, table, columns, q, k, v, offsets, layer, order='fp64'):
    """Reference ``mt_paged_decode_batch`` on the host.

    Appends K/V [B,H,1,D] at offsets[b] (src/paged_attention_kernel.cu:131),
    then attends over offsets[b] + 1 keys (src/paged_attention_kernel.cu:43,133).
    Mutates ``pool``. Returns float64 ('fp64') or float32 ('fp32') outputs
    [B,H,1,D]; ``order='fp32'`` uses ``attention_fp32_reference_order``.
    """
    b, h, _, d = q.shape
    table = np.asarray(table, np.int32).reshape(b, columns)
    paged_append(pool, table, columns, k, v, layer, offsets=offsets)
    qf = decode(q, pool.dtype)
    out = np.zeros((b, h, 1, d), np.float64 if order == 'fp64' else np.float32)
    for bi in range(b):
        length = max(int(offsets[bi]) + 1, 0)
        for hi in range(h):
            keys, vals = gather(pool, table[bi], columns, layer, hi, length)
            if order == 'fp64':
                out[bi, hi, 0] = attention_fp64(qf[bi, hi, 0], keys, vals)
            else:
                out[bi, hi, 0] = attention_fp32_reference_order(qf[bi, hi, 0], keys, vals)
    return out


def paged_attention(pool, table, columns, q, layer, offset, nk):
    """Reference ``mt_paged_attention`` (causal, nq >= 1) in float64.

    Query qi attends keys kj < nk with kj <= offset + qi
    (src/paged_attention_kernel.cu:59). Does not append.
    """
    b, h, nq, d = q.shape
    table = np.asarray(table, np.int32).reshape(b, columns)
    qf = decode(q, pool.dtype)
    out = np.zeros((b, h, nq, d))
    for bi in range(b):
        for hi in range(h):
            keys, vals = gather(pool, table[bi], columns, layer, hi, nk)
            for qi in range(nq):
                hi_key = min(offset + qi + 1, nk)
                out[bi, hi, qi] = attention_fp64(qf[bi, hi, qi], keys[:hi_key], vals[:hi_key])
    return out


# ------------------------------------------------------------ token I/O ---
def embedding_gather(weights, ids):
    """dst[t] = W[ids[t]]; NaN row for a non-finite, negative, >= vocab or
    non-integer id (src/inference_kernels.cu:7-14). Pinned by numpy fancy
    indexing on valid ids and by the explicit invalid-id cases."""
    weights = np.asarray(weights, np.float32)
    ids = np.asarray(ids, np.float32).reshape(-1)
    vocab, dim = weights.shape
    out = np.full((ids.size, dim), np.nan, np.float32)
    with np.errstate(invalid='ignore'):
        ok = np.isfinite(ids) & (ids >= 0) & (ids < vocab) & (ids == np.floor(ids))
    out[ok] = weights[ids[ok].astype(np.int64)]
    return out


def row_argmax(rows):
    """Index of the first maximum per row, NaN beating numbers (numpy.argmax
    semantics, minitorch/kv_cache.py:43-44). Returned as float32."""
    rows = np.asarray(rows, np.float32)
    return np.argmax(rows, axis=-1).astype(np.float32)


def last_row(x):
    """x[:, -1:, :] for [B, n, W] (src/inference_kernels.cu:28-30)."""
    return np.ascontiguousarray(np.asarray(x)[:, -1:, :])


# ------------------------------------------- vectorized image-based forms ---
# The functions below work on a pool image [num_slabs, layers, 2, pps, H, P, D]
# (storage dtype) instead of flat slabs. They compute the same thing as the
# element_index-based forms above, vectorized over positions; tests pin them
# against those forms on small pools.
def image_slots(image_shape, table_row, columns, positions, present=None):
    """(ok, slab, slot) arrays for positions of one request (page validity as
    in src/paged_attention_kernel.cu:11-16)."""
    num_slabs, _, _, pps, _, page_size, _ = image_shape
    positions = np.asarray(positions, np.int64)
    logical = positions // page_size
    ok = (logical >= 0) & (logical < columns)
    phys = np.where(ok, np.asarray(table_row)[np.clip(logical, 0, columns - 1)], -1).astype(np.int64)
    ok &= (phys >= 0) & (phys < num_slabs * pps)
    slab = np.where(ok, phys // pps, 0)
    slot = np.where(ok, phys % pps, 0)
    if present is not None:
        ok &= np.asarray(present, bool)[slab]
    return ok, slab, slot


def image_gather(image, dtype, table_row, columns, layer, head, length, present=None):
    """K, V [length, D] float32 of one (request, head); NaN rows for missing pages."""
    page_size, dim = image.shape[5], image.shape[6]
    pos = np.arange(length)
    ok, slab, slot = image_slots(image.shape, table_row, columns, pos, present)
    keys = np.full((length, dim), np.nan, np.float32)
    vals = np.full((length, dim), np.nan, np.float32)
    keys[ok] = decode(image[slab[ok], layer, 0, slot[ok], head, pos[ok] % page_size], dtype)
    vals[ok] = decode(image[slab[ok], layer, 1, slot[ok], head, pos[ok] % page_size], dtype)
    return keys, vals


def image_append(image, table, columns, k, v, layer, offsets=None, offset=0, present=None):
    """Vectorized ``paged_append`` on an image (mutates it)."""
    b, h, n, d = k.shape
    page_size = image.shape[5]
    table = np.asarray(table).reshape(b, columns)
    for bi in range(b):
        base = int(offsets[bi]) if offsets is not None else offset
        pos = base + np.arange(n)
        ok, slab, slot = image_slots(image.shape, table[bi], columns, pos, present)
        for j in np.nonzero(ok)[0]:
            image[slab[j], layer, 0, slot[j], :, pos[j] % page_size] = k[bi, :, j]
            image[slab[j], layer, 1, slot[j], :, pos[j] % page_size] = v[bi, :, j]


def image_decode_batch(image, dtype, table, columns, q, k, v, offsets, layer, present=None,
                       rows=None):
    """``mt_paged_decode_batch`` on an image in float64 (mutates ``image``).

    ``rows`` optionally restricts the attention to a subset of (b, h) pairs;
    the append always covers every request. Returns [B, H, 1, D] float64 with
    NaN for rows not computed.
    """
    b, h, _, d = q.shape
    table = np.asarray(table, np.int32).reshape(b, columns)
    image_append(image, table, columns, k, v, layer, offsets=offsets, present=present)
    qf = decode(q, dtype)
    out = np.full((b, h, 1, d), np.nan)
    pairs = [(bi, hi) for bi in range(b) for hi in range(h)] if rows is None else rows
    for bi, hi in pairs:
        length = max(int(offsets[bi]) + 1, 0)
        keys, vals = image_gather(image, dtype, table[bi], columns, layer, hi, length, present)
        out[bi, hi, 0] = attention_fp64(qf[bi, hi, 0], keys, vals)
    return out


def image_paged_attention(image, dtype, table, columns, q, layer, offset, nk, present=None):
    """``mt_paged_attention`` (causal, nq >= 1) on an image, float64."""
    b, h, nq, d = q.shape
    table = np.asarray(table, np.int32).reshape(b, columns)
    qf = decode(q, dtype)
    out = np.zeros((b, h, nq, d))
    for bi in range(b):
        for hi in range(h):
            keys, vals = image_gather(image, dtype, table[bi], columns, layer, hi, nk, present)
            for qi in range(nq):
                top = min(offset + qi + 1, nk)
                out[bi, hi, qi] = attention_fp64(qf[bi, hi, qi], keys[:top], vals[:top])
    return out
