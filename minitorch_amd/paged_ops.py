"""Thin Python wrappers over the paged-attention and token-I/O C-ABI.

Argument order and meaning follow the reference's ctypes call sites
(minitorch/paged_kv_cache.py:205-221, minitorch/paged_decode.py:65-69,
minitorch/kv_cache.py:35,52, minitorch/pretrained_gpt2.py:30-31). Every call
goes to ``cuda_kernels/paged_attention_kernel.so`` or
``cuda_kernels/inference_kernels.so``.
"""
import ctypes as ct
from functools import lru_cache
import numpy as np
from .runtime import library, call, P, I, Z, DeviceTensor, runtime
from .dtypes import dtype_code


def paged_library():
    return library('paged_attention_kernel')


def inference_library():
    return library('inference_kernels')


def paged_append(k, v, slab_table, block_table, *, b, h, n, d, page_size, pages_per_slab,
                 num_slabs, columns, layer, layers, offset, dtype):
    """``mt_paged_append`` (reference src/paged_attention_kernel.cu:96-106)."""
    call(paged_library(), 'mt_paged_append', [P] * 4 + [I] * 12,
         k, v, slab_table, block_table, b, h, n, d, page_size, pages_per_slab, num_slabs,
         columns, layer, layers, offset, dtype_code(dtype))


def paged_attention(out, q, slab_table, block_table, *, b, h, nq, nk, d, page_size,
                    pages_per_slab, num_slabs, columns, layer, layers, offset, dtype):
    """``mt_paged_attention`` (reference src/paged_attention_kernel.cu:108-117)."""
    call(paged_library(), 'mt_paged_attention', [P] * 4 + [I] * 13,
         out, q, slab_table, block_table, b, h, nq, nk, d, page_size, pages_per_slab,
         num_slabs, columns, layer, layers, offset, dtype_code(dtype))


def paged_prefill(out, q, k, v, slab_table, block_table, *, b, h, n, d, page_size, pages_per_slab,
                  num_slabs, columns, layer, layers, offset, dtype, qkv_stride=0, out_stride=0):
    """``mt_paged_prefill``: append + causal attention of n tokens per request
    over token-major rows (q/k/v [b, n, qkv_stride], out [b, n, out_stride])."""
    call(paged_library(), 'mt_paged_prefill', [P] * 6 + [I] * 14,
         out, q, k, v, slab_table, block_table, b, h, n, d, page_size, pages_per_slab, num_slabs,
         columns, layer, layers, offset, dtype_code(dtype), qkv_stride, out_stride)


def paged_prefill_ragged(out, q, k, v, slab_table, tables, tokens, offsets, *, h, d, page_size, pages_per_slab,
                         num_slabs, columns, layer, layers, dtype, qkv_stride=0, out_stride=0):
    """``mt_paged_prefill_ragged``: ``paged_prefill`` for prompts of different
    lengths in one call; ``tables`` (device pointers to each prompt's table
    row), ``tokens`` and ``offsets`` are per prompt, rows token-major and
    concatenated in prompt order."""
    r = len(tokens)
    if not (len(tables) == len(offsets) == r):
        raise ValueError('tables, tokens and offsets need one entry per prompt')
    call(paged_library(), 'mt_paged_prefill_ragged', [P] * 8 + [I] * 12,
         out, q, k, v, slab_table, (P * r)(*tables), (I * r)(*tokens), (I * r)(*offsets), r, h, d,
         page_size, pages_per_slab, num_slabs, columns, layer, layers, dtype_code(dtype), qkv_stride, out_stride)


def paged_decode_batch(out, q, k, v, slab_table, block_table, offsets, *, b, h, d, page_size,
                       pages_per_slab, num_slabs, columns, layer, layers, dtype):
    """``mt_paged_decode_batch`` (reference src/paged_attention_kernel.cu:121-137)."""
    call(paged_library(), 'mt_paged_decode_batch', [P] * 7 + [I] * 10,
         out, q, k, v, slab_table, block_table, offsets, b, h, d, page_size, pages_per_slab,
         num_slabs, columns, layer, layers, dtype_code(dtype))


@lru_cache(maxsize=4096)
def decode_workspace_bytes(*, b, h, page_size, columns, split_tokens=0):
    """Workspace size for ``mt_paged_decode_split`` (0 when no row can split);
    a pure function of its arguments, memoized."""
    out = ct.c_size_t()
    call(paged_library(), 'mt_paged_decode_workspace_bytes', [I] * 5 + [ct.POINTER(ct.c_size_t)],
         b, h, page_size, columns, split_tokens, ct.byref(out))
    return out.value


@lru_cache(maxsize=4096)
def split_tokens_for(*, page_size, columns, requested=0):
    """Split length the decode uses for a table of ``columns`` pages; a pure
    function of its arguments, memoized."""
    out = ct.c_int()
    call(paged_library(), 'mt_paged_decode_split_tokens', [I, I, I, ct.POINTER(ct.c_int)],
         page_size, columns, requested, ct.byref(out))
    return out.value


def paged_decode_order(offsets, *, b, h, page_size, columns, list_out, count_out, split_tokens=0,
                       compute_units=0):
    """``mt_paged_decode_order``: the work list of :func:`decode_work_list`
    built on the device from the device ``offsets`` (what
    ``mt_paged_decode_batch`` does for batches it does not rank in-kernel)."""
    call(paged_library(), 'mt_paged_decode_order', [P, I, I, I, I, I, I, P, P],
         offsets, b, h, page_size, columns, split_tokens, compute_units, list_out, count_out)


SPLIT_ARGTYPES = [P] * 7 + [I] * 14 + [P, I, I, P, Z]


def paged_decode_split(out, q, k, v, slab_table, block_table, offsets, *, b, h, d, page_size,
                       pages_per_slab, num_slabs, columns, layer, layers, dtype,
                       split_tokens=0, unroll=0, waves=0, qkv_stride=0, work=None, work_items=0,
                       merge_rows=0, workspace=None, workspace_bytes=0):
    """``mt_paged_decode_split``: the decode of ``mt_paged_decode_batch`` with a
    caller-owned workspace, an explicit split length (0 = automatic), stream
    unroll and waves per workgroup (0 = defaults), the row stride of q/k/v
    (0 = contiguous) and an optional device work list from
    :func:`decode_work_list`."""
    call(paged_library(), 'mt_paged_decode_split', SPLIT_ARGTYPES,
         out, q, k, v, slab_table, block_table, offsets, b, h, d, page_size, pages_per_slab,
         num_slabs, columns, layer, layers, dtype_code(dtype), split_tokens, unroll, waves,
         qkv_stride, work, work_items, merge_rows, workspace, workspace_bytes)


def decode_work_list(lengths, heads, split_tokens, compute_units):
    """Work list for ``mt_paged_decode_split``: returns (int32 array,
    work_items, merge_rows).

    Every (row, split) of contexts ``lengths`` (keys attended, new token
    included) is one entry of ``heads`` workgroups. Entries are ordered by
    their token count, longest first (LPT), and every other dispatch pass of
    ``compute_units`` workgroups is reversed, so a compute unit that received
    one of the longest entries in one pass receives one of the shorter
    entries of the next ("snake" order). The rows with more than one split
    follow the pairs.
    """
    if len(lengths) <= 32 and all(0 < int(n) <= split_tokens for n in lengths):
        # one split per row (the common small decode batch): the same list in
        # plain Python, cheaper than numpy at this size
        return _small_work_list([int(n) for n in lengths], heads, compute_units)
    return _numpy_work_list(lengths, heads, split_tokens, compute_units)


def _numpy_work_list(lengths, heads, split_tokens, compute_units):
    L = np.asarray(lengths, np.int64)
    nsplit = np.maximum(1, -(-L // split_tokens))
    rows = np.repeat(np.arange(len(L)), nsplit)
    first = np.repeat(np.cumsum(nsplit) - nsplit, nsplit)
    splits = np.arange(len(rows)) - first
    tokens = np.clip(L[rows] - splits * split_tokens, 0, split_tokens)
    lpt = np.lexsort((rows, -tokens))
    per = max(1, compute_units // max(1, heads))
    passes = [lpt[i:i + per] for i in range(0, len(lpt), per)]
    order = np.concatenate([p if k % 2 == 0 else p[::-1] for k, p in enumerate(passes)])
    merge = np.flatnonzero(nsplit > 1)
    work = np.concatenate([np.stack([rows[order], splits[order]], 1).ravel(), merge])
    return work.astype(np.int32), len(order), len(merge)


def _small_work_list(lengths, heads, compute_units):
    """decode_work_list for rows of one split each: rows longest first
    (stable, ties by row), every other pass of compute_units // heads rows
    reversed; no merge rows."""
    lpt = sorted(range(len(lengths)), key=lambda r: -lengths[r])
    per = max(1, compute_units // max(1, heads))
    order = []
    for k, i in enumerate(range(0, len(lpt), per)):
        chunk = lpt[i:i + per]
        order += chunk[::-1] if k % 2 else chunk
    work = np.empty(2 * len(order), np.int32)
    work[0::2] = order
    work[1::2] = 0
    return work, len(order), 0


def embedding_gather(dst, weights, ids, tokens, vocab, dim):
    """``mt_embedding_gather`` (reference src/inference_kernels.cu:15-19)."""
    call(inference_library(), 'mt_embedding_gather', [P, P, P, I, I, I],
         dst, weights, ids, tokens, vocab, dim)


def row_argmax(dst, src, rows, width, dtype):
    """``mt_row_argmax`` (reference src/inference_kernels.cu:73-79)."""
    call(inference_library(), 'mt_row_argmax', [P, P, I, I, I], dst, src, rows, width,
         dtype_code(dtype))


def row_argmax_feedback(dst, slot_tokens, slots, num_slots, src, rows, width, dtype):
    """``mt_row_argmax_feedback``: ``row_argmax`` that also stores each row's
    token in ``slot_tokens[slots[r]]`` (the device-side token feedback of the
    sync-free decode loop)."""
    call(inference_library(), 'mt_row_argmax_feedback', [P, P, P, I, P, I, I, I], dst, slot_tokens,
         slots, num_slots, src, rows, width, dtype_code(dtype))


def row_argmax_commit(dst, slot_tokens, slots, num_slots, slot_len, tokens, src, rows, width, dtype):
    """``mt_row_argmax_commit``: ``row_argmax_feedback`` that also adds
    ``tokens`` to each row's committed length ``slot_len[slots[r]]`` (the
    decode step's commit in the same launch)."""
    call(inference_library(), 'mt_row_argmax_commit', [P, P, P, I, P, I, P, I, I, I], dst, slot_tokens,
         slots, num_slots, slot_len, tokens, src, rows, width, dtype_code(dtype))


def gather_slot_tokens(ids, slot_tokens, slots, num_slots, rows):
    """``mt_gather_slot_tokens``: ``ids[r] = slot_tokens[slots[r]]`` (NaN for a
    slot outside the table)."""
    call(inference_library(), 'mt_gather_slot_tokens', [P, P, P, I, I], ids, slot_tokens, slots,
         num_slots, rows)


def embed_tokens(x, wte, wpe, ids, positions, tokens, vocab, n_positions, dim, *, slot_tokens=None,
                 slots=None, num_slots=0):
    """``mt_embed_tokens``: ``x = wte[id] + wpe[position]`` per token, the ids
    from ``ids`` or, with ``slot_tokens``, from the pool's per-slot last tokens."""
    call(inference_library(), 'mt_embed_tokens', [P, P, P, P, P, P, I, P, I, I, I, I], x, wte, wpe, ids,
         slot_tokens, slots, num_slots, positions, tokens, vocab, n_positions, dim)


def last_row(dst, src, b, n, w, dtype):
    """``mt_last_row`` (reference src/inference_kernels.cu:66-72)."""
    call(inference_library(), 'mt_last_row', [P, P, I, I, I, I], dst, src, b, n, w,
         dtype_code(dtype))
