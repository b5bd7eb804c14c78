"""The C-ABI libraries load here (no GPU), export every symbol their header
declares, and reject the shapes the reference rejects before any device work.
"""
import ctypes as ct
import re
import subprocess
from pathlib import Path

import pytest

from minitorch_amd.runtime import library, P, I, Z

ROOT = Path(__file__).resolve().parents[1]
HEADERS = {
    'mt_paged.h': 'paged_attention_kernel',
    'mt_inference.h': 'inference_kernels',
    'mt_runtime.h': 'cuda_runtime',
    'mt_sched.h': 'sched_kernels',
    'mt_model.h': 'model_kernels',
}


def declared(header):
    text = (ROOT / 'include' / header).read_text()
    return re.findall(r'^\s*(?:int|const char\*|size_t)\s+(mt_\w+)\s*\(', text, re.M)


@pytest.mark.parametrize('header', sorted(HEADERS))
def test_header_symbols_exported(header):
    path = ROOT / 'include' / header
    if not path.exists():
        pytest.skip(f'{header} not present')
    names = declared(header)
    assert names, header
    lib = library(HEADERS[header])
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f'{HEADERS[header]}.so lacks {missing}'


def test_headers_compile_as_c_and_cpp():
    for header in sorted((ROOT / 'include').glob('*.h')):
        for lang in ('c', 'c++'):
            r = subprocess.run(['gcc', '-x', lang, '-fsyntax-only', '-Wall', '-Werror', str(header)],
                               capture_output=True, text=True)
            assert r.returncode == 0, r.stderr


def _decode_batch(**overrides):
    lib = library('paged_attention_kernel')
    f = lib.mt_paged_decode_batch
    f.argtypes, f.restype = [P] * 7 + [I] * 10, I
    args = dict(out=8, q=8, k=8, v=8, slabs=8, table=8, offsets=8, b=4, h=12, d=64, page_size=16,
                pps=4, num_slabs=16, columns=8, layer=0, layers=1, dtype=0)
    args.update(overrides)
    return f(*args.values())


@pytest.mark.parametrize('bad', [
    dict(b=0), dict(h=0), dict(d=0), dict(d=129), dict(page_size=12), dict(page_size=64),
    dict(pps=0), dict(num_slabs=0), dict(columns=0), dict(layer=1), dict(layer=-1),
    dict(layers=0), dict(b=65536, h=1), dict(b=300, h=300), dict(dtype=3), dict(dtype=-1),
    dict(out=None), dict(offsets=None), dict(table=None),
    dict(pps=2 ** 30, num_slabs=4), dict(b=2 ** 16 - 1, h=1, columns=2 ** 16),
])
def test_decode_rejects_invalid_shapes(bad):
    assert _decode_batch(**bad) == 1


def test_append_and_attention_reject_invalid_shapes():
    lib = library('paged_attention_kernel')
    app = lib.mt_paged_append
    app.argtypes, app.restype = [P] * 4 + [I] * 12, I
    base = [8, 8, 8, 8, 2, 3, 5, 64, 16, 4, 4, 4, 0, 1, 0, 0]
    bad_offset = list(base)
    bad_offset[14] = -1
    assert app(*bad_offset) == 1                      # offset < 0
    too_long = list(base)
    too_long[14] = 60                                  # offset + n > columns * P
    assert app(*too_long) == 1
    att = lib.mt_paged_attention
    att.argtypes, att.restype = [P] * 4 + [I] * 13, I
    # nq + offset != nk
    assert att(8, 8, 8, 8, 2, 3, 5, 6, 64, 16, 4, 4, 4, 0, 1, 0, 0) == 1
    # nk beyond the table
    assert att(8, 8, 8, 8, 2, 3, 5, 70, 64, 16, 4, 4, 4, 0, 1, 65, 0) == 1


def test_split_entry_validation_and_workspace_size():
    lib = library('paged_attention_kernel')
    ws = lib.mt_paged_decode_workspace_bytes
    ws.argtypes, ws.restype = [I] * 5 + [ct.POINTER(ct.c_size_t)], I
    out = ct.c_size_t()
    assert ws(64, 12, 16, 128, 0, ct.byref(out)) == 0
    # 2048-token table, automatic 1024-token splits: (max, denominator, 128
    # accumulators) per (row, head, split)
    assert out.value == 768 * 2 * 130 * 4
    assert ws(64, 12, 16, 64, 256, ct.byref(out)) == 0 and out.value == 768 * 4 * 130 * 4
    assert ws(64, 12, 16, 64, 0, ct.byref(out)) == 0 and out.value == 0   # cap 1024: one split
    assert ws(64, 12, 16, 64, 100, ct.byref(out)) == 1                     # not a multiple of 64
    assert ws(64, 12, 16, 64, 4096, ct.byref(out)) == 1                    # beyond 2048
    assert ws(64, 12, 12, 64, 0, ct.byref(out)) == 1                       # page size
    st = lib.mt_paged_decode_split_tokens
    st.argtypes, st.restype = [I, I, I, ct.POINTER(ct.c_int)], I
    s = ct.c_int()
    assert st(16, 64, 0, ct.byref(s)) == 0 and s.value == 1024
    assert st(16, 1024, 0, ct.byref(s)) == 0 and s.value == 2048        # 16384 tokens: 8 splits of 2048
    assert st(16, 100, 0, ct.byref(s)) == 0 and s.value == 1024
    assert st(8, 64, 256, ct.byref(s)) == 0 and s.value == 256
    assert st(16, 64, 96, ct.byref(s)) == 1                             # not a multiple of 64
    split = lib.mt_paged_decode_split
    split.argtypes, split.restype = [P] * 7 + [I] * 14 + [P, I, I, P, Z], I
    common = (8, 8, 8, 8, 8, 8, 8, 4, 12, 64, 16, 4, 16)
    # a splitting launch without a workspace is rejected
    assert split(*common, 128, 0, 1, 0, 0, 0, 0, 0, None, 0, 0, None, 0) == 1
    # waves must be 4 or 8
    assert split(*common, 64, 0, 1, 0, 0, 0, 6, 0, None, 0, 0, None, 0) == 1
    # a work list needs an explicit split length and counts within the batch
    assert split(*common, 64, 0, 1, 0, 0, 0, 0, 0, 8, 4, 0, None, 0) == 1
    assert split(*common, 64, 0, 1, 0, 1024, 0, 0, 0, 8, 5, 0, None, 0) == 1   # 5 > 4 rows x 1 split
    assert split(*common, 64, 0, 1, 0, 1024, 0, 0, 0, 8, 4, 5, None, 0) == 1   # 5 merge rows > 4
    assert split(*common, 64, 0, 1, 0, 1024, 0, 0, 0, 8, -1, 0, None, 0) == 1
    # q/k/v row stride below h*d is rejected
    assert split(*common, 64, 0, 1, 0, 0, 0, 0, 700, None, 0, 0, None, 0) == 1
    # an empty work list launches nothing
    assert split(*common, 64, 0, 1, 0, 1024, 0, 0, 0, 8, 0, 0, None, 0) == 0


def test_order_entry_rejects_invalid_arguments():
    # mt_paged_decode_order refuses before any launch: batch outside
    # 1..2048, no heads, page size, split length, negative compute units,
    # null pointers
    f = library('paged_attention_kernel').mt_paged_decode_order
    f.argtypes, f.restype = [P, I, I, I, I, I, I, P, P], I
    ok = (8, 4, 12, 16, 64, 0, 0, 8, 8)
    for i, bad in [(1, 0), (1, 2049), (2, 0), (3, 12), (4, 0), (5, 96), (5, 4096), (6, -1),
                   (0, None), (7, None), (8, None)]:
        args = list(ok)
        args[i] = bad
        assert f(*args) == 1, (i, bad)


def test_inference_entries_reject_invalid_shapes():
    lib = library('inference_kernels')
    g = lib.mt_embedding_gather
    g.argtypes, g.restype = [P, P, P, I, I, I], I
    assert g(8, 8, 8, 0, 10, 4) == 1
    assert g(8, 8, 8, 1, 0, 4) == 1
    assert g(8, 8, 8, 2 ** 20, 10, 2 ** 12) == 1
    a = lib.mt_row_argmax
    a.argtypes, a.restype = [P, P, I, I, I], I
    assert a(8, 8, 1, 2 ** 24 + 1, 0) == 1
    assert a(8, 8, 0, 10, 0) == 1
    assert a(8, 8, 1, 10, 5) == 1
    lr = lib.mt_last_row
    lr.argtypes, lr.restype = [P, P, I, I, I, I], I
    assert lr(8, 8, 0, 1, 1, 0) == 1
    assert lr(8, 8, 1, 1, 1, 7) == 1


def test_error_strings():
    lib = library('cuda_runtime')
    lib.mt_error.argtypes, lib.mt_error.restype = [I], ct.c_char_p
    assert lib.mt_error(0)
    assert lib.mt_error(1)


# The reference's CudaRuntime binds exactly these names from cuda_runtime.so
# (minitorch/cuda_storage.py:29-40), then mt_error (:41-42), and calls
# mt_blas_create at start-up (:43-45).
REFERENCE_RUNTIME_SIGNATURES = {
    'mt_malloc': [ct.POINTER(P), Z], 'mt_free': [P],
    'mt_copy': [P, P, Z, I], 'mt_sync': [], 'mt_fill': [P, I, ct.c_float],
    'mt_random': [P, I, ct.c_ulonglong], 'mt_one_hot': [P, P, I, I],
    'mt_sequence': [P, I, I], 'mt_blas_create': [ct.POINTER(P)],
    'mt_blas_destroy': [P], 'mt_gemm': [P, P, P, P, I, I, I],
    'mt_event_create': [ct.POINTER(P)], 'mt_event_record': [P],
    'mt_event_elapsed': [ct.POINTER(ct.c_float), P, P], 'mt_event_destroy': [P],
}


def test_runtime_binds_the_reference_signature_table():
    # The reference's binding loop, run against a fresh handle of this build's
    # cuda_runtime.so: every getattr succeeds and each symbol is a function of
    # this library (not only reachable through another one).
    lib = ct.CDLL(str(ROOT / 'minitorch_amd' / 'cuda_kernels' / 'cuda_runtime.so'))
    for name, args in REFERENCE_RUNTIME_SIGNATURES.items():
        f = getattr(lib, name)
        f.argtypes, f.restype = args, I
    lib.mt_error.argtypes, lib.mt_error.restype = [I], ct.c_char_p
    out = subprocess.run(['nm', '-D', '--defined-only',
                          str(ROOT / 'minitorch_amd' / 'cuda_kernels' / 'cuda_runtime.so')],
                         capture_output=True, text=True, check=True).stdout
    defined = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = sorted(set(REFERENCE_RUNTIME_SIGNATURES) - defined)
    assert not missing, missing


def test_runtime_generators_reject_invalid_arguments():
    # Host-side checks only (no launch reaches a device).
    lib = library('cuda_runtime')
    for name, args in REFERENCE_RUNTIME_SIGNATURES.items():
        f = getattr(lib, name)
        f.argtypes, f.restype = args, I
    assert lib.mt_random(None, -1, 0) == 1
    assert lib.mt_random(None, 4, 0) == 1
    assert lib.mt_one_hot(8, 8, -1, 3) == 1
    assert lib.mt_one_hot(8, 8, 6, 0) == 1
    assert lib.mt_one_hot(8, None, 6, 3) == 1
    assert lib.mt_sequence(8, -1, 0) == 1
    assert lib.mt_sequence(8, 4, -2) == 1
    assert lib.mt_sequence(None, 4, 2) == 1
    assert lib.mt_gemm(None, 8, 8, 8, 1, 1, 1) == 1


def test_paged_prefill_rejects_invalid_arguments():
    lib = library('paged_attention_kernel')
    f = lib.mt_paged_prefill
    f.argtypes, f.restype = [P] * 6 + [I] * 14, I
    ptrs = (8, 8, 8, 8, 8, 8)
    #       b  h  n  d   P   pps slabs cols layer layers offset dtype qkv_stride out_stride
    assert f(*ptrs, 2, 3, 5, 64, 16, 4, 4, 8, 0, 1, 0, 1, 100, 0) == 1      # qkv_stride < h*d
    assert f(*ptrs, 2, 3, 5, 64, 16, 4, 4, 8, 0, 1, 0, 1, 0, 100) == 1      # out_stride < h*d
    assert f(*ptrs, 2, 3, 5, 64, 12, 4, 4, 8, 0, 1, 0, 1, 0, 0) == 1        # page size
    assert f(*ptrs, 2, 3, 5, 64, 16, 4, 4, 8, 0, 1, 0, 3, 0, 0) == 1        # dtype
    assert f(*ptrs, 2, 3, 5, 64, 16, 4, 4, 8, 1, 1, 0, 1, 0, 0) == 1        # layer >= layers
    assert f(None, *ptrs[1:], 2, 3, 5, 64, 16, 4, 4, 8, 0, 1, 0, 1, 0, 0) == 1


def test_token_feedback_entries_reject_invalid_arguments():
    lib = library('inference_kernels')
    a = lib.mt_row_argmax_feedback
    a.argtypes, a.restype = [P, P, P, I, P, I, I, I], I
    assert a(8, 8, None, 4, 8, 1, 10, 0) == 1          # slot table without slots
    assert a(8, 8, 8, 0, 8, 1, 10, 0) == 1             # empty slot table
    assert a(8, None, None, 0, 8, 0, 10, 0) == 1       # no rows
    assert a(8, None, None, 0, 8, 1, 10, 3) == 1       # dtype
    assert a(None, None, None, 0, 8, 1, 10, 0) == 1
    g = lib.mt_gather_slot_tokens
    g.argtypes, g.restype = [P, P, P, I, I], I
    assert g(8, 8, 8, 4, 0) == 1
    assert g(8, 8, 8, 0, 1) == 1
    assert g(None, 8, 8, 4, 1) == 1
    c = lib.mt_row_argmax_commit
    c.argtypes, c.restype = [P, P, P, I, P, I, P, I, I, I], I
    assert c(8, None, None, 0, 8, 1, 8, 1, 10, 0) == 1  # a commit needs the slot table
    assert c(8, 8, None, 4, 8, 1, 8, 1, 10, 0) == 1     # slot table without slots
    assert c(8, 8, 8, 4, 8, 1, 8, 0, 10, 0) == 1        # no rows
    assert c(8, 8, 8, 4, 8, 1, 8, 1, 10, 5) == 1        # dtype


def test_fused_prepare_embed_rejects_invalid_arguments():
    # mt_sched_decode_prepare_embed refuses before any launch: pool geometry,
    # metadata arguments and the embedding's (null, unaligned, width not a
    # multiple of 4, no slot table or one longer than the pool's slots)
    f = library('sched_kernels').mt_sched_decode_prepare_embed
    f.argtypes, f.restype = [P, I, I, I, I, I, ct.c_uint64, ct.c_uint64] + [P, I, I, I, I, P, P, P, P, P,
                                                                        P, P, P, P, I, I, I, I], I
    # state at 256 (16-byte aligned); 16 slabs of 16 pages, 1024 slots of 16 columns
    pool = (256, 256, 16, 1024, 16, 16, 256, 4096)
    ok = [256, 2, 4, 16, -1, 256, 256, 256, 256, 256, 256, 256, 256, 256, 8, 100, 64, 64]
    # the valid shape passes validation (without a GPU the launch itself fails with another status)
    assert f(*pool, *ok) != 1
    for i, bad in [(1, 0), (2, 0), (2, 2000), (3, 12), (4, -2), (5, None), (10, None), (11, 8), (13, None),
                   (14, 0), (14, 1025), (15, 0), (16, 0), (17, 6), (17, 0)]:
        args = list(ok)
        args[i] = bad
        assert f(*pool, *args) == 1, (i, bad)
    assert f(None, *pool[1:], *ok) == 1


class _Layer(ct.Structure):
    # mt_decoder_layer (include/mt_model.h), the tiled weight copies last
    _fields_ = [(n, P) for n in ('ln1_gamma', 'ln1_beta', 'w_qkv', 'b_qkv', 'w_o', 'b_o',
                                 'ln2_gamma', 'ln2_beta', 'w_fc', 'b_fc', 'w_proj', 'b_proj',
                                 'w_qkv_tiled', 'w_o_tiled', 'w_fc_tiled', 'w_proj_tiled')]


class _Prefill(ct.Structure):
    _fields_ = [('slabs', P), ('table', P), ('page_size', I), ('pages_per_slab', I), ('num_slabs', I),
                ('columns', I), ('layers', I), ('offset', I)]


def test_prefill_layers_rejects_invalid_arguments():
    lib = library('model_kernels')
    f = lib.mt_prefill_layers
    f.argtypes = [P, P, I, P, P, P, P, P, P, I, I, I, I, I, ct.c_float, I, I, P, Z, P]
    f.restype = I
    layer = _Layer(*([8] * 12))
    att = _Prefill(8, 8, 16, 4, 4, 8, 1, 0)
    need = lib.mt_decoder_scratch_bytes
    need.argtypes, need.restype = [I, I, I], Z
    scratch = need(2 * 5, 64, 1)
    args = dict(handle=8, layers=ct.byref(layer), n_layer=1, x=8, h=8, fg=8, fb=8, head=8, logits=8, vocab=10,
                batch=2, n=5, d=64, heads=2, eps=1e-5, dtype=1, gelu=1, scratch=8, scratch_bytes=scratch,
                att=ct.byref(att))

    def call(**over):
        a = dict(args, **over)
        return f(*a.values())
    assert call(handle=None) == 1
    assert call(heads=3) == 1                     # d % heads
    assert call(scratch_bytes=scratch - 1) == 1   # scratch too small
    assert call(batch=0) == 1
    assert call(dtype=5) == 1
    assert call(logits=8, head=None) == 1         # logits need the head weight
    assert call(att=None) == 1


def test_ragged_prefill_entries_reject_invalid_arguments():
    # validation only: every call below returns before any device work
    lib = library('paged_attention_kernel')
    f = lib.mt_paged_prefill_ragged
    f.argtypes, f.restype = [P] * 8 + [I] * 12, I
    tables = (P * 2)(8, 8)

    def call(tokens=(5, 7), offsets=(0, 3), requests=2, h=3, d=64, page=16, dtype=1, qkv_stride=0,
             out_stride=0, tabs=tables, layer=0):
        return f(8, 8, 8, 8, 8, tabs, (I * 2)(*tokens), (I * 2)(*offsets), requests, h, d, page, 4, 4, 8,
                 layer, 1, dtype, qkv_stride, out_stride)
    assert call(tokens=(5, 0)) == 1             # an empty prompt
    assert call(offsets=(0, -1)) == 1           # negative offset
    assert call(tokens=(5, 200)) == 1           # beyond columns * page_size
    assert call(requests=0) == 1
    assert call(page=12) == 1
    assert call(dtype=3) == 1
    assert call(qkv_stride=100) == 1            # < h * d
    assert call(layer=1) == 1                   # layer >= layers
    assert call(tabs=(P * 2)(8, None)) == 1     # a null table row
    assert f(None, 8, 8, 8, 8, tables, (I * 2)(5, 7), (I * 2)(0, 0), 2, 3, 64, 16, 4, 4, 8, 0, 1, 1, 0, 0) == 1

    lib = library('model_kernels')
    g = lib.mt_prefill_layers_ragged
    g.argtypes = [P, P, I, P, P, P, P, P, P, I, I, P, I, I, ct.c_float, I, I, P, Z, P]
    g.restype = I
    layer = _Layer(*([8] * 12))
    atts = (_Prefill * 2)(_Prefill(8, 8, 16, 4, 4, 8, 1, 0), _Prefill(8, 8, 16, 4, 4, 8, 1, 0))
    need = lib.mt_decoder_scratch_bytes
    need.argtypes, need.restype = [I, I, I], Z
    scratch = need(12, 64, 1)

    def layers_call(tokens=(5, 7), requests=2, scratch_bytes=scratch, heads=2, att=atts):
        return g(8, ct.byref(layer), 1, 8, 8, 8, 8, 8, 8, 10, requests, (I * 2)(*tokens), 64, heads, 1e-5, 1, 1,
                 8, scratch_bytes, att)
    assert layers_call(tokens=(5, 0)) == 1            # an empty prompt
    assert layers_call(scratch_bytes=scratch - 1) == 1
    assert layers_call(heads=3) == 1                  # d % heads
    assert layers_call(requests=0) == 1
    assert layers_call(att=None) == 1
    other = (_Prefill * 2)(_Prefill(8, 8, 16, 4, 4, 8, 1, 0), _Prefill(8, 8, 32, 4, 4, 8, 1, 0))
    assert layers_call(att=other) == 1                # prompts of different pools


def test_decode_projection_entries_reject_invalid_arguments():
    # Host-side validation of the decode projection entries (16-byte aligned
    # stand-in pointers that are never dereferenced: every call is invalid).
    lib = library('model_kernels')
    pr = lib.mt_decode_projection
    pr.argtypes, pr.restype = [P, P, P, P, I, I, I, I, I, I, I], I
    A = 256
    #          out x  w  bias  m    n     k    splits epi dtype layout
    for args in [(A, A, A, 0, 0, 1024, 1024, 1, 0, 2, 0),      # no rows
                 (A, A, A, 0, 257, 1024, 1024, 1, 0, 2, 0),    # more rows than the kernel takes
                 (A, A, A, 0, 4, 40, 1024, 1, 0, 2, 0),        # n not a multiple of 16
                 (A, A, A, 0, 4, 1024, 100, 1, 0, 2, 0),       # k not a multiple of 32
                 (A, A, A, 0, 4, 1024, 1024, 3, 2, 2, 0),      # splits not a power of two
                 (A, A, A, 0, 4, 1024, 1024, 2, 0, 2, 0),      # a split needs the partial-sum epilogue
                 (A, A, A, 0, 4, 1024, 1024, 1, 0, 0, 0),      # fp32
                 (A, A + 2, A, 0, 4, 1024, 1024, 1, 0, 2, 0),  # misaligned activations
                 (None, A, A, 0, 4, 1024, 1024, 1, 0, 2, 0),
                 (A, A, A, 0, 4, 1024, 1024, 2, 2, 2, 2),      # split partials are written row-major
                 (A, A, A, 0, 4, 48, 1024, 1, 0, 2, 2),        # a tiled output needs n a multiple of 32
                 (A, A, A, 0, 4, 1024, 1024, 1, 0, 2, 8)]:     # no such layout bit
        assert pr(*args) == 1, args
    ln = lib.mt_decode_projection_ln
    ln.argtypes, ln.restype = [P, P, P, P, I, P, P, P, ct.c_float, P, P, I, I, I, I, I, I], I
    #          out x_in x_out part splits pbias gamma beta eps w bias m n k epi dtype layout
    for args in [(A, A, A, A, 4, 0, A, A, 1e-5, A, 0, 4, 1024, 1024, 0, 2, 0),          # x_out is x_in
                 (A, A, 2 * A, A, 4, 0, A, A, 1e-5, A, 0, 4, 1024, 1280, 0, 2, 0),      # k above 1024
                 (A, A, 2 * A, A, 3, 0, A, A, 1e-5, A, 0, 4, 1024, 1024, 0, 2, 0),      # 3 partial splits
                 (A, A, 2 * A, 0, 4, 0, A, A, 1e-5, A, 0, 4, 1024, 1024, 0, 2, 0),      # splits without partials
                 (A, A, 2 * A, 0, 0, A, A, A, 1e-5, A, 0, 4, 1024, 1024, 0, 2, 0),      # a bias without partials
                 (A, A, 2 * A, A, 4, 0, A, A, 1e-5, A, 0, 17, 1024, 1024, 0, 2, 0),     # more than 16 rows
                 (A, A, 2 * A, A, 4, 0, A, A, 1e-5, A, 0, 4, 1024, 1024, 2, 2, 0),      # partial-sum epilogue
                 (A, A, 2 * A, A, 4, 0, A, A, 1e-5, A, 0, 4, 1024, 1024, 0, 2, 1)]:     # only the weights may be tiled
        assert ln(*args) == 1, args
    rp = lib.mt_residual_layernorm_partials
    rp.argtypes, rp.restype = [P, P, P, I, P, P, P, I, I, ct.c_float, I, I], I
    for args in [(A, A, A, 1, 0, A, A, 4, 1000, 1e-5, 2, 0),   # width not a multiple of 256
                 (A, A, A, 9, 0, A, A, 4, 1024, 1e-5, 2, 0),   # more than 8 splits
                 (A, A, A, 1, 0, A, A, 4, 1024, 1e-5, 0, 0),   # fp32
                 (A, A, A, 1, 0, A, A, 0, 1024, 1e-5, 2, 0),   # no rows
                 (A, A, A, 1, 0, A, A, 4, 0, 1e-5, 2, 0),      # zero width
                 (A, A, A, 1, 0, A, A, 4, -256, 1e-5, 2, 0),   # negative width (a multiple of 256)
                 (A, A, A, 1, 0, A, A, 4, -2048, 1e-5, 2, 0),
                 (A, A, A, 1, 0, A, A, 4, 1024, 1e-5, 2, 1)]:  # layout 1 (a tiled input) is not taken
        assert rp(*args) == 1, args


class _DecodeAtt(ct.Structure):
    _fields_ = [('slabs', P), ('table', P), ('offsets', P), ('page_size', I), ('pages_per_slab', I),
                ('num_slabs', I), ('columns', I), ('layers', I), ('split_tokens', I), ('work', P),
                ('work_items', I), ('merge_rows', I), ('partials', P), ('partial_bytes', Z)]


def test_mixed_layers_and_batched_pool_entries_reject_invalid_arguments():
    # validation only: every call below returns before any device work
    lib = library('model_kernels')
    g = lib.mt_mixed_layers
    g.argtypes = [P, P, I, P, P, P, P, P, P, I, I, I, P, I, I, ct.c_float, I, I, P, Z, P, P]
    g.restype = I
    layer = _Layer(*([8] * 12))
    need = lib.mt_decoder_scratch_bytes
    need.argtypes, need.restype = [I, I, I], Z
    scratch = need(3 + 12, 64, 1)
    datt = _DecodeAtt(8, 8, 8, 16, 4, 4, 8, 1, 1024, 8, 3, 0, 8, 1024)
    atts = (_Prefill * 2)(_Prefill(8, 8, 16, 4, 4, 8, 1, 0), _Prefill(8, 8, 16, 4, 4, 8, 1, 0))

    def call(decode_rows=3, tokens=(5, 7), requests=2, scratch_bytes=scratch, heads=2, d_att=datt, att=atts):
        return g(8, ct.byref(layer), 1, 8, 8, 8, 8, 8, 8, 10, decode_rows, requests, (I * 2)(*tokens), 64, heads,
                 1e-5, 1, 1, 8, scratch_bytes, None if d_att is None else ct.byref(d_att), att)
    assert call(decode_rows=0) == 1
    assert call(decode_rows=65535) == 1             # more decode rows than the head gather takes
    assert call(tokens=(5, 0)) == 1                 # an empty prompt
    assert call(requests=0) == 1
    assert call(scratch_bytes=scratch - 1) == 1
    assert call(heads=3) == 1                       # d % heads
    assert call(d_att=None) == 1
    assert call(att=None) == 1
    other = _DecodeAtt(8, 8, 8, 32, 4, 4, 8, 1, 1024, 8, 3, 0, 8, 1024)
    assert call(d_att=other) == 1                   # decode rows and prompts on different pools

    sched = library('sched_kernels')
    geometry = [P, I, I, I, I, I, ct.c_ulonglong, ct.c_ulonglong]
    acquire = sched.mt_pool_acquire_lists
    acquire.argtypes, acquire.restype = geometry + [P, P, I, P], I
    lengths = sched.mt_sched_add_lengths
    lengths.argtypes, lengths.restype = geometry + [P, P, I], I
    pool = (8, 16, 4, 16, 4, 4, 8, 1 << 20)
    assert acquire(*pool, 8, 8, 0, 8) == 1           # no cache
    assert acquire(*pool, None, 8, 2, 8) == 1
    assert acquire(*pool, 8, 8, 2, None) == 1        # no scratch
    assert acquire(8, 16, 4, 16, 4, 5, 8, 1 << 20, 8, 8, 2, 8) == 1   # slabs * pages_per_slab != pages
    assert lengths(*pool, 8, 8, 0) == 1
    assert lengths(*pool, 8, None, 2) == 1
