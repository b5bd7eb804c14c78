"""Precision context for caches (reference minitorch/amp.py:15-28).

``autocast('float16'|'bfloat16')`` selects the KV cache element type and the
model's GEMM input type inside the block; outside it the path is fp32.
"""
from contextlib import contextmanager
from contextvars import ContextVar
from .dtypes import normalize_dtype

_dtype = ContextVar('minitorch_amd_autocast', default=None)


def autocast_dtype():
    return _dtype.get()


@contextmanager
def autocast(dtype='float16', enabled=True):
    token = _dtype.set(normalize_dtype(dtype) if enabled else None)
    try:
        yield
    finally:
        _dtype.reset(token)
