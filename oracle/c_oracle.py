"""ctypes loader for the C restatement (oracle/paged_oracle.c). TEST INFRASTRUCTURE ONLY.

Used by tests as a second checker and by bench.py as the reported CPU
baseline (kind "port").
"""
import ctypes as ct
import subprocess
from pathlib import Path
import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / '_build' / 'liboracle_paged.so'
CODES = {'float32': 0, 'float16': 1, 'bfloat16': 2}


def build():
    subprocess.run(['make', '-s', '-C', str(HERE)], check=True)
    return LIB


def library():
    if not LIB.exists():
        raise RuntimeError(f'{LIB} is not built; run `make -C oracle`')
    lib = ct.CDLL(str(LIB))
    P, I = ct.c_void_p, ct.c_int
    lib.oracle_paged_decode_batch.argtypes = [P] * 7 + [I] * 11
    lib.oracle_paged_decode_batch.restype = I
    lib.oracle_paged_attention.argtypes = [P] * 4 + [I] * 14
    lib.oracle_paged_attention.restype = I
    lib.oracle_max_threads.argtypes = []
    lib.oracle_max_threads.restype = I
    return lib


class HostCase:
    """Host buffers of a PagedDecodeCase for the C oracle (image copied so the
    append can be repeated from the original state)."""

    def __init__(self, case):
        self.case = case
        self.image = np.ascontiguousarray(case.image.copy())
        c = case
        base = self.image.ctypes.data
        self.slabs = np.array([base + s * c.slab_bytes for s in range(c.num_slabs)], np.uint64)
        self.table = np.ascontiguousarray(c.table, np.int32)
        self.offsets = np.ascontiguousarray(c.offsets, np.int32)
        self.q, self.k, self.v = (np.ascontiguousarray(x) for x in (c.q, c.k, c.v))
        self.out = np.zeros_like(self.q)

    def run(self, lib, threads=0):
        c = self.case
        status = lib.oracle_paged_decode_batch(
            self.out.ctypes.data, self.q.ctypes.data, self.k.ctypes.data, self.v.ctypes.data,
            self.slabs.ctypes.data, self.table.ctypes.data, self.offsets.ctypes.data,
            c.batch, c.heads, c.dim, c.page_size, c.pages_per_slab, c.num_slabs, c.columns,
            c.layer, c.layers, CODES[c.dtype], threads)
        if status:
            raise RuntimeError(f'oracle_paged_decode_batch returned {status}')
        return self.out


def paged_attention(lib, case, q, nq, nk, offset, image=None, threads=0):
    """Causal attention of q [B, H, nq, D] (stored values) over the pages of
    ``case`` (or of ``image``, an image of the same shape) through
    oracle_paged_attention; returns the output in storage format."""
    c = case
    image = np.ascontiguousarray(c.image if image is None else image)
    base = image.ctypes.data
    slabs = np.array([base + s * c.slab_bytes for s in range(c.num_slabs)], np.uint64)
    table = np.ascontiguousarray(c.table, np.int32)
    q = np.ascontiguousarray(q)
    out = np.zeros_like(q)
    status = lib.oracle_paged_attention(out.ctypes.data, q.ctypes.data, slabs.ctypes.data, table.ctypes.data,
                                        c.batch, c.heads, nq, nk, c.dim, c.page_size, c.pages_per_slab,
                                        c.num_slabs, c.columns, c.layer, c.layers, offset, CODES[c.dtype],
                                        threads)
    if status:
        raise RuntimeError(f'oracle_paged_attention returned {status}')
    return out
