"""Element types and bf16 host transport.

Names and codes are the reference's (minitorch/dtypes.py:7-11): float32 = 0,
float16 = 1, bfloat16 = 2. bfloat16 travels host<->device as uint16 bit
patterns with round-to-nearest-even and quiet NaNs (minitorch/dtypes.py:37-51).
"""
import numpy as np

FLOAT32 = 'float32'
FLOAT16 = 'float16'
BFLOAT16 = 'bfloat16'
INT32 = 'int32'
_CODES = {FLOAT32: 0, FLOAT16: 1, BFLOAT16: 2}
_ITEMSIZE = {FLOAT32: 4, FLOAT16: 2, BFLOAT16: 2, INT32: 4}


def normalize_dtype(dtype):
    name = dtype if isinstance(dtype, str) else np.dtype(dtype).name
    if name not in _ITEMSIZE:
        raise ValueError(f'Unsupported dtype {dtype!r}; use float32, float16, bfloat16 or int32')
    return name


def dtype_code(dtype):
    name = normalize_dtype(dtype)
    if name not in _CODES:
        raise ValueError(f'{name} has no floating-point dtype code')
    return _CODES[name]


def itemsize(dtype):
    return _ITEMSIZE[normalize_dtype(dtype)]


def encode_host(value, dtype):
    """Host array in the device storage layout of ``dtype`` (flat)."""
    dtype = normalize_dtype(dtype)
    if dtype != BFLOAT16:
        return np.ascontiguousarray(value, dtype=dtype).reshape(-1)
    bits = np.ascontiguousarray(value, dtype=np.float32).reshape(-1).view(np.uint32)
    rounded = ((bits + np.uint32(0x7fff) + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = ((bits & 0x7f800000) == 0x7f800000) & ((bits & 0x007fffff) != 0)
    return np.where(nan, (bits >> 16).astype(np.uint16) | np.uint16(0x40), rounded).astype(np.uint16)


def decode_host(value, dtype):
    """Storage array -> numpy values (bf16 bits become float32)."""
    if normalize_dtype(dtype) == BFLOAT16:
        return (np.asarray(value).astype(np.uint32) << 16).view(np.float32)
    return value


def storage_numpy_dtype(dtype):
    dtype = normalize_dtype(dtype)
    return np.uint16 if dtype == BFLOAT16 else np.dtype(dtype)
