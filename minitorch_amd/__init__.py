"""MI355X-native paged-KV continuous-batching decode path with MiniTorch's API.

The compute runs in hand-written HIP kernels for gfx950 behind a C-ABI
(``include/*.h``), loaded with ctypes exactly as the reference loads its
``.so`` files. Python holds the host-side mirror of the reference's
interfaces: ``KVPagePool``, ``PagedKVCache``, ``PagedDecodeBatch``,
``greedy_token`` and ``ContinuousBatcher``.
"""
from .dtypes import normalize_dtype, dtype_code, itemsize, encode_host, decode_host
from .runtime import runtime, RawDeviceBuffer, DeviceTensor, CudaEvent, call, pointer, P, I, F

__all__ = [
    'normalize_dtype', 'dtype_code', 'itemsize', 'encode_host', 'decode_host',
    'runtime', 'RawDeviceBuffer', 'DeviceTensor', 'CudaEvent', 'call', 'pointer', 'P', 'I', 'F',
]
