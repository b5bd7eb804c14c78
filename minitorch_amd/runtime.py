"""Device runtime over the C-ABI: library loading, buffers, typed device arrays.

Mirrors the reference's FFI layer (minitorch/cuda_storage.py:14-147,258-271;
minitorch/cuda_resident_ops.py:33-47): one device, one stream (the calling thread's default stream, where the libraries launch; the reference's legacy null stream), ctypes
``call(lib, name, argtypes, *args)`` that raises ``RuntimeError('CUDA: ...')``
on a nonzero status, byte buffers for metadata and slabs, and events.
Everything runs in ``cuda_kernels/*.so`` built from ``csrc/*.hip``; there is
no CPU fallback, so a missing library is an error.
"""
import ctypes as ct
from functools import lru_cache
from pathlib import Path
import weakref
import numpy as np
from .dtypes import normalize_dtype, itemsize, encode_host, decode_host, storage_numpy_dtype

LIB_DIR = Path(__file__).resolve().parent / 'cuda_kernels'
P, I, F, Z = ct.c_void_p, ct.c_int, ct.c_float, ct.c_size_t


@lru_cache(maxsize=None)
def library(name):
    """ctypes handle of ``cuda_kernels/<name>.so``; raises if it was not built."""
    path = LIB_DIR / f'{name}.so'
    try:
        return ct.CDLL(str(path))
    except OSError as error:
        raise RuntimeError(f'HIP library {path.name} is missing or failed to load; '
                           f'build it with `python -m minitorch_amd._build` ({error})') from error


class HipRuntime:
    """Loads ``cuda_runtime.so`` and keeps allocation/transfer counters."""

    def __init__(self):
        self.lib = library('cuda_runtime')
        self.stats = dict(active_bytes=0, peak_active_bytes=0, reserved_bytes=0,
                          peak_reserved_bytes=0, allocations=0, frees=0,
                          h2d_bytes=0, d2h_bytes=0, d2d_bytes=0)
        signatures = {
            'mt_malloc': [ct.POINTER(P), Z], 'mt_free': [P],
            'mt_copy': [P, P, Z, I], 'mt_copy_async': [P, P, Z, I], 'mt_sync': [],
            'mt_fill': [P, I, F], 'mt_fill_words': [P, Z, ct.c_uint],
            'mt_event_create': [ct.POINTER(P)], 'mt_event_record': [P],
            'mt_event_elapsed': [ct.POINTER(F), P, P], 'mt_event_destroy': [P],
            'mt_event_synchronize': [P], 'mt_event_query': [P],
            'mt_device_count': [ct.POINTER(I)], 'mt_compute_units': [ct.POINTER(I)],
            'mt_host_alloc': [ct.POINTER(P), Z], 'mt_host_free': [P],
            'mt_fill_random': [P, ct.c_longlong, ct.c_ulonglong, I],
            'mt_graph_begin': [], 'mt_graph_end': [ct.POINTER(P)], 'mt_graph_launch': [P],
            'mt_graph_destroy': [P],
        }
        for name, args in signatures.items():
            f = getattr(self.lib, name)
            f.argtypes, f.restype = args, I
        self.lib.mt_error.argtypes = [I]
        self.lib.mt_error.restype = ct.c_char_p
        self._staging = None

    def check(self, status):
        if status:
            raise RuntimeError(f'CUDA: {self.lib.mt_error(status).decode()}')

    def synchronize(self):
        self.check(self.lib.mt_sync())

    def compute_units(self):
        if getattr(self, '_compute_units', None) is None:
            n = I()
            self.check(self.lib.mt_compute_units(ct.byref(n)))
            self._compute_units = n.value
        return self._compute_units

    def malloc(self, nbytes):
        pointer = P()
        self.check(self.lib.mt_malloc(ct.byref(pointer), nbytes))
        s = self.stats
        s['allocations'] += 1
        s['active_bytes'] += nbytes
        s['reserved_bytes'] += nbytes
        s['peak_active_bytes'] = max(s['peak_active_bytes'], s['active_bytes'])
        s['peak_reserved_bytes'] = max(s['peak_reserved_bytes'], s['reserved_bytes'])
        return pointer

    def _free(self, pointer, nbytes):
        if self.lib.mt_free(pointer) == 0:
            self.stats['active_bytes'] -= nbytes
            self.stats['reserved_bytes'] -= nbytes
            self.stats['frees'] += 1

    def h2d(self, dst, array):
        """Copy a host array to device memory. Arrays up to STAGED_UPLOAD_BYTES
        are copied into pinned staging memory and uploaded asynchronously on
        the default stream (stream-ordered before any later launch or read-back),
        so a small upload does not wait for the work already queued; larger
        ones use a blocking copy."""
        a = np.ascontiguousarray(array)
        if a.nbytes <= STAGED_UPLOAD_BYTES:
            if self._staging is None:
                self._staging = _StagingRing()
            self._staging.upload(dst, a)
            return
        self.check(self.lib.mt_copy(dst, a.ctypes.data, a.nbytes, 1))
        self.stats['h2d_bytes'] += a.nbytes

    def d2h(self, out, src):
        self.check(self.lib.mt_copy(out.ctypes.data, src, out.nbytes, 2))
        self.stats['d2h_bytes'] += out.nbytes
        return out

    def d2d(self, dst, src, nbytes):
        self.check(self.lib.mt_copy(dst, src, nbytes, 3))
        self.stats['d2d_bytes'] += nbytes

    def snapshot(self):
        return dict(self.stats)


_runtime = None


def runtime():
    global _runtime
    if _runtime is None:
        _runtime = HipRuntime()
    return _runtime


def call(lib, name, signature, *args):
    """Call an ``int mt_*`` entry point and raise on a nonzero status
    (reference minitorch/cuda_resident_ops.py:41-44)."""
    f = getattr(lib, name)
    f.argtypes, f.restype = signature, I
    runtime().check(f(*args))


class RawDeviceBuffer:
    """Byte allocation for metadata and page slabs (reference
    minitorch/cuda_storage.py:112-147); closes idempotently."""

    def __init__(self, nbytes):
        if type(nbytes) is not int or nbytes < 1:
            raise ValueError('RawDeviceBuffer requires positive byte size')
        self.runtime = runtime()
        self.nbytes = nbytes
        self.pointer = self.runtime.malloc(nbytes)
        self._release = weakref.finalize(self, self.runtime._free, self.pointer, nbytes)

    @property
    def ptr(self):
        if not self._release.alive:
            raise ValueError('RawDeviceBuffer is closed')
        return self.pointer.value

    @property
    def closed(self):
        return not self._release.alive

    def upload(self, array, byte_offset=0):
        a = np.ascontiguousarray(array)
        if a.dtype.hasobject or type(byte_offset) is not int or byte_offset < 0 or byte_offset + a.nbytes > self.nbytes:
            raise ValueError('Invalid raw metadata upload')
        self.runtime.h2d(self.ptr + byte_offset, a)

    def download(self, dtype, count=None, byte_offset=0):
        dtype = np.dtype(dtype)
        count = (self.nbytes - byte_offset) // dtype.itemsize if count is None else count
        if byte_offset < 0 or byte_offset + count * dtype.itemsize > self.nbytes:
            raise ValueError('Invalid raw metadata download')
        return self.runtime.d2h(np.empty(count, dtype), self.ptr + byte_offset)

    def fill_words(self, value=0):
        self.runtime.check(self.runtime.lib.mt_fill_words(self.ptr, self.nbytes // 4, value))

    def close(self):
        self._release()


class CachingAllocator:
    """Reuses freed device blocks by size class instead of hipFree.

    hipFree synchronizes the device, so per-step tensors must not be freed to
    the driver. Blocks are rounded up to 256 bytes below 1 MiB and to powers of
    two above it (the reference's MemoryPool, minitorch/memory_pool.py:24-83,
    uses powers of two). On the single stream, a block released by the
    host may be reused at once: later kernels run after every kernel that used
    the block before.
    """

    def __init__(self, rt):
        self.runtime = rt
        self.free = {}
        self.cached_bytes = 0

    @staticmethod
    def size_class(nbytes):
        if nbytes <= 1 << 20:
            return max(256, (nbytes + 255) // 256 * 256)
        return 1 << (nbytes - 1).bit_length()

    def acquire(self, nbytes):
        size = self.size_class(nbytes)
        blocks = self.free.get(size)
        if blocks:
            self.cached_bytes -= size
            return blocks.pop(), size
        try:
            return self.runtime.malloc(size).value, size
        except RuntimeError:
            self.empty()  # out of memory: return cached blocks and retry once
            return self.runtime.malloc(size).value, size

    def release(self, pointer, size):
        self.free.setdefault(size, []).append(pointer)
        self.cached_bytes += size

    def empty(self):
        for size, blocks in self.free.items():
            for pointer in blocks:
                self.runtime._free(P(pointer), size)
        self.free.clear()
        self.cached_bytes = 0


class PooledBuffer:
    """Device bytes from the caching allocator, returned to it when dropped."""

    def __init__(self, nbytes):
        alloc = allocator()
        self.pointer, self.nbytes = alloc.acquire(nbytes)
        self._release = weakref.finalize(self, alloc.release, self.pointer, self.nbytes)

    @property
    def ptr(self):
        return self.pointer

    def download(self, dtype, count=None, byte_offset=0):
        dtype = np.dtype(dtype)
        count = (self.nbytes - byte_offset) // dtype.itemsize if count is None else count
        return runtime().d2h(np.empty(count, dtype), self.pointer + byte_offset)

    def fill_words(self, value=0):
        rt = runtime()
        rt.check(rt.lib.mt_fill_words(self.pointer, self.nbytes // 4, value))


_allocator = None


def allocator():
    global _allocator
    if _allocator is None:
        _allocator = CachingAllocator(runtime())
    return _allocator


STAGED_UPLOAD_BYTES = 1 << 16
HIP_ERROR_NOT_READY = 600


class _StagingRing:
    """Pinned staging buffers used round-robin by small uploads; a buffer is
    reused only after the upload that last read it has run."""

    def __init__(self, count=16):
        self.buffers = [PinnedHostBuffer(STAGED_UPLOAD_BYTES) for _ in range(count)]
        self.next = 0

    def upload(self, dst, array):
        buffer = self.buffers[self.next]
        self.next = (self.next + 1) % len(self.buffers)
        buffer.upload_async(dst, array)


class PinnedHostBuffer:
    """Pinned host staging memory for asynchronous host-to-device uploads."""

    def __init__(self, nbytes):
        self.runtime = runtime()
        self.nbytes = int(nbytes)
        self.pointer = P()
        self.runtime.check(self.runtime.lib.mt_host_alloc(ct.byref(self.pointer), self.nbytes))
        self._release = weakref.finalize(self, self.runtime.lib.mt_host_free, self.pointer)
        self.array = np.ctypeslib.as_array((ct.c_uint8 * self.nbytes).from_address(self.pointer.value))
        self._copied = None  # event recorded after the last enqueued upload

    def upload_async(self, dst, array):
        """Copy ``array`` into this staging buffer and enqueue its upload to ``dst``
        on the default stream. Before overwriting the staging memory it waits for
        the previous upload from it to have run (normally long finished)."""
        a = np.ascontiguousarray(array)
        if a.nbytes > self.nbytes:
            raise ValueError('staging buffer too small')
        if self._copied is not None:
            self._copied.synchronize()
        self.array[:a.nbytes] = a.view(np.uint8).reshape(-1)
        self.runtime.check(self.runtime.lib.mt_copy_async(dst, self.pointer.value, a.nbytes, 1))
        self.runtime.stats['h2d_bytes'] += a.nbytes
        if self._copied is None:
            self._copied = CudaEvent()
        self._copied.record()


class DeviceTensor:
    """Contiguous typed device array (shape, dtype, pointer).

    Stands where the reference passes a device-resident MiniTorch ``Tensor``
    to its kernels (``pointer(t, typed=True)``, minitorch/cuda_resident_ops.py:33-38).
    A tensor may be a view into another tensor's allocation (``base``).
    """

    def __init__(self, shape, dtype='float32', *, buffer=None, byte_offset=0):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = normalize_dtype(dtype)
        self.size = int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1
        self.nbytes = self.size * itemsize(self.dtype)
        if buffer is None:
            buffer = PooledBuffer(max(self.nbytes, 1))
            byte_offset = 0
        if byte_offset + self.nbytes > buffer.nbytes:
            raise ValueError('DeviceTensor view exceeds its buffer')
        self.buffer = buffer
        self.byte_offset = byte_offset

    @property
    def ptr(self):
        return self.buffer.ptr + self.byte_offset

    @property
    def dims(self):
        return len(self.shape)

    @classmethod
    def empty(cls, shape, dtype='float32'):
        return cls(shape, dtype)

    @classmethod
    def from_numpy(cls, value, dtype='float32'):
        value = np.asarray(value)
        t = cls(value.shape, dtype)
        runtime().h2d(t.ptr, encode_host(value, t.dtype))
        return t

    @classmethod
    def zeros(cls, shape, dtype='float32'):
        t = cls(shape, dtype)
        t.buffer.fill_words(0)
        return t

    def to_numpy(self):
        out = np.empty(self.size, storage_numpy_dtype(self.dtype))
        runtime().d2h(out, self.ptr)
        return np.asarray(decode_host(out, self.dtype)).reshape(self.shape)

    def raw_numpy(self):
        """Storage bit patterns (bf16 as uint16)."""
        out = np.empty(self.size, storage_numpy_dtype(self.dtype))
        return runtime().d2h(out, self.ptr).reshape(self.shape)

    def view(self, *shape):
        shape = tuple(int(s) for s in (shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape))
        if int(np.prod(shape, dtype=np.int64)) != self.size:
            raise ValueError(f'Cannot view {self.shape} as {shape}')
        return DeviceTensor(shape, self.dtype, buffer=self.buffer, byte_offset=self.byte_offset)

    def rows(self, start, stop):
        """View of rows [start, stop) along the first dimension."""
        row = self.size // self.shape[0] * itemsize(self.dtype)
        return DeviceTensor((stop - start,) + self.shape[1:], self.dtype, buffer=self.buffer,
                            byte_offset=self.byte_offset + start * row)

    def contiguous(self):
        return self

    def __repr__(self):
        return f'DeviceTensor(shape={self.shape}, dtype={self.dtype})'


def pointer(tensor, typed=False):
    """Raw device address of a tensor; FP32 unless ``typed`` (reference
    minitorch/cuda_resident_ops.py:33-38)."""
    if not isinstance(tensor, DeviceTensor):
        raise TypeError('Native operation requires a DeviceTensor')
    if not typed and tensor.dtype != 'float32':
        raise TypeError('This native kernel requires float32')
    return tensor.ptr


class CudaEvent:
    """Null-stream event with elapsed seconds (reference minitorch/cuda_storage.py:258-271)."""

    def __init__(self):
        self.runtime = runtime()
        self.handle = P()
        self.runtime.check(self.runtime.lib.mt_event_create(ct.byref(self.handle)))
        weakref.finalize(self, self.runtime.lib.mt_event_destroy, self.handle)

    def record(self):
        self.runtime.check(self.runtime.lib.mt_event_record(self.handle))

    def synchronize(self):
        self.runtime.check(self.runtime.lib.mt_event_synchronize(self.handle))

    def query(self):
        """True once the work before the last record has completed."""
        status = self.runtime.lib.mt_event_query(self.handle)
        if status == HIP_ERROR_NOT_READY:
            return False
        self.runtime.check(status)
        return True

    def seconds_since(self, start):
        ms = F()
        self.runtime.check(self.runtime.lib.mt_event_elapsed(ct.byref(ms), start.handle, self.handle))
        return ms.value / 1000
