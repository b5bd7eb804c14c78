"""Cache transaction base and token helpers (reference minitorch/kv_cache.py).

``CacheBase`` keeps the reference's transaction state machine
(prepare_append / commit_append / abort_append, one write per layer,
validation of model, precision and weight version; kv_cache.py:56-160).
``greedy_token`` and ``last_position`` run ``mt_row_argmax`` and
``mt_last_row`` from ``cuda_kernels/inference_kernels.so``
(kv_cache.py:26-53). This build has no autograd, so the reference's no_grad
checks have nothing to check.
"""
import weakref
import numpy as np
from .amp import autocast_dtype
from .runtime import DeviceTensor, PinnedHostBuffer, CudaEvent, runtime
from . import paged_ops


def last_position(x):
    """Copy the last sequence position of a device [B, T, C] tensor (reference
    minitorch/kv_cache.py:26-36)."""
    if not isinstance(x, DeviceTensor) or x.dims != 3:
        raise ValueError('last_position requires no_grad and device [B,T,C] input')
    b, n, w = x.shape
    if min(b, n, w) < 1:
        raise ValueError('Empty last-position input')
    out = DeviceTensor((b, 1, w), x.dtype)
    paged_ops.last_row(out.ptr, x.ptr, b, n, w, x.dtype)
    return out


def greedy_token(logits, feedback=None):
    """GPU argmax over [B, 1, V] logits, returning fp32 token IDs [B, 1]; ties
    and NaNs choose the first index, like numpy.argmax (reference
    minitorch/kv_cache.py:39-53). With ``feedback`` (a paged cache of B rows,
    or a sequence of B paged caches of one row each, on one pool) the tokens
    are also stored as the slots' last tokens in the pool, where the next
    decode step reads them without a host round trip."""
    if not isinstance(logits, DeviceTensor) or logits.dims != 3 or logits.shape[1] != 1:
        raise ValueError('greedy_token requires no_grad and device logits [B,1,V]')
    b, _, v = logits.shape
    if b < 1 or not 1 <= v <= 2 ** 24:
        raise ValueError('Vocabulary must fit exact FP32 token IDs')
    out = DeviceTensor((b, 1), 'float32')
    if feedback is None:
        paged_ops.row_argmax(out.ptr, logits.ptr, b, v, logits.dtype)
    elif isinstance(feedback, (list, tuple)):
        pool = feedback[0].pool if feedback else None
        if (len(feedback) != b or pool is None or pool.closed or
                any(c.pool is not pool or c.batch_size != 1 for c in feedback)):
            raise ValueError('Feedback caches must be live, share a pool and hold one row per logits row')
        slots = DeviceTensor.from_numpy(np.array([c.slot for c in feedback], np.int32), 'int32')
        paged_ops.row_argmax_feedback(out.ptr, pool.slot_tokens.ptr, slots.ptr, pool.max_slots,
                                      logits.ptr, b, v, logits.dtype)
    else:
        pool = feedback.pool
        if feedback.batch_size != b or pool.closed:
            raise ValueError('Feedback cache must be live and have one row per logits row')
        paged_ops.row_argmax_feedback(out.ptr, pool.slot_tokens.ptr, feedback.slots_ptr, pool.max_slots,
                                      logits.ptr, b, v, logits.dtype)
    return out


class TokenReadback:
    """Token IDs copied to pinned host memory without waiting for the device:
    ``push`` enqueues the copy of a [B, 1] fp32 id tensor behind the work
    that produces it and returns a ticket; ``ready`` polls it and ``read``
    waits for it and returns the ids as int64. Tickets are served in order.
    Used by the sync-free decode loop, where the host schedules the next step
    before the tokens of the last one have arrived."""

    def __init__(self, depth=8):
        self.depth = depth
        self._buffers = [None] * depth
        self._events = [None] * depth
        self._rows = [0] * depth
        self._issued = 0
        self._read = 0

    def push(self, ids):
        if self._issued - self._read >= self.depth:
            raise RuntimeError('Too many unread token readbacks')
        k = self._issued % self.depth
        nbytes = 4 * ids.size
        if self._buffers[k] is None or self._buffers[k].nbytes < nbytes:
            self._buffers[k] = PinnedHostBuffer(max(nbytes, 4096))
        rt = runtime()
        rt.check(rt.lib.mt_copy_async(self._buffers[k].pointer.value, ids.ptr, nbytes, 2))
        if self._events[k] is None:
            self._events[k] = CudaEvent()
        self._events[k].record()
        self._rows[k] = ids.size
        self._issued += 1
        return self._issued - 1

    @property
    def pending(self):
        return self._issued - self._read

    @property
    def issued(self):
        """Ticket of the next push."""
        return self._issued

    def ready(self, ticket):
        return self._events[ticket % self.depth].query()

    def read(self, ticket):
        if ticket != self._read:
            raise ValueError('Token readbacks are read in order')
        k = ticket % self.depth
        self._events[k].synchronize()
        raw = self._buffers[k].array[:4 * self._rows[k]].view(np.float32)
        self._read += 1
        return raw.astype(np.int64)


class CacheBase:
    """Transaction state shared by inference caches (reference minitorch/kv_cache.py:56-160)."""

    def __init__(self, model, batch_size=1, capacity=None):
        if getattr(model, 'training', False):
            raise ValueError('Call model.eval() before creating an inference cache')
        capacity = model.n_positions if capacity is None else capacity
        if (type(batch_size) is not int or batch_size < 1 or type(capacity) is not int
                or not 1 <= capacity <= model.n_positions):
            raise ValueError('Invalid cache batch size or capacity')
        layers = model.transformer_layers()
        if any(l.attention.attn_hidden_dim > 128 for l in layers):
            raise ValueError('Cached inference requires head_dim<=128')
        self.model = weakref.ref(model)
        self.batch_size, self.capacity = batch_size, capacity
        self.dtype = autocast_dtype() or 'float32'
        self.length, self.valid, self.closed = 0, True, False
        self.layout = tuple((l.attention.n_head, l.attention.attn_hidden_dim) for l in layers)
        self._pending_tokens = None
        self._written_layers = set()
        self.weights = self._weights()
        self.last_attention_path = None

    def _weights(self):
        model = self.model()
        if model is None:
            raise ValueError('Cache model no longer exists')
        return model.weights_version()

    def prefill_attention(self, layer, q, k, v):
        if self.length != 0:
            raise ValueError('prefill attention requires empty cache')
        return self._attention(layer, q, k, v, prefill=True)

    def decode_attention(self, layer, q, k, v):
        if self.length == 0 or self._pending_tokens != 1:
            raise ValueError('decode attention requires populated cache and one token')
        return self._attention(layer, q, k, v, prefill=False)

    def attention(self, layer, q, k, v):
        return (self.prefill_attention if self.length == 0 else self.decode_attention)(layer, q, k, v)

    def _validate_model(self, model):
        if self.closed or not self.valid:
            raise ValueError('Cache is closed or invalid; reset/create a cache')
        if self.model() is not model:
            raise ValueError('Cache/model/backend mismatch')
        if getattr(model, 'training', False):
            raise ValueError('Cached inference requires eval and no_grad')
        if self.dtype != (autocast_dtype() or 'float32') or self.weights != self._weights():
            raise ValueError('Cache precision or model weights changed; reset/create a cache')

    def validate(self, model, idx, prefill):
        self._validate_model(model)
        if not isinstance(idx, DeviceTensor):
            raise ValueError('Cache/model/backend mismatch')
        if idx.dims != 2 or idx.shape[0] != self.batch_size or idx.dtype != 'float32':
            raise ValueError('Expected FP32 token IDs [cache_batch, sequence]')
        if prefill and self.length != 0:
            raise ValueError('prefill requires an empty cache')
        if not prefill and (self.length == 0 or idx.shape[1] != 1):
            raise ValueError('decode_step requires a populated cache and one token per batch')
        if idx.shape[1] < 1 or self.length + idx.shape[1] > self.capacity:
            raise ValueError('KV cache capacity exceeded or empty prompt')

    def prepare_append(self, tokens):
        if self.closed or not self.valid or self._pending_tokens is not None:
            raise ValueError('Cache closed, invalid, or append already pending')
        if self.dtype != (autocast_dtype() or 'float32'):
            raise ValueError('Cache writes require no_grad and matching precision')
        if type(tokens) is not int or tokens < 1 or self.length + tokens > self.capacity:
            raise ValueError('Invalid append size or cache capacity exceeded')
        self._pending_tokens = tokens
        self._written_layers.clear()

    def _check_attention(self, layer, q, k, v):
        if (self.closed or not self.valid or self._pending_tokens is None
                or type(layer) is not int or not 0 <= layer < len(self.layout)
                or layer in self._written_layers):
            raise ValueError('Invalid cache append transaction or layer')
        h, d = self.layout[layer]
        expected = (self.batch_size, h, self._pending_tokens, d)
        if any(not isinstance(t, DeviceTensor) or t.shape != expected or t.dtype != self.dtype
               for t in (q, k, v)):
            raise ValueError('Cache append shape/dtype/backend mismatch')

    def commit_append(self):
        if self._pending_tokens is None or len(self._written_layers) != len(self.layout):
            raise ValueError('Cannot commit an incomplete cache append')
        self.length += self._pending_tokens
        self._pending_tokens = None
        self._written_layers.clear()

    def abort_append(self):
        self._pending_tokens = None
        self._written_layers.clear()
        self.valid = False

    def reset(self):
        if self.closed:
            raise ValueError('Cannot reset a closed cache')
        self.weights = self._weights()
        self.length, self.valid = 0, True
        self._pending_tokens = None
        self._written_layers.clear()
