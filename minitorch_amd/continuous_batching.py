"""Iteration-level continuous batching over a shared paged KV pool
(reference minitorch/continuous_batching.py).

Same scheduling as the reference: FIFO admission under a logical reservation
of each request's maximum page demand, decode of every active request before
admissions, at most ``max_prefills_per_step`` prefills per step within
``prefill_token_budget`` (the first prefill of a step is exempt), finish on
EOS or length, cancel of queued or active requests, and the same per-step
statistics. Page IDs, tables and offsets of every decode step are built on
the device (``PagedDecodeBatch``); the host reads back only the new tokens.

With ``token_feedback=True`` the decode loop is sync-free: each step's
greedy tokens stay on the device as the next step's input (the pool's
per-slot last tokens), requests without an EOS token finish by count, and
the token values reach the host through asynchronous copies that ``step``
delivers one step later (a step returns the events of the tokens that
arrived during it; a step that admits requests waits for all its tokens, so
first tokens are not delayed). Scheduling decisions, pages and tokens are the same as in
the synchronous mode; a step whose batch has a request with an EOS token
waits for its tokens, since finishing then depends on their values. With
``graph=True`` as well, each decode step's device work is replayed from a HIP
graph captured per batch size (``DecoderLM.decode_greedy(graph=True)``). With
``merge_prefill=True`` (sync-free) a step whose batch has no EOS token decides
its admissions before its decode runs -- the requests that end with the step's
token leave the batch first, as their count already decides -- and runs the
decode and the admissions' prefill as one layer loop
(``DecoderLM.decode_prefill_greedy``): same decisions, pages and tokens.
"""
from collections import deque
from contextlib import nullcontext
from dataclasses import dataclass, field
import math
import time
import numpy as np

from .amp import autocast
from .kv_cache import greedy_token, TokenReadback
from .paged_kv_cache import KVPagePool
from .runtime import DeviceTensor


@dataclass
class GenerationRequest:
    request_id: str
    prompt_ids: tuple
    max_new_tokens: int
    eos_token_id: int | None
    submitted_at: float
    capacity: int
    reserved_pages: int
    state: str = 'queued'
    finish_reason: str | None = None
    admitted_at: float | None = None
    finished_at: float | None = None
    output_ids: list = field(default_factory=list)
    token_times: list = field(default_factory=list)
    cache: object = field(default=None, repr=False)
    generated: int = 0  # tokens produced on the device, delivered or not

    @property
    def done(self):
        return self.state in ('completed', 'cancelled', 'rejected', 'failed')

    @property
    def ttft_seconds(self):
        return self.token_times[0] - self.submitted_at if self.token_times else None


class ContinuousBatcher:
    """Submit requests between steps; each step yields newly available tokens
    (reference minitorch/continuous_batching.py:45-195)."""

    def __init__(self, model, *, max_batch_size=4, page_size=16, kv_budget_bytes=256 * 1024 ** 2,
                 pages_per_slab=4, precision='fp32', max_prefills_per_step=1,
                 prefill_token_budget=512, clock=time.perf_counter, token_feedback=False, graph=False,
                 merge_prefill=False):
        for value in (max_batch_size, max_prefills_per_step, prefill_token_budget):
            if type(value) is not int or value < 1:
                raise ValueError('Positive integer batch size and prefill limits required')
        if precision not in ('fp32', 'fp16', 'bf16'):
            raise ValueError('precision must be fp32, fp16 or bf16')
        if any(l.attention.attention_impl != 'flash' for l in model.transformer_layers()):
            raise ValueError('Continuous batching requires FlashAttention')
        self.model, self.precision = model, precision
        self.max_batch_size = max_batch_size
        self.max_prefills_per_step = max_prefills_per_step
        self.prefill_token_budget = prefill_token_budget
        self.clock = clock
        with self._precision_context():
            self.pool = KVPagePool(model, page_size=page_size, max_bytes=kv_budget_bytes,
                                   pages_per_slab=pages_per_slab)
        self.requests, self.active, self.pending = {}, {}, deque()
        self.reserved_pages = 0
        self.peak_used_pages = 0
        self.iteration = 0
        self.last_step = None
        self.closed = False
        if (graph or merge_prefill) and not token_feedback:
            raise ValueError('graph replay and merged prefills need the sync-free loop (token_feedback=True)')
        self.token_feedback = bool(token_feedback)
        self.graph = bool(graph)
        self.merge_prefill = bool(merge_prefill)
        self._readback = TokenReadback(max_prefills_per_step + 4) if self.token_feedback else None
        self._inflight = deque()  # (readback ticket, requests) in issue order

    def _precision_context(self):
        if self.precision == 'fp32':
            return nullcontext()
        return autocast('float16' if self.precision == 'fp16' else 'bfloat16')

    @property
    def has_work(self):
        return bool(self.active or self.pending or self._inflight)

    def submit(self, request_id, prompt_ids, *, max_new_tokens=32, eos_token_id=None):
        if self.closed:
            raise ValueError('Batcher is closed')
        if not isinstance(request_id, str) or not request_id or request_id in self.requests:
            raise ValueError('Nonempty unique request ID required')
        ids = np.asarray(prompt_ids)
        if (ids.ndim != 1 or ids.size < 1 or ids.dtype.kind not in 'iu' or
                np.any(ids < 0) or np.any(ids >= self.model.n_vocab)):
            raise ValueError('prompt_ids must be nonempty 1-D integer vocabulary IDs')
        if type(max_new_tokens) is not int or max_new_tokens < 1:
            raise ValueError('Positive integer max_new_tokens required')
        if eos_token_id is not None and (type(eos_token_id) is not int or not 0 <= eos_token_id < self.model.n_vocab):
            raise ValueError('Invalid EOS token ID')
        capacity = int(ids.size) + max_new_tokens - 1
        if capacity > self.model.n_positions:
            raise ValueError('Prompt plus output exceeds model position capacity')
        request = GenerationRequest(request_id, tuple(int(x) for x in ids), max_new_tokens, eos_token_id,
                                    self.clock(), capacity, math.ceil(capacity / self.pool.page_size))
        self.requests[request_id] = request
        if request.reserved_pages > self.pool.max_pages:
            request.state, request.finish_reason, request.finished_at = 'rejected', 'kv_budget', self.clock()
        else:
            self.pending.append(request)
        return request

    def _finish(self, request, state, reason):
        if request.request_id in self.active:
            del self.active[request.request_id]
            self.reserved_pages -= request.reserved_pages
        if request.cache is not None:
            request.cache.close()
            request.cache = None
        request.state, request.finish_reason, request.finished_at = state, reason, self.clock()

    def cancel(self, request_id):
        request = self.requests[request_id]
        if request.done:
            return False
        if request.state == 'queued':
            self.pending.remove(request)
        self._finish(request, 'cancelled', 'cancelled')
        return True

    def _emit(self, request, token_id, arrival):
        request.generated += 1
        return self._deliver(request, token_id, arrival, finish=True)

    def _deliver(self, request, token_id, arrival, finish):
        request.output_ids.append(int(token_id))
        request.token_times.append(arrival)
        reason = ('eos' if token_id == request.eos_token_id else
                  'length' if len(request.output_ids) >= request.max_new_tokens else None)
        if reason is not None and finish and not request.done:
            self._finish(request, 'completed', reason)
        return dict(request_id=request.request_id, token_id=int(token_id),
                    output_index=len(request.output_ids) - 1, arrival_time=arrival, finish_reason=reason)

    # ------------------------------------------------ sync-free decoding ---
    def _issue(self, requests, ids):
        """Queue the read-back of the device tokens ``ids`` of ``requests`` and
        finish, by count, the requests that reached their length. Requests
        with an EOS token finish when their tokens are delivered."""
        self._inflight.append((self._readback.push(ids), list(requests)))
        for request in requests:
            request.generated += 1
            if request.eos_token_id is None and request.generated >= request.max_new_tokens and not request.done:
                self._finish(request, 'completed', 'length')

    @staticmethod
    def _ended_early(request):
        """Ended by cancel, an early finish or a failure rather than by its own
        tokens: nothing is delivered to it afterwards, as the reference emits
        nothing after a cancel (minitorch/continuous_batching.py:117-122)."""
        return request.state in ('cancelled', 'failed') or (
            request.state == 'completed' and request.finish_reason not in ('length', 'eos'))

    def _drain(self, keep=0, block=True):
        """Deliver arrived tokens in issue order, leaving ``keep`` read-backs
        in flight; without ``block`` only those already complete."""
        events = []
        while len(self._inflight) > keep:
            ticket, requests = self._inflight[0]
            if not block and not self._readback.ready(ticket):
                break
            tokens = self._readback.read(ticket)
            self._inflight.popleft()
            arrival = self.clock()
            for request, token in zip(requests, tokens):
                if self._ended_early(request):
                    continue  # cancelled, finished or failed while the token was in flight
                finish = request.eos_token_id is not None
                events.append(self._deliver(request, int(token), arrival, finish))
        return events

    def step(self):
        if self.closed:
            raise ValueError('Batcher is closed')
        start = self.clock()
        events, decode_ids, prefill_ids = [], list(self.active), []
        if self.token_feedback:
            events.extend(self._drain(block=False))
            first_ticket = self._readback.issued
        prefill_tokens = 0
        with self._precision_context():
            merged = None
            if decode_ids and self.merge_prefill and all(self.active[rid].eos_token_id is None for rid in decode_ids):
                # the step's decode runs with its admissions' prefills (below):
                # the requests that end with this step's token leave the batch
                # now, as their token's count already decides
                batch = [self.active[rid] for rid in decode_ids]
                ending = [r for r in batch if r.generated + 1 >= r.max_new_tokens]
                needs = sum(1 for r in batch if r.cache.length % self.pool.page_size == 0)
                merged = (batch, ending, self.pool.used_pages + needs)
                for request in ending:
                    del self.active[request.request_id]
                    self.reserved_pages -= request.reserved_pages
                    request.state, request.finish_reason, request.finished_at = 'completed', 'length', self.clock()
            elif decode_ids and self.token_feedback:
                batch = [self.active[rid] for rid in decode_ids]
                try:
                    ids = self.model.decode_greedy([r.cache for r in batch], graph=self.graph)
                    self.peak_used_pages = max(self.peak_used_pages, self.pool.used_pages)
                    self._issue(batch, ids)
                    if any(r.eos_token_id is not None for r in batch):
                        events.extend(self._drain())
                except Exception:
                    for request in batch:
                        if not request.done:
                            self._finish(request, 'failed', 'decode_error')
                    raise
            elif decode_ids:
                batch = [self.active[rid] for rid in decode_ids]
                try:
                    ids = DeviceTensor.from_numpy(np.array([[r.output_ids[-1]] for r in batch], np.float32))
                    logits = self.model.decode_batch(ids, [r.cache for r in batch])
                    self.peak_used_pages = max(self.peak_used_pages, self.pool.used_pages)
                    tokens = greedy_token(logits).to_numpy()[:, 0]
                    arrival = self.clock()
                    events.extend(self._emit(r, t, arrival) for r, t in zip(batch, tokens))
                except Exception:
                    for request in batch:
                        if not request.done:
                            self._finish(request, 'failed', 'decode_error')
                    raise
            decode_seconds = self.clock() - start
            admitted = []
            while self.pending and len(self.active) < self.max_batch_size and len(prefill_ids) < self.max_prefills_per_step:
                request = self.pending[0]
                if self.reserved_pages + request.reserved_pages > self.pool.max_pages:
                    break
                if prefill_ids and prefill_tokens + len(request.prompt_ids) > self.prefill_token_budget:
                    break
                self.pending.popleft()
                self.active[request.request_id] = request
                self.reserved_pages += request.reserved_pages
                request.state, request.admitted_at = 'active', self.clock()
                try:
                    request.cache = self.model.create_kv_cache(1, request.capacity, cache_impl='paged',
                                                               page_size=self.pool.page_size, page_pool=self.pool)
                except Exception:
                    self._finish(request, 'failed', 'prefill_error')
                    raise
                admitted.append(request)
                prefill_ids.append(request.request_id)
                prefill_tokens += len(request.prompt_ids)
            if merged is not None:
                events.extend(self._merged_step(*merged, admitted))
            elif admitted:
                events.extend(self._prefill(admitted))
        if self.token_feedback:
            # Only the read-backs issued in this step stay in flight: the
            # previous step's tokens are delivered while this step runs. A
            # step that admitted requests delivers everything, so that a first
            # token is not held back a step (time to first token).
            keep = 0 if prefill_ids else sum(1 for t, _ in self._inflight if t >= first_ticket)
            events.extend(self._drain(keep=keep))
        capacity_bytes = sum(r.cache.nbytes for r in self.active.values())
        live_bytes = sum(r.cache.length * self.pool.page_bytes // self.pool.page_size for r in self.active.values())
        self.last_step = dict(iteration=self.iteration, decode_request_ids=decode_ids,
                              decode_batch_size=len(decode_ids), prefill_request_ids=prefill_ids,
                              prefill_tokens=prefill_tokens, active_request_ids=list(self.active),
                              queued_requests=len(self.pending), logical_reserved_pages=self.reserved_pages,
                              decode_seconds=decode_seconds, kv_live_bytes=live_bytes,
                              kv_capacity_bytes=capacity_bytes,
                              kv_slot_utilization=live_bytes / capacity_bytes if capacity_bytes else None,
                              peak_used_pages=self.peak_used_pages, step_seconds=self.clock() - start,
                              token_feedback=self.token_feedback, tokens_in_flight=len(self._inflight),
                              **self.pool.memory_stats())
        self.iteration += 1
        return events

    def _merged_step(self, batch, ending, used_after_decode, admitted):
        """The decode of ``batch`` and the prefill of ``admitted`` as one
        layer loop (``DecoderLM.decode_prefill_greedy``), the caches of the
        ``ending`` requests closed inside it once the step's pages are taken
        (without admissions: ``decode_greedy``, then those caches closed).
        Issues the read-back of every token of the step. The logical
        reservation of every active request's whole demand keeps both the
        decode's and the prompts' pages within the budget, as it does for
        separate passes."""
        try:
            if admitted:
                ids = self.model.decode_prefill_greedy(
                    [r.cache for r in batch], [np.array(r.prompt_ids) for r in admitted],
                    [r.cache for r in admitted], finished=[r.cache for r in ending])
            else:
                ids = self.model.decode_greedy([r.cache for r in batch], graph=self.graph)
                self.pool.close_caches([r.cache for r in ending])
        except Exception:
            ended = {id(r) for r in ending}
            for request in batch:
                if id(request) in ended or not request.done:
                    self._finish(request, 'failed', 'decode_error')
            for request in admitted:
                if not request.done:
                    self._finish(request, 'failed', 'prefill_error')
            raise
        for request in ending:
            request.cache = None
        self.peak_used_pages = max(self.peak_used_pages, used_after_decode, self.pool.used_pages)
        self._issue(batch + admitted, ids)
        return []

    def _prefill(self, admitted):
        """Prefill the requests admitted in this step and emit (or, sync-free,
        issue) their first tokens. One request goes through ``prefill`` as in
        the reference; several admitted together go through one
        ``prefill_batch`` call (pages acquired in admission order, as
        consecutive prefills would)."""
        events = []
        try:
            if len(admitted) == 1:
                request = admitted[0]
                ids = DeviceTensor.from_numpy(np.array([request.prompt_ids], np.float32))
                logits, _ = self.model.prefill(ids, request.cache)
                feedback = request.cache
            else:
                logits = self.model.prefill_batch([np.array(r.prompt_ids) for r in admitted],
                                                  [r.cache for r in admitted])
                feedback = [r.cache for r in admitted]
            self.peak_used_pages = max(self.peak_used_pages, self.pool.used_pages)
            if self.token_feedback:
                self._issue(admitted, greedy_token(logits, feedback=feedback))
                if any(r.eos_token_id is not None for r in admitted):
                    events.extend(self._drain())
            else:
                tokens = greedy_token(logits).to_numpy()[:, 0]
                arrival = self.clock()
                events.extend(self._emit(r, t, arrival) for r, t in zip(admitted, tokens))
        except Exception:
            for request in admitted:
                if not request.done:
                    self._finish(request, 'failed', 'prefill_error')
            raise
        return events

    def close(self):
        if self.closed:
            return
        if self._inflight:
            self._drain()
        for request in tuple(self.requests.values()):
            if not request.done:
                self.cancel(request.request_id)
        self.pool.close()
        self.closed = True

    def __enter__(self):
        return self

    def __exit__(self, *args):
        self.close()


class ContinuousBatchingEngine(ContinuousBatcher):
    """The batcher under the admit / finish / cancel vocabulary: ``admit``
    queues a request for FIFO admission (``submit``), ``finish`` ends an active
    or queued request early and returns its pages, ``cancel`` as above."""

    def admit(self, request_id, prompt_ids, *, max_new_tokens=32, eos_token_id=None):
        return self.submit(request_id, prompt_ids, max_new_tokens=max_new_tokens, eos_token_id=eos_token_id)

    def finish(self, request_id, reason='finished'):
        request = self.requests[request_id]
        if request.done:
            return False
        if request.state == 'queued':
            self.pending.remove(request)
        self._finish(request, 'completed', reason)
        return True
