"""End-to-end decode harnesses for the benchmark configurations 3 and 4.

Config 3 replays the reference's continuous-batching benchmark shape
(project/benchmark_continuous_batching.py:84-97,122) on a random-init
DistilGPT-2: requests arrive by wall clock (Poisson), the batcher steps while
there is work, and throughput is reported both with the reference's formula
(generated tokens / (end - start), arrival gaps included) and as busy-step
decode throughput (sum of decode batch sizes / sum of decode seconds).

Config 4 holds a steady state of concurrent requests on a random-init
GPT-2-medium: every step decodes all of them, then each request is replaced
with a seeded 5 % probability (or when it reaches its capacity) by a fresh
prefilled one, exercising page free/reuse. Decode tokens/s counts decode
steps only.
"""
import math
import time
import numpy as np

from .continuous_batching import ContinuousBatcher
from .kv_cache import greedy_token
from .paged_kv_cache import KVPagePool
from .runtime import DeviceTensor, CudaEvent, runtime
from .amp import autocast


def config3_trace(seed=0, requests=256, rate=32.0, vocab=50257, n_positions=1024):
    """(arrival_seconds, request_id, prompt_ids, max_new_tokens) for config 3:
    Poisson arrivals, prompts U{32..512}, outputs geometric with mean 128,
    capped so prompt + output <= n_positions."""
    rng = np.random.default_rng([seed, 3])
    arrivals = np.cumsum(rng.exponential(1.0 / rate, requests))
    arrivals -= arrivals[0]
    out = []
    for i in range(requests):
        n = int(rng.integers(32, 513))
        prompt = rng.integers(0, vocab, n)
        new = int(min(rng.geometric(1.0 / 128), n_positions - n + 1))
        out.append((float(arrivals[i]), f'r{i}', prompt, new))
    return out


def config3_step_trace(seed=0, step_seconds=1e-3, **kwargs):
    """``config3_trace`` on a step-indexed clock: one scheduler step stands for
    ``step_seconds`` and an arrival at t seconds becomes step
    floor(t / step_seconds). Replaying it submits request i just before that
    step runs, so decisions do not depend on wall-clock timing."""
    return [(int(math.floor(a / step_seconds)), rid, prompt, new)
            for a, rid, prompt, new in config3_trace(seed, **kwargs)]


def _progress(message):
    import sys
    print(message, file=sys.stderr, flush=True)


def run_config3(model, trace, *, precision='fp16', max_batch_size=256, page_size=16, kv_pages=16384,
                max_prefills_per_step=1, prefill_token_budget=512, clock=time.perf_counter,
                report_every=200, token_feedback=False, graph=False, merge_prefill=False):
    """Replay a config-3 trace through the batcher (``merge_prefill``: steps
    that admit requests run their decode and the prefills as one layer loop). ``busy_step_tokens_per_sec``
    is decode tokens over the wall time of the steps (decode, prefill and
    scheduling, idle gaps between arrivals excluded), comparable between the
    synchronous and the sync-free (``token_feedback``) loop;
    ``busy_decode_tokens_per_sec`` (synchronous loop only) counts just the
    decode part of each step up to its tokens on the host."""
    itemsize = 4 if precision == 'fp32' else 2
    page_bytes = 2 * model.n_layer * model.n_embd * page_size * itemsize
    batcher = ContinuousBatcher(model, max_batch_size=max_batch_size, page_size=page_size,
                                kv_budget_bytes=kv_pages * page_bytes, precision=precision,
                                max_prefills_per_step=max_prefills_per_step,
                                prefill_token_budget=prefill_token_budget, clock=clock,
                                token_feedback=token_feedback, graph=graph, merge_prefill=merge_prefill)
    pending = list(trace)
    steps = []
    start = clock()
    while pending or batcher.has_work:
        now = clock() - start
        while pending and pending[0][0] <= now:
            _, rid, prompt, new = pending.pop(0)
            batcher.submit(rid, prompt, max_new_tokens=new)
        if batcher.has_work:
            batcher.step()
            steps.append(batcher.last_step)
            if report_every and len(steps) % report_every == 0:
                _progress(f'config 3: step {len(steps)}, {clock() - start:.1f} s, '
                          f'decode batch {steps[-1]["decode_batch_size"]}, queued {steps[-1]["queued_requests"]}')
        elif pending:
            time.sleep(max(0.0, pending[0][0] - (clock() - start)))
    elapsed = clock() - start
    generated = sum(len(r.output_ids) for r in batcher.requests.values())
    decode_tokens = sum(s['decode_batch_size'] for s in steps)
    decode_seconds = sum(s['decode_seconds'] for s in steps if s['decode_batch_size'])
    step_seconds = sum(s['step_seconds'] for s in steps)
    ttft = [r.ttft_seconds for r in batcher.requests.values() if r.ttft_seconds is not None]
    result = dict(
        token_feedback=token_feedback, graph=graph,
        generated_tokens=generated, elapsed_seconds=elapsed,
        output_tokens_per_sec=generated / elapsed,
        busy_decode_tokens_per_sec=(decode_tokens / decode_seconds if decode_seconds and not token_feedback
                                    else None),
        busy_step_tokens_per_sec=decode_tokens / step_seconds, step_seconds=step_seconds,
        decode_tokens=decode_tokens, decode_seconds=decode_seconds, steps=len(steps),
        max_decode_batch_size=max(s['decode_batch_size'] for s in steps),
        mean_decode_batch_size=float(np.mean([s['decode_batch_size'] for s in steps if s['decode_batch_size']])),
        ttft_p50_ms=float(np.median(ttft) * 1e3), ttft_p95_ms=float(np.percentile(ttft, 95) * 1e3),
        completed=sum(r.state == 'completed' for r in batcher.requests.values()),
        kv_pool_used_pages_after=steps[-1]['kv_pool_used_pages'],
        peak_used_pages=batcher.peak_used_pages,
        page_reuses=steps[-1]['kv_pool_page_reuses'])
    batcher.close()
    return result


def config4_lengths(rng, n):
    return np.clip(np.round(np.exp(rng.normal(np.log(256.0), 1.2, n))), 16, 1024).astype(int)


def run_config4(model, *, seed=0, concurrent=128, steps=40, warmup=5, replace_rate=0.05,
                precision='bf16', page_size=16, kv_pages=None, token_feedback=False, batch_prefills=True,
                graph=False, merge_prefill=False):
    """Steady-state decode throughput; returns a dict of measurements.

    ``decode_tokens_per_sec`` times each step's decode: in the synchronous
    loop up to its tokens on the host (wall clock), in the sync-free loop
    between events recorded on the stream before and after it (gaps the host
    leaves in the stream included). ``loop_tokens_per_sec`` times the whole
    timed loop (decode steps plus the replacement prefills, synchronized only
    at its start and end), which is comparable between the synchronous loop
    and the sync-free one (``token_feedback``: tokens stay on the device as
    the next step's input and are never read). With ``batch_prefills`` the
    requests replaced in a step are prefilled together
    (``DecoderLM.prefill_batch``), else one ``prefill`` call each; the random
    draws, and so the replacements and prompts, are the same either way.
    With ``merge_prefill`` (sync-free only) a step that replaces requests runs
    its decode and the replacements' prefill as one layer loop
    (``DecoderLM.decode_prefill_greedy``; the replaced requests' caches are
    closed inside it, after the step's pages are taken): same replacements,
    prompts and page IDs; only the loop's rate is reported, since the decode
    step is no longer timed on its own."""
    dtype = {'fp16': 'float16', 'bf16': 'bfloat16', 'fp32': 'float32'}[precision]
    rng = np.random.default_rng([seed, 4])
    rt = runtime()
    itemsize = 4 if precision == 'fp32' else 2
    page_bytes = 2 * model.n_layer * model.n_embd * page_size * itemsize
    kv_pages = kv_pages or concurrent * ((model.n_positions + page_size - 1) // page_size)
    with autocast(dtype) if precision != 'fp32' else _null():
        pool = KVPagePool(model, page_size=page_size, max_bytes=kv_pages * page_bytes, pages_per_slab=16)
        caches, last = [], []

        def draw():
            # context length L counts the token being decoded: prompt of L - 1
            length = int(config4_lengths(rng, 1)[0]) - 1
            return rng.integers(0, model.n_vocab, length)

        def admit(prompts):
            """New caches prefilled with ``prompts``, and their first tokens."""
            new = [model.create_kv_cache(1, model.n_positions, page_size=page_size, page_pool=pool)
                   for _ in prompts]
            if batch_prefills:
                logits = model.prefill_batch(prompts, new)
            else:
                logits = [model.prefill(DeviceTensor.from_numpy(p[None].astype(np.float32)), c)[0]
                          for p, c in zip(prompts, new)]
            if token_feedback:
                if batch_prefills:
                    greedy_token(logits, feedback=new)
                else:
                    for c, l in zip(new, logits):
                        greedy_token(l, feedback=c)
                return new, [None] * len(new)
            if batch_prefills:
                return new, [int(t) for t in greedy_token(logits).to_numpy()[:, 0]]
            return new, [int(greedy_token(l).to_numpy()[0, 0]) for l in logits]

        for c0 in range(0, concurrent, 32):
            new, first = admit([draw() for _ in range(min(32, concurrent - c0))])
            caches += new
            last += first
        decode_seconds, tokens, replaced, context, step_events = 0.0, 0, 0, [], []
        loop0 = None
        if merge_prefill and not token_feedback:
            raise ValueError('merge_prefill needs the sync-free loop (token_feedback=True)')
        for step in range(warmup + steps):
            context.append(sum(c.length + 1 for c in caches))
            if step == warmup:
                rt.synchronize()
                loop0 = time.perf_counter()
            if merge_prefill:
                # the replacements are drawn as after the step (the condition
                # on the length counts the step's token), then run with it
                slots, prompts = [], []
                for i in range(len(caches)):
                    if rng.random() < replace_rate or caches[i].length + 2 >= caches[i].capacity:
                        slots.append(i)
                        prompts.append(draw())
                if slots:
                    new = [model.create_kv_cache(1, model.n_positions, page_size=page_size, page_pool=pool)
                           for _ in prompts]
                    model.decode_prefill_greedy(caches, prompts, new, finished=[caches[i] for i in slots])
                    for i, c in zip(slots, new):
                        caches[i] = c
                    replaced += len(slots)
                else:
                    model.decode_greedy(caches, graph=graph)
                if step >= warmup:
                    tokens += len(caches)
                continue
            if token_feedback:
                if step >= warmup:
                    # events around the decode step: its time on the device,
                    # host-induced gaps included, replacement prefills not
                    e0, e1 = CudaEvent(), CudaEvent()
                    e0.record()
                model.decode_greedy(caches, graph=graph)
                if step >= warmup:
                    e1.record()
                    step_events.append((e0, e1))
                    tokens += len(caches)
            else:
                ids = DeviceTensor.from_numpy(np.array(last, np.float32)[:, None])
                rt.synchronize()
                t0 = time.perf_counter()
                logits = model.decode_batch(ids, caches)
                nxt = greedy_token(logits).to_numpy()[:, 0]
                t1 = time.perf_counter()
                if step >= warmup:
                    decode_seconds += t1 - t0
                    tokens += len(caches)
                last = [int(t) for t in nxt]
                if step % 10 == 0:
                    _progress(f'config 4: step {step}, decode {(t1 - t0) * 1e3:.2f} ms')
            slots, prompts = [], []
            for i in range(len(caches)):
                if rng.random() < replace_rate or caches[i].length + 1 >= caches[i].capacity:
                    caches[i].close()
                    slots.append(i)
                    prompts.append(draw())
            if slots:
                new, first = admit(prompts)
                for i, c, t in zip(slots, new, first):
                    caches[i], last[i] = c, t
                replaced += len(slots)
        rt.synchronize()
        loop_seconds = time.perf_counter() - loop0
        if step_events:
            decode_seconds = sum(e1.seconds_since(e0) for e0, e1 in step_events)
        stats = pool.memory_stats()
        for c in caches:
            c.close()
        pool.close()
    return dict(token_feedback=token_feedback, graph=graph, batch_prefills=batch_prefills,
                merge_prefill=merge_prefill,
                decode_tokens_per_sec=tokens / decode_seconds if decode_seconds else None,
                decode_seconds=decode_seconds, loop_tokens_per_sec=tokens / loop_seconds,
                loop_seconds=loop_seconds, steps=steps, concurrent=concurrent,
                mean_context_tokens=float(np.mean(context) / concurrent),
                replaced_requests=replaced, page_reuses=stats['kv_pool_page_reuses'],
                ms_per_step=decode_seconds / steps * 1e3 if decode_seconds else None,
                loop_ms_per_step=loop_seconds / steps * 1e3)


class _null:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False
