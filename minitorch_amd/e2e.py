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


# The reference's published serial-vs-continuous trace
# (project/benchmark_continuous_batching.py:26-33): request id, arrival (ms
# after the start), prompt tokens, new tokens.
REFERENCE_TRACE = (('A', 0, 32, 12), ('B', 0, 128, 8), ('C', 30, 256, 16), ('D', 60, 512, 8),
                   ('E', 100, 32, 12), ('F', 180, 128, 4))
REFERENCE_PROMPT_LENGTHS = (32, 128, 256, 512)   # project/benchmark_inference.py:26


def reference_prompts(seed, vocab, lengths=REFERENCE_PROMPT_LENGTHS):
    """One prompt of random token IDs per length. The reference tokenizes a
    fixed prose text to these lengths (project/benchmark_inference.py:36-52);
    its tokenizer files are not available here, so the IDs are synthetic."""
    rng = np.random.default_rng([seed, 9])
    return {n: rng.integers(0, vocab, n).tolist() for n in lengths}


def independent_tokens(model, prompt, new_tokens, precision='fp32'):
    """Greedy tokens of one request by prefill then decode_step on its own
    paged cache (the reference's untimed validation generation,
    project/benchmark_continuous_batching.py:50-66)."""
    from .amp import autocast as _autocast
    ctx = _autocast('float16' if precision == 'fp16' else 'bfloat16') if precision != 'fp32' else None
    if ctx:
        ctx.__enter__()
    try:
        cache = model.create_kv_cache(1, len(prompt) + new_tokens - 1)
        logits, _ = model.prefill(DeviceTensor.from_numpy(np.array([prompt], np.float32)), cache)
        out = []
        for step in range(new_tokens):
            if step:
                logits = model.decode_step(token, cache)
            token = greedy_token(logits)
            out.append(int(token.to_numpy()[0, 0]))
        cache.close()
        return out
    finally:
        if ctx:
            ctx.__exit__(None, None, None)


def run_reference_trace(model, prompts, *, mode, precision='fp32', max_batch_size=4, page_size=16,
                        budget_bytes=256 * 1024 ** 2, pages_per_slab=4, max_prefills_per_step=1,
                        prefill_token_budget=512, trace=REFERENCE_TRACE, clock=time.perf_counter):
    """One run of the reference's trace (project/benchmark_continuous_batching.py:69-138):
    ``serial`` is the batcher at max_batch_size 1, ``continuous`` at
    ``max_batch_size``; requests are submitted when their arrival time has
    passed on the wall clock, the batcher steps while it has work, TTFT is
    counted from each request's scheduled arrival, throughput is generated
    tokens / (end - start) with the idle arrival gaps included."""
    if mode not in ('serial', 'continuous'):
        raise ValueError('Unknown benchmark mode')
    batcher = ContinuousBatcher(model, precision=precision, max_batch_size=1 if mode == 'serial' else max_batch_size,
                                page_size=page_size, kv_budget_bytes=budget_bytes, pages_per_slab=pages_per_slab,
                                max_prefills_per_step=max_prefills_per_step,
                                prefill_token_budget=prefill_token_budget, clock=clock)
    pending = sorted(trace, key=lambda r: r[1])
    steps = []
    runtime().synchronize()
    start = clock()
    index = 0
    while index < len(pending) or batcher.has_work:
        elapsed_ms = (clock() - start) * 1e3
        while index < len(pending) and pending[index][1] <= elapsed_ms:
            rid, _, n, new = pending[index]
            batcher.submit(rid, np.array(prompts[n]), max_new_tokens=new)
            index += 1
        if not batcher.has_work:
            if index < len(pending):
                time.sleep(min(1e-3, max(0.0, pending[index][1] / 1e3 - (clock() - start))))
            continue
        batcher.step()
        steps.append(dict(batcher.last_step))
    end = clock()
    rows = {}
    for rid, arrival_ms, n, new in trace:
        r = batcher.requests[rid]
        scheduled = start + arrival_ms / 1e3
        rows[rid] = dict(state=r.state, tokens=list(r.output_ids),
                         ttft_ms=(r.token_times[0] - scheduled) * 1e3 if r.token_times else None)
    stats = batcher.pool.memory_stats()
    counts = [s['decode_batch_size'] for s in steps if s['decode_batch_size']]
    ttft = [v['ttft_ms'] for v in rows.values() if v['ttft_ms'] is not None]
    generated = sum(len(v['tokens']) for v in rows.values())
    summary = dict(mode=mode, elapsed_seconds=end - start, generated_tokens=generated,
                   output_tokens_per_sec=generated / (end - start),
                   completed_requests=sum(v['state'] == 'completed' for v in rows.values()),
                   ttft_ms=ttft, max_decode_batch_size=max(counts, default=0),
                   mean_decode_batch_size=float(np.mean(counts)) if counts else 0.0,
                   peak_used_pages=batcher.peak_used_pages,
                   kv_pool_reserved_bytes=stats['kv_pool_reserved_bytes'],
                   kv_pool_physical_bytes=stats['kv_pool_physical_bytes'],
                   kv_pool_used_pages_after=stats['kv_pool_used_pages'],
                   reserved_pages_after=batcher.reserved_pages)
    batcher.close()
    return summary, rows


def run_reference_scenarios(model, *, seed=0, precision='fp32', warmup=1, repeats=3, max_batch_size=4,
                            new_tokens=16):
    """The reference's two published DistilGPT-2 scenarios on this build:

    * the serial (max batch 1) vs continuous (max batch 4) trace, 1 warmup and
      ``repeats`` measured runs with the mode order alternating per run
      (project/benchmark_continuous_batching.py:171-178,193-211): tok/s over
      the measured runs, TTFT p50/p95 over their requests, max and mean
      non-empty decode batch, KV reserved peak (logical, the reference's
      figure, and physical), pages left after the run, and every completed
      request's tokens against independent generation;
    * batch-1 paged inference at prompts of 32/128/256/512 tokens with
      ``new_tokens`` new tokens (project/benchmark_inference.py:92-175):
      TTFT from before the cache is created to the first token on the host,
      end-to-end tok/s = new tokens / request time, decode tok/s = (new
      tokens - 1) / time from the first to the last token, medians and sums
      over the measured runs, and the tokens against independent generation."""
    prompts = reference_prompts(seed, model.n_vocab)
    gold = {rid: independent_tokens(model, prompts[n], new, precision) for rid, _, n, new in REFERENCE_TRACE}
    runs = {'serial': [], 'continuous': []}
    parity = True
    for repeat in range(warmup + repeats):
        order = ('serial', 'continuous') if repeat % 2 == 0 else ('continuous', 'serial')
        for mode in order:
            summary, rows = run_reference_trace(model, prompts, mode=mode, precision=precision,
                                                max_batch_size=max_batch_size)
            parity &= all(v['tokens'] == gold[rid] for rid, v in rows.items() if v['state'] == 'completed')
            if repeat >= warmup:
                runs[mode].append(summary)
    trace = {}
    for mode, measured in runs.items():
        seconds = sum(s['elapsed_seconds'] for s in measured)
        ttft = [t for s in measured for t in s['ttft_ms']]
        trace[mode] = dict(
            output_tokens_per_sec=sum(s['generated_tokens'] for s in measured) / seconds,
            completed_requests=sum(s['completed_requests'] for s in measured),
            ttft_p50_ms=float(np.median(ttft)), ttft_p95_ms=float(np.percentile(ttft, 95)),
            max_decode_batch_size=max(s['max_decode_batch_size'] for s in measured),
            mean_decode_batch_size=float(np.mean([s['mean_decode_batch_size'] for s in measured])),
            kv_reserved_peak_mib=max(s['kv_pool_reserved_bytes'] for s in measured) / 2 ** 20,
            kv_physical_mib=max(s['kv_pool_physical_bytes'] for s in measured) / 2 ** 20,
            unreturned_pages=max(s['kv_pool_used_pages_after'] for s in measured),
            unreturned_reservations=max(s['reserved_pages_after'] for s in measured))
    trace['continuous_vs_serial'] = trace['continuous']['output_tokens_per_sec'] / trace['serial']['output_tokens_per_sec']
    trace['token_parity_vs_independent_generation'] = bool(parity)

    modes = {}
    for n, prompt in prompts.items():
        gold_n = independent_tokens(model, prompt, new_tokens, precision)
        measured, match = [], True
        for repeat in range(warmup + repeats):
            r = _paged_request(model, prompt, new_tokens)
            match &= r.pop('tokens') == gold_n
            if repeat >= warmup:
                measured.append(r)
        seconds = sum(r['request_seconds'] for r in measured)
        decode = sum(r['decode_seconds'] for r in measured)
        modes[n] = dict(median_ttft_ms=float(np.median([r['ttft_seconds'] for r in measured])) * 1e3,
                        output_tokens_per_sec=new_tokens * len(measured) / seconds,
                        decode_tokens_per_sec=(new_tokens - 1) * len(measured) / decode,
                        kv_reserved_bytes=measured[-1]['kv_reserved_bytes'],
                        tokens_match_independent_generation=bool(match))
    return dict(precision=precision, warmup=warmup, repeats=repeats, trace=trace, inference_modes=modes)


def _paged_request(model, prompt, new_tokens, clock=time.perf_counter):
    """One batch-1 paged request timed as the reference's run_request
    (project/benchmark_inference.py:92-160): the cache is created inside the
    timed region, each step's token is read on the host."""
    runtime().synchronize()
    start = clock()
    cache = model.create_kv_cache(1, len(prompt) + new_tokens - 1, page_size=16,
                                  kv_budget_bytes=256 * 1024 ** 2, pages_per_slab=4)
    tokens, first, ids = [], None, None
    for step in range(new_tokens):
        if step == 0:
            logits, _ = model.prefill(DeviceTensor.from_numpy(np.array([prompt], np.float32)), cache)
        else:
            logits = model.decode_step(ids, cache)
        ids = greedy_token(logits)
        tokens.append(int(ids.to_numpy()[0, 0]))
        arrival = clock()
        if first is None:
            first = arrival
    reserved = cache.memory_stats()['kv_pool_reserved_bytes']
    cache.close()
    return dict(ttft_seconds=first - start, request_seconds=arrival - start, decode_seconds=arrival - first,
                kv_reserved_bytes=reserved, tokens=tokens)
