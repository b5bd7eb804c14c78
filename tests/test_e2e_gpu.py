"""End-to-end configurations 3 and 4 on the GPU.

Config 3: the 256-request DistilGPT-2 trace (random init, Poisson arrivals at
32 req/s, prompts U{32..512}, outputs geometric with mean 128, EOS off, 16384
pages of 16 tokens, FIFO with the reference defaults max_prefills_per_step 1
and prefill_token_budget 512, max_batch_size 256) replayed on a step-indexed
clock (1 ms of arrivals per step), with the reference benchmark's gates
(project/benchmark_continuous_batching.py:50-66,115,189-191): in fp32 every
completed request's tokens equal independent per-request generation, and the
pool drains. Beyond the reference: the first 16 requests' tokens equal the
float64 numpy GPT-2 oracle, and after every step the decisions, KV counters,
each active request's page list and the device free stack equal the
scheduling restatement (BatcherOracle) fed with the GPU's tokens. The fp16
trace is checked the same way except for the token oracles.

Config 4: GPT-2-medium (24 layers, d 1024, 16 heads, random init) in bf16,
128 concurrent requests with contexts lognormal(median 256, sigma 1.2) in
[16, 1024], each replaced with a seeded 5 % probability per step: after every
step the device free stack, the pool header's counters and every cache's page
list equal a PoolOracle / CacheOracle replay (page free and reuse bit-exact,
reference minitorch/paged_kv_cache.py:71-103); one layer's decode attention
over the live pool equals the C oracle; the pool drains at close.
"""
import numpy as np
import pytest

from minitorch_amd.amp import autocast
from minitorch_amd.continuous_batching import ContinuousBatcher
from minitorch_amd.dtypes import encode_host, decode_host
from minitorch_amd.e2e import config3_step_trace, config4_lengths
from minitorch_amd.kv_cache import greedy_token
from minitorch_amd.model import distilgpt2, gpt2_medium
from minitorch_amd.paged_kv_cache import KVPagePool
from minitorch_amd import paged_ops
from minitorch_amd.runtime import DeviceTensor, RawDeviceBuffer, runtime
from minitorch_amd.workloads import PagedDecodeCase
from oracle import gpt2_oracle as go
from oracle import c_oracle
from oracle.pool_oracle import PoolOracle, CacheOracle, BatcherOracle
from tolerances import assert_attention_close

pytestmark = pytest.mark.gpu

SCHEDULE_KEYS = ('decode_request_ids', 'prefill_request_ids', 'logical_reserved_pages', 'peak_used_pages',
                 'kv_pool_used_pages', 'kv_pool_free_pages', 'kv_pool_reserved_bytes', 'kv_pool_page_acquires',
                 'kv_pool_page_releases', 'kv_pool_page_reuses')
PAGE_SIZE = 16
CONFIG3_PAGES = 16384


@pytest.fixture(scope='module')
def distil():
    return distilgpt2(seed=0)


@pytest.fixture(scope='module')
def trace3():
    return config3_step_trace(0)


class Run(dict):
    """A replay's tokens by request ID, with ``schedule``: every step's
    decisions and pool counters (SCHEDULE_KEYS)."""


def replay_config3(model, trace, precision):
    """Replay the step trace through ContinuousBatcher and, in lockstep, the
    scheduling restatement fed with the GPU's tokens; compare after every step
    that did work. Returns the batcher's outputs and the number of steps."""
    page_bytes = 2 * model.n_layer * model.n_embd * PAGE_SIZE * (4 if precision == 'fp32' else 2)
    budget = CONFIG3_PAGES * page_bytes
    batcher = ContinuousBatcher(model, max_batch_size=256, page_size=PAGE_SIZE, kv_budget_bytes=budget,
                                precision=precision, max_prefills_per_step=1, prefill_token_budget=512)
    pool_o = PoolOracle(page_bytes=page_bytes, page_size=PAGE_SIZE, max_bytes=budget,
                        pages_per_slab=batcher.pool.pages_per_slab)
    ob = BatcherOracle(pool_o, lambda rid, i: batcher.requests[rid].output_ids[i], max_batch_size=256,
                       max_prefills_per_step=1, prefill_token_budget=512, n_positions=model.n_positions)
    pending = list(trace)
    worked = 0
    schedule = []
    while pending or batcher.has_work:
        while pending and pending[0][0] <= batcher.iteration:
            _, rid, prompt, new = pending.pop(0)
            batcher.submit(rid, prompt, max_new_tokens=new)
            ob.submit(rid, prompt.tolist(), new)
        batcher.step()
        ob.step()
        s, o = batcher.last_step, ob.steps[-1]
        schedule.append({key: s[key] for key in SCHEDULE_KEYS})
        if not (s['decode_batch_size'] or s['prefill_request_ids']):
            assert not (o['decode_request_ids'] or o['prefill_request_ids'])
            continue
        worked += 1
        for key in SCHEDULE_KEYS:
            assert s[key] == o[key], (s['iteration'], key, s[key], o[key])
        for rid in s['active_request_ids']:
            assert batcher.requests[rid].cache.pages()[0] == ob.requests[rid].cache.pages[0], (s['iteration'], rid)
        assert batcher.pool.free_stack() == pool_o.free, s['iteration']
    assert not ob.has_work
    for _, rid, _, new in trace:
        r = batcher.requests[rid]
        assert (r.state, r.finish_reason, len(r.output_ids)) == ('completed', 'length', new), rid
        assert r.output_ids == ob.requests[rid].output
    # reference gate: every page returned (benchmark_continuous_batching.py:115)
    stats = batcher.pool.memory_stats()
    assert stats['kv_pool_used_pages'] == 0 and batcher.reserved_pages == 0
    assert batcher.pool.header()['leased'] == 0 and not pool_o.leased
    outputs = Run({rid: list(batcher.requests[rid].output_ids) for _, rid, _, _ in trace})
    outputs.schedule = schedule
    print(f'config 3 {precision}: {worked} working steps, peak {batcher.peak_used_pages} pages, '
          f'{stats["kv_pool_page_reuses"]} reuses, max decode batch '
          f'{max(len(x["decode_request_ids"]) for x in ob.steps)}', flush=True)
    batcher.close()
    return outputs



@pytest.fixture(scope='module')
def config3_fp32(distil, trace3):
    print('config 3 fp32 trace: 256 requests', flush=True)
    return replay_config3(distil, trace3, 'fp32')


def test_config3_fp32_trace_schedule_pages_and_drain(config3_fp32, trace3):
    assert len(config3_fp32) == 256
    assert sum(map(len, config3_fp32.values())) == sum(t[3] for t in trace3)


def generate(model, prompt, steps):
    """Independent generation, one request: prefill, then decode_step per
    token (the reference's reference_tokens, benchmark_continuous_batching.py:50-66)."""
    cache = model.create_kv_cache(1, len(prompt) + steps - 1, page_size=PAGE_SIZE)
    logits, _ = model.prefill(DeviceTensor.from_numpy(np.array([prompt], np.float32)), cache)
    out = [int(greedy_token(logits).to_numpy()[0, 0])]
    for _ in range(steps - 1):
        logits = model.decode_step(DeviceTensor.from_numpy(np.array([[out[-1]]], np.float32)), cache)
        out.append(int(greedy_token(logits).to_numpy()[0, 0]))
    cache.close()
    return out


def test_config3_fp32_tokens_equal_independent_generation(distil, config3_fp32, trace3):
    # the reference gate (benchmark_continuous_batching.py:189-191), on all 256
    mismatched = []
    for i, (_, rid, prompt, new) in enumerate(trace3):
        if generate(distil, prompt.tolist(), new) != config3_fp32[rid]:
            mismatched.append(rid)
        if i % 64 == 63:
            print(f'independent generation: {i + 1} of 256', flush=True)
    assert not mismatched, mismatched


def test_config3_fp32_prefix_equals_gpt2_oracle(distil, config3_fp32, trace3):
    # the first 16 requests, their first 128 tokens (or all of them), against
    # the float64 numpy GPT-2 (pinned to transformers' GPT2LMHeadModel);
    # top-1/top-2 margins are reported on a mismatch
    first = trace3[:16]
    counts = [min(new, 128) for *_, new in first]
    tokens, margins = go.greedy_cached(distil.state, [p for _, _, p, _ in first], counts,
                                       n_head=distil.n_head, n_layer=distil.n_layer)
    for (_, rid, _, _), n, ref, m in zip(first, counts, tokens, margins):
        got = config3_fp32[rid][:n]
        if got != ref:
            k = next(j for j in range(n) if got[j] != ref[j])
            pytest.fail(f'{rid}: token {k} is {got[k]}, oracle {ref[k]} (margin {m[k]:.3g}, '
                        f'smallest margin before it {min(m[:k + 1]):.3g})')


def test_config3_fp32_merged_sync_free_loop_equals_synchronous(distil, config3_fp32, trace3):
    # the same trace through the sync-free loop whose admitting steps run the
    # decode and the prefill as one layer loop (merge_prefill): every step's
    # decisions and pool counters, and every request's tokens, equal the
    # synchronous replay (itself checked against the scheduling oracle)
    page_bytes = 2 * distil.n_layer * distil.n_embd * PAGE_SIZE * 4
    batcher = ContinuousBatcher(distil, max_batch_size=256, page_size=PAGE_SIZE,
                                kv_budget_bytes=CONFIG3_PAGES * page_bytes, precision='fp32',
                                max_prefills_per_step=1, prefill_token_budget=512, token_feedback=True,
                                merge_prefill=True)
    pending = list(trace3)
    schedule = []
    while pending or batcher.has_work:
        while pending and pending[0][0] <= batcher.iteration:
            _, rid, prompt, new = pending.pop(0)
            batcher.submit(rid, prompt, max_new_tokens=new)
        batcher.step()
        schedule.append({key: batcher.last_step[key] for key in SCHEDULE_KEYS})
    sync = config3_fp32.schedule
    assert len(schedule) >= len(sync)
    for i, (a, b) in enumerate(zip(sync, schedule)):
        assert a == b, (i, a, b)
    for extra in schedule[len(sync):]:  # trailing steps only deliver tokens
        assert not extra['decode_request_ids'] and not extra['prefill_request_ids']
    mismatched = [rid for _, rid, _, _ in trace3 if batcher.requests[rid].output_ids != config3_fp32[rid]]
    assert not mismatched, mismatched[:5]
    assert batcher.pool.memory_stats()['kv_pool_used_pages'] == 0
    batcher.close()


def test_config3_fp16_trace_completes_with_oracle_schedule(distil, trace3):
    print('config 3 fp16 trace: 256 requests', flush=True)
    outputs = replay_config3(distil, trace3, 'fp16')
    assert len(outputs) == 256


# ---------------------------------------------------------------- config 4 ---

def _layer_block(pool, layer):
    """Host copy of one layer's K/V planes of every opened slab, as an image
    [num_slabs, 1, 2, pps, H, P, D] in storage format."""
    pps, h, d = pool.pages_per_slab, pool.heads, pool.dim
    elems = 2 * pps * h * PAGE_SIZE * d
    raw = np.empty((pool.num_slabs, 1, 2, pps, h, PAGE_SIZE, d), np.uint16)
    for s in range(pool.num_slabs):
        raw[s] = pool.kv.download(np.uint16, elems, s * pool.slab_bytes + layer * elems * 2).reshape(
            1, 2, pps, h, PAGE_SIZE, d)
    return raw


def test_config4_gpt2_medium_pages_reuse_and_attention():
    model = gpt2_medium(seed=0)
    concurrent, steps, layer = 128, 12, 7
    rng = np.random.default_rng([0, 4])
    page_bytes = 2 * model.n_layer * model.n_embd * PAGE_SIZE * 2
    max_bytes = concurrent * (model.n_positions // PAGE_SIZE) * page_bytes
    with autocast('bfloat16'):
        pool = KVPagePool(model, page_size=PAGE_SIZE, max_bytes=max_bytes, pages_per_slab=16)
        po = PoolOracle(page_bytes=page_bytes, page_size=PAGE_SIZE, max_bytes=max_bytes, pages_per_slab=16)
        caches, shadows, last = [], [], []

        def draw():
            return rng.integers(0, model.n_vocab, int(config4_lengths(rng, 1)[0]) - 1)

        def admit(prompts):
            new = [model.create_kv_cache(1, model.n_positions, page_size=PAGE_SIZE, page_pool=pool)
                   for _ in prompts]
            logits = model.prefill_batch(prompts, new)
            first = [int(t) for t in greedy_token(logits).to_numpy()[:, 0]]
            shadow = []
            for p in prompts:   # the batched prefill takes pages prompt by prompt
                c = CacheOracle(po, 1, model.n_positions)
                c.prepare_append(len(p))
                c.commit_append()
                shadow.append(c)
            return new, shadow, first

        def check(where):
            hdr = pool.header()
            assert (hdr['leased'], hdr['acquires'], hdr['releases'], hdr['reuses']) == (
                len(po.leased), po.page_acquires, po.page_releases, po.page_reuses), where
            assert pool.free_stack() == po.free, where
            for i, (c, o) in enumerate(zip(caches, shadows)):
                assert c.pages()[0] == o.pages[0], (where, i)
                assert c.length == o.length, (where, i)

        for c0 in range(0, concurrent, 32):
            new, shadow, first = admit([draw() for _ in range(32)])
            caches += new
            shadows += shadow
            last += first
        check('admission')
        replaced = 0
        for step in range(steps):
            ids = DeviceTensor.from_numpy(np.array(last, np.float32)[:, None])
            last = [int(t) for t in greedy_token(model.decode_batch(ids, caches)).to_numpy()[:, 0]]
            for o in shadows:
                o.prepare_append(1)
            for o in shadows:
                o.commit_append()
            check(f'decode step {step}')
            slots, prompts = [], []
            for i in range(concurrent):
                if rng.random() < 0.05 or caches[i].length + 1 >= caches[i].capacity:
                    caches[i].close()
                    shadows[i].close()
                    slots.append(i)
                    prompts.append(draw())
            if slots:
                new, shadow, first = admit(prompts)
                for i, c, o, t in zip(slots, new, shadow, first):
                    caches[i], shadows[i], last[i] = c, o, t
                replaced += len(slots)
            check(f'replacement step {step}')
        assert replaced > 0 and po.page_reuses > 0
        print(f'config 4: {replaced} replacements, {po.page_reuses} page reuses, '
              f'{pool.num_slabs} slabs', flush=True)

        # One layer's decode attention over the live pool against the C
        # oracle: random bf16 q/k/v, every request appending at its last
        # committed position (its pages exist), layer 7 of 24.
        b, h, d = concurrent, model.n_head, model.n_embd // model.n_head
        lengths = np.array([c.length for c in caches], np.int64)
        tables = [c.pages()[0] for c in caches]
        columns = max(map(len, tables))
        table = np.full((b, columns), -1, np.int32)
        for i, t in enumerate(tables):
            table[i, :len(t)] = t
        image = _layer_block(pool, layer)
        q, k, v = (encode_host(rng.standard_normal((b, h, 1, d), dtype=np.float32), 'bfloat16')
                   .reshape(b, h, 1, d) for _ in range(3))
        case = PagedDecodeCase(b, h, d, PAGE_SIZE, pool.pages_per_slab, pool.num_slabs, 1, 0, 'bfloat16',
                               lengths, table, image, q, k, v)
        host = c_oracle.HostCase(case)
        ref = decode_host(host.run(c_oracle.library()), 'bfloat16').reshape(b, h, 1, d)
        dq, dk, dv, dout = (DeviceTensor((b, h, 1, d), 'bfloat16') for _ in range(4))
        for t, a in ((dq, q), (dk, k), (dv, v)):
            runtime().h2d(t.ptr, a)
        dtable, doffs = RawDeviceBuffer(table.nbytes), RawDeviceBuffer(4 * b)
        dtable.upload(table)
        doffs.upload((lengths - 1).astype(np.int32))
        paged_ops.paged_decode_batch(dout.ptr, dq.ptr, dk.ptr, dv.ptr, pool.slab_table.ptr, dtable.ptr,
                                     doffs.ptr, b=b, h=h, d=d, page_size=PAGE_SIZE,
                                     pages_per_slab=pool.pages_per_slab, num_slabs=pool.num_slabs,
                                     columns=columns, layer=layer, layers=model.n_layer, dtype='bfloat16')
        runtime().synchronize()
        assert_attention_close(dout.to_numpy(), ref, 'bfloat16', context='config 4 layer 7', ref_rounded=True)
        assert np.array_equal(_layer_block(pool, layer), host.image), 'append into the live pool differs'

        for c, o in zip(caches, shadows):
            c.close()
            o.close()
        assert pool.free_stack() == po.free
        assert pool.used_pages == 0 and pool.header()['leased'] == 0 and not po.leased
        pool.close()
