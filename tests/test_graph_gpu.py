"""Captured decode steps (HIP graphs) against eager steps.

A sync-free decode step with ``graph=True`` replays its device work (page
pops and metadata, embeddings, the layer loop, greedy selection, length
commit) from a graph captured per batch size after a few eager steps. Every
replay must give the eager step's tokens bit for bit and the same pages; the
replays are interleaved with eager work of the program (prefills, other
batches) and host synchronizations, and each one is checked.
"""
import numpy as np
import pytest

from minitorch_amd.amp import autocast
from minitorch_amd.continuous_batching import ContinuousBatcher
from minitorch_amd.kv_cache import greedy_token
from minitorch_amd.model import DecoderLM, GRAPH_WARMUP
from minitorch_amd.paged_kv_cache import KVPagePool
from minitorch_amd.runtime import DeviceTensor, runtime

pytestmark = pytest.mark.gpu


def tiny(seed=0, d=128, heads=2, layers=2, vocab=512, positions=160):
    return DecoderLM(n_vocab=vocab, n_embd=d, n_head=heads, n_layer=layers, n_positions=positions, seed=seed)


def steady_loop(model, graph, steps, seed, concurrent=12, dtype=None, replace=0.2):
    """A config-4-style loop on its own pool: ``concurrent`` requests decoded
    every step (sync-free), each replaced with probability ``replace`` by a
    fresh prefilled one. Returns per-step token arrays, the pages of every
    cache after each step, and the final free stack."""
    rng = np.random.default_rng(seed)
    ctx = autocast(dtype) if dtype else None
    if ctx:
        ctx.__enter__()
    try:
        pool = KVPagePool(model, page_size=16, max_bytes=64 << 20, pages_per_slab=4)

        def admit(n):
            if n == 0:
                return []
            prompts = [rng.integers(0, model.n_vocab, int(rng.integers(1, 100))) for _ in range(n)]
            caches = [model.create_kv_cache(1, model.n_positions, page_size=16, page_pool=pool) for _ in prompts]
            greedy_token(model.prefill_batch(prompts, caches), feedback=caches)
            return caches

        caches = admit(concurrent)
        tokens, pages = [], []
        for step in range(steps):
            ids = model.decode_greedy(caches, graph=graph)
            tokens.append(ids.to_numpy()[:, 0].copy())     # a host synchronization between replays
            pages.append([c.pages()[0] for c in caches])
            slots = [i for i in range(concurrent)
                     if rng.random() < replace or caches[i].length + 1 >= caches[i].capacity]
            for i in slots:
                caches[i].close()
            for i, c in zip(slots, admit(len(slots))):      # eager prefills between replays
                caches[i] = c
        stack = pool.free_stack()
        for c in caches:
            c.close()
        ws = pool._decode_workspace
        captured = len(ws.graphs)
        pool.close()
        return tokens, pages, stack, captured
    finally:
        if ctx:
            ctx.__exit__(None, None, None)


@pytest.mark.parametrize('dtype', [None, 'bfloat16'])
def test_graph_replays_equal_eager_steps(dtype):
    model = tiny(seed=41)
    steps = GRAPH_WARMUP + 12
    eager = steady_loop(model, False, steps, seed=41, dtype=dtype)
    graph = steady_loop(model, True, steps, seed=41, dtype=dtype)
    assert graph[3] == 1, 'one batch size: one captured step'
    for k in range(steps):
        assert np.array_equal(eager[0][k], graph[0][k]), f'step {k}: tokens differ'
        assert eager[1][k] == graph[1][k], f'step {k}: pages differ'
    assert eager[2] == graph[2]


def test_graph_batcher_matches_eager_batcher():
    # The sync-free batcher with graph replay: batch sizes change as requests
    # arrive and finish (a graph per size), budget-limited admission; same
    # tokens, decisions and pages as without graphs.
    model = tiny(seed=43)
    rng = np.random.default_rng(43)
    trace = [(int(rng.integers(0, 30)), f'r{i}', rng.integers(0, model.n_vocab, int(rng.integers(3, 90))),
              int(rng.integers(5, 40))) for i in range(24)]
    trace.sort(key=lambda t: t[0])

    def run(graph):
        b = ContinuousBatcher(model, max_batch_size=6, kv_budget_bytes=2 * 2 * 128 * 16 * 4 * 60,
                              token_feedback=True, graph=graph)
        pending, steps = list(trace), []
        while pending or b.has_work:
            while pending and pending[0][0] <= b.iteration:
                _, rid, p, n = pending.pop(0)
                b.submit(rid, p, max_new_tokens=n)
            b.step()
            steps.append({k: b.last_step[k] for k in ('decode_request_ids', 'prefill_request_ids',
                                                      'kv_pool_used_pages', 'kv_pool_page_acquires',
                                                      'kv_pool_page_reuses')})
        out = {rid: list(r.output_ids) for rid, r in b.requests.items()}
        stack = b.pool.free_stack()
        graphs = len(b.pool._decode_workspace.graphs)
        b.close()
        return out, steps, stack, graphs

    eager, graph = run(False), run(True)
    assert graph[3] >= 2, 'several batch sizes captured'
    assert graph[0] == eager[0]
    assert graph[1] == eager[1]
    assert graph[2] == eager[2]


@pytest.mark.parametrize('concurrent', [4, 16])
def test_graph_distilgpt2_shape_replays(concurrent):
    # DistilGPT-2 shapes (d 768, 12 heads, vocab 50257) in fp16; 4 requests
    # take the decode loop with the LayerNorm inside the QKV and fc
    # projections, 16 the one with separate residual LayerNorm kernels
    model = DecoderLM(n_vocab=50257, n_embd=768, n_head=12, n_layer=6, n_positions=1024, seed=45)
    steps = GRAPH_WARMUP + 6
    eager = steady_loop(model, False, steps, seed=45, concurrent=concurrent, dtype='float16', replace=0.1)
    graph = steady_loop(model, True, steps, seed=45, concurrent=concurrent, dtype='float16', replace=0.1)
    for k in range(steps):
        assert np.array_equal(eager[0][k], graph[0][k]), f'step {k}'
        assert eager[1][k] == graph[1][k], f'step {k}: pages differ'


def test_failed_capture_falls_back_to_eager_steps(monkeypatch):
    # A capture that fails (forced from the host here) leaves that batch size
    # running eagerly, with the eager loop's tokens and pages.
    model = tiny(seed=49)

    def refuse(*args, **kwargs):
        raise RuntimeError('CUDA: operation not permitted when stream is capturing')

    steps = GRAPH_WARMUP + 4
    eager = steady_loop(model, False, steps, seed=49)
    monkeypatch.setattr(model, '_capture_decode', refuse)
    fallback = steady_loop(model, True, steps, seed=49)
    assert fallback[3] == 0
    for k in range(steps):
        assert np.array_equal(eager[0][k], fallback[0][k]), f'step {k}'
        assert eager[1][k] == fallback[1][k]
