"""Failure handling of the decode path, with errors forced from the host.

A native entry returning a nonzero status raises ``RuntimeError('CUDA: ...')``
in ``runtime.call`` (reference minitorch/cuda_resident_ops.py:41-44). These
tests make the model's native layer loops return status 1 from the host side
(no kernel is made to fail) and check what the reference's Python does with
it:
* a failed decode step marks every request of the batch ``failed`` with
  ``decode_error`` and returns its pages (minitorch/continuous_batching.py:149-152);
* a failed prefill marks the admitted request ``failed`` with
  ``prefill_error`` (:172-174) and leaves the others running;
* ``PagedDecodeBatch`` aborts every prepared cache on a failure, returning
  the pages the step took and invalidating the caches
  (minitorch/paged_decode.py:85-93, minitorch/kv_cache.py:149-152);
* changing the model's weights invalidates live caches
  (minitorch/kv_cache.py:78-82,104).
"""
import numpy as np
import pytest

from minitorch_amd import model as model_module
from minitorch_amd.continuous_batching import ContinuousBatcher
from minitorch_amd.kv_cache import greedy_token
from minitorch_amd.model import DecoderLM
from minitorch_amd.paged_kv_cache import KVPagePool
from minitorch_amd.runtime import DeviceTensor, runtime

pytestmark = pytest.mark.gpu


def tiny(seed=0):
    return DecoderLM(n_vocab=256, n_embd=64, n_head=2, n_layer=2, n_positions=128, seed=seed)


def generate(model, prompt, steps):
    cache = model.create_kv_cache(1, len(prompt) + steps - 1, page_size=16)
    logits, _ = model.prefill(DeviceTensor.from_numpy(np.array([prompt], np.float32)), cache)
    out = [int(greedy_token(logits).to_numpy()[0, 0])]
    for _ in range(steps - 1):
        logits = model.decode_step(DeviceTensor.from_numpy(np.array([[out[-1]]], np.float32)), cache)
        out.append(int(greedy_token(logits).to_numpy()[0, 0]))
    cache.close()
    return out


class FailOnce:
    """Stands in for ``runtime.call`` in the model module: the first call of
    ``name`` returns status 1 (as a native entry rejecting its arguments
    would), so ``call`` raises; every other call goes through."""

    def __init__(self, name):
        self.name, self.fired, self.real = name, 0, model_module.call

    def __call__(self, lib, name, signature, *args):
        if name == self.name and not self.fired:
            self.fired += 1
            runtime().check(1)
        return self.real(lib, name, signature, *args)


def test_decode_error_fails_the_batch_and_returns_its_pages(monkeypatch):
    model = tiny(1)
    rng = np.random.default_rng(1)
    prompts = {f'r{i}': rng.integers(0, 256, n) for i, n in enumerate((20, 31, 5, 12))}
    b = ContinuousBatcher(model, max_batch_size=3, kv_budget_bytes=64 << 20)
    for rid, p in prompts.items():
        b.submit(rid, p, max_new_tokens=8)
    for _ in range(4):                      # r0..r2 admitted and decoding, r3 queued
        b.step()
    assert list(b.active) == ['r0', 'r1', 'r2'] and b.requests['r3'].state == 'queued'
    assert b.pool.used_pages > 0
    fail = FailOnce('mt_decoder_layers')
    monkeypatch.setattr(model_module, 'call', fail)
    with pytest.raises(RuntimeError, match='CUDA'):
        b.step()
    assert fail.fired == 1
    for rid in ('r0', 'r1', 'r2'):
        r = b.requests[rid]
        assert (r.state, r.finish_reason, r.cache) == ('failed', 'decode_error', None), rid
    assert b.pool.used_pages == 0 and b.reserved_pages == 0 and not b.active
    hdr = b.pool.header()
    assert hdr['leased'] == 0 and hdr['error'] == 0
    assert len(b.pool.free_stack()) == b.pool.num_slabs * b.pool.pages_per_slab
    # the queued request still runs to completion, with the tokens of an
    # independent generation
    while b.has_work:
        b.step()
    r3 = b.requests['r3']
    assert r3.state == 'completed' and r3.output_ids == generate(model, prompts['r3'].tolist(), 8)
    assert b.pool.used_pages == 0
    b.close()


def test_prefill_error_fails_the_request_and_keeps_the_others(monkeypatch):
    model = tiny(2)
    rng = np.random.default_rng(2)
    prompts = {f'r{i}': rng.integers(0, 256, n) for i, n in enumerate((17, 40, 9))}
    b = ContinuousBatcher(model, max_batch_size=4, kv_budget_bytes=64 << 20)
    b.submit('r0', prompts['r0'], max_new_tokens=6)
    b.step()                                # r0 prefilled
    used = b.pool.used_pages
    b.submit('r1', prompts['r1'], max_new_tokens=6)
    b.submit('r2', prompts['r2'], max_new_tokens=6)
    fail = FailOnce('mt_prefill_layers')
    monkeypatch.setattr(model_module, 'call', fail)
    with pytest.raises(RuntimeError, match='CUDA'):
        b.step()                            # decodes r0, then r1's prefill fails
    r1 = b.requests['r1']
    assert (r1.state, r1.finish_reason, r1.cache) == ('failed', 'prefill_error', None)
    # r0 decoded one more token in that step (one new page at most); r1's
    # pages and reservation are gone; r2 is still queued
    assert b.requests['r0'].state == 'active' and len(b.requests['r0'].output_ids) == 2
    assert b.pool.used_pages == b.requests['r0'].cache.nbytes // b.pool.page_bytes >= used
    assert b.reserved_pages == b.requests['r0'].reserved_pages
    assert b.requests['r2'].state == 'queued'
    while b.has_work:
        b.step()
    for rid in ('r0', 'r2'):
        r = b.requests[rid]
        assert r.state == 'completed' and r.output_ids == generate(model, prompts[rid].tolist(), 6), rid
    assert b.pool.used_pages == 0 and b.reserved_pages == 0
    b.close()


def test_failed_decode_batch_aborts_every_cache(monkeypatch):
    # Rows at a page boundary take a page in prepare; the failure returns
    # those pages in row order (as the pool restatement does), leaves the
    # committed lengths, and invalidates the caches.
    from oracle.pool_oracle import PoolOracle, CacheOracle, decode_batch_metadata
    model = tiny(3)
    rng = np.random.default_rng(3)
    pool = KVPagePool(model, page_size=16, max_bytes=64 << 20)
    po = PoolOracle(page_bytes=pool.page_bytes, page_size=16, max_bytes=64 << 20, pages_per_slab=pool.pages_per_slab)
    caches, shadows, last = [], [], []
    for n in (16, 32, 7):
        c = model.create_kv_cache(1, 60, page_size=16, page_pool=pool)
        logits, _ = model.prefill(DeviceTensor.from_numpy(rng.integers(0, 256, (1, n)).astype(np.float32)), c)
        caches.append(c)
        last.append(int(greedy_token(logits).to_numpy()[0, 0]))
        o = CacheOracle(po, 1, 60)
        o.prepare_append(n)
        o.commit_append()
        shadows.append(o)
    used = pool.used_pages
    monkeypatch.setattr(model_module, 'call', FailOnce('mt_decoder_layers'))
    with pytest.raises(RuntimeError, match='CUDA'):
        model.decode_batch(DeviceTensor.from_numpy(np.array(last, np.float32)[:, None]), caches)
    decode_batch_metadata(shadows)          # the step's prepare: two rows take a page
    for o in shadows:
        o.abort_append()
    assert po.page_acquires == pool.header()['acquires'] and len(po.leased) == used
    assert pool.used_pages == used and pool.free_stack() == po.free
    assert pool.header()['leased'] == used
    assert [c.length for c in caches] == [16, 32, 7]
    assert [c.pages()[0] for c in caches] == [o.pages[0] for o in shadows]
    assert not any(c.valid for c in caches)
    with pytest.raises(ValueError, match='invalid'):
        model.decode_batch(DeviceTensor.from_numpy(np.array(last, np.float32)[:, None]), caches)
    for c, o in zip(caches, shadows):
        c.close()
        o.close()
    assert pool.used_pages == 0 and pool.header()['leased'] == 0 and pool.free_stack() == po.free
    pool.close()


def test_weight_change_invalidates_live_caches():
    model = tiny(4)
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, 256, 10)
    cache = model.create_kv_cache(1, 30, page_size=16)
    logits, _ = model.prefill(DeviceTensor.from_numpy(prompt[None].astype(np.float32)), cache)
    token = greedy_token(logits).to_numpy()
    state = {k: v.copy() for k, v in model.state.items()}
    state['transformer.h.0.mlp.c_fc.bias'] = state['transformer.h.0.mlp.c_fc.bias'] + 0.5
    model.load_state(state)
    with pytest.raises(ValueError, match='weights changed'):
        model.decode_step(DeviceTensor.from_numpy(token), cache)
    with pytest.raises(ValueError, match='weights changed'):
        model.decode_batch(DeviceTensor.from_numpy(token), [cache])
    # reset re-binds the cache to the new weights (reference kv_cache.py:154-160)
    cache.reset()
    logits, _ = model.prefill(DeviceTensor.from_numpy(prompt[None].astype(np.float32)), cache)
    fresh = model.create_kv_cache(1, 30, page_size=16)
    ref, _ = model.prefill(DeviceTensor.from_numpy(prompt[None].astype(np.float32)), fresh)
    assert np.array_equal(logits.to_numpy(), ref.to_numpy())
    cache.close()
    fresh.close()
