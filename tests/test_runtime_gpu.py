"""GPU tests of the host runtime's asynchronous paths: small uploads through
the pinned staging ring (reused only after its previous copy ran), in-order
token read-backs, and the sync-free batcher when requests are cancelled or
finished while their tokens are still in flight."""
import numpy as np
import pytest

from minitorch_amd.runtime import runtime, DeviceTensor, RawDeviceBuffer, STAGED_UPLOAD_BYTES
from minitorch_amd.kv_cache import TokenReadback

pytestmark = pytest.mark.gpu


def test_staged_uploads_survive_ring_reuse():
    # Far more small uploads than staging buffers, queued behind a slow copy,
    # each to its own destination: every destination must hold its own data.
    rt = runtime()
    rng = np.random.default_rng(0)
    big = RawDeviceBuffer(256 << 20)
    big2 = RawDeviceBuffer(256 << 20)
    rt.d2d(big2.ptr, big.ptr, 256 << 20)           # keep the queue busy
    arrays = [rng.integers(0, 1 << 30, int(rng.integers(1, STAGED_UPLOAD_BYTES // 4)), dtype=np.int32)
              for _ in range(100)]
    dests = [RawDeviceBuffer(a.nbytes) for a in arrays]
    for d, a in zip(dests, arrays):
        d.upload(a)
    for d, a in zip(dests, arrays):
        assert np.array_equal(d.download(np.int32), a)


def test_upload_then_overwrite_source_keeps_uploaded_values():
    # The staged copy takes the host data at call time.
    a = np.arange(1000, dtype=np.float32)
    t = DeviceTensor.from_numpy(a)
    a[:] = -1
    assert np.array_equal(t.to_numpy(), np.arange(1000, dtype=np.float32))


def test_token_readback_in_order():
    rb = TokenReadback(depth=4)
    ids = [DeviceTensor.from_numpy(np.arange(k, k + 5, dtype=np.float32)[:, None]) for k in range(4)]
    tickets = [rb.push(t) for t in ids]
    assert rb.pending == 4
    with pytest.raises(RuntimeError):
        rb.push(ids[0])                              # depth exhausted
    with pytest.raises(ValueError):
        rb.read(tickets[1])                          # out of order
    for k, t in enumerate(tickets):
        assert rb.read(t).tolist() == list(range(k, k + 5))
    assert rb.pending == 0 and rb.ready(tickets[-1])


def test_sync_free_batcher_cancel_and_finish_in_flight():
    # Cancel and finish requests right after steps that left their tokens in
    # flight: the pages come back, every delivered token belongs to a step
    # before the cancel/finish, and the tokens delivered equal the synchronous
    # loop's prefix for those requests.
    from minitorch_amd.model import DecoderLM
    from minitorch_amd.continuous_batching import ContinuousBatchingEngine
    model = DecoderLM(n_vocab=256, n_embd=64, n_head=2, n_layer=2, n_positions=128, seed=3)
    rng = np.random.default_rng(3)
    prompts = {f'r{i}': rng.integers(0, 256, int(rng.integers(3, 30))) for i in range(5)}

    def run(feedback):
        eng = ContinuousBatchingEngine(model, max_batch_size=4, kv_budget_bytes=64 << 20,
                                       token_feedback=feedback)
        for rid, p in prompts.items():
            eng.admit(rid, p, max_new_tokens=20)
        for _ in range(6):
            eng.step()
        eng.cancel('r0')
        eng.finish('r1')
        while eng.has_work:
            eng.step()
        out = {rid: (r.state, r.finish_reason, list(r.output_ids)) for rid, r in eng.requests.items()}
        stats = eng.pool.memory_stats()
        eng.close()
        return out, stats

    sync, s_stats = run(False)
    fb, f_stats = run(True)
    assert s_stats['kv_pool_used_pages'] == 0 and f_stats['kv_pool_used_pages'] == 0
    assert fb['r0'][:2] == ('cancelled', 'cancelled') and fb['r1'][:2] == ('completed', 'finished')
    for rid in prompts:
        # same states and the same tokens, including those generated before the
        # cancel/finish but delivered after it in the sync-free loop
        assert fb[rid] == sync[rid], rid
