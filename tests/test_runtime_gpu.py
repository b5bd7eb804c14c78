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
    # flight: the pages come back, nothing is delivered to those requests
    # after the cancel/finish (their in-flight tokens are dropped, as the
    # reference emits nothing after a cancel), what they did receive is a
    # prefix of the synchronous loop's tokens, and every other request gets
    # exactly the synchronous loop's tokens.
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
        at_end = {rid: len(eng.requests[rid].output_ids) for rid in ('r0', 'r1')}
        eng.cancel('r0')
        eng.finish('r1')
        late = []
        while eng.has_work:
            late += [e['request_id'] for e in eng.step()]
        out = {rid: (r.state, r.finish_reason, list(r.output_ids)) for rid, r in eng.requests.items()}
        stats = eng.pool.memory_stats()
        eng.close()
        return out, stats, late, at_end

    sync, s_stats, s_late, s_end = run(False)
    fb, f_stats, f_late, f_end = run(True)
    assert s_stats['kv_pool_used_pages'] == 0 and f_stats['kv_pool_used_pages'] == 0
    assert fb['r0'][:2] == ('cancelled', 'cancelled') and fb['r1'][:2] == ('completed', 'finished')
    for late, end, out in ((s_late, s_end, sync), (f_late, f_end, fb)):
        assert 'r0' not in late and 'r1' not in late
        assert all(len(out[rid][2]) == end[rid] for rid in ('r0', 'r1'))
    assert f_end['r0'] < s_end['r0']                    # a token was in flight and was dropped
    for rid in prompts:
        if rid in ('r0', 'r1'):
            assert fb[rid][:2] == sync[rid][:2]
            assert fb[rid][2] == sync[rid][2][:len(fb[rid][2])], rid
        else:
            assert fb[rid] == sync[rid], rid


def _reference_runtime():
    # The reference's CudaRuntime binding loop over this build's cuda_runtime.so.
    import ctypes as ct
    from minitorch_amd.runtime import LIB_DIR, P, I, Z
    lib = ct.CDLL(str(LIB_DIR / 'cuda_runtime.so'))
    sig = {'mt_random': [P, I, ct.c_ulonglong], 'mt_one_hot': [P, P, I, I], 'mt_sequence': [P, I, I],
           'mt_blas_create': [ct.POINTER(P)], 'mt_blas_destroy': [P], 'mt_gemm': [P, P, P, P, I, I, I],
           'mt_sync': []}
    for name, args in sig.items():
        f = getattr(lib, name)
        f.argtypes, f.restype = args, I
    return lib


def _splitmix_unit(seed, n):
    # SplitMix64's output function of seed * gamma + i, top 24 bits / 2^24.
    with np.errstate(over='ignore'):
        z = np.uint64(seed) * np.uint64(0x9E3779B97F4A7C15) + np.arange(n, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z ^= z >> np.uint64(31)
    return (z >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)


def test_runtime_random_known_answers_and_range():
    lib = _reference_runtime()
    out = DeviceTensor.empty((100003,))
    assert lib.mt_random(out.ptr, 100003, 1) == 0
    a = out.to_numpy()
    # seed 1, index 0 is SplitMix64's first output for state 0: 0xE220A8397B1DCDAF
    assert a[0] == np.float32(0xE220A8 / 2 ** 24)
    assert lib.mt_random(out.ptr, 1, 2) == 0
    # seed 2, index 0 is its second output: 0x6E789E6AA1B965F4
    assert out.to_numpy()[0] == np.float32(0x6E789E / 2 ** 24)
    assert np.array_equal(a, _splitmix_unit(1, 100003))
    assert a.min() >= 0 and a.max() < 1
    # uniform: 64 bins, chi-square well inside its 99.9 % bound (df 63: 103.4)
    counts = np.histogram(a, bins=64, range=(0, 1))[0]
    expected = len(a) / 64
    assert ((counts - expected) ** 2 / expected).sum() < 103.4
    assert lib.mt_random(out.ptr, 100003, 1) == 0
    assert np.array_equal(out.to_numpy(), a)          # deterministic per seed
    assert lib.mt_random(out.ptr, 100003, 7) == 0
    assert not np.array_equal(out.to_numpy(), a)
    assert lib.mt_random(None, 0, 3) == 0              # nothing to launch


def test_runtime_one_hot_and_sequence():
    lib = _reference_runtime()
    ids = np.array([0, 4, 2.7, -1, np.nan, 1e10, 3, -0.5], np.float32)
    classes = 5
    d_ids = DeviceTensor.from_numpy(ids)
    out = DeviceTensor.empty((len(ids), classes))
    assert lib.mt_one_hot(out.ptr, d_ids.ptr, len(ids) * classes, classes) == 0
    # truncation toward zero; NaN reads as 0; out-of-range ids match nothing
    want = np.zeros((len(ids), classes), np.float32)
    for r, x in enumerate([0, 4, 2, -1, 0, None, 3, 0]):
        if x is not None and 0 <= x < classes:
            want[r, x] = 1
    assert np.array_equal(out.to_numpy(), want)
    seq = DeviceTensor.empty((37,))
    assert lib.mt_sequence(seq.ptr, 37, 0) == 0
    assert np.array_equal(seq.to_numpy(), np.arange(37, dtype=np.float32))
    w = 6
    mask = DeviceTensor.empty((w, w))
    assert lib.mt_sequence(mask.ptr, w * w, w) == 0
    i = np.arange(w * w)
    want = np.where(i % w > i // w, np.float32(-3.402823466e38), np.float32(0)).reshape(w, w)
    assert np.array_equal(mask.to_numpy(), want)
    assert np.array_equal(want, np.triu(np.full((w, w), np.float32(-3.402823466e38)), 1))


def test_runtime_blas_handle_and_gemm_forward_to_hipblaslt():
    import ctypes as ct
    from minitorch_amd.runtime import library, P, I
    lib = _reference_runtime()
    handle = P()
    assert lib.mt_blas_create(ct.byref(handle)) == 0 and handle.value
    rng = np.random.default_rng(5)
    m, n, k = 37, 53, 300
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    da, db, dc = DeviceTensor.from_numpy(a), DeviceTensor.from_numpy(b), DeviceTensor.empty((m, n))
    assert lib.mt_gemm(handle, dc.ptr, da.ptr, db.ptr, m, n, k) == 0
    ref = a.astype(np.float64) @ b.astype(np.float64)
    got = dc.to_numpy()
    # fp32 accumulation over k terms: |err| <= k * eps32 * sum |a||b| per element
    bound = k * 2.0 ** -23 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(got - ref) <= bound)
    # the same handle drives model_kernels.so's own GEMM
    mk = library('model_kernels')
    mk.mt_gemm.argtypes, mk.mt_gemm.restype = [P, P, P, P, I, I, I], I
    dc2 = DeviceTensor.empty((m, n))
    assert mk.mt_gemm(handle, dc2.ptr, da.ptr, db.ptr, m, n, k) == 0
    assert np.array_equal(dc2.to_numpy(), got)
    assert lib.mt_blas_destroy(handle) == 0
