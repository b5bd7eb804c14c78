"""One decode step and the prefill of newly admitted requests in a single
layer loop (DecoderLM.decode_prefill_greedy over mt_mixed_layers) against the
same work as separate calls -- decode_greedy, closing the requests that end,
prefill_batch -- run on an identical second pool: page IDs, every cache's
page list, the free list and the pool counters bit-exact after every step;
fp32 greedy tokens (decode rows and first tokens) equal. In fp16 the decode
rows take hipBLASLt in the merged loop and the matrix-core projection kernel
in the separate one, so tokens are compared where both worlds still hold the
same tokens."""
import numpy as np
import pytest

from minitorch_amd.amp import autocast
from minitorch_amd.kv_cache import greedy_token
from minitorch_amd.model import DecoderLM
from minitorch_amd.paged_kv_cache import KVPagePool
from minitorch_amd.runtime import DeviceTensor, runtime

pytestmark = pytest.mark.gpu


def tiny(seed=0, layers=2, d=128, heads=2, vocab=512, positions=256):
    return DecoderLM(n_vocab=vocab, n_embd=d, n_head=heads, n_layer=layers, n_positions=positions, seed=seed)


class World:
    """A pool, its live caches (in a fixed order) and their last tokens."""

    def __init__(self, model, prompts, page_size):
        self.model = model
        self.pool = KVPagePool(model, page_size=page_size, max_bytes=4096 * 2 * model.n_layer * model.n_embd *
                               page_size * 4, pages_per_slab=5)
        self.caches = self.new_caches(len(prompts))
        logits = model.prefill_batch(prompts, self.caches)
        self.tokens = greedy_token(logits, feedback=list(self.caches)).to_numpy()[:, 0].astype(int).tolist()

    def new_caches(self, n):
        return [self.model.create_kv_cache(1, self.model.n_positions, page_size=self.pool.page_size,
                                           page_pool=self.pool) for _ in range(n)]

    def separate(self, finished, prompts):
        ids = self.model.decode_greedy(self.caches)
        for i in finished:
            self.caches[i].close()
        new = self.new_caches(len(prompts))
        first = greedy_token(self.model.prefill_batch(prompts, new), feedback=new) if prompts else None
        out = ids.to_numpy()[:, 0].tolist() + (first.to_numpy()[:, 0].tolist() if prompts else [])
        self._advance(finished, new)
        return [int(t) for t in out]

    def merged(self, finished, prompts):
        new = self.new_caches(len(prompts))
        ids = self.model.decode_prefill_greedy(self.caches, prompts, new,
                                               finished=[self.caches[i] for i in finished])
        out = [int(t) for t in ids.to_numpy()[:, 0]]
        self._advance(finished, new)
        return out

    def _advance(self, finished, new):
        self.caches = [c for i, c in enumerate(self.caches) if i not in finished] + new

    def close(self):
        for c in self.caches:
            c.close()
        assert self.pool.used_pages == 0
        self.pool.close()


def assert_same_pools(a, b):
    assert a.pool.free_stack() == b.pool.free_stack(), 'free list differs'
    ha, hb = a.pool.header(), b.pool.header()
    assert ha == hb, (ha, hb)
    assert a.pool.memory_stats() == b.pool.memory_stats()
    assert [c.pages() for c in a.caches] == [c.pages() for c in b.caches]
    assert [c.length for c in a.caches] == [c.length for c in b.caches]


def plan(rng, live, vocab, max_new=3):
    """Requests that end with this step (positions in the live list) and the
    prompts admitted after them."""
    finished = sorted(int(i) for i in np.nonzero(rng.random(live) < 0.3)[0])[:live - 1]
    prompts = [rng.integers(0, vocab, int(rng.integers(1, 70))) for _ in range(int(rng.integers(1, max_new + 1)))]
    return finished, prompts


@pytest.mark.parametrize('page_size', [8, 16])
def test_mixed_step_equals_separate_calls_fp32(page_size):
    model = tiny(seed=page_size)
    rng = np.random.default_rng(page_size)
    prompts = [rng.integers(0, model.n_vocab, int(n)) for n in rng.integers(1, 90, 6)]
    a, b = World(model, prompts, page_size), World(model, prompts, page_size)
    assert a.tokens == b.tokens
    for step in range(8):
        finished, new = plan(rng, len(a.caches), model.n_vocab)
        ta = a.separate(finished, new)
        tb = b.merged(finished, new)
        runtime().synchronize()
        assert ta == tb, f'step {step}: tokens differ at {[i for i, (x, y) in enumerate(zip(ta, tb)) if x != y]}'
        assert_same_pools(a, b)
    a.close()
    b.close()


def test_mixed_step_pages_and_tokens_fp16():
    model = tiny(seed=3, layers=3, d=256, heads=4)
    rng = np.random.default_rng(3)
    with autocast('float16'):
        prompts = [rng.integers(0, model.n_vocab, int(n)) for n in rng.integers(20, 200, 24)]
        a, b = World(model, prompts, 16), World(model, prompts, 16)
        assert a.tokens == b.tokens
        same = agree = 0
        for step in range(6):
            finished, new = plan(rng, len(a.caches), model.n_vocab, max_new=5)
            ta = a.separate(finished, new)
            tb = b.merged(finished, new)
            runtime().synchronize()
            if step == 0:
                # identical inputs: only the decode projections' rounding differs
                same += len(ta)
                agree += sum(x == y for x, y in zip(ta, tb))
            assert_same_pools(a, b)
        assert agree >= 0.9 * same, f'{agree} of {same} first-step tokens agree'
        a.close()
        b.close()


def test_mixed_step_argument_checks():
    model = tiny()
    rng = np.random.default_rng(0)
    w = World(model, [rng.integers(0, model.n_vocab, 9) for _ in range(2)], 16)
    other = w.new_caches(1)
    with pytest.raises(ValueError):   # a finished cache that is not decoded in the step
        model.decode_prefill_greedy(w.caches[:1], [np.arange(4)], other, finished=[w.caches[1]])
    with pytest.raises(ValueError):   # a new cache that is also decoded
        model.decode_prefill_greedy(w.caches, [np.arange(4)], [w.caches[0]])
    with pytest.raises(ValueError):   # one prompt per new cache
        model.decode_prefill_greedy(w.caches, [np.arange(4), np.arange(3)], other)
    runtime().synchronize()
    assert [c.length for c in w.caches] == [9, 9]
    for c in other:
        c.close()
    w.close()


def test_mixed_step_budget_exhaustion_changes_nothing():
    # the prompts together need more pages than the budget holds: the merged
    # step raises MemoryError before any change (no decode committed, the
    # ending cache still open, no new cache holding pages); the caller then
    # runs the separate calls, which fail at the same prompt, and both worlds
    # decode the next step to the same tokens and pool state
    model = tiny(seed=5)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, model.n_vocab, 40) for _ in range(3)]

    def world():
        w = World.__new__(World)
        w.model = model
        w.pool = KVPagePool(model, page_size=16, max_bytes=14 * 2 * model.n_layer * model.n_embd * 16 * 4,
                            pages_per_slab=2)
        w.caches = w.new_caches(len(prompts))
        w.tokens = greedy_token(model.prefill_batch(prompts, w.caches), feedback=list(w.caches))
        return w

    a, b = world(), world()
    big = [rng.integers(0, model.n_vocab, n) for n in (30, 60, 40)]   # 2 + 4 + 3 pages
    new_b = b.new_caches(3)
    before = (b.pool.free_stack(), b.pool.header(), b.pool.memory_stats(), [c.pages() for c in b.caches])
    with pytest.raises(MemoryError):
        b.model.decode_prefill_greedy(b.caches, big, new_b, finished=[b.caches[1]])
    runtime().synchronize()
    assert (b.pool.free_stack(), b.pool.header(), b.pool.memory_stats(), [c.pages() for c in b.caches]) == before
    assert [c.length for c in b.caches] == [40, 40, 40] and all(c.valid and not c.closed for c in b.caches)
    assert [c.length for c in new_b] == [0, 0, 0] and b.pool.used_pages == 9
    for c in new_b:
        c.close()
    for w in (a, b):
        # the separate calls, as the caller's fallback
        w.model.decode_greedy(w.caches)
        w.caches[1].close()
        new = w.new_caches(3)
        with pytest.raises(MemoryError):
            w.model.prefill_batch(big, new)
        for c in new:
            assert c.length == 0
            c.close()
        w._advance([1], [])
    runtime().synchronize()
    assert_same_pools(a, b)
    ta = a.model.decode_greedy(a.caches).to_numpy()[:, 0].tolist()
    tb = b.model.decode_greedy(b.caches).to_numpy()[:, 0].tolist()
    assert ta == tb
    assert_same_pools(a, b)
    a.close()
    b.close()


@pytest.mark.parametrize('dtype', ['float16', 'bfloat16'])
def test_mixed_step_logits_near_oracle(dtype):
    # The merged step's logits in fp16/bf16 (4 layers, d 256): every decode
    # row and every new prompt's last row against the fp64 numpy GPT-2 on its
    # own sequence, within 2 % of the logits' range (the bound of the other
    # low-precision model tests; a wrong row, layer or position misses it by
    # far), and the returned tokens are the first maxima of those logits.
    from oracle import gpt2_oracle as go
    model = tiny(seed=41, layers=4, d=256, heads=4)
    rng = np.random.default_rng(41)
    with autocast(dtype):
        prompts = [rng.integers(0, model.n_vocab, int(n)) for n in rng.integers(5, 120, 12)]
        w = World(model, prompts, 16)
        seqs = [list(p) + [t] for p, t in zip(prompts, w.tokens)]
        new_prompts = [rng.integers(0, model.n_vocab, int(n)) for n in (3, 50, 97)]
        new = w.new_caches(len(new_prompts))
        ids, logits = model.decode_prefill_greedy(w.caches, new_prompts, new, finished=[w.caches[4]],
                                                  return_logits=True)
        got = logits.to_numpy()[:, 0].astype(np.float64)
        assert np.array_equal(ids.to_numpy()[:, 0].astype(int), got.argmax(axis=1))
        w._advance([4], new)
        w.close()
    for i, seq in enumerate(seqs + [list(p) for p in new_prompts]):
        ref = go.forward(model.state, seq, n_head=model.n_head, n_layer=model.n_layer)[-1]
        err = np.abs(got[i] - ref).max()
        assert err <= 0.02 * (ref.max() - ref.min()), (i, err, ref.max() - ref.min())
