"""Pin the numpy GPT-2 oracle (oracle/gpt2_oracle.py) against transformers'
GPT2LMHeadModel built locally from a GPT2Config (no download), in float64,
with non-trivial LayerNorm gains and biases. This is the reference's own
oracle for its model (project/benchmark_inference.py:62-71)."""
import numpy as np
import pytest

from oracle import gpt2_oracle as go
from minitorch_amd.model import init_gpt2_state


def test_oracle_matches_hf_gpt2_float64():
    torch = pytest.importorskip('torch')
    transformers = pytest.importorskip('transformers')
    cfg = transformers.GPT2Config(vocab_size=97, n_positions=64, n_embd=32, n_layer=2, n_head=4,
                                  activation_function='gelu_new', resid_pdrop=0.0, embd_pdrop=0.0,
                                  attn_pdrop=0.0, bos_token_id=0, eos_token_id=0)
    state = init_gpt2_state(n_vocab=97, n_embd=32, n_layer=2, n_positions=64, seed=3)
    rng = np.random.default_rng(0)
    for k in state:
        if k.endswith('bias') or '.ln_' in k:
            state[k] = (state[k] + 0.1 * rng.standard_normal(state[k].shape)).astype(np.float32)
    model = transformers.GPT2LMHeadModel(cfg).double().eval()
    model.load_state_dict({k: torch.tensor(v, dtype=torch.float64) for k, v in state.items()}, strict=False)
    ids = rng.integers(0, 97, 23)
    with torch.no_grad():
        ref = model(torch.tensor(ids)[None]).logits[0].numpy()
    ours = go.forward(state, ids, n_head=4, n_layer=2)
    assert np.abs(ref - ours).max() <= 1e-12 * np.abs(ref).max()


def test_greedy_margins_reported():
    state = init_gpt2_state(n_vocab=50, n_embd=16, n_layer=1, n_positions=32, seed=1)
    tokens, margins = go.greedy(state, [1, 2, 3], 5, n_head=2, n_layer=1)
    assert len(tokens) == 5 and all(m >= 0 for m in margins)
    logits = go.forward(state, [1, 2, 3] + tokens[:2], n_head=2, n_layer=1)[-1]
    assert tokens[2] == int(np.argmax(logits))


@pytest.mark.parametrize('dtype,tol', [(np.float64, 1e-10), (np.float32, 2e-4)])
def test_cached_decode_step_equals_full_forward(dtype, tol):
    # The KV-cached batched decode (the CPU baseline of the end-to-end
    # configs) gives, row by row, the last-position logits of the full
    # forward over the whole sequence; a wrong position, a stale cache row or
    # a row mixed into another's attention fails it.
    state = init_gpt2_state(n_vocab=97, n_embd=32, n_layer=2, n_positions=64, seed=5)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 97, n).tolist() for n in (1, 7, 20)]
    caches, seqs = [], []
    for p in prompts:
        cache, last = go.prefill_cache(state, p, n_head=4, n_layer=2, capacity=len(p) + 4, dtype=dtype)
        full = go.forward(state, p, n_head=4, n_layer=2)[-1]
        assert np.abs(last - full).max() <= tol * np.abs(full).max()
        caches.append(cache)
        seqs.append(list(p) + [int(np.argmax(full))])
    for _ in range(4):
        logits = go.decode_step(state, caches, [s[-1] for s in seqs], n_head=4, n_layer=2, dtype=dtype)
        for r, s in enumerate(seqs):
            full = go.forward(state, s, n_head=4, n_layer=2)[-1]
            assert np.abs(logits[r] - full).max() <= tol * np.abs(full).max(), r
            s.append(int(np.argmax(full)))
    assert [c['length'] for c in caches] == [len(s) - 1 for s in seqs]


def test_greedy_cached_equals_greedy():
    # The batched KV-cached greedy (used for long end-to-end traces) gives the
    # full-recompute greedy's tokens and margins for prompts of different
    # lengths and output counts.
    state = init_gpt2_state(n_vocab=61, n_embd=32, n_layer=2, n_positions=64, seed=9)
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, 61, n).tolist() for n in (1, 5, 13)]
    steps = [6, 1, 9]
    tokens, margins = go.greedy_cached(state, prompts, steps, n_head=4, n_layer=2)
    for p, n, t, m in zip(prompts, steps, tokens, margins):
        ref, ref_m = go.greedy(state, p, n, n_head=4, n_layer=2)
        assert t == ref
        assert np.allclose(m, ref_m, rtol=1e-9, atol=1e-12)
