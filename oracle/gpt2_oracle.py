"""numpy GPT-2 forward restating the reference's decoder math. TEST INFRASTRUCTURE ONLY.

Follows minitorch/modules_transformer.py:258-284 (pre-LayerNorm residual
block), :81-107 (Q/K/V projections split into heads), the paged/flash
attention semantics softmax(q.k / sqrt(D)) with a causal mask, the fused
LayerNorm's one-pass variance E[x^2] - mean^2 clamped at 0 plus eps
(src/layernorm_kernel.cu:37-99), tanh GELU (minitorch/nn.py:222-226) and the
tied head (minitorch/pretrained_gpt2.py:35-49). Weights use the GPT-2
checkpoint layout (Conv1D [in, out]). Computed in float64 by default.

Pinned against transformers' GPT2LMHeadModel built locally from a GPT2Config
(no download) with the same weights, in tests/test_gpt2_oracle.py.
"""
import math
import numpy as np


def layernorm(x, gamma, beta, eps=1e-5):
    mean = x.mean(-1, keepdims=True)
    var = np.maximum((x * x).mean(-1, keepdims=True) - mean * mean, 0) + eps
    return gamma * ((x - mean) / np.sqrt(var)) + beta


def gelu(x):
    return 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def forward(state, ids, *, n_head, n_layer, eps=1e-5, dtype=np.float64):
    """Logits [n, V] for token ids [n] at positions 0..n-1."""
    g = {k: np.asarray(v, dtype) for k, v in state.items()}
    ids = np.asarray(ids, np.int64)
    n = ids.size
    x = g['transformer.wte.weight'][ids] + g['transformer.wpe.weight'][np.arange(n)]
    d = x.shape[-1]
    hd = d // n_head
    mask = np.triu(np.full((n, n), -np.inf), 1)
    for i in range(n_layer):
        p = f'transformer.h.{i}.'
        h = layernorm(x, g[p + 'ln_1.weight'], g[p + 'ln_1.bias'], eps)
        qkv = h @ g[p + 'attn.c_attn.weight'] + g[p + 'attn.c_attn.bias']
        q, k, v = (qkv[:, j * d:(j + 1) * d].reshape(n, n_head, hd).transpose(1, 0, 2) for j in range(3))
        s = q @ k.transpose(0, 2, 1) / math.sqrt(hd) + mask
        s = s - s.max(-1, keepdims=True)
        a = np.exp(s)
        a = a / a.sum(-1, keepdims=True)
        o = (a @ v).transpose(1, 0, 2).reshape(n, d)
        x = x + o @ g[p + 'attn.c_proj.weight'] + g[p + 'attn.c_proj.bias']
        h = layernorm(x, g[p + 'ln_2.weight'], g[p + 'ln_2.bias'], eps)
        f = gelu(h @ g[p + 'mlp.c_fc.weight'] + g[p + 'mlp.c_fc.bias'])
        x = x + f @ g[p + 'mlp.c_proj.weight'] + g[p + 'mlp.c_proj.bias']
    x = layernorm(x, g['transformer.ln_f.weight'], g['transformer.ln_f.bias'], eps)
    return x @ g['transformer.wte.weight'].T


def greedy(state, prompt, steps, *, n_head, n_layer, eps=1e-5):
    """Greedy tokens after ``prompt`` (first token from the prompt's last
    position), and the top-1/top-2 logit margin at each step."""
    ids = list(int(t) for t in prompt)
    out, margins = [], []
    for _ in range(steps):
        logits = forward(state, ids, n_head=n_head, n_layer=n_layer, eps=eps)[-1]
        top = np.argsort(logits)[-2:]
        margins.append(float(logits[top[1]] - logits[top[0]]))
        token = int(np.argmax(logits))
        out.append(token)
        ids.append(token)
    return out, margins


def prefill_cache(state, ids, *, n_head, n_layer, capacity=None, eps=1e-5, dtype=np.float32):
    """K/V cache of a prompt and the logits of its last position, computed as
    ``forward`` does. The cache is {'length': n, 'k': [...], 'v': [...]} with
    per-layer K and V arrays [n_head, capacity, hd] (capacity defaults to n)."""
    g = _cast(state, dtype)
    ids = np.asarray(ids, np.int64)
    n = ids.size
    capacity = n if capacity is None else capacity
    x = g['transformer.wte.weight'][ids] + g['transformer.wpe.weight'][np.arange(n)]
    d = x.shape[-1]
    hd = d // n_head
    mask = np.triu(np.full((n, n), -np.inf, dtype), 1)
    cache = {'length': n, 'k': [], 'v': []}
    for i in range(n_layer):
        p = f'transformer.h.{i}.'
        h = layernorm(x, g[p + 'ln_1.weight'], g[p + 'ln_1.bias'], eps)
        qkv = h @ g[p + 'attn.c_attn.weight'] + g[p + 'attn.c_attn.bias']
        q, k, v = (qkv[:, j * d:(j + 1) * d].reshape(n, n_head, hd).transpose(1, 0, 2) for j in range(3))
        for name, t in (('k', k), ('v', v)):
            buf = np.zeros((n_head, capacity, hd), dtype)
            buf[:, :n] = t
            cache[name].append(buf)
        s = q @ k.transpose(0, 2, 1) / np.sqrt(dtype(hd)) + mask
        a = np.exp(s - s.max(-1, keepdims=True))
        a = a / a.sum(-1, keepdims=True)
        o = (a @ v).transpose(1, 0, 2).reshape(n, d)
        x = x + o @ g[p + 'attn.c_proj.weight'] + g[p + 'attn.c_proj.bias']
        h = layernorm(x, g[p + 'ln_2.weight'], g[p + 'ln_2.bias'], eps)
        x = x + gelu(h @ g[p + 'mlp.c_fc.weight'] + g[p + 'mlp.c_fc.bias']) @ g[p + 'mlp.c_proj.weight'] + g[p + 'mlp.c_proj.bias']
    x = layernorm(x[-1:], g['transformer.ln_f.weight'], g['transformer.ln_f.bias'], eps)
    return cache, (x @ g['transformer.wte.weight'].T)[0]


def decode_step(state, caches, ids, *, n_head, n_layer, eps=1e-5, dtype=np.float32):
    """One batched decode step with K/V caches (reference DecoderLM.decode_batch,
    minitorch/modules_transformer.py:373-390): token ids[b] at position
    caches[b]['length']; writes each row's K/V into its cache, advances the
    lengths and returns logits [B, V]. The projections run on the whole batch
    at once, attention per row over its own cache."""
    g = _cast(state, dtype)
    ids = np.asarray(ids, np.int64)
    pos = np.array([c['length'] for c in caches], np.int64)
    x = g['transformer.wte.weight'][ids] + g['transformer.wpe.weight'][pos]
    b, d = x.shape
    hd = d // n_head
    scale = 1 / np.sqrt(dtype(hd))
    for i in range(n_layer):
        p = f'transformer.h.{i}.'
        h = layernorm(x, g[p + 'ln_1.weight'], g[p + 'ln_1.bias'], eps)
        qkv = h @ g[p + 'attn.c_attn.weight'] + g[p + 'attn.c_attn.bias']
        o = np.empty((b, d), dtype)
        for r, cache in enumerate(caches):
            n = cache['length']
            q, k, v = (qkv[r, j * d:(j + 1) * d].reshape(n_head, hd) for j in range(3))
            kc, vc = cache['k'][i], cache['v'][i]
            kc[:, n], vc[:, n] = k, v
            s = np.einsum('hd,hnd->hn', q, kc[:, :n + 1]) * scale
            a = np.exp(s - s.max(-1, keepdims=True))
            a = a / a.sum(-1, keepdims=True)
            o[r] = np.einsum('hn,hnd->hd', a, vc[:, :n + 1]).reshape(d)
        x = x + o @ g[p + 'attn.c_proj.weight'] + g[p + 'attn.c_proj.bias']
        h = layernorm(x, g[p + 'ln_2.weight'], g[p + 'ln_2.bias'], eps)
        x = x + gelu(h @ g[p + 'mlp.c_fc.weight'] + g[p + 'mlp.c_fc.bias']) @ g[p + 'mlp.c_proj.weight'] + g[p + 'mlp.c_proj.bias']
    for c in caches:
        c['length'] += 1
    x = layernorm(x, g['transformer.ln_f.weight'], g['transformer.ln_f.bias'], eps)
    return x @ g['transformer.wte.weight'].T


def greedy_cached(state, prompts, steps, *, n_head, n_layer, eps=1e-5, dtype=np.float64):
    """``greedy`` for several prompts at once through ``prefill_cache`` and
    batched ``decode_step`` (each row's math is the full forward's, so the
    tokens equal ``greedy``'s): ``steps[i]`` tokens after ``prompts[i]``.
    Returns (tokens, margins), one list per prompt."""
    g = _cast(state, dtype)
    caches, out, margins = [], [], []
    for prompt, n in zip(prompts, steps):
        cache, last = prefill_cache(g, prompt, n_head=n_head, n_layer=n_layer, capacity=len(prompt) + n,
                                    eps=eps, dtype=dtype)
        top = np.argsort(last)[-2:]
        caches.append(cache)
        out.append([int(np.argmax(last))])
        margins.append([float(last[top[1]] - last[top[0]])])
    while True:
        rows = [i for i, n in enumerate(steps) if len(out[i]) < n]
        if not rows:
            return out, margins
        logits = decode_step(g, [caches[i] for i in rows], [out[i][-1] for i in rows], n_head=n_head,
                             n_layer=n_layer, eps=eps, dtype=dtype)
        for i, row in zip(rows, logits):
            top = np.argsort(row)[-2:]
            out[i].append(int(np.argmax(row)))
            margins[i].append(float(row[top[1]] - row[top[0]]))


def _cast(state, dtype):
    if all(np.asarray(v).dtype == dtype for v in state.values()):
        return state
    return {k: np.asarray(v, dtype) for k, v in state.items()}
