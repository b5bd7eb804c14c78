"""GPT-2 decoder for the end-to-end decode configurations.

Mirrors the reference model's inference entry points
(minitorch/modules_transformer.py:355-410: ``create_kv_cache``, ``prefill``,
``decode_step``, ``decode_batch``) and the GPT-2 layer math of
``TransformerLayer.forward`` (:258-284) with the pretrained adapter's layout
(minitorch/pretrained_gpt2.py:52-127): fp32 residual stream, LayerNorm in
fp32, Q/K/V/out/MLP projections, tanh GELU, tied output head. Weights are a
seeded random init (N(0, 0.02) matrices and embeddings, zero biases, unit
LayerNorm gains, as HF GPT-2 initializes them) or a host state dict.

MI355X-first choices: projection weights are kept resident on the device in
the compute type (the reference re-casts fp32 masters on every matmul,
minitorch/tensor.py:226-231); Q, K and V come from one fused [d, 3d]
projection (GPT-2's c_attn) whose output the paged decode reads as three
column blocks (no split copies); the batched decode step runs its whole layer
loop in one native call (mt_decoder_layers), with the residual adds fused into
the following LayerNorms. In fp16/bf16 a decode step of up to 128 rows runs
its projections on the matrix-core projection kernel, reading a second copy of
each projection weight stored fragment-tiled (``fragment_tiled``: each operand
fragment one contiguous 1 KB run); prefill, larger batches and fp32 use one
hipBLASLt call per projection with the bias (and for the MLP's fc, the GELU)
as its epilogue.
"""
import ctypes as ct
import numpy as np

from .amp import autocast_dtype
from .dtypes import dtype_code
from .runtime import DeviceTensor, library, call, runtime, P, I, F
from . import paged_ops



def model_library():
    return library('model_kernels')


class _Attention:
    def __init__(self, n_head, head_dim):
        self.n_head = n_head
        self.attn_hidden_dim = head_dim
        self.attention_impl = 'flash'


class _Layer:
    def __init__(self, n_head, head_dim):
        self.attention = _Attention(n_head, head_dim)


# Whether the fc projection's tanh GELU runs as hipBLASLt's GELU epilogue
# (else as a separate pass of mt_gelu after the GEMM).
FUSED_GELU = True


class _Blas:
    def __init__(self):
        self.handle = P()
        call(model_library(), 'mt_blas_create', [ct.POINTER(P)], ct.byref(self.handle))



class DecoderLayerStruct(ct.Structure):
    """``mt_decoder_layer`` (include/mt_model.h)."""
    _fields_ = [(name, P) for name in ('ln1_gamma', 'ln1_beta', 'w_qkv', 'b_qkv', 'w_o', 'b_o',
                                       'ln2_gamma', 'ln2_beta', 'w_fc', 'b_fc', 'w_proj', 'b_proj',
                                       'w_qkv_tiled', 'w_o_tiled', 'w_fc_tiled', 'w_proj_tiled')]


class PrefillAttentionStruct(ct.Structure):
    """``mt_prefill_attention`` (include/mt_model.h)."""
    _fields_ = [('slabs', P), ('table', P), ('page_size', I), ('pages_per_slab', I), ('num_slabs', I),
                ('columns', I), ('layers', I), ('offset', I)]


class DecodeAttentionStruct(ct.Structure):
    """``mt_decode_attention`` (include/mt_model.h)."""
    _fields_ = [('slabs', P), ('table', P), ('offsets', P),
                ('page_size', I), ('pages_per_slab', I), ('num_slabs', I), ('columns', I),
                ('layers', I), ('split_tokens', I),
                ('work', P), ('work_items', I), ('merge_rows', I),
                ('partials', P), ('partial_bytes', ct.c_size_t)]


def init_gpt2_state(*, n_vocab, n_embd, n_layer, n_positions, seed=0, std=0.02):
    """Seeded HF-style random GPT-2 weights as a dict of fp32 numpy arrays in
    the GPT-2 checkpoint layout (Conv1D weights are [in, out])."""
    rng = np.random.default_rng(seed)
    d = n_embd

    def normal(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)

    state = {'transformer.wte.weight': normal(n_vocab, d), 'transformer.wpe.weight': normal(n_positions, d),
             'transformer.ln_f.weight': np.ones(d, np.float32), 'transformer.ln_f.bias': np.zeros(d, np.float32)}
    for i in range(n_layer):
        p = f'transformer.h.{i}.'
        state[p + 'ln_1.weight'] = np.ones(d, np.float32)
        state[p + 'ln_1.bias'] = np.zeros(d, np.float32)
        state[p + 'ln_2.weight'] = np.ones(d, np.float32)
        state[p + 'ln_2.bias'] = np.zeros(d, np.float32)
        state[p + 'attn.c_attn.weight'] = normal(d, 3 * d)
        state[p + 'attn.c_attn.bias'] = np.zeros(3 * d, np.float32)
        state[p + 'attn.c_proj.weight'] = normal(d, d)
        state[p + 'attn.c_proj.bias'] = np.zeros(d, np.float32)
        state[p + 'mlp.c_fc.weight'] = normal(d, 4 * d)
        state[p + 'mlp.c_fc.bias'] = np.zeros(4 * d, np.float32)
        state[p + 'mlp.c_proj.weight'] = normal(4 * d, d)
        state[p + 'mlp.c_proj.bias'] = np.zeros(d, np.float32)
    return state


def fragment_tiled(a):
    """A [rows, width] matrix (width a multiple of 32) in the fragment-tiled
    layout the decode projection kernel reads (include/mt_model.h,
    mt_decode_projection), flat, rows padded with zeros to a multiple of 16:
    the 16 x 32 block (R, K) at element (R * width / 32 + K) * 512, its
    element (r, c) at ((c // 8) * 16 + r) * 8 + c % 8 -- the lane order of a
    matrix-core operand fragment, so that one wave reads a fragment as 1 KB of
    consecutive 16-byte loads."""
    a = np.asarray(a)
    rows, width = a.shape
    if width % 32:
        raise ValueError('fragment_tiled: width must be a multiple of 32')
    mp = -(-rows // 16) * 16
    p = np.zeros((mp, width), a.dtype)
    p[:rows] = a
    return np.ascontiguousarray(p.reshape(mp // 16, 16, width // 32, 4, 8).transpose(0, 2, 3, 1, 4)).reshape(-1)


class _DeviceWeights:
    """Device copies of the weights for one compute type."""

    def __init__(self, state, n_layer, d, dtype):
        self.dtype = dtype

        def put(name, dt=dtype, array=None):
            a = state[name] if array is None else array
            return DeviceTensor.from_numpy(np.ascontiguousarray(a), dt)

        self.wte = put('transformer.wte.weight', 'float32')
        self.wpe = put('transformer.wpe.weight', 'float32')
        self.head = put('transformer.wte.weight')          # tied head, [V, d] in the compute type
        self.ln_f = (put('transformer.ln_f.weight', 'float32'), put('transformer.ln_f.bias', 'float32'))
        self.layers = []
        for i in range(n_layer):
            p = f'transformer.h.{i}.'
            layer = dict(
                ln_1=(put(p + 'ln_1.weight', 'float32'), put(p + 'ln_1.bias', 'float32')),
                ln_2=(put(p + 'ln_2.weight', 'float32'), put(p + 'ln_2.bias', 'float32')),
                # projection weights stored [out, in] (the GPT-2 [in, out] arrays
                # transposed once): hipBLASLt's kernels for K-contiguous weights
                # run these shapes 11-20 % faster
                qkv=(put(p + 'attn.c_attn.weight', array=state[p + 'attn.c_attn.weight'].T),   # [3d, d]
                     put(p + 'attn.c_attn.bias')),
                o=(put(p + 'attn.c_proj.weight', array=state[p + 'attn.c_proj.weight'].T),
                   put(p + 'attn.c_proj.bias')),
                fc=(put(p + 'mlp.c_fc.weight', array=state[p + 'mlp.c_fc.weight'].T), put(p + 'mlp.c_fc.bias')),
                proj=(put(p + 'mlp.c_proj.weight', array=state[p + 'mlp.c_proj.weight'].T),
                      put(p + 'mlp.c_proj.bias')))
            if dtype != 'float32':
                # the decode projection kernel's copies: coalesced weight fragments
                for key, name in (('qkv', 'attn.c_attn'), ('o', 'attn.c_proj'), ('fc', 'mlp.c_fc'),
                                  ('proj', 'mlp.c_proj')):
                    layer[key + '_tiled'] = put(p + name + '.weight',
                                                array=fragment_tiled(state[p + name + '.weight'].T))
            self.layers.append(layer)

        def tiled_ptr(L, key):
            return L[key + '_tiled'].ptr if key + '_tiled' in L else None

        self.layer_array = (DecoderLayerStruct * n_layer)(*[
            DecoderLayerStruct(L['ln_1'][0].ptr, L['ln_1'][1].ptr, L['qkv'][0].ptr, L['qkv'][1].ptr,
                               L['o'][0].ptr, L['o'][1].ptr, L['ln_2'][0].ptr, L['ln_2'][1].ptr,
                               L['fc'][0].ptr, L['fc'][1].ptr, L['proj'][0].ptr, L['proj'][1].ptr,
                               tiled_ptr(L, 'qkv'), tiled_ptr(L, 'o'), tiled_ptr(L, 'fc'), tiled_ptr(L, 'proj'))
            for L in self.layers])


class DecoderLM:
    """GPT-2-architecture decoder with paged-KV inference entry points."""

    def __init__(self, *, n_vocab=50257, n_embd=768, n_head=12, n_layer=6, n_positions=1024,
                 ln_eps=1e-5, seed=0, state=None):
        if n_embd % n_head or n_embd // n_head > 128:
            raise ValueError('head_dim must divide n_embd and be <= 128')
        self.n_vocab, self.n_embd, self.n_head, self.n_layer = n_vocab, n_embd, n_head, n_layer
        self.n_positions, self.ln_eps = n_positions, ln_eps
        self.head_dim = n_embd // n_head
        self.state = state if state is not None else init_gpt2_state(
            n_vocab=n_vocab, n_embd=n_embd, n_layer=n_layer, n_positions=n_positions, seed=seed)
        self.training = False
        self._version = 0
        self._layers = tuple(_Layer(n_head, self.head_dim) for _ in range(n_layer))
        self._device = {}
        self._blas = None

    # ---------------------------------------------------------- plumbing ---
    def transformer_layers(self):
        return self._layers

    def weights_version(self):
        return self._version

    def eval(self):
        self.training = False
        return self

    def load_state(self, state):
        """Replace the weights (invalidates caches, like a parameter update)."""
        self.state = state
        self._device.clear()
        self._version += 1

    def _weights(self, dtype):
        if dtype not in self._device:
            self._device[dtype] = _DeviceWeights(self.state, self.n_layer, self.n_embd, dtype)
        return self._device[dtype]

    def blas(self):
        if self._blas is None:
            self._blas = _Blas()
        return self._blas

    def create_kv_cache(self, batch_size=1, capacity=None, *, cache_impl='paged', page_size=16,
                        page_pool=None, kv_budget_bytes=256 * 1024 ** 2, pages_per_slab=4,
                        paged_prefill_impl='flash'):
        if cache_impl != 'paged':
            raise ValueError('This build provides the paged cache (cache_impl="paged")')
        from .paged_kv_cache import PagedKVCache
        return PagedKVCache(self, batch_size, capacity, page_size=page_size, page_pool=page_pool,
                            kv_budget_bytes=kv_budget_bytes, pages_per_slab=pages_per_slab,
                            paged_prefill_impl=paged_prefill_impl)

    # -------------------------------------------------------------- ops ---
    def _embed(self, w, ids, positions, rows=None, feedback=None):
        """Token + position embeddings [rows, d] fp32 in one launch (reference
        minitorch/modules_transformer.py:384, pretrained_gpt2.py:16-32); with
        ``feedback`` = (pool, device slots) the token ids are the slots' last
        tokens instead of ``ids``."""
        rows = ids.size if rows is None else rows
        d = self.n_embd
        x = DeviceTensor((rows, d), 'float32')
        if feedback is None:
            paged_ops.embed_tokens(x.ptr, w.wte.ptr, w.wpe.ptr, ids.ptr, positions.ptr, rows, self.n_vocab,
                                   self.n_positions, d)
        else:
            pool, slots = feedback
            paged_ops.embed_tokens(x.ptr, w.wte.ptr, w.wpe.ptr, None, positions.ptr, rows, self.n_vocab,
                                   self.n_positions, d, slot_tokens=pool.slot_tokens.ptr, slots=slots,
                                   num_slots=pool.max_slots)
        return x

    # ------------------------------------------------- inference entries ---
    def prefill(self, idx, cache=None):
        """Evaluate a prompt [B, n] of fp32 token IDs; returns (last-position
        logits [B, 1, V], cache) (reference modules_transformer.py:355-365)."""
        owns = cache is None
        cache = self.create_kv_cache(idx.shape[0]) if owns else cache
        try:
            return self._cached_forward(idx, cache, True), cache
        except Exception:
            if owns:
                cache.close()
            raise

    def decode_step(self, idx, cache):
        """One new token per batch row of one cache (reference :367-371)."""
        return self._cached_forward(idx, cache, False)

    def prefill_batch(self, prompts, caches):
        """Prefill prompts of different lengths, each into its own empty paged
        cache of batch size 1 (all on one pool), in one native layer loop
        (``mt_prefill_layers_ragged``): the projections run once over every
        prompt row, attention per prompt over its own pages. Returns the
        last-position logits [R, 1, V], row r for prompt r. Pages are acquired
        cache by cache in the given order, as consecutive ``prefill`` calls
        would. No reference counterpart (the reference prefills one request per
        call, minitorch/continuous_batching.py:164-170)."""
        caches, prompts, pool, tokens = self._check_prefill(prompts, caches, 'prefill_batch')
        dtype, d = caches[0].dtype, self.n_embd
        w = self._weights(dtype)
        prepared = []
        try:
            for cache, n in zip(caches, tokens):
                cache.prepare_append(n)
                prepared.append(cache)
            total = sum(tokens)
            ids = DeviceTensor.from_numpy(np.concatenate(prompts).astype(np.float32)[None], 'float32')
            positions = DeviceTensor.from_numpy(
                np.concatenate([np.arange(n, dtype=np.float32) for n in tokens])[None], 'float32')
            x = self._embed(w, ids, positions)                      # [total, d] fp32
            h = DeviceTensor((total, d), dtype)
            lib = model_library()
            scratch_bytes = _scratch_bytes(lib, total, d, dtype)
            scratch = DeviceTensor(((scratch_bytes + 3) // 4,), 'float32')
            att = _prefill_attention(pool, caches)
            counts = (I * len(caches))(*tokens)
            logits = DeviceTensor((len(caches), 1, self.n_vocab), dtype)
            call(lib, 'mt_prefill_layers_ragged',
                 [P, P, I, P, P, P, P, P, P, I, I, P, I, I, F, I, I, P, ct.c_size_t, P],
                 self.blas().handle, w.layer_array, self.n_layer, x.ptr, h.ptr, w.ln_f[0].ptr, w.ln_f[1].ptr,
                 w.head.ptr, logits.ptr, self.n_vocab, len(caches), counts, d, self.n_head, self.ln_eps,
                 dtype_code(dtype), 1 if FUSED_GELU else 0, scratch.ptr, scratch_bytes, att)
            for cache in caches:
                cache._written_layers.update(range(len(cache.layout)))
                cache.last_attention_path = 'paged_prefill'
                cache.commit_append()
            return logits
        except Exception:
            for cache in prepared:
                if cache._pending_tokens is not None:
                    cache.abort_append()
            raise

    def _check_prefill(self, prompts, caches, name):
        """Validated (caches, prompts, pool, token counts) of a batched
        prefill: one nonempty 1-D prompt per distinct empty paged cache of
        batch size 1, all on one pool, each within its cache's capacity."""
        from .paged_kv_cache import PagedKVCache
        caches = tuple(caches)
        prompts = [np.asarray(p) for p in prompts]
        if not caches or len(prompts) != len(caches) or len({id(c) for c in caches}) != len(caches):
            raise ValueError(f'{name} needs one prompt per distinct cache')
        pool = getattr(caches[0], 'pool', None)
        for cache, prompt in zip(caches, prompts):
            if not isinstance(cache, PagedKVCache) or cache.pool is not pool or cache.batch_size != 1:
                raise ValueError(f'{name} requires paged caches of batch size 1 on one pool')
            if prompt.ndim != 1 or prompt.size < 1 or prompt.dtype.kind not in 'iuf':
                raise ValueError('Each prompt must be a nonempty 1-D array of token IDs')
            cache._validate_model(self)
            if cache.length != 0:
                raise ValueError('prefill requires an empty cache')
            if prompt.size > cache.capacity:
                raise ValueError('KV cache capacity exceeded or empty prompt')
        return caches, prompts, pool, [int(p.size) for p in prompts]

    def _cached_forward(self, idx, cache, prefill):
        cache.validate(self, idx, prefill)
        b, n = idx.shape
        offset = cache.length
        dtype = cache.dtype
        w = self._weights(dtype)
        try:
            cache.prepare_append(n)
            positions = DeviceTensor.from_numpy(
                np.tile(np.arange(offset, offset + n, dtype=np.float32), (b, 1)), 'float32')
            x = self._embed(w, idx, positions)                      # [b*n, d] fp32
            logits = self._paged_layers(w, x, cache, b, n, offset, dtype, prefill)
            cache.commit_append()
            return logits
        except Exception:
            cache.abort_append()
            raise

    def _paged_layers(self, w, x, cache, b, n, offset, dtype, prefill):
        """The whole layer loop and the last position's logits in one native
        call (``mt_prefill_layers``), for a paged cache: every layer appends
        its K/V at ``offset`` and runs causal paged attention."""
        pool = cache.pool
        h = DeviceTensor((b * n, self.n_embd), dtype)
        lib = model_library()
        scratch_bytes = _scratch_bytes(lib, b * n, self.n_embd, dtype)
        scratch = DeviceTensor(((scratch_bytes + 3) // 4,), 'float32')
        att = PrefillAttentionStruct(pool.slab_table.ptr, cache.block_table.ptr, cache.page_size,
                                     pool.pages_per_slab, pool.num_slabs, pool.max_cols, len(cache.layout),
                                     offset)
        logits = DeviceTensor((b, 1, self.n_vocab), dtype)
        call(lib, 'mt_prefill_layers', [P, P, I, P, P, P, P, P, P, I, I, I, I, I, F, I, I, P, ct.c_size_t, P],
             self.blas().handle, w.layer_array, self.n_layer, x.ptr, h.ptr, w.ln_f[0].ptr, w.ln_f[1].ptr,
             w.head.ptr, logits.ptr, self.n_vocab, b, n, self.n_embd, self.n_head, self.ln_eps,
             dtype_code(dtype), 1 if FUSED_GELU else 0, scratch.ptr, scratch_bytes, ct.byref(att))
        cache._written_layers.update(range(len(cache.layout)))
        cache.last_attention_path = ('paged_reference_prefill' if prefill and cache.paged_prefill_impl == 'paged_reference'
                                     else 'paged_prefill' if prefill else 'paged_decode')
        return logits

    def decode_batch(self, idx, caches):
        """One token per independent paged request in one model batch; rows
        may have different context lengths (reference modules_transformer.py:373-390)."""
        return self._decode_batch(idx, caches, greedy=False)

    def decode_greedy(self, caches, idx=None, *, graph=False):
        """``decode_batch`` with greedy selection on the device, for the
        sync-free decode loop: the input token of each row is ``idx`` or, when
        None, the last token its cache slot holds in the pool (written by the
        previous step's selection); the chosen tokens are written back there
        and returned as fp32 IDs [B, 1] on the device. Nothing waits for the
        device. No reference counterpart (the reference reads every step's
        tokens on the host, minitorch/continuous_batching.py:143,146).

        With ``graph`` (and ``idx`` None) the step's device work (page pops
        and metadata, embeddings, the layer loop, the greedy selection and the
        length commit) is replayed from a HIP graph captured for the batch
        size; the first ``GRAPH_WARMUP`` steps of a batch size run eagerly, so
        that the projections' hipBLASLt algorithms are chosen (and timed)
        outside any capture. The returned IDs then live in the captured step's
        buffer and are overwritten by its next replay."""
        if graph and idx is None:
            return self._decode_greedy_graph(caches)
        return self._decode_batch(idx, caches, greedy=True)

    def decode_prefill_greedy(self, caches, prompts, new_caches, *, finished=(), return_logits=False):
        """One sync-free greedy decode step of ``caches`` (as ``decode_greedy``
        with ``idx`` None) and the prefill of ``prompts`` into the empty caches
        ``new_caches`` (one each, as ``prefill_batch``), run as one native
        layer loop (``mt_mixed_layers``): the projections cover both sets of
        rows at once. ``finished`` names caches of ``caches`` whose requests end
        with this step: they are closed once the step's pages are taken and its
        lengths committed, and before ``new_caches`` take their pages, which is
        the order of ``decode_greedy``, then closing them, then
        ``prefill_batch`` -- page IDs, tables and the free list come out the
        same. Returns the greedy token IDs [len(caches) + len(prompts), 1] fp32
        on the device (the decode rows, then each prompt's first token), which
        also become each cache's last token for the next step. Nothing waits
        for the device. With ``return_logits`` the result is (ids, logits
        [len(caches) + len(prompts), 1, V]) in the compute type.

        The step's whole page demand (the decode rows' new pages, less what
        the ending requests return, plus the prompts' pages) is checked on the
        host before anything changes: a step that does not fit raises
        MemoryError with every cache, page and length as it was, and the
        caller may run the separate calls instead. If the native layer loop
        fails after the decode rows' lengths were committed, those caches are
        marked invalid (their K/V for the step was not written). No reference
        counterpart (the reference runs a step's decode batch and its
        prefills as separate forward passes,
        minitorch/continuous_batching.py:140-176)."""
        from .paged_decode import PagedDecodeBatch
        new_caches, prompts, pool, tokens = self._check_prefill(prompts, new_caches, 'decode_prefill_greedy')
        caches = tuple(caches)
        ids_of = {id(c) for c in caches}
        if any(id(c) not in ids_of for c in finished) or ids_of & {id(c) for c in new_caches}:
            raise ValueError('finished caches must be decoded in the step and new caches must not')
        if caches and caches[0].pool is not pool:
            raise ValueError('decode_prefill_greedy requires the decode and new caches on one pool')
        with PagedDecodeBatch(self, None, caches) as batch:
            ps = pool.page_size
            grows = {id(c): int(c.length % ps == 0) for c in caches}
            free = pool.max_pages - pool.used_pages
            decode_pages = sum(grows.values())
            returned = sum(c._counts[0] + grows[id(c)] for c in finished)
            prompt_pages = sum(-(-n // ps) for n in tokens)
            if decode_pages > free or decode_pages - returned + prompt_pages > free:
                raise MemoryError('KV page budget exhausted')
            b, dtype, d = batch.batch_size, batch.dtype, self.n_embd
            w = self._weights(dtype)
            # the decode rows' embeddings come from the metadata launch (the
            # slots' last tokens at their committed lengths), the prompts'
            # from their IDs below
            x = DeviceTensor((b + sum(tokens), d), 'float32')
            batch.prepare(embed=(x.ptr, w.wte.ptr, w.wpe.ptr, self.n_vocab, self.n_positions, d))
            datt = batch.attention_metadata()
            slots = batch.device_slots
            # the decode half's lengths are committed before any page changes
            # hands; its kernels read the step's own table and offsets
            batch.mark_layers_written()
            batch.commit()
        pool.close_caches(finished)
        total, r = sum(tokens), len(new_caches)
        # one upload: the new caches' slots, page counts and tokens
        # (append_lists), then the prompts' token IDs and positions (fp32)
        lists = pool.append_lists(new_caches, tokens)
        blob = DeviceTensor.from_numpy(np.concatenate([
            np.array(lists, np.int32), np.concatenate(prompts).astype(np.float32).view(np.int32),
            np.concatenate([np.arange(n, dtype=np.float32) for n in tokens]).view(np.int32)]), 'int32')
        new_slots, prompt_ids, prompt_positions = blob.ptr, blob.ptr + 12 * r, blob.ptr + 12 * r + 4 * total
        prepared = []
        try:
            pool.prepare_appends(new_caches, tokens, blob.ptr)
            prepared = list(new_caches)
            paged_ops.embed_tokens(x.ptr + 4 * b * d, w.wte.ptr, w.wpe.ptr, prompt_ids, prompt_positions, total,
                                   self.n_vocab, self.n_positions, d)
            h = DeviceTensor((b + total, d), dtype)
            lib = model_library()
            scratch_bytes = _scratch_bytes(lib, b + total, d, dtype)
            scratch = DeviceTensor(((scratch_bytes + 3) // 4,), 'float32')
            logits = DeviceTensor((b + r, 1, self.n_vocab), dtype)
            call(lib, 'mt_mixed_layers',
                 [P, P, I, P, P, P, P, P, P, I, I, I, P, I, I, F, I, I, P, ct.c_size_t, P, P],
                 self.blas().handle, w.layer_array, self.n_layer, x.ptr, h.ptr, w.ln_f[0].ptr, w.ln_f[1].ptr,
                 w.head.ptr, logits.ptr, self.n_vocab, b, r, (I * r)(*tokens), d, self.n_head, self.ln_eps,
                 dtype_code(dtype), 1 if FUSED_GELU else 0, scratch.ptr, scratch_bytes, ct.byref(datt),
                 _prefill_attention(pool, new_caches))
            out = DeviceTensor((b + r, 1), 'float32')
            row_bytes = self.n_vocab * (logits.nbytes // logits.size)
            paged_ops.row_argmax_feedback(out.ptr, pool.slot_tokens.ptr, slots.ptr, pool.max_slots, logits.ptr, b,
                                          self.n_vocab, dtype)
            paged_ops.row_argmax_feedback(out.ptr + 4 * b, pool.slot_tokens.ptr, new_slots, pool.max_slots,
                                          logits.ptr + b * row_bytes, r, self.n_vocab, dtype)
            for cache in new_caches:
                cache._written_layers.update(range(len(cache.layout)))
                cache.last_attention_path = 'paged_prefill'
            pool.commit_appends(new_caches, blob.ptr)
            return (out, logits) if return_logits else out
        except Exception:
            for cache in prepared:
                if cache._pending_tokens is not None:
                    cache.abort_append()
            for cache in caches:
                if not cache.closed:
                    cache.valid = False
            raise

    def _decode_greedy_graph(self, caches):
        from .paged_decode import PagedDecodeBatch
        rt = runtime()
        with PagedDecodeBatch(self, None, caches) as batch:
            batch.prepare(graph=True)
            pool, b, dtype, ws = batch.pool, batch.batch_size, batch.dtype, batch._ws
            w = self._weights(dtype)
            att = batch.attention_metadata()
            deps = (w, self.blas(), ws.buffer, ws.partials, pool.slot_tokens, pool.state)
            step = ws.graphs.get(b)
            if step is not None and not step.matches(deps):
                step.close()
                del ws.graphs[b]
                step = None
            if step is None and ws.eager_steps.get(b, 0) >= GRAPH_WARMUP and b not in ws.uncapturable:
                try:
                    step = ws.graphs[b] = self._capture_decode(batch, w, att, deps)
                except RuntimeError:
                    # this batch size keeps running eagerly (the capture was
                    # ended and discarded; nothing of it ran)
                    ws.uncapturable.add(b)
            if step is None:
                ws.eager_steps[b] = ws.eager_steps.get(b, 0) + 1
                ids = self._issue_decode(batch, w, att, _StepBuffers(model_library(), b, self.n_embd,
                                                                     self.n_vocab, dtype))
                batch.mark_layers_written()
                batch.commit(device=False)  # the greedy selection committed on the device
                return ids
            rt.check(rt.lib.mt_graph_launch(step.exec))
            batch._device_prepared = True
            batch.mark_layers_written()
            batch.commit(device=False)
            return step.buffers.ids

    def _capture_decode(self, batch, w, att, deps):
        """Capture the device work of one decode step into a graph (nothing
        runs until it is launched)."""
        rt = runtime()
        buffers = _StepBuffers(model_library(), batch.batch_size, self.n_embd, self.n_vocab, batch.dtype)
        exec_ptr = P()
        rt.check(rt.lib.mt_graph_begin())
        try:
            self._issue_decode(batch, w, att, buffers)
        except Exception:
            rt.lib.mt_graph_end(ct.byref(exec_ptr))     # ends and discards the capture
            if exec_ptr.value:
                rt.lib.mt_graph_destroy(exec_ptr)
            raise
        finally:
            batch._device_prepared = False              # nothing has run yet
        rt.check(rt.lib.mt_graph_end(ct.byref(exec_ptr)))
        return _CapturedStep(exec_ptr.value, buffers, deps)

    def _issue_decode(self, batch, w, att, buffers):
        """The device work of a sync-free decode step: its metadata and the
        embeddings of each slot's last token in one launch
        (``mt_sched_decode_prepare_embed``), the native layer loop with the
        tied head, and the greedy selection with token feedback and the step's
        commit (each row's committed length + 1, ``mt_row_argmax_commit``),
        into ``buffers``; returns the IDs."""
        b, d, dtype, pool = batch.batch_size, self.n_embd, batch.dtype, batch.pool
        batch.prepare_device(embed=(buffers.x.ptr, w.wte.ptr, w.wpe.ptr, self.n_vocab, self.n_positions, d))
        call(model_library(), 'mt_decoder_layers', [P, P, I, P, P, P, P, P, P, I, I, I, I, F, I, I, P, ct.c_size_t, P],
             self.blas().handle, w.layer_array, self.n_layer, buffers.x.ptr, buffers.h.ptr, w.ln_f[0].ptr,
             w.ln_f[1].ptr, w.head.ptr, buffers.logits.ptr, self.n_vocab, b, d, self.n_head, self.ln_eps,
             dtype_code(dtype), 1 if FUSED_GELU else 0, buffers.scratch.ptr, buffers.scratch_bytes, ct.byref(att))
        paged_ops.row_argmax_commit(buffers.ids.ptr, pool.slot_tokens.ptr, batch.device_slots.ptr,
                                    pool.max_slots, pool.slot_len_ptr, 1, buffers.logits.ptr, b, self.n_vocab,
                                    dtype)
        return buffers.ids

    def _decode_batch(self, idx, caches, greedy):
        from .paged_decode import PagedDecodeBatch
        with PagedDecodeBatch(self, idx, caches) as batch:
            dtype = batch.dtype
            w = self._weights(dtype)
            b, d = batch.batch_size, self.n_embd
            pool = batch.pool
            # A sync-free greedy step fuses as the captured step does: the
            # metadata launch also embeds each slot's last token, and the
            # greedy selection also commits the lengths.
            fused = idx is None and greedy
            if fused:
                x = DeviceTensor((b, d), 'float32')
                batch.prepare(embed=(x.ptr, w.wte.ptr, w.wpe.ptr, self.n_vocab, self.n_positions, d))
            else:
                batch.prepare()
                feedback = (pool, batch.device_slots.ptr) if idx is None else None
                x = self._embed(w, idx, batch.position_ids, rows=b, feedback=feedback)
            h = DeviceTensor((b, d), dtype)
            lib = model_library()
            scratch_bytes = _scratch_bytes(lib, b, d, dtype)
            scratch = DeviceTensor(((scratch_bytes + 3) // 4,), 'float32')
            att = batch.attention_metadata()
            logits = DeviceTensor((b, 1, self.n_vocab), dtype)
            call(lib, 'mt_decoder_layers', [P, P, I, P, P, P, P, P, P, I, I, I, I, F, I, I, P, ct.c_size_t, P],
                 self.blas().handle, w.layer_array, self.n_layer, x.ptr, h.ptr, w.ln_f[0].ptr,
                 w.ln_f[1].ptr, w.head.ptr, logits.ptr, self.n_vocab, b, d, self.n_head, self.ln_eps,
                 dtype_code(dtype), 1 if FUSED_GELU else 0, scratch.ptr, scratch_bytes, ct.byref(att))
            batch.mark_layers_written()
            if fused:
                ids = DeviceTensor((b, 1), 'float32')
                paged_ops.row_argmax_commit(ids.ptr, pool.slot_tokens.ptr, batch.device_slots.ptr, pool.max_slots,
                                            pool.slot_len_ptr, 1, logits.ptr, b, self.n_vocab, dtype)
                batch.commit(device=False)  # the lengths were committed by the selection
                return ids
            if greedy:
                ids = DeviceTensor((b, 1), 'float32')
                paged_ops.row_argmax_feedback(ids.ptr, pool.slot_tokens.ptr, batch.device_slots.ptr,
                                              pool.max_slots, logits.ptr, b, self.n_vocab, dtype)
            batch.commit()
            return ids if greedy else logits


# Eager steps of a batch size before its decode step is captured: the
# decoder loop times its projections' algorithms on the third call of a shape.
GRAPH_WARMUP = 3


class _CapturedStep:
    """A captured decode step: the instantiated graph, the device buffers it
    writes, and the objects whose memory it reads (kept alive, and compared
    before each replay)."""

    def __init__(self, exec_ptr, buffers, deps):
        self.exec, self.buffers, self.deps = exec_ptr, buffers, deps

    def matches(self, deps):
        return len(deps) == len(self.deps) and all(a is b for a, b in zip(deps, self.deps))

    def close(self):
        if self.exec:
            rt = runtime()
            rt.check(rt.lib.mt_graph_destroy(self.exec))
            self.exec = None


class _StepBuffers:
    def __init__(self, lib, b, d, n_vocab, dtype):
        self.x = DeviceTensor((b, d), 'float32')
        self.h = DeviceTensor((b, d), dtype)
        self.scratch_bytes = _scratch_bytes(lib, b, d, dtype)
        self.scratch = DeviceTensor(((self.scratch_bytes + 3) // 4,), 'float32')
        self.logits = DeviceTensor((b, 1, n_vocab), dtype)
        self.ids = DeviceTensor((b, 1), 'float32')


def _prefill_attention(pool, caches):
    """``mt_prefill_attention`` of each empty cache (offset 0), as a ctypes array."""
    return (PrefillAttentionStruct * len(caches))(*[
        PrefillAttentionStruct(pool.slab_table.ptr, c.block_table.ptr, c.page_size, pool.pages_per_slab,
                               pool.num_slabs, pool.max_cols, len(c.layout), 0) for c in caches])


def _scratch_bytes(lib, rows, d, dtype):
    f = lib.mt_decoder_scratch_bytes
    f.argtypes, f.restype = [I, I, I], ct.c_size_t
    return int(f(rows, d, dtype_code(dtype)))


def distilgpt2(seed=0):
    """Config 3 architecture: 6 layers, d 768, 12 heads, vocab 50257, 1024 positions."""
    return DecoderLM(n_vocab=50257, n_embd=768, n_head=12, n_layer=6, n_positions=1024, seed=seed)


def gpt2_medium(seed=0):
    """Config 4 architecture: 24 layers, d 1024, 16 heads, vocab 50257, 1024 positions."""
    return DecoderLM(n_vocab=50257, n_embd=1024, n_head=16, n_layer=24, n_positions=1024, seed=seed)
