/* Token I/O of the decode step: C-ABI of
 * minitorch_amd/cuda_kernels/inference_kernels.so (gfx950).
 * Status and dtype conventions as in mt_paged.h.
 */
#ifndef MT_INFERENCE_H
#define MT_INFERENCE_H

#ifdef __cplusplus
extern "C" {
#endif

/* dst[t, :] = weights[ids[t], :] for fp32 ids [tokens] and weights
 * [vocab, dim]; a non-finite, negative, >= vocab or non-integer id gives a NaN
 * row. Replaces reference mt_embedding_gather (src/inference_kernels.cu:15-19). */
int mt_embedding_gather(float* dst, const float* weights, const float* ids, int tokens, int vocab,
                        int dim);

/* dst[r] = index of the first maximum of src[r, :] as fp32, a NaN beating
 * every number (numpy.argmax). Replaces reference mt_row_argmax
 * (src/inference_kernels.cu:73-79). */
int mt_row_argmax(float* dst, const void* src, int rows, int width, int dtype);

/* Token feedback of a sync-free decode loop: every cache slot of a page pool
 * keeps its request's last token on the device (slot_tokens, fp32 ids,
 * num_slots entries), so the next step reads it there instead of from the
 * host. mt_row_argmax_feedback is mt_row_argmax that also writes
 * slot_tokens[slots[r]] = dst[r] (slots outside [0, num_slots) are skipped;
 * slot_tokens == NULL writes dst only). mt_gather_slot_tokens sets
 * ids[r] = slot_tokens[slots[r]] (NaN for a slot outside the table).
 * No reference counterpart: they replace the per-step host round trip of the
 * token ids (reference minitorch/continuous_batching.py:143,146,
 * minitorch/kv_cache.py:39-53). */
int mt_row_argmax_feedback(float* dst, float* slot_tokens, const int* slots, int num_slots,
                           const void* src, int rows, int width, int dtype);
int mt_gather_slot_tokens(float* ids, const float* slot_tokens, const int* slots, int num_slots,
                          int rows);
/* mt_row_argmax_feedback that also commits the decode step of each row whose
 * slot is in the table: slot_len[slots[r]] += tokens, where slot_len is the
 * page pool's per-slot committed lengths (device, mt_pool_layout offset 5;
 * at least num_slots entries, so num_slots must not exceed the pool's slots).
 * The same launch thus replaces mt_row_argmax_feedback followed by
 * mt_sched_add_length. slot_len NULL commits nothing; a non-null slot_len
 * needs slot_tokens. No reference counterpart (the reference commits each
 * cache on the host, minitorch/paged_decode.py:80-86). */
int mt_row_argmax_commit(float* dst, float* slot_tokens, const int* slots, int num_slots, int* slot_len,
                         int tokens, const void* src, int rows, int width, int dtype);

/* x[t, :] = wte[id_t, :] + wpe[positions[t], :] (fp32) in one launch, with
 * id_t = ids[t], or slot_tokens[slots[t]] when slot_tokens is not null (token
 * feedback); an id or position that is non-finite, negative, too large or not
 * an integer gives a NaN row, as mt_embedding_gather. dim % 4 == 0 and
 * 16-byte aligned x/wte/wpe. No reference counterpart as one call (reference
 * minitorch/pretrained_gpt2.py:16-32 gathers both tables with
 * mt_embedding_gather and adds them, minitorch/modules_transformer.py:384). */
int mt_embed_tokens(float* x, const float* wte, const float* wpe, const float* ids,
                    const float* slot_tokens, const int* slots, int num_slots, const float* positions,
                    int tokens, int vocab, int n_positions, int dim);

/* dst[b, 0, :] = src[b, n - 1, :] for src [b, n, w]. Replaces reference
 * mt_last_row (src/inference_kernels.cu:66-72). */
int mt_last_row(void* dst, const void* src, int b, int n, int w, int dtype);

#ifdef __cplusplus
}
#endif
#endif /* MT_INFERENCE_H */
