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

/* dst[b, 0, :] = src[b, n - 1, :] for src [b, n, w]. Replaces reference
 * mt_last_row (src/inference_kernels.cu:66-72). */
int mt_last_row(void* dst, const void* src, int b, int n, int w, int dtype);

#ifdef __cplusplus
}
#endif
#endif /* MT_INFERENCE_H */
