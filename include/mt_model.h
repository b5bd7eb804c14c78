/* Model-side support for the end-to-end decode configs: C-ABI of
 * minitorch_amd/cuda_kernels/model_kernels.so (gfx950, links hipBLASLt).
 * Status convention as in mt_paged.h (hipBLASLt failures return 1000 + the
 * hipblasStatus_t value). dtype 0 = float32, 1 = float16, 2 = bfloat16.
 */
#ifndef MT_MODEL_H
#define MT_MODEL_H

#ifdef __cplusplus
extern "C" {
#endif

/* hipBLASLt handle with a 64 MiB workspace and per-shape plans.
 * Replace reference mt_blas_create / mt_blas_destroy (src/cuda_runtime.cu:22-23). */
int mt_blas_create(void** handle);
int mt_blas_destroy(void* handle);

/* Row-major fp32 out[m, n] = a[m, k] @ b[k, n].
 * Replaces reference mt_gemm (src/cuda_runtime.cu:24-30). */
int mt_gemm(void* handle, float* out, const float* a, const float* b, int m, int n, int k);

/* fp16/bf16 inputs, fp32 accumulation, output fp32 (out_dtype 0) or the input type.
 * Replaces reference mt_typed_gemm (src/mixed_precision.cu:103-122). */
int mt_typed_gemm(void* handle, void* out, const void* a, const void* b, int m, int n, int k,
                  int dtype, int out_dtype);

/* 1 for fp16 and bf16 on gfx950.
 * Replaces reference mt_low_gemm_supported (src/mixed_precision.cu:98-102). */
int mt_low_gemm_supported(int dtype);

/* out[m, n] = a[m, k] @ op(b) + bias[n] (bias may be null), op(b) = b [k, n]
 * or, with transb = 1, b^T for b [n, k] (the tied head). fp32 accumulation.
 * No reference counterpart (bias epilogue of the reference's Linear,
 * minitorch/modules_basic.py:132-149, fused into the GEMM). */
int mt_gemm_ex(void* handle, void* out, const void* a, const void* b, const void* bias, int m,
               int n, int k, int transb, int dtype, int out_dtype);

/* LayerNorm of fp32 rows written in out_dtype: one-pass variance
 * E[x^2] - mean^2 clamped at 0, plus eps. Replaces reference mt_layernorm_fw
 * (src/layernorm_kernel.cu:449-456) fused with the cast to the GEMM input type. */
int mt_layernorm_typed(void* out, const float* x, const float* gamma, const float* beta, int rows,
                       int width, float eps, int out_dtype);

/* In-place tanh GELU. Replaces the reference's elementwise chain
 * (minitorch/nn.py:222-226). */
int mt_gelu(void* x, long long n, int dtype);

/* x[i] += y[i], fp32 residual x, y in dtype. Replaces the reference's
 * residual add (minitorch/modules_transformer.py:276,282). */
int mt_residual_add(float* x, const void* y, long long n, int dtype);

/* out = a + b (fp32): token + position embeddings
 * (minitorch/modules_transformer.py:384). */
int mt_add_f32(float* out, const float* a, const float* b, long long n);

/* Element type conversion (reference Tensor.to, mixed_precision.cu casts). */
int mt_cast(void* out, const void* in, long long n, int in_dtype, int out_dtype);

/* split = 1: out [b, h, n, d] <- in [b, n, h*d]; split = 0: the inverse
 * (reference view/permute/contiguous, minitorch/modules_transformer.py:96-104,179-181). */
int mt_heads(void* out, const void* in, int b, int n, int h, int d, int split, int dtype);

#ifdef __cplusplus
}
#endif
#endif /* MT_MODEL_H */
