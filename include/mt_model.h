/* Model-side support for the end-to-end decode configs: C-ABI of
 * minitorch_amd/cuda_kernels/model_kernels.so (gfx950, links hipBLASLt).
 * Status convention as in mt_paged.h (hipBLASLt failures return 1000 + the
 * hipblasStatus_t value). dtype 0 = float32, 1 = float16, 2 = bfloat16.
 */
#ifndef MT_MODEL_H
#define MT_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weights of one GPT-2 layer for mt_decoder_layers / mt_prefill_layers: fp32
 * LayerNorm parameters; projection weights row-major [out, in] (GPT-2's
 * [in, out] Conv1D arrays transposed once, so that the GEMMs read them
 * K-contiguous) and biases [out] in the compute type; w_qkv is the fused
 * [3d, d] query/key/value projection. */
typedef struct mt_decoder_layer {
  const float* ln1_gamma; const float* ln1_beta;
  const void* w_qkv; const void* b_qkv;
  const void* w_o; const void* b_o;
  const float* ln2_gamma; const float* ln2_beta;
  const void* w_fc; const void* b_fc;
  const void* w_proj; const void* b_proj;
  /* The four projection weights again in the fragment-tiled layout of
   * mt_decode_projection (fp16/bf16 only; null: the decode projections read
   * the row-major copies above, which hipBLASLt always reads). */
  const void* w_qkv_tiled; const void* w_o_tiled; const void* w_fc_tiled; const void* w_proj_tiled;
} mt_decoder_layer;

/* Paged-cache metadata of one decode batch, as mt_paged_decode_split takes it
 * (include/mt_paged.h); the layer index is supplied per layer. */
typedef struct mt_decode_attention {
  const uint64_t* slabs; const int* table; const int* offsets;
  int page_size, pages_per_slab, num_slabs, columns, layers, split_tokens;
  const int* work; int work_items, merge_rows;
  void* partials; size_t partial_bytes;
} mt_decode_attention;

/* Paged-cache metadata of one prefill (n new tokens per request at a common
 * offset), as mt_paged_prefill takes it (include/mt_paged.h); the layer index
 * is supplied per layer. */
typedef struct mt_prefill_attention {
  const uint64_t* slabs; const int* table;
  int page_size, pages_per_slab, num_slabs, columns, layers, offset;
} mt_prefill_attention;

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

/* split = 1: out [b, h, n, d] <- in [b, n, *] whose rows are in_stride
 * elements apart (0 = h*d; e.g. 3*h*d for one column block of a fused QKV
 * output); split = 0: the inverse, contiguous, in_stride 0
 * (reference view/permute/contiguous, minitorch/modules_transformer.py:96-104,179-181). */
int mt_heads(void* out, const void* in, int b, int n, int h, int d, int split, int in_stride,
             int dtype);

/* out[m, n] = epilogue(a[m, k] @ b[k, n] + bias[n]) in dtype, fp32
 * accumulation; epilogue 0 = none, 1 = tanh GELU, computed by hipBLASLt's
 * fused GELU epilogue when fused_gelu != 0, else by the mt_gelu kernel after
 * the GEMM. No reference counterpart (Linear + GELU of
 * minitorch/modules_transformer.py:278-282 in one call). */
int mt_gemm_epilogue(void* handle, void* out, const void* a, const void* b, const void* bias, int m,
                     int n, int k, int dtype, int epilogue, int fused_gelu);

/* x[r, :] += y[r, :] (fp32 x, y in dtype), then out[r, :] = LayerNorm(x[r, :])
 * in dtype, as mt_layernorm_typed. Replaces the reference's residual add
 * followed by the next LayerNorm (minitorch/modules_transformer.py:272-282). */
int mt_residual_layernorm(void* out, float* x, const void* y, const float* gamma, const float* beta,
                          int rows, int width, float eps, int dtype);

/* Decode projection on the matrix cores for fp16/bf16 (dtype 1/2):
 * out = epilogue(x[m, k] @ w[n, k]^T) with fp32 accumulation, for
 * 1 <= m <= 256 rows. epilogue 0: + bias[n] (bias in dtype, may be null),
 * out [m, n] in dtype; 1: + bias, then tanh GELU in fp32, out in dtype;
 * 2: out [splits, m, n] fp32 partial sums over `splits` (1, 2, 4 or 8)
 * equal k ranges, no bias (epilogues 0 and 1 take splits = 1). Requires n a
 * multiple of 16, k / splits = 32 * s * w for some w <= 16 and s <= 4
 * (s <= 2 when m > 64), x and w 16-byte aligned, out 8-byte (16-byte for
 * epilogue 2) aligned; hipErrorInvalidValue otherwise. layout bit 0: x is in
 * the fragment-tiled layout, bit 1: out (epilogues 0 and 1, n a multiple of
 * 32) is written in it, bit 2: w [n, k] is in it (fragment_tiled in
 * minitorch_amd/model.py writes it). That layout stores a 16-bit [rows, width] matrix
 * (width a multiple of 32) as ceil(rows / 16) * 16 rows: element (r, c) at
 * ((r / 16) * (width / 32) + c / 32) * 512 + (((c / 8) % 4) * 16 + r % 16) * 8
 * + c % 8, i.e. each 16 x 32 block as one 1 KB run in the order the matrix
 * cores take it; rows past m are read and never affect the result. Weights
 * are read once per call. No reference counterpart (the reference's Linear,
 * minitorch/modules_basic.py:132-149, calls cuBLAS). */
int mt_decode_projection(void* out, const void* x, const void* w, const void* bias, int m, int n, int k,
                         int splits, int epilogue, int dtype, int layout);

/* mt_decode_projection (epilogue 0 or 1, one split) whose activations are
 * LayerNorm(x_in + part_bias + sum_s partials[s]) for rows r < m: v[r, :] =
 * x_in[r, :] + part_bias + sum over s < splits of partials[s, r, :] (fp32;
 * splits 0, 1, 2 or 4; 0 means no partials and no part_bias), h = gamma *
 * ((v - mean) * rsqrt(var + eps)) + beta with one-pass mean and variance as
 * mt_residual_layernorm, rounded to dtype, out = epilogue(h @ w[n, k]^T +
 * bias); x_out[r, :] = v[r, :] (x_out must not be x_in). 1 <= m <= 16, k a
 * multiple of 256 up to 1024, n a multiple of 16, 16-byte aligned
 * x_in/x_out/partials/gamma/beta/w, 8-byte aligned out/bias/part_bias;
 * hipErrorInvalidValue otherwise. The residual add and LayerNorm of a decode
 * step fused into the QKV and fc projections for small batches. layout 0: w
 * row-major, 4: w in the fragment-tiled layout (mt_decode_projection). No
 * reference counterpart (minitorch/modules_transformer.py:272-282 around the Linear of
 * minitorch/modules_basic.py:132-149). */
int mt_decode_projection_ln(void* out, const float* x_in, float* x_out, const float* partials, int splits,
                            const void* part_bias, const float* gamma, const float* beta, float eps, const void* w,
                            const void* bias, int m, int n, int k, int epilogue, int dtype, int layout);

/* x[r, :] += bias + sum_s partials[s, r, :] (fp32), then out[r, :] =
 * LayerNorm(x[r, :]) in dtype (1 or 2): the residual add and LayerNorm after
 * a split projection (mt_decode_projection epilogue 2), as
 * mt_residual_layernorm. width a multiple of 256, at most 2048; 1 <= splits
 * <= 8; layout 0: out [rows, width] row-major, 2: out in the fragment-tiled
 * layout of mt_decode_projection. No reference counterpart
 * (minitorch/modules_transformer.py:272-282 with the projection's split-k
 * reduction folded in). */
int mt_residual_layernorm_partials(void* out, float* x, const float* partials, int splits, const void* bias,
                                   const float* gamma, const float* beta, int rows, int width, float eps,
                                   int dtype, int layout);

/* Scratch bytes mt_decoder_layers needs for `rows` tokens of width d. */
size_t mt_decoder_scratch_bytes(int rows, int d, int dtype);

/* The layer loop of one batched decode step, all launches issued from here on
 * the default stream: for each layer, LayerNorm (fused with the previous
 * residual add), fused QKV GEMM, paged decode attention
 * (mt_paged_decode_split reading q/k/v as column blocks of the QKV output),
 * out-projection, residual add + LayerNorm, fc GEMM + GELU, proj GEMM; after
 * the last layer the residual add is fused with the final LayerNorm
 * (final_gamma/final_beta). x [rows, d] fp32 is the residual stream, updated
 * in place; h [rows, d] in dtype receives the final LayerNorm output and,
 * when logits is not null, logits [rows, vocab] = h @ head_weight^T (the tied
 * head, head_weight [vocab, d]). For fp16/bf16 the layer projections run on
 * mt_decode_projection (reading the layer's tiled weight copies where given):
 * for rows <= 8 and d <= 1024 the residual add and LayerNorm move into the
 * QKV and fc projections (mt_decode_projection_ln, the residual stream
 * alternating between x and a scratch copy) and the out- and proj-projections
 * leave split-k partial sums; for 9 <= rows <= 128 (d a multiple of 256) the
 * LayerNorms (mt_residual_layernorm_partials after the split out- and
 * proj-projections) and the fc epilogue write the activations of QKV, fc and
 * proj in the fragment-tiled layout, and the out-projection runs split while
 * rows <= 32 or it takes at most 4 splits. Otherwise (larger batches, fp32,
 * other shapes, MT_DECODE_PROJECTIONS=0 in the environment) the QKV and fc
 * projections take the kernel up to 16 rows and the out- and proj-projections
 * up to 32, on row-major activations, and hipBLASLt the rest; hipBLASLt
 * chooses its algorithm by timing (cold caches) on the third call of a shape,
 * as does the tied head. MT_DECODE_TILED_ROWS=<rows> moves the tiled path's
 * upper bound (0: off).
 * Replaces the reference's per-op layer loop of DecoderLM.decode_batch
 * (minitorch/modules_transformer.py:373-390,258-284). */
int mt_decoder_layers(void* handle, const mt_decoder_layer* layers, int n_layer, float* x, void* h,
                      const float* final_gamma, const float* final_beta, const void* head_weight,
                      void* logits, int vocab, int rows, int d, int heads, float eps, int dtype,
                      int fused_gelu, void* scratch, size_t scratch_bytes,
                      const mt_decode_attention* att);

/* The layer loop of a prefill of n tokens for each of batch requests, all
 * launches issued from here on the default stream: as mt_decoder_layers, with
 * rows = batch * n token rows (x [rows, d] fp32, updated in place; h [rows, d]
 * in dtype) and, per layer, mt_paged_prefill appending K/V at att->offset and
 * computing causal attention, with q/k/v read as column blocks of the fused
 * QKV output and the output written with heads merged. When logits is not
 * null, logits [batch, vocab] = final-LayerNorm(x)[last position of each
 * request] @ head_weight^T. The projections keep hipBLASLt's first heuristic
 * choice (prompt lengths vary). Scratch as mt_decoder_scratch_bytes(rows).
 * Replaces the reference's per-op layer loop of DecoderLM.prefill
 * (minitorch/modules_transformer.py:355-365,258-284). */
int mt_prefill_layers(void* handle, const mt_decoder_layer* layers, int n_layer, float* x, void* h,
                      const float* final_gamma, const float* final_beta, const void* head_weight,
                      void* logits, int vocab, int batch, int n, int d, int heads, float eps,
                      int dtype, int fused_gelu, void* scratch, size_t scratch_bytes,
                      const mt_prefill_attention* att);

/* The prefill of `requests` prompts of different lengths in one layer loop:
 * tokens[r] rows for request r (host array), token-major and concatenated in
 * request order (x [sum tokens, d] fp32, updated in place; h [sum tokens, d]
 * in dtype). The projections, LayerNorms and GELU run once over all rows;
 * per layer, each request's K/V are appended and its causal attention
 * computed over its own pages (mt_paged_prefill_ragged), att[r] (host array of
 * `requests` structs: the request's table row and offset; all must describe
 * the same pool).
 * When logits is not null, logits [requests, vocab] = final-LayerNorm(x)[last
 * row of each request] @ head_weight^T. Scratch as
 * mt_decoder_scratch_bytes(sum tokens). Results equal one mt_prefill_layers
 * call per request up to the projections' algorithm choice for the row
 * count. No reference counterpart (the reference prefills one request per
 * call, minitorch/continuous_batching.py:164-170). */
int mt_prefill_layers_ragged(void* handle, const mt_decoder_layer* layers, int n_layer, float* x,
                             void* h, const float* final_gamma, const float* final_beta,
                             const void* head_weight, void* logits, int vocab, int requests,
                             const int* tokens, int d, int heads, float eps, int dtype, int fused_gelu,
                             void* scratch, size_t scratch_bytes, const mt_prefill_attention* att);

/* One decode step and one ragged prefill in a single layer loop: rows
 * [0, decode_rows) of x [decode_rows + sum tokens, d] fp32 (updated in place)
 * are the decode batch (datt, as mt_decoder_layers takes it), the rest the
 * prompts, tokens[r] rows for request r in request order (patt[r], as
 * mt_prefill_layers_ragged takes them; all on the decode batch's pool). The
 * projections (hipBLASLt, first heuristic choice), LayerNorms and GELU run
 * once over every row; per layer the decode rows' append and attention run
 * before the prompts' appends and attention, so that pages the prompts were
 * given after a decode row's request ended (its pages released once the
 * step's pages were taken) are written, layer by layer, only after that row
 * has read them. When logits is not null, logits [decode_rows + requests,
 * vocab] = final-LayerNorm(x)[decode rows, then each prompt's last row] @
 * head_weight^T. decode_rows <= 65471. Scratch as
 * mt_decoder_scratch_bytes(decode_rows + sum tokens). Results equal
 * mt_decoder_layers followed by mt_prefill_layers_ragged up to the
 * projections' algorithm choice for the row count. No reference counterpart
 * (the reference runs a step's decode batch and its prefills as separate
 * forward passes, minitorch/continuous_batching.py:140-176). */
int mt_mixed_layers(void* handle, const mt_decoder_layer* layers, int n_layer, float* x, void* h,
                    const float* final_gamma, const float* final_beta, const void* head_weight, void* logits,
                    int vocab, int decode_rows, int requests, const int* tokens, int d, int heads, float eps,
                    int dtype, int fused_gelu, void* scratch, size_t scratch_bytes,
                    const mt_decode_attention* datt, const mt_prefill_attention* patt);

#ifdef __cplusplus
}
#endif
#endif /* MT_MODEL_H */
