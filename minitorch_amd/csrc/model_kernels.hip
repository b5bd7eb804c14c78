// Model-side support for the end-to-end decode configs on gfx950: dense
// projections through hipBLASLt and the elementwise steps of a GPT-2 layer
// (LayerNorm, GELU, residual add, embedding sum, head split/merge, casts).
//
// The reference runs these through cuBLAS (src/cuda_runtime.cu:24-30,
// src/mixed_precision.cu:103-122), its fused fp32 LayerNorm
// (src/layernorm_kernel.cu:37-99) and chains of typed map/zip kernels
// (src/mixed_precision.cu:29-97, minitorch/nn.py:222-226). Here weights stay
// resident in the compute type (no per-call casts), the projection bias is a
// hipBLASLt epilogue, and each elementwise step is one kernel.
#include "mt_device.h"
#include <hipblaslt/hipblaslt.h>
#include <climits>
#include <cmath>
#include <map>
#include <mutex>
#include <tuple>

using namespace mt;

namespace {

hipDataType hip_type(int dtype) {
  return dtype == kF32 ? HIP_R_32F : dtype == kF16 ? HIP_R_16F : HIP_R_16BF;
}

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo;
  bool ok = false;
};

// A hipBLASLt handle, a 64 MiB workspace and the plans (descriptors plus the
// heuristic's first algorithm) per GEMM shape, created on first use.
struct Blas {
  hipblasLtHandle_t handle = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = size_t(64) << 20;
  std::mutex mutex;
  std::map<std::tuple<int, int, int, int, int, int, int>, Plan> plans;
};

int blas_status(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS ? 0 : 1000 + int(s); }

// Row-major C[m, n] = A[m, k] @ op(B) (+ bias[n]) where op(B) = B [k, n] or,
// with transb, B^T for B [n, k]. Column-major view: C^T = op(B)^T A^T, i.e. a
// column-major GEMM with rows n, columns m; the bias is per row of C^T.
int gemm(Blas* blas, void* out, const void* a, const void* b, const void* bias, int m, int n,
         int k, int transb, int dtype, int out_dtype) {
  std::lock_guard<std::mutex> lock(blas->mutex);
  auto key = std::make_tuple(m, n, k, transb, dtype, out_dtype, bias ? 1 : 0);
  Plan& p = blas->plans[key];
  if (!p.ok) {
    hipblasStatus_t s;
    const hipDataType in = hip_type(dtype), outt = hip_type(out_dtype);
    if ((s = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F))) return blas_status(s);
    hipblasOperation_t opa = transb ? HIPBLAS_OP_T : HIPBLAS_OP_N, opb = HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa));
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb));
    if (bias) {
      hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
      hipDataType bt = outt;
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi));
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt));
    }
    // A' = B (col-major [n, k], or [k, n] transposed), B' = A (col-major [k, m]).
    if ((s = transb ? hipblasLtMatrixLayoutCreate(&p.la, in, k, n, k)
                    : hipblasLtMatrixLayoutCreate(&p.la, in, n, k, n)))
      return blas_status(s);
    if ((s = hipblasLtMatrixLayoutCreate(&p.lb, in, k, m, k))) return blas_status(s);
    if ((s = hipblasLtMatrixLayoutCreate(&p.lc, outt, n, m, n))) return blas_status(s);
    hipblasLtMatmulPreference_t pref;
    if ((s = hipblasLtMatmulPreferenceCreate(&pref))) return blas_status(s);
    uint64_t ws = blas->workspace_bytes;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    hipblasLtMatmulHeuristicResult_t heur;
    int returned = 0;
    s = hipblasLtMatmulAlgoGetHeuristic(blas->handle, p.desc, p.la, p.lb, p.lc, p.lc, pref, 1, &heur,
                                        &returned);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (s) return blas_status(s);
    if (returned < 1) return blas_status(HIPBLAS_STATUS_NOT_SUPPORTED);
    p.algo = heur.algo;
    p.ok = true;
  }
  if (bias)
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
  const float alpha = 1.f, beta = 0.f;
  return blas_status(hipblasLtMatmul(blas->handle, p.desc, &alpha, b, p.la, a, p.lb, &beta, out,
                                     p.lc, out, p.lc, &p.algo, blas->workspace,
                                     blas->workspace_bytes, nullptr));
}

int blocks_for(int64_t n, int threads = 256) {
  const int64_t b = (n + threads - 1) / threads;
  return int(b < (1 << 20) ? b : (1 << 20));
}

// LayerNorm of fp32 rows (reference src/layernorm_kernel.cu:37-99): one-pass
// mean and E[x^2] - mean^2 clamped at 0, plus eps, then
// gamma * ((x - mean) * rsqrt(var)) + beta, written in the output type.
template <int DT>
__global__ __launch_bounds__(256) void layernorm_kernel(void* out, const float* x, const float* gamma,
                                                        const float* beta, int width, float eps) {
  using T = typename Elem<DT>::T;
  __shared__ float s_sum[8], s_sq[8];
  const float* row = x + int64_t(blockIdx.x) * width;
  float sum = 0.f, sq = 0.f;
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    const float v = row[i];
    sum += v;
    sq += v * v;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sum += __shfl_xor(sum, off);
    sq += __shfl_xor(sq, off);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { s_sum[wave] = sum; s_sq[wave] = sq; }
  __syncthreads();
  float tsum = 0.f, tsq = 0.f;
  for (int w = 0; w < int(blockDim.x >> 6); ++w) { tsum += s_sum[w]; tsq += s_sq[w]; }
  const float mean = tsum / width;
  const float var = fmaxf(tsq / width - mean * mean, 0.f) + eps;
  const float inv = 1.f / sqrtf(var);
  T* o = static_cast<T*>(out) + int64_t(blockIdx.x) * width;
  for (int i = threadIdx.x; i < width; i += blockDim.x)
    o[i] = from_f32<DT>(gamma[i] * ((row[i] - mean) * inv) + beta[i]);
}

// tanh-form GELU in place (reference minitorch/nn.py:222-226):
// 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), computed in fp32.
template <int DT>
__global__ __launch_bounds__(256) void gelu_kernel(void* x, int64_t n) {
  using T = typename Elem<DT>::T;
  T* p = static_cast<T*>(x);
  const float c = 0.7978845608028654f;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const float v = to_f32<DT>(p[i]);
    p[i] = from_f32<DT>(0.5f * v * (1.f + tanhf(c * (v + 0.044715f * v * v * v))));
  }
}

// x[i] += y[i] with fp32 x (the residual stream) and y in its own type.
template <int DT>
__global__ __launch_bounds__(256) void residual_kernel(float* x, const void* y, int64_t n) {
  using T = typename Elem<DT>::T;
  const T* q = static_cast<const T*>(y);
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    x[i] += to_f32<DT>(q[i]);
}

__global__ __launch_bounds__(256) void add_kernel(float* out, const float* a, const float* b, int64_t n) {
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    out[i] = a[i] + b[i];
}

template <int DI, int DO>
__global__ __launch_bounds__(256) void cast_kernel(void* out, const void* in, int64_t n) {
  const auto* src = static_cast<const typename Elem<DI>::T*>(in);
  auto* dst = static_cast<typename Elem<DO>::T*>(out);
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    dst[i] = from_f32<DO>(to_f32<DI>(src[i]));
}

// [b, n, h*d] <-> [b, h, n, d] (split = 1: to heads; 0: back).
template <class T>
__global__ __launch_bounds__(256) void heads_kernel(T* out, const T* in, int b, int n, int h, int d, int split) {
  const int64_t total = int64_t(b) * n * h * d;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    // i indexes the [b, h, n, d] tensor
    const int col = int(i % d);
    const int64_t r = i / d;
    const int t = int(r % n);
    const int64_t r2 = r / n;
    const int hh = int(r2 % h);
    const int bb = int(r2 / h);
    const int64_t j = ((int64_t(bb) * n + t) * h + hh) * d + col;  // [b, n, h, d]
    if (split) out[i] = in[j];
    else out[j] = in[i];
  }
}

bool dtype_ok(int d) { return d >= 0 && d <= 2; }

}  // namespace

extern "C" {

// Replaces reference mt_blas_create / mt_blas_destroy (src/cuda_runtime.cu:22-23).
int mt_blas_create(void** handle) {
  if (!handle) return hipErrorInvalidValue;
  Blas* b = new Blas();
  hipblasStatus_t s = hipblasLtCreate(&b->handle);
  if (s) { delete b; return blas_status(s); }
  hipError_t e = hipMalloc(&b->workspace, b->workspace_bytes);
  if (e != hipSuccess) { hipblasLtDestroy(b->handle); delete b; return e; }
  *handle = b;
  return 0;
}

int mt_blas_destroy(void* handle) {
  Blas* b = static_cast<Blas*>(handle);
  if (!b) return hipErrorInvalidValue;
  for (auto& kv : b->plans) {
    Plan& p = kv.second;
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  }
  hipFree(b->workspace);
  hipblasLtDestroy(b->handle);
  delete b;
  return 0;
}

// Row-major fp32 out[m, n] = a[m, k] @ b[k, n] (reference mt_gemm, src/cuda_runtime.cu:24-30).
int mt_gemm(void* handle, float* out, const float* a, const float* b, int m, int n, int k) {
  if (!handle || !out || !a || !b || m < 1 || n < 1 || k < 1) return hipErrorInvalidValue;
  return gemm(static_cast<Blas*>(handle), out, a, b, nullptr, m, n, k, 0, kF32, kF32);
}

// fp16/bf16 inputs, fp32 accumulation, output fp32 or the input type
// (reference mt_typed_gemm, src/mixed_precision.cu:103-122).
int mt_typed_gemm(void* handle, void* out, const void* a, const void* b, int m, int n, int k,
                  int dtype, int out_dtype) {
  if (dtype < 1 || dtype > 2 || (out_dtype != 0 && out_dtype != dtype)) return hipErrorInvalidValue;
  if (!handle || !out || !a || !b || m < 1 || n < 1 || k < 1) return hipErrorInvalidValue;
  return gemm(static_cast<Blas*>(handle), out, a, b, nullptr, m, n, k, 0, dtype, out_dtype);
}

// Reference mt_low_gemm_supported (src/mixed_precision.cu:98-102): gfx950
// supports fp16 and bf16 inputs.
int mt_low_gemm_supported(int dtype) { return dtype == 1 || dtype == 2; }

// out[m, n] = a[m, k] @ op(b) + bias[n] (bias may be null); op(b) = b [k, n]
// or, with transb, b^T for b [n, k]; fp32 accumulation; dtype 0/1/2 for the
// inputs and the bias' and output's out_dtype (0 or dtype). No reference
// counterpart (bias epilogue and transposed weights for the tied head).
int mt_gemm_ex(void* handle, void* out, const void* a, const void* b, const void* bias, int m,
               int n, int k, int transb, int dtype, int out_dtype) {
  if (!dtype_ok(dtype) || (out_dtype != 0 && out_dtype != dtype)) return hipErrorInvalidValue;
  if (!handle || !out || !a || !b || m < 1 || n < 1 || k < 1 || (transb != 0 && transb != 1))
    return hipErrorInvalidValue;
  return gemm(static_cast<Blas*>(handle), out, a, b, bias, m, n, k, transb, dtype, out_dtype);
}

// out[r, :] = LayerNorm(x[r, :]) in out_dtype for fp32 x [rows, width].
int mt_layernorm_typed(void* out, const float* x, const float* gamma, const float* beta, int rows,
                       int width, float eps, int out_dtype) {
  if (!out || !x || !gamma || !beta || rows < 1 || width < 1 || !dtype_ok(out_dtype))
    return hipErrorInvalidValue;
  if (out_dtype == kF32) layernorm_kernel<kF32><<<rows, 256>>>(out, x, gamma, beta, width, eps);
  else if (out_dtype == kF16) layernorm_kernel<kF16><<<rows, 256>>>(out, x, gamma, beta, width, eps);
  else layernorm_kernel<kBF16><<<rows, 256>>>(out, x, gamma, beta, width, eps);
  return hipGetLastError();
}

int mt_gelu(void* x, long long n, int dtype) {
  if (!x || n < 0 || !dtype_ok(dtype)) return hipErrorInvalidValue;
  if (!n) return 0;
  if (dtype == kF32) gelu_kernel<kF32><<<blocks_for(n), 256>>>(x, n);
  else if (dtype == kF16) gelu_kernel<kF16><<<blocks_for(n), 256>>>(x, n);
  else gelu_kernel<kBF16><<<blocks_for(n), 256>>>(x, n);
  return hipGetLastError();
}

int mt_residual_add(float* x, const void* y, long long n, int dtype) {
  if (!x || !y || n < 0 || !dtype_ok(dtype)) return hipErrorInvalidValue;
  if (!n) return 0;
  if (dtype == kF32) residual_kernel<kF32><<<blocks_for(n), 256>>>(x, y, n);
  else if (dtype == kF16) residual_kernel<kF16><<<blocks_for(n), 256>>>(x, y, n);
  else residual_kernel<kBF16><<<blocks_for(n), 256>>>(x, y, n);
  return hipGetLastError();
}

int mt_add_f32(float* out, const float* a, const float* b, long long n) {
  if (!out || !a || !b || n < 0) return hipErrorInvalidValue;
  if (n) add_kernel<<<blocks_for(n), 256>>>(out, a, b, n);
  return hipGetLastError();
}

int mt_cast(void* out, const void* in, long long n, int in_dtype, int out_dtype) {
  if (!out || !in || n < 0 || !dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return hipErrorInvalidValue;
  if (!n) return 0;
#define MT_CAST(DI, DO) if (in_dtype == DI && out_dtype == DO) cast_kernel<DI, DO><<<blocks_for(n), 256>>>(out, in, n);
  MT_CAST(kF32, kF32) MT_CAST(kF32, kF16) MT_CAST(kF32, kBF16)
  MT_CAST(kF16, kF32) MT_CAST(kF16, kF16) MT_CAST(kF16, kBF16)
  MT_CAST(kBF16, kF32) MT_CAST(kBF16, kF16) MT_CAST(kBF16, kBF16)
#undef MT_CAST
  return hipGetLastError();
}

// split = 1: out [b, h, n, d] <- in [b, n, h*d]; split = 0: the inverse.
int mt_heads(void* out, const void* in, int b, int n, int h, int d, int split, int dtype) {
  if (!out || !in || b < 1 || n < 1 || h < 1 || d < 1 || !dtype_ok(dtype)) return hipErrorInvalidValue;
  const int64_t total = int64_t(b) * n * h * d;
  if (dtype == kF32)
    heads_kernel<float><<<blocks_for(total), 256>>>(static_cast<float*>(out), static_cast<const float*>(in), b, n, h, d, split);
  else
    heads_kernel<uint16_t><<<blocks_for(total), 256>>>(static_cast<uint16_t*>(out), static_cast<const uint16_t*>(in), b, n, h, d, split);
  return hipGetLastError();
}

}  // extern "C"
