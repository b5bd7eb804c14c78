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
#include "../../include/mt_paged.h"
#include "../../include/mt_model.h"
#include <hipblaslt/hipblaslt.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <climits>
#include <cstdlib>
#include <cmath>
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <vector>

using namespace mt;

namespace {

hipDataType hip_type(int dtype) {
  return dtype == kF32 ? HIP_R_32F : dtype == kF16 ? HIP_R_16F : HIP_R_16BF;
}

#ifndef MT_GEMM_CANDIDATES
#define MT_GEMM_CANDIDATES 8
#endif
constexpr int kCandidates = MT_GEMM_CANDIDATES;
// Calls of one shape before its algorithm is chosen by timing: shapes a step
// repeats (the decode projections) are tuned, one-off shapes (a prefill's
// prompt length) keep the heuristic's first choice and pay no timing.
constexpr int kTuneAfterCalls = 3;

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo;
  hipblasLtMatmulHeuristicResult_t heur[kCandidates];
  int candidates = 0;
  int calls = 0;
  bool ok = false;
  bool tunable = false;
};

// One-off shapes (prefill row counts, which batched prefills make nearly
// unique) keep at most this many cached plans; beyond it they are all
// released and rebuilt on demand. Tuned shapes (the decode step's) stay.
constexpr int kMaxOneOffPlans = 256;

// A hipBLASLt handle, a 64 MiB workspace and the plans (descriptors plus the
// chosen algorithm) per GEMM shape, created on first use.
struct Blas {
  hipblasLtHandle_t handle = nullptr;
  void* workspace = nullptr;
  void* flush = nullptr;  // written between timed runs; allocated on the first tuning
  bool tune = true;       // MT_GEMM_TUNE=0 keeps the heuristic's first choice everywhere
  size_t workspace_bytes = size_t(64) << 20;
  std::mutex mutex;
  std::map<std::tuple<int, int, int, int, int, int, int, int, int>, Plan> plans;
  int oneoff_plans = 0;
  // Algorithm per problem class of the one-off shapes (rows rounded up to a
  // multiple of kRowBucket, any row stride): the heuristic's first choice for
  // the class's largest row count.
  std::map<std::tuple<int, int, int, int, int, int, int, int>, hipblasLtMatmulAlgo_t> class_algos;
};

// One-off shapes (a prefill's prompt length, its last-position head with a
// row stride that follows the prompt length) would each cost a heuristic
// query (~0.1 ms of host time, on the prefill's critical path). Rows above
// kRowBucket share the algorithm of their class when hipBLASLt accepts it for
// the exact shape; the class algorithm is a function of the class only, so
// the choice does not depend on which shapes came first.
constexpr int kRowBucket = 64;

int blas_status(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS ? 0 : 1000 + int(s); }

enum Epilogue : int { kEpiNone = 0, kEpiGelu = 1 };

// Projections of the decode step (called through mt_decoder_layers) repeat
// every step with the same shapes, so on the kTuneAfterCalls-th call of such a
// shape the heuristic's candidates are timed on the call's own operands and
// the fastest is kept. Each timed run follows a write of kFlushBytes, so the
// weights come from HBM as they do in a step (a step's weights do not stay in
// the L2/Infinity Cache across its layers); on cache-resident weights other
// candidates win (config 4: 52.2 K vs 49.1 K tokens/s). Other shapes (prefill
// prompt lengths, one-off calls) keep the heuristic's first choice and pay no
// timing, which would otherwise stall serving.
constexpr size_t kFlushBytes = size_t(256) << 20;

// Whether work issued now is being captured into a graph (per-thread stream).
bool stream_capturing() {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(hipStreamPerThread, &status) == hipSuccess && status != hipStreamCaptureStatusNone;
}

int pick_fastest(Blas* blas, Plan& p, const hipblasLtMatmulHeuristicResult_t* heur, int count,
                 void* out, const void* a, const void* b) {
  if (count == 1) { p.algo = heur[0].algo; return 0; }
  if (!blas->flush && hipMalloc(&blas->flush, kFlushBytes) != hipSuccess) {
    blas->flush = nullptr;
    (void)hipGetLastError();
  }
  const float alpha = 1.f, beta = 0.f;
  hipEvent_t start, stop;
  if (hipEventCreate(&start) != hipSuccess) return hipErrorOutOfMemory;
  if (hipEventCreate(&stop) != hipSuccess) { hipEventDestroy(start); return hipErrorOutOfMemory; }
  float best = INFINITY;
  int chosen = -1;
  for (int i = 0; i < count; ++i) {
    auto run = [&]() {
      return hipblasLtMatmul(blas->handle, p.desc, &alpha, b, p.la, a, p.lb, &beta, out, p.lc, out,
                             p.lc, &heur[i].algo, blas->workspace, blas->workspace_bytes, hipStreamPerThread);
    };
    if (run() != HIPBLAS_STATUS_SUCCESS) continue;  // warm-up; unusable candidates drop out
    float total = 0.f;
    bool ok = true;
    for (int r = 0; r < 2 && ok; ++r) {
      if (blas->flush) ok = hipMemsetAsync(blas->flush, r, kFlushBytes, hipStreamPerThread) == hipSuccess;
      hipEventRecord(start, hipStreamPerThread);
      ok = ok && run() == HIPBLAS_STATUS_SUCCESS;
      hipEventRecord(stop, hipStreamPerThread);
      float ms = 0.f;
      ok = ok && hipEventSynchronize(stop) == hipSuccess && hipEventElapsedTime(&ms, start, stop) == hipSuccess;
      total += ms;
    }
    if (ok && total < best) { best = total; chosen = i; }
  }
  hipEventDestroy(start);
  hipEventDestroy(stop);
  p.algo = heur[chosen >= 0 ? chosen : 0].algo;
  return 0;
}

// Row-major C[m, n] = A[m, k] @ op(B) (+ bias[n]) (then GELU) where op(B) =
// B [k, n] or, with transb, B^T for B [n, k]. Column-major view: C^T =
// op(B)^T A^T, i.e. a column-major GEMM with rows n, columns m; the bias is
// per row of C^T.
void release_plan(Plan& p) {
  if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
  if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
  if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = Plan();
}

// The heuristic's first choice for a row-major [m, k] x [k, n] problem with
// the descriptor of `p`, through temporary layouts (lda = k).
bool class_algorithm(Blas* blas, const Plan& p, int m, int n, int k, hipDataType in, hipDataType outt,
                     hipblasLtMatmulAlgo_t* algo) {
  hipblasLtMatrixLayout_t rb = nullptr, rc = nullptr;
  hipblasLtMatmulPreference_t pref = nullptr;
  hipblasLtMatmulHeuristicResult_t h[1];
  int got = 0;
  uint64_t ws = blas->workspace_bytes;
  bool ok = !hipblasLtMatrixLayoutCreate(&rb, in, k, m, k) && !hipblasLtMatrixLayoutCreate(&rc, outt, n, m, n) &&
            !hipblasLtMatmulPreferenceCreate(&pref);
  if (ok) {
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    ok = !hipblasLtMatmulAlgoGetHeuristic(blas->handle, p.desc, p.la, rb, rc, rc, pref, 1, h, &got) && got > 0;
    if (ok) *algo = h[0].algo;
  }
  if (pref) hipblasLtMatmulPreferenceDestroy(pref);
  if (rb) hipblasLtMatrixLayoutDestroy(rb);
  if (rc) hipblasLtMatrixLayoutDestroy(rc);
  return ok;
}

// Descriptors and algorithm candidates of one exact GEMM shape.
int make_plan(Blas* blas, Plan& p, int m, int n, int k, int transb, int dtype, int out_dtype,
              const void* bias, int epilogue, bool tunable, int lda) {
  hipblasStatus_t s;
  const hipDataType in = hip_type(dtype), outt = hip_type(out_dtype);
  if ((s = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F))) return blas_status(s);
  hipblasOperation_t opa = transb ? HIPBLAS_OP_T : HIPBLAS_OP_N, opb = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb));
  hipblasLtEpilogue_t epi = epilogue == kEpiGelu
                                ? (bias ? HIPBLASLT_EPILOGUE_GELU_BIAS : HIPBLASLT_EPILOGUE_GELU)
                                : (bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT);
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi));
  if (bias) {
    hipDataType bt = outt;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt));
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
  }
  // A' = B (col-major [n, k], or [k, n] transposed), B' = A (col-major [k, m]).
  if ((s = transb ? hipblasLtMatrixLayoutCreate(&p.la, in, k, n, k)
                  : hipblasLtMatrixLayoutCreate(&p.la, in, n, k, n)))
    return blas_status(s);
  if ((s = hipblasLtMatrixLayoutCreate(&p.lb, in, k, m, lda))) return blas_status(s);
  if ((s = hipblasLtMatrixLayoutCreate(&p.lc, outt, n, m, n))) return blas_status(s);
  if (!tunable && (m > kRowBucket || lda != k)) {
    const int mb = m > kRowBucket ? (m + kRowBucket - 1) / kRowBucket * kRowBucket : m;
    const auto ckey = std::make_tuple(mb, n, k, transb, dtype, out_dtype, bias ? 1 : 0, epilogue);
    auto it = blas->class_algos.find(ckey);
    if (it == blas->class_algos.end()) {
      hipblasLtMatmulAlgo_t algo;
      if (class_algorithm(blas, p, mb, n, k, in, outt, &algo))
        it = blas->class_algos.emplace(ckey, algo).first;
    }
    if (it != blas->class_algos.end()) {
      const float one = 1.f, zero = 0.f;
      hipblasLtMatmulAlgo_t algo = it->second;
      size_t need = 0;
      if (hipblaslt_ext::matmulIsAlgoSupported(blas->handle, p.desc, &one, p.la, p.lb, &zero, p.lc, p.lc,
                                               algo, need) == HIPBLAS_STATUS_SUCCESS &&
          need <= blas->workspace_bytes) {
        p.heur[0].algo = algo;
        p.candidates = 1;
        p.algo = algo;
        p.ok = true;
        return 0;
      }
    }
  }
  hipblasLtMatmulPreference_t pref;
  if ((s = hipblasLtMatmulPreferenceCreate(&pref))) return blas_status(s);
  uint64_t ws = blas->workspace_bytes;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
  int returned = 0;
  s = hipblasLtMatmulAlgoGetHeuristic(blas->handle, p.desc, p.la, p.lb, p.lc, p.lc, pref, kCandidates,
                                      p.heur, &returned);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (s) return blas_status(s);
  if (returned < 1) return blas_status(HIPBLAS_STATUS_NOT_SUPPORTED);
  p.candidates = returned;
  p.algo = p.heur[0].algo;
  p.ok = true;
  return 0;
}

int gemm(Blas* blas, void* out, const void* a, const void* b, const void* bias, int m, int n,
         int k, int transb, int dtype, int out_dtype, int epilogue = kEpiNone, bool tunable = false,
         int lda = 0) {
  if (lda == 0) lda = k;  // elements between consecutive rows of a
  std::lock_guard<std::mutex> lock(blas->mutex);
  auto key = std::make_tuple(m, n, k, transb, dtype, out_dtype, bias ? 1 : 0, epilogue, lda);
  if (!tunable && blas->oneoff_plans >= kMaxOneOffPlans && !blas->plans.count(key)) {
    for (auto it = blas->plans.begin(); it != blas->plans.end();) {
      if (!it->second.tunable) {
        release_plan(it->second);
        it = blas->plans.erase(it);
      } else {
        ++it;
      }
    }
    blas->oneoff_plans = 0;
  }
  Plan& p = blas->plans[key];
  if (p.ok && tunable && !p.tunable) {
    // First built for a one-off call (one class algorithm, never timed): a
    // repeating shape rebuilds it with the heuristic's candidates to time.
    release_plan(p);
    --blas->oneoff_plans;
  }
  if (!p.ok) {
    // On failure the partial plan is released so a later call can retry.
    const int st = make_plan(blas, p, m, n, k, transb, dtype, out_dtype, bias, epilogue, tunable, lda);
    if (st) {
      release_plan(p);
      blas->plans.erase(key);
      return st;
    }
    p.tunable = tunable;
    if (!tunable) ++blas->oneoff_plans;
  }
  // No timing (events, synchronization, cache flushes) inside a stream
  // capture: a captured step keeps the algorithm chosen so far.
  if (tunable && !stream_capturing() && ++p.calls == kTuneAfterCalls && p.candidates > 1 && blas->tune) {
    if (bias)
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
    const int e = pick_fastest(blas, p, p.heur, p.candidates, out, a, b);
    if (e) return e;
  }
  if (bias)
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
  const float alpha = 1.f, beta = 0.f;
  return blas_status(hipblasLtMatmul(blas->handle, p.desc, &alpha, b, p.la, a, p.lb, &beta, out,
                                     p.lc, out, p.lc, &p.algo, blas->workspace,
                                     blas->workspace_bytes, hipStreamPerThread));
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

// Residual add fused with the next LayerNorm: x[r, :] += y[r, :] (y in DT,
// the fp32 residual stream updated in place), then out = LayerNorm(x[r, :])
// exactly as layernorm_kernel computes it.
template <int DT>
__global__ __launch_bounds__(256) void residual_layernorm_kernel(void* out, float* x, const void* y,
                                                                 const float* gamma, const float* beta,
                                                                 int width, float eps) {
  using T = typename Elem<DT>::T;
  __shared__ float s_sum[8], s_sq[8];
  float* row = x + int64_t(blockIdx.x) * width;
  const T* yr = static_cast<const T*>(y) + int64_t(blockIdx.x) * width;
  float sum = 0.f, sq = 0.f;
  for (int i = threadIdx.x; i < width; i += blockDim.x) {
    const float v = row[i] + to_f32<DT>(yr[i]);
    row[i] = v;
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
  // each thread reads back only the elements it wrote above
  for (int i = threadIdx.x; i < width; i += blockDim.x)
    o[i] = from_f32<DT>(gamma[i] * ((row[i] - mean) * inv) + beta[i]);
}

// Fragment-tiled layout of a 16-bit [rows, width] activation matrix (width a
// multiple of 32, rows padded to a multiple of 16): the 16 x 32 block of row
// tile R and column tile K is 1 KB at element ((R * width / 32) + K) * 512,
// stored in the order lane (c, g) of v_mfma_f32_16x16x32 takes it as its B
// operand: row 16 R + c, columns 32 K + 8 g .. 8 g + 7 at element
// (16 g + c) * 8 of the block. A wave then reads a B fragment as one 1 KB run
// of consecutive 16-byte lane loads, which the memory pipeline coalesces;
// from row-major rows the same fragment is 16 separate 64-byte pieces, served
// at about a third of the rate (MI355X: ~35 against ~110 GB/s per compute
// unit from L2). kProjXTiled: x is tiled; kProjOutTiled: out (epilogues 0
// and 1) is written tiled; kProjWTiled: the weights [n, k] are tiled (their
// A fragments have the same lane order). A tiled buffer holds
// ceil(rows / 16) * 16 rows; the rows past `rows` are read but never affect a
// stored result.
enum ProjLayout : int { kProjXTiled = 1, kProjOutTiled = 2, kProjWTiled = 4 };
__host__ __device__ __forceinline__ int64_t tiled_offset(int row, int col, int width) {
  return ((int64_t(row >> 4) * (width >> 5) + (col >> 5)) << 9) + ((((col >> 3) & 3) << 4) + (row & 15)) * 8 +
         (col & 7);
}

// The same residual add + LayerNorm with one wave per row, for widths that are
// a multiple of 256 (at most 256 * NJ): lane l owns columns 4l + 256j of
// every 256-column block j. All loads of a row (x, y, gamma, beta) are issued
// at once and the row stays in registers, so the kernel makes one dependent
// memory round trip and reduces within the wave (no LDS, no barrier).
// XOR-butterfly sums leave every lane with the row total. Blocks past the
// row's last (j >= width / 256) repeat the last one and add nothing to the
// sums, so that the code has no branch on the width (a branch made the
// compiler wait for the residual stores before the output stores).
template <int DT, int NJ, bool RES>
__global__ __launch_bounds__(256) void residual_layernorm_wave_kernel(void* __restrict__ out, float* __restrict__ x,
                                                                      const void* __restrict__ y,
                                                                      const float* __restrict__ gamma,
                                                                      const float* __restrict__ beta, int rows,
                                                                      int width, float eps, int out_tiled) {
  using T = typename Elem<DT>::T;
  using R = typename std::conditional<DT == kF32, float4, uint2>::type;  // 4 elements of y
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * int(blockDim.x >> 6) + int(threadIdx.x >> 6);
  if (row >= rows) return;
  const int nj = width >> 8;
  float* xr = x + int64_t(row) * width;
  const T* yr = static_cast<const T*>(y) + int64_t(row) * width;
  int col[NJ];
  float4 v[NJ], g[NJ], b[NJ];
  R r[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    col[j] = 256 * (j < nj ? j : nj - 1) + 4 * lane;
    v[j] = *reinterpret_cast<const float4*>(xr + col[j]);
    g[j] = *reinterpret_cast<const float4*>(gamma + col[j]);
    b[j] = *reinterpret_cast<const float4*>(beta + col[j]);
    if constexpr (RES) r[j] = *reinterpret_cast<const R*>(yr + col[j]);
  }
  float sum = 0.f, sq = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if constexpr (RES) {
      if constexpr (DT == kF32) {
        v[j].x += r[j].x; v[j].y += r[j].y; v[j].z += r[j].z; v[j].w += r[j].w;
      } else {
        v[j].x += to_f32<DT>(T(r[j].x & 0xffffu)); v[j].y += to_f32<DT>(T(r[j].x >> 16));
        v[j].z += to_f32<DT>(T(r[j].y & 0xffffu)); v[j].w += to_f32<DT>(T(r[j].y >> 16));
      }
      *reinterpret_cast<float4*>(xr + col[j]) = v[j];  // a repeated block stores the same values again
    }
    const float keep = j < nj ? 1.f : 0.f;
    sum += keep * ((v[j].x + v[j].y) + (v[j].z + v[j].w));
    sq += keep * ((v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sum += __shfl_xor(sum, off);
    sq += __shfl_xor(sq, off);
  }
  const float mean = sum / width;
  const float var = fmaxf(sq / width - mean * mean, 0.f) + eps;
  const float inv = 1.f / sqrtf(var);
  T* o = static_cast<T*>(out);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = col[j];
    const int64_t at = out_tiled ? tiled_offset(row, c, width) : int64_t(row) * width + c;
    const float r0 = g[j].x * ((v[j].x - mean) * inv) + b[j].x;
    const float r1 = g[j].y * ((v[j].y - mean) * inv) + b[j].y;
    const float r2 = g[j].z * ((v[j].z - mean) * inv) + b[j].z;
    const float r3 = g[j].w * ((v[j].w - mean) * inv) + b[j].w;
    if constexpr (DT == kF32) {
      *reinterpret_cast<float4*>(o + at) = float4{r0, r1, r2, r3};
    } else {
      *reinterpret_cast<uint2*>(o + at) =
          uint2{uint32_t(from_f32<DT>(r0)) | (uint32_t(from_f32<DT>(r1)) << 16),
                uint32_t(from_f32<DT>(r2)) | (uint32_t(from_f32<DT>(r3)) << 16)};
    }
  }
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

// Rows (one wave each) per workgroup of the one-wave-per-row LayerNorm
// kernels. A decode step's LayerNorms are latency-bound; 2 rows per workgroup
// spread GPT-2-medium's 128 rows over 64 compute units (steps 3.5 % faster
// than with 4 rows per workgroup on MI355X; 1 row is no faster).
#ifndef MT_LN_ROWS_PER_BLOCK
#define MT_LN_ROWS_PER_BLOCK 2
#endif
constexpr int kLnRowsPerBlock = MT_LN_ROWS_PER_BLOCK;
static_assert(kLnRowsPerBlock >= 1 && kLnRowsPerBlock * 64 <= 256,
              "the one-wave-per-row LayerNorm kernels are built for at most 256 threads per workgroup");

// ---------------------------------------------------------------------------
// Decode projections on the matrix cores: out[m, n] = x[m, :] . w[n, :] for
// the few rows of a decode step (m <= kProjMaxRows) against weights stored
// [n, k] (fp16/bf16, fp32 accumulation). At these row counts a projection
// moves a few MB (the weights, read once) through short chains of dependent
// loads, so the kernel is built for memory-level parallelism: many waves,
// each with a short k range whose loads are all issued before its first
// MFMA, instead of long per-wave k loops that wait one memory latency per
// step.
//
// C^T = W X^T on v_mfma_f32_16x16x32: A = 16 weight rows, B = 16 activation
// rows, both contiguous along k and loaded 16 bytes per lane straight from
// global memory; lane (c, g) ends up holding C^T[4g + i][c], i.e. 4
// consecutive features of one row. A workgroup owns 16 NT features, 16 MT
// rows (blockIdx.z selects the row block) and k range blockIdx.y of
// `splits`; its WK waves (blockDim.x / 64) split that range into kc-wide
// pieces of at most SMAX 32-wide steps, and their sums meet in LDS. Weights
// are read with non-temporal loads (a step's weights do not fit the caches);
// the activations, which every workgroup reads, stay cached.
//
// Epilogues: kProjBias: + bias (type T) -> T; kProjGelu: + bias, tanh GELU
// in fp32 -> T; kProjPartials: the fp32 sums of split blockIdx.y into
// out[split][m][n] (no bias), which residual_layernorm_partials_kernel adds
// into the residual stream together with the bias.
constexpr int kProjMaxRows = 256;
constexpr int kProjMaxSplits = 8;
constexpr int kProjMaxWaves = 16;
// Row counts up to which a decode step on row-major activations (the layer
// loop's fallback when neither the fused nor the tiled path takes the shapes)
// uses this kernel rather than hipBLASLt, measured on MI355X with captured
// DistilGPT-2 and GPT-2-medium steps: unsplit projections to 16 rows, split
// ones plus their LayerNorm reduction to 32. The tiled path also takes its
// out-projection (row-major: attention's output) split up to kProjSplitRows.
constexpr int kProjDirectRows = 16;
constexpr int kProjSplitRows = 32;
enum ProjEpilogue : int { kProjBias = 0, kProjGelu = 1, kProjPartials = 2 };


struct ProjArgs {
  void* out;
  const void* x;
  const void* w;
  const void* bias;
  int m, n, k;
  int kc;  // k per wave: k / (splits * waves), a multiple of 32, at most 32 * SMAX
  int w_tiled;  // w is [n, k] in the fragment-tiled layout
  // LayerNorm prologue (projection_kernel with PS >= 0): the activations are
  // LayerNorm(x_in + part_bias + sum of the PS partial rows part[s, r, :]),
  // computed by every workgroup; workgroup (0, 0, 0) writes the sum to x_out.
  const float* x_in;
  float* x_out;
  const float* part;
  const void* part_bias;
  const float* gamma;
  const float* beta;
  float eps;
};

// Rows up to which the decode step fuses the residual add and LayerNorm into
// the QKV and fc projections (every workgroup re-reads m * d * (4 + 4 splits)
// bytes, which outweighs the saved launch beyond a few rows), and the largest
// width the prologue takes.
#ifndef MT_PROJ_FUSED_ROWS
#define MT_PROJ_FUSED_ROWS 8
#endif
constexpr int kProjFusedRows = MT_PROJ_FUSED_ROWS;
constexpr int kProjFusedMaxWidth = 1024;

__device__ __forceinline__ float gelu_tanh(float v) {
  const float c = 0.7978845608028654f;
  return 0.5f * v * (1.f + tanhf(c * (v + 0.044715f * v * v * v)));
}

// Steps of 32 a wave may hold in flight: 2 with 8 row tiles (the loads and
// accumulators then fill the 128 registers a 16-wave workgroup allows), 4
// with fewer. (4 steps in 8-wave workgroups at 8 row tiles, which halves the
// cross-wave reduction, measured 4-8 % slower on MI355X: fewer loads in
// flight per compute unit.)
template <int MT>
constexpr int proj_max_steps() { return MT >= 8 ? 2 : 4; }

// LayerNorm prologue of projection_kernel (PS >= 0, one row tile): pass 1
// spreads the m x k sums v = x_in + part_bias + sum_s part[s] over all
// threads (every load in flight at once) into vbuf, and gamma/beta into gb;
// pass 2 takes one wave per row for the mean and variance (one-pass, as the
// LayerNorm kernels) and writes the normalized rows in T to the activation
// tile xt (row stride xs).
template <int DT, int PS>
__device__ __forceinline__ void ln_prologue(const ProjArgs& p, float* vbuf, float* gb, typename Elem<DT>::T* xt,
                                            int xs, int wave, int waves, int lane) {
  using T = typename Elem<DT>::T;
  const int tid = int(threadIdx.x), nt = int(blockDim.x);
  const int k4 = p.k >> 2;
  const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
  for (int i = tid; i < p.m * k4; i += nt) {
    const int r = i / k4, c = 4 * (i - r * k4);
    float4 v = *reinterpret_cast<const float4*>(p.x_in + r * p.k + c);
    if constexpr (PS > 0) {
      float4 q[PS];
#pragma unroll
      for (int s = 0; s < PS; ++s) q[s] = *reinterpret_cast<const float4*>(p.part + (s * p.m + r) * p.k + c);
      const uint2 b = p.part_bias ? *reinterpret_cast<const uint2*>(static_cast<const T*>(p.part_bias) + c)
                                  : uint2{0u, 0u};
      v.x += to_f32<DT>(T(b.x & 0xffffu)); v.y += to_f32<DT>(T(b.x >> 16));
      v.z += to_f32<DT>(T(b.y & 0xffffu)); v.w += to_f32<DT>(T(b.y >> 16));
#pragma unroll
      for (int s = 0; s < PS; ++s) { v.x += q[s].x; v.y += q[s].y; v.z += q[s].z; v.w += q[s].w; }
    }
    *reinterpret_cast<float4*>(vbuf + r * p.k + c) = v;
    if (writer) *reinterpret_cast<float4*>(p.x_out + r * p.k + c) = v;
  }
  for (int i = tid; i < k4; i += nt) {
    *reinterpret_cast<float4*>(gb + 4 * i) = *reinterpret_cast<const float4*>(p.gamma + 4 * i);
    *reinterpret_cast<float4*>(gb + p.k + 4 * i) = *reinterpret_cast<const float4*>(p.beta + 4 * i);
  }
  __syncthreads();
  const int nj = p.k >> 8;
  for (int r = wave; r < p.m; r += waves) {
    float sum = 0.f, sq = 0.f;
    for (int j = 0; j < nj; ++j) {
      const float4 v = *reinterpret_cast<const float4*>(vbuf + r * p.k + 256 * j + 4 * lane);
      sum += (v.x + v.y) + (v.z + v.w);
      sq += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      sum += __shfl_xor(sum, off);
      sq += __shfl_xor(sq, off);
    }
    const float mean = sum / p.k;
    const float var = fmaxf(sq / p.k - mean * mean, 0.f) + p.eps;
    const float inv = 1.f / sqrtf(var);
    for (int j = 0; j < nj; ++j) {
      const int c = 256 * j + 4 * lane;
      const float4 v = *reinterpret_cast<const float4*>(vbuf + r * p.k + c);
      const float4 g = *reinterpret_cast<const float4*>(gb + c);
      const float4 b = *reinterpret_cast<const float4*>(gb + p.k + c);
      const float r0 = g.x * ((v.x - mean) * inv) + b.x;
      const float r1 = g.y * ((v.y - mean) * inv) + b.y;
      const float r2 = g.z * ((v.z - mean) * inv) + b.z;
      const float r3 = g.w * ((v.w - mean) * inv) + b.w;
      *reinterpret_cast<uint2*>(xt + r * xs + c) =
          uint2{uint32_t(from_f32<DT>(r0)) | (uint32_t(from_f32<DT>(r1)) << 16),
                uint32_t(from_f32<DT>(r2)) | (uint32_t(from_f32<DT>(r3)) << 16)};
    }
  }
  __syncthreads();
}

// PS < 0: activations read from p.x (row-major, or tiled with LAY &
// kProjXTiled). PS >= 0 (one row tile, one feature tile, one split): the
// activations come from the LayerNorm prologue through LDS; the weight loads
// are issued before it, so their HBM latency overlaps it. LAY &
// kProjOutTiled writes out tiled. A workgroup owns NT feature tiles and MT
// row tiles: each wave's step loads NT weight and MT activation fragments and
// runs NT * MT MFMAs.
template <int DT, int MT, int EPI, int PS = -1, int LAY = 0, int NT = 1>
__global__ __launch_bounds__(1024) void projection_kernel(ProjArgs p) {
  using T = typename Elem<DT>::T;
  using V8 = typename Mfma<DT>::v8;
  constexpr int SMAX = proj_max_steps<MT * NT>();
  constexpr int NL = NT + MT;  // 16-byte loads per lane and step
  constexpr int NQ = NT * MT;  // output tiles
  constexpr bool LN = PS >= 0;
  constexpr bool XT = (LAY & kProjXTiled) != 0;
  constexpr int XSTEP = XT ? 512 : 32;  // elements between a lane's activations of consecutive 32-wide steps
  static_assert(!LN || (MT == 1 && NT == 1), "the LayerNorm prologue takes one row and one feature tile");
  static_assert(!LN || LAY == 0, "the LayerNorm prologue reads its activations from LDS");
  static_assert(EPI != kProjPartials || !(LAY & kProjOutTiled), "split partials are written row-major");
  // [waves][NQ][64] sums | LN: v [m][k] fp32, gamma/beta [2][k] fp32, tile [16][k + 8] T
  extern __shared__ floatx4 red[];
  const int waves = int(blockDim.x >> 6);
  const int wave = int(threadIdx.x >> 6), lane = int(threadIdx.x & 63);
  const int col = lane & 15, grp = lane >> 4;
  const int f0 = int(blockIdx.x) * 16 * NT;
  const int r0 = int(blockIdx.z) * 16 * MT;
  const int k0 = (int(blockIdx.y) * waves + wave) * p.kc + 8 * grp;
  const int kt = (k0 - 8 * grp) >> 5;  // the wave's first 32-wide step
  const int steps = p.kc >> 5;
  // weights [n, k] row-major, or tiled (p.w_tiled) as the activations are
  const T* w = p.w_tiled ? static_cast<const T*>(p.w) + ((int64_t(f0 >> 4) * (p.k >> 5) + kt) << 9) + lane * 8
                         : static_cast<const T*>(p.w) + int64_t(f0 + col) * p.k + k0;
  const int wstep = p.w_tiled ? 512 : 32;  // elements between a lane's weights of consecutive steps
  const int wtile = p.k << 4;              // and of consecutive feature tiles (16 rows of k in both layouts)
  const T* x = static_cast<const T*>(p.x);
  int xoff[MT];  // element offsets of this lane's activations at the first step
  if constexpr (XT) {
    // row tiles past the last one repeat it (their columns are never stored)
    const int last = (p.m - 1) >> 4;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int rt = (r0 >> 4) + t < last ? (r0 >> 4) + t : last;
      xoff[t] = ((rt * (p.k >> 5) + kt) << 9) + lane * 8;
    }
  } else {
    // rows past m repeat row m - 1
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int row = r0 + 16 * t + col < p.m ? r0 + 16 * t + col : p.m - 1;
      xoff[t] = row * p.k + k0;
    }
  }
  // the bias of the output tile this wave finishes first (q = wave), loaded
  // with the operands instead of after the reduction
  uint2 bias0 = uint2{0u, 0u};
  if (EPI != kProjPartials && p.bias && wave < NQ)
    bias0 = *reinterpret_cast<const uint2*>(static_cast<const T*>(p.bias) + f0 + 16 * (wave / MT) + 4 * grp);
  u32x4 buf[SMAX][NL];
  if constexpr (LN) {
    float* vbuf = reinterpret_cast<float*>(red + waves * 64);
    float* gb = vbuf + p.m * p.k;
    T* xt = reinterpret_cast<T*>(gb + 2 * p.k);
    const int xs = p.k + 8;
#pragma unroll
    for (int s = 0; s < SMAX; ++s)
      if (s < steps) buf[s][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + wstep * s));
    ln_prologue<DT, PS>(p, vbuf, gb, xt, xs, wave, waves, lane);
    const int row = col < p.m ? col : p.m - 1;
#pragma unroll
    for (int s = 0; s < SMAX; ++s)
      if (s < steps) buf[s][1] = *reinterpret_cast<const u32x4*>(xt + row * xs + k0 + 32 * s);
  } else {
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      if (s < steps) {
#pragma unroll
        for (int f = 0; f < NT; ++f)
          buf[s][f] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w + wtile * f + wstep * s));
#pragma unroll
        for (int t = 0; t < MT; ++t)
          buf[s][NT + t] = *global_view(reinterpret_cast<const u32x4*>(x + xoff[t] + XSTEP * s));
      }
    }
  }
  floatx4 acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < SMAX; ++s) {
    if (s < steps) {
#pragma unroll
      for (int f = 0; f < NT; ++f)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          acc[f * MT + t] = Mfma<DT>::run(__builtin_bit_cast(V8, buf[s][f]), __builtin_bit_cast(V8, buf[s][NT + t]),
                                          acc[f * MT + t]);
    }
  }

#pragma unroll
  for (int q = 0; q < NQ; ++q) red[(wave * NQ + q) * 64 + lane] = acc[q];
  __syncthreads();
  for (int q = wave; q < NQ; q += waves) {
    floatx4 a = red[q * 64 + lane];
    for (int v = 1; v < waves; ++v) {
      const floatx4 b = red[(v * NQ + q) * 64 + lane];
      a[0] += b[0]; a[1] += b[1]; a[2] += b[2]; a[3] += b[3];
    }
    const int row = r0 + 16 * (q % MT) + col;
    if (row >= p.m) continue;
    const int feat = f0 + 16 * (q / MT) + 4 * grp;
    float v[4] = {a[0], a[1], a[2], a[3]};
    if constexpr (EPI == kProjPartials) {
      float* o = static_cast<float*>(p.out) + (int64_t(blockIdx.y) * p.m + row) * p.n + feat;
      *reinterpret_cast<float4*>(o) = float4{v[0], v[1], v[2], v[3]};
    } else {
      if (p.bias) {
        const uint2 b = q == wave ? bias0 : *reinterpret_cast<const uint2*>(static_cast<const T*>(p.bias) + feat);
        v[0] += to_f32<DT>(T(b.x & 0xffffu)); v[1] += to_f32<DT>(T(b.x >> 16));
        v[2] += to_f32<DT>(T(b.y & 0xffffu)); v[3] += to_f32<DT>(T(b.y >> 16));
      }
      if constexpr (EPI == kProjGelu) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = gelu_tanh(v[i]);
      }
      T* o = static_cast<T*>(p.out) + ((LAY & kProjOutTiled) ? tiled_offset(row, feat, p.n) : int64_t(row) * p.n + feat);
      *reinterpret_cast<uint2*>(o) =
          uint2{uint32_t(from_f32<DT>(v[0])) | (uint32_t(from_f32<DT>(v[1])) << 16),
                uint32_t(from_f32<DT>(v[2])) | (uint32_t(from_f32<DT>(v[3])) << 16)};
    }
  }
}

// x[r, :] += bias + sum over the S splits of partials[s, r, :] (fp32);
// out[r, :] = LayerNorm(x[r, :]) in T. One wave per row, as
// residual_layernorm_wave_kernel; every load of a row (x, bias, the S
// partials, which other XCDs wrote, gamma and beta) is issued before the
// first add, so the kernel waits for one memory round trip (loading gamma and
// beta after the reduction made GPT-2-medium decode steps 2-4 % slower).
// Blocks past the row's last repeat it and add nothing to the sums, and a
// missing bias is read from gamma and zeroed, so that no branch makes the
// output stores wait for the residual stores.
template <int DT, int NJ, int S>
__global__ __launch_bounds__(256) void residual_layernorm_partials_kernel(void* __restrict__ out, float* __restrict__ x,
                                                                          const float* __restrict__ part,
                                                                          const void* __restrict__ bias,
                                                                          const float* __restrict__ gamma,
                                                                          const float* __restrict__ beta, int rows,
                                                                          int width, float eps, int out_tiled) {
  using T = typename Elem<DT>::T;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * int(blockDim.x >> 6) + int(threadIdx.x >> 6);
  if (row >= rows) return;
  const int nj = width >> 8;
  float* xr = x + int64_t(row) * width;
  const int64_t split_stride = int64_t(rows) * width;
  const float* pr = part + int64_t(row) * width;
  const bool has_bias = bias != nullptr;
  const T* bp = has_bias ? static_cast<const T*>(bias) : reinterpret_cast<const T*>(gamma);
  int col[NJ];
  float4 v[NJ], q[NJ][S], gm[NJ], bt[NJ];
  uint2 b[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    col[j] = 256 * (j < nj ? j : nj - 1) + 4 * lane;
    const int c = col[j];
    v[j] = *reinterpret_cast<const float4*>(xr + c);
    b[j] = *reinterpret_cast<const uint2*>(bp + c);
#pragma unroll
    for (int s = 0; s < S; ++s) q[j][s] = *reinterpret_cast<const float4*>(pr + s * split_stride + c);
    gm[j] = *reinterpret_cast<const float4*>(gamma + c);
    bt[j] = *reinterpret_cast<const float4*>(beta + c);
  }
  float sum = 0.f, sq = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint2 bj = has_bias ? b[j] : uint2{0u, 0u};
    v[j].x += to_f32<DT>(T(bj.x & 0xffffu)); v[j].y += to_f32<DT>(T(bj.x >> 16));
    v[j].z += to_f32<DT>(T(bj.y & 0xffffu)); v[j].w += to_f32<DT>(T(bj.y >> 16));
#pragma unroll
    for (int s = 0; s < S; ++s) {
      v[j].x += q[j][s].x; v[j].y += q[j][s].y; v[j].z += q[j][s].z; v[j].w += q[j][s].w;
    }
    *reinterpret_cast<float4*>(xr + col[j]) = v[j];  // a repeated block stores the same values again
    const float keep = j < nj ? 1.f : 0.f;
    sum += keep * ((v[j].x + v[j].y) + (v[j].z + v[j].w));
    sq += keep * ((v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    sum += __shfl_xor(sum, off);
    sq += __shfl_xor(sq, off);
  }
  const float mean = sum / width;
  const float var = fmaxf(sq / width - mean * mean, 0.f) + eps;
  const float inv = 1.f / sqrtf(var);
  T* o = static_cast<T*>(out);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int c = col[j];
    const int64_t at = out_tiled ? tiled_offset(row, c, width) : int64_t(row) * width + c;
    const float4 g = gm[j], bb = bt[j];
    const float r0 = g.x * ((v[j].x - mean) * inv) + bb.x;
    const float r1 = g.y * ((v[j].y - mean) * inv) + bb.y;
    const float r2 = g.z * ((v[j].z - mean) * inv) + bb.z;
    const float r3 = g.w * ((v[j].w - mean) * inv) + bb.w;
    *reinterpret_cast<uint2*>(o + at) =
        uint2{uint32_t(from_f32<DT>(r0)) | (uint32_t(from_f32<DT>(r1)) << 16),
              uint32_t(from_f32<DT>(r2)) | (uint32_t(from_f32<DT>(r3)) << 16)};
  }
}

bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0; }

// Row tiles (mt) and feature tiles (nt) of 16 a workgroup holds for m rows of
// an n-feature projection (more rows take several row blocks of 16 mt). Every
// workgroup takes in (16 mt + 16 nt) k elements for 256 mt nt outputs: from
// 33 rows on, 32 features (n a multiple of 32) by 32 or 64 rows read a
// fifth to a third less than 16 features by 64 or 128 rows, with the same
// number of workgroups.
struct ProjTiles {
  int mt, nt;
};
ProjTiles proj_tiles(int m, int n) {
  if (m <= 16) return {1, 1};
  if (m <= 32) return {2, 1};
  if (n % 32 == 0) return {m <= 64 ? 2 : 4, 2};
  return {m <= 64 ? 4 : 8, 1};
}

// Waves per workgroup for a k range of `range` per split and q = mt * nt
// output tiles: the most (at most kProjMaxWaves) that leave each wave a whole
// number of 32-wide steps, at most as many as it can hold in flight; 0 if none
// does.
int proj_waves(int range, int q) {
  const int smax = q >= 8 ? proj_max_steps<8>() : proj_max_steps<4>();
  for (int wv = kProjMaxWaves; wv >= 1; --wv)
    if (range % (32 * wv) == 0 && range / (32 * wv) <= smax) return wv;
  return 0;
}

// Whether the decode projection kernel takes out = epi(x [m, k] @ w[n, k]^T):
// fp16/bf16, m <= kProjMaxRows, n a multiple of 16, k split into `splits`
// ranges that some wave count divides into short whole-step pieces, 16-byte
// aligned rows.
bool projection_ok(const void* out, const void* x, const void* w, const void* bias, int m, int n, int k,
                   int splits, int epilogue, int dtype, int layout = 0) {
  if (dtype != kF16 && dtype != kBF16) return false;
  if (m < 1 || m > kProjMaxRows || n < 16 || n % 16 || k < 32) return false;
  if (splits != 1 && splits != 2 && splits != 4 && splits != 8) return false;
  if (epilogue < 0 || epilogue > kProjPartials || (epilogue != kProjPartials && splits != 1)) return false;
  if (layout < 0 || layout > (kProjXTiled | kProjOutTiled | kProjWTiled)) return false;
  if ((layout & kProjOutTiled) && (epilogue == kProjPartials || n % 32)) return false;
  const ProjTiles pt = proj_tiles(m, n);
  if (k % splits || proj_waves(k / splits, pt.mt * pt.nt) == 0) return false;
  const int64_t mp = (int64_t(m) + 15) / 16 * 16;  // rows of a tiled buffer
  if (mp * k > INT32_MAX || int64_t(n) * k > INT32_MAX || int64_t(splits) * mp * n > INT32_MAX) return false;
  return out && x && w && aligned(x, 16) && aligned(w, 16) && aligned(out, epilogue == kProjPartials ? 16 : 8) &&
         (!bias || aligned(bias, 8));
}

// MT_DECODE_PROJECTIONS=0 sends the decode step's projections to hipBLASLt.
bool decode_projections_enabled() {
  static const bool on = [] {
    const char* v = std::getenv("MT_DECODE_PROJECTIONS");
    return !(v && v[0] == '0');
  }();
  return on;
}

// Rows up to which a decode step past the fused rows runs on the projection
// kernel with tiled activations (MT_DECODE_TILED_ROWS overrides it, 0 turns
// the tiled path off). Captured GPT-2-medium steps on MI355X: 1.80 against
// 1.91 ms at 128 rows, 2.86 against 2.72 ms at 256 (hipBLASLt's tiles win
// there).
constexpr int kProjTiledRows = 128;
int decode_tiled_rows() {
  static const int rows = [] {
    const char* v = std::getenv("MT_DECODE_TILED_ROWS");
    return v && *v ? std::atoi(v) : kProjTiledRows;
  }();
  return rows;
}

// Splits of k for an [m, n] x [n, k] projection whose partial sums are
// reduced downstream: the fewest that give at least one workgroup per compute
// unit (n / 16 feature tiles per split), while the projection kernel still
// takes each split's range.
int projection_splits(int m, int n, int k) {
  static const int cus = [] {
    int dev = 0, c = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c < 1)
      c = 256;
    return c;
  }();
  const ProjTiles pt = proj_tiles(m, n);
  const int tiles = n / (16 * pt.nt) * ((m + 16 * pt.mt - 1) / (16 * pt.mt));
  auto takes = [&](int s) { return k % s == 0 && proj_waves(k / s, pt.mt * pt.nt) > 0; };
  int s = 1;
  while (s < kProjMaxSplits && !takes(s)) s *= 2;
  while (s < kProjMaxSplits && int64_t(tiles) * s < cus && takes(2 * s)) s *= 2;
  return s;
}

template <int DT, int MT, int NT, int EPI, int LAY>
void launch_projection_mt(ProjArgs a, int splits) {
  const int waves = proj_waves(a.k / splits, MT * NT);
  a.kc = a.k / (splits * waves);
  const dim3 grid(unsigned(a.n / (16 * NT)), unsigned(splits), unsigned((a.m + 16 * MT - 1) / (16 * MT)));
  projection_kernel<DT, MT, EPI, -1, LAY, NT>
      <<<grid, 64 * waves, size_t(waves) * MT * NT * 64 * sizeof(floatx4)>>>(a);
}

template <int DT, int EPI, int LAY>
void launch_projection_lay(const ProjArgs& a, int splits) {
  const ProjTiles pt = proj_tiles(a.m, a.n);
  if (pt.nt == 2) {
    if (pt.mt == 2) launch_projection_mt<DT, 2, 2, EPI, LAY>(a, splits);
    else launch_projection_mt<DT, 4, 2, EPI, LAY>(a, splits);
  } else if (pt.mt == 1) {
    launch_projection_mt<DT, 1, 1, EPI, LAY>(a, splits);
  } else if (pt.mt == 2) {
    launch_projection_mt<DT, 2, 1, EPI, LAY>(a, splits);
  } else if (pt.mt == 4) {
    launch_projection_mt<DT, 4, 1, EPI, LAY>(a, splits);
  } else {
    launch_projection_mt<DT, 8, 1, EPI, LAY>(a, splits);
  }
}

template <int DT, int EPI>
void launch_projection_epi(const ProjArgs& a, int splits, int layout) {
  if constexpr (EPI == kProjPartials) {
    if (layout & kProjXTiled) launch_projection_lay<DT, EPI, kProjXTiled>(a, splits);
    else launch_projection_lay<DT, EPI, 0>(a, splits);
  } else {
    switch (layout) {
      case 0: launch_projection_lay<DT, EPI, 0>(a, splits); break;
      case kProjXTiled: launch_projection_lay<DT, EPI, kProjXTiled>(a, splits); break;
      case kProjOutTiled: launch_projection_lay<DT, EPI, kProjOutTiled>(a, splits); break;
      default: launch_projection_lay<DT, EPI, kProjXTiled | kProjOutTiled>(a, splits); break;
    }
  }
}

// Whether the LayerNorm-prologue projection takes out = epi(LayerNorm(x_in +
// part_bias + sum of splits partial rows) @ w^T): fp16/bf16, 1 <= m <= 16,
// one split, k a multiple of 256 up to kProjFusedMaxWidth, partial splits
// 0, 1, 2 or 4 (0: no partials and no part_bias), x_out distinct from x_in;
// layout 0 or kProjWTiled.
bool projection_ln_ok(const void* out, const float* x_in, const float* x_out, const float* part, int splits,
                      const void* part_bias, const float* gamma, const float* beta, const void* w,
                      const void* bias, int m, int n, int k, int epilogue, int dtype, int layout = 0) {
  if (dtype != kF16 && dtype != kBF16) return false;
  if (layout != 0 && layout != kProjWTiled) return false;
  if (m < 1 || m > 16 || n < 16 || n % 16 || k < 256 || k % 256 || k > kProjFusedMaxWidth) return false;
  if (epilogue != kProjBias && epilogue != kProjGelu) return false;
  if (splits != 0 && splits != 1 && splits != 2 && splits != 4) return false;
  if ((splits == 0) != (part == nullptr) || (splits == 0 && part_bias)) return false;
  if (proj_waves(k, 1) == 0 || int64_t(n) * k > INT32_MAX) return false;
  if (!out || !x_in || !x_out || x_in == x_out || !gamma || !beta || !w) return false;
  return aligned(out, 8) && aligned(x_in, 16) && aligned(x_out, 16) && (!part || aligned(part, 16)) &&
         (!part_bias || aligned(part_bias, 8)) && aligned(gamma, 16) && aligned(beta, 16) && aligned(w, 16) &&
         (!bias || aligned(bias, 8));
}

template <int DT, int EPI, int PS>
void launch_projection_ln_ps(const ProjArgs& a) {
  const int waves = proj_waves(a.k, 1);
  ProjArgs b = a;
  b.kc = a.k / waves;
  const size_t lds = size_t(waves) * 64 * sizeof(floatx4) + sizeof(float) * (size_t(a.m) * a.k + 2 * a.k) +
                     sizeof(typename Elem<DT>::T) * 16 * size_t(a.k + 8);
  projection_kernel<DT, 1, EPI, PS><<<dim3(unsigned(a.n / 16), 1, 1), 64 * waves, lds>>>(b);
}

template <int DT, int EPI>
void launch_projection_ln_epi(const ProjArgs& a, int splits) {
  if (splits == 0) launch_projection_ln_ps<DT, EPI, 0>(a);
  else if (splits == 1) launch_projection_ln_ps<DT, EPI, 1>(a);
  else if (splits == 2) launch_projection_ln_ps<DT, EPI, 2>(a);
  else launch_projection_ln_ps<DT, EPI, 4>(a);
}

// Caller has checked projection_ln_ok.
hipError_t projection_ln(void* out, const float* x_in, float* x_out, const float* part, int splits,
                         const void* part_bias, const float* gamma, const float* beta, float eps, const void* w,
                         const void* bias, int m, int n, int k, int epilogue, int dtype, int layout = 0) {
  ProjArgs a{};
  a.out = out; a.w = w; a.bias = bias;
  a.m = m; a.n = n; a.k = k;
  a.w_tiled = layout == kProjWTiled;
  a.x_in = x_in; a.x_out = x_out; a.part = part; a.part_bias = part_bias;
  a.gamma = gamma; a.beta = beta; a.eps = eps;
  if (dtype == kF16) {
    if (epilogue == kProjBias) launch_projection_ln_epi<kF16, kProjBias>(a, splits);
    else launch_projection_ln_epi<kF16, kProjGelu>(a, splits);
  } else {
    if (epilogue == kProjBias) launch_projection_ln_epi<kBF16, kProjBias>(a, splits);
    else launch_projection_ln_epi<kBF16, kProjGelu>(a, splits);
  }
  return hipGetLastError();
}

// Caller has checked projection_ok.
hipError_t projection(void* out, const void* x, const void* w, const void* bias, int m, int n, int k, int splits,
                      int epilogue, int dtype, int layout = 0) {
  ProjArgs a{};
  a.out = out; a.x = x; a.w = w; a.bias = bias;
  a.m = m; a.n = n; a.k = k;
  a.w_tiled = (layout & kProjWTiled) != 0;
  layout &= kProjXTiled | kProjOutTiled;
  if (dtype == kF16) {
    if (epilogue == kProjBias) launch_projection_epi<kF16, kProjBias>(a, splits, layout);
    else if (epilogue == kProjGelu) launch_projection_epi<kF16, kProjGelu>(a, splits, layout);
    else launch_projection_epi<kF16, kProjPartials>(a, splits, layout);
  } else {
    if (epilogue == kProjBias) launch_projection_epi<kBF16, kProjBias>(a, splits, layout);
    else if (epilogue == kProjGelu) launch_projection_epi<kBF16, kProjGelu>(a, splits, layout);
    else launch_projection_epi<kBF16, kProjPartials>(a, splits, layout);
  }
  return hipGetLastError();
}

// Whether residual_layernorm_partials takes the row shape (width a positive
// multiple of 256, at most 2048, 16-byte aligned rows).
bool partials_ln_ok(const void* out, const float* x, const float* part, const void* bias, const float* gamma,
                    const float* beta, int width, int dtype) {
  return (dtype == kF16 || dtype == kBF16) && width >= 256 && width % 256 == 0 && width <= 2048 && aligned(x, 16) &&
         aligned(part, 16) && aligned(gamma, 16) && aligned(beta, 16) && aligned(out, 8) && (!bias || aligned(bias, 8));
}

template <int DT, int S>
void launch_partials_ln(void* out, float* x, const float* part, const void* bias, const float* gamma,
                        const float* beta, int rows, int width, float eps, int tiled) {
  constexpr int R = kLnRowsPerBlock;  // rows (waves) per workgroup
  const int blocks = (rows + R - 1) / R;
  if (width <= 1024)
    residual_layernorm_partials_kernel<DT, 4, S>
        <<<blocks, 64 * R>>>(out, x, part, bias, gamma, beta, rows, width, eps, tiled);
  else
    residual_layernorm_partials_kernel<DT, 8, S>
        <<<blocks, 64 * R>>>(out, x, part, bias, gamma, beta, rows, width, eps, tiled);
}

template <int DT>
void launch_partials_ln_dt(void* out, float* x, const float* part, int splits, const void* bias, const float* gamma,
                           const float* beta, int rows, int width, float eps, int tiled) {
  switch (splits) {
    case 1: launch_partials_ln<DT, 1>(out, x, part, bias, gamma, beta, rows, width, eps, tiled); break;
    case 2: launch_partials_ln<DT, 2>(out, x, part, bias, gamma, beta, rows, width, eps, tiled); break;
    case 3: launch_partials_ln<DT, 3>(out, x, part, bias, gamma, beta, rows, width, eps, tiled); break;
    case 4: launch_partials_ln<DT, 4>(out, x, part, bias, gamma, beta, rows, width, eps, tiled); break;
    case 5: launch_partials_ln<DT, 5>(out, x, part, bias, gamma, beta, rows, width, eps, tiled); break;
    case 6: launch_partials_ln<DT, 6>(out, x, part, bias, gamma, beta, rows, width, eps, tiled); break;
    case 7: launch_partials_ln<DT, 7>(out, x, part, bias, gamma, beta, rows, width, eps, tiled); break;
    default: launch_partials_ln<DT, 8>(out, x, part, bias, gamma, beta, rows, width, eps, tiled); break;
  }
}

// Caller has checked partials_ln_ok and 1 <= splits <= kProjMaxSplits. tiled:
// out in the fragment-tiled layout (ceil(rows / 16) * 16 rows).
hipError_t residual_layernorm_partials(void* out, float* x, const float* part, int splits, const void* bias,
                                       const float* gamma, const float* beta, int rows, int width, float eps,
                                       int dtype, int tiled = 0) {
  if (dtype == kF16) launch_partials_ln_dt<kF16>(out, x, part, splits, bias, gamma, beta, rows, width, eps, tiled);
  else launch_partials_ln_dt<kBF16>(out, x, part, splits, bias, gamma, beta, rows, width, eps, tiled);
  return hipGetLastError();
}

// The weights a decode projection reads: a layer's fragment-tiled copy where
// it has one (kProjWTiled), else the row-major one.
struct ProjWeight {
  const void* w;
  int layout;
};
ProjWeight pick_weight(const void* row_major, const void* tiled) {
  return tiled ? ProjWeight{tiled, kProjWTiled} : ProjWeight{row_major, 0};
}
ProjWeight qkv_weight(const mt_decoder_layer& L) { return pick_weight(L.w_qkv, L.w_qkv_tiled); }
ProjWeight out_weight(const mt_decoder_layer& L) { return pick_weight(L.w_o, L.w_o_tiled); }
ProjWeight fc_weight(const mt_decoder_layer& L) { return pick_weight(L.w_fc, L.w_fc_tiled); }
ProjWeight proj_weight(const mt_decoder_layer& L) { return pick_weight(L.w_proj, L.w_proj_tiled); }

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

// [b, n, h*d] <-> [b, h, n, d] (split = 1: to heads, the [b, n, *] rows
// `stride` elements apart; 0: back, contiguous).
template <class T>
__global__ __launch_bounds__(256) void heads_kernel(T* out, const T* in, int b, int n, int h, int d, int split,
                                                    int64_t stride) {
  const int64_t total = int64_t(b) * n * h * d;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    // i indexes the [b, h, n, d] tensor
    const int col = int(i % d);
    const int64_t r = i / d;
    const int t = int(r % n);
    const int64_t r2 = r / n;
    const int hh = int(r2 % h);
    const int bb = int(r2 / h);
    if (split) out[i] = in[(int64_t(bb) * n + t) * stride + int64_t(hh) * d + col];
    else out[((int64_t(bb) * n + t) * h + hh) * d + col] = in[i];
  }
}

bool dtype_ok(int d) { return d >= 0 && d <= 2; }

// One wave per row when the row fits the wave kernel (width a multiple of 256,
// at most 2048, 16-byte aligned rows); y == nullptr means no residual.
bool wave_rows(const void* out, const float* x, const void* y, const float* gamma, const float* beta,
               int width, int dtype) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const bool y_ok = !y || (dtype == kF32 ? a16(y) : (reinterpret_cast<uintptr_t>(y) & 7u) == 0);
  return width % 256 == 0 && width <= 2048 && a16(x) && a16(gamma) && a16(beta) && y_ok &&
         (dtype == kF32 ? a16(out) : (reinterpret_cast<uintptr_t>(out) & 7u) == 0);
}

// Blocks of 256 columns a lane carries: exactly the width's for 768 and 1024
// (DistilGPT-2, GPT-2-medium), else 3 or 8 (repeated blocks past the width).
template <int DT, bool RES>
void launch_wave_rows_res(int blocks, int threads, void* out, float* x, const void* y, const float* gamma,
                          const float* beta, int rows, int width, float eps, int tiled) {
  const int nj = width >> 8;
  if (nj <= 3)
    residual_layernorm_wave_kernel<DT, 3, RES><<<blocks, threads>>>(out, x, y, gamma, beta, rows, width, eps, tiled);
  else if (nj == 4)
    residual_layernorm_wave_kernel<DT, 4, RES><<<blocks, threads>>>(out, x, y, gamma, beta, rows, width, eps, tiled);
  else
    residual_layernorm_wave_kernel<DT, 8, RES><<<blocks, threads>>>(out, x, y, gamma, beta, rows, width, eps, tiled);
}

template <int DT>
void launch_wave_rows(void* out, float* x, const void* y, const float* gamma, const float* beta,
                      int rows, int width, float eps, int tiled) {
  constexpr int R = kLnRowsPerBlock;  // one wave per row
  const int blocks = (rows + R - 1) / R;
  if (y) launch_wave_rows_res<DT, true>(blocks, 64 * R, out, x, y, gamma, beta, rows, width, eps, tiled);
  else launch_wave_rows_res<DT, false>(blocks, 64 * R, out, x, y, gamma, beta, rows, width, eps, tiled);
}

// tiled: out in the fragment-tiled layout (fp16/bf16, rows that the
// one-wave-per-row kernel takes; anything else is rejected).
hipError_t layernorm(void* out, const float* x, const float* gamma, const float* beta, int rows,
                     int width, float eps, int dtype, int tiled = 0) {
  const bool wave = wave_rows(out, x, nullptr, gamma, beta, width, dtype);
  if (tiled && (!wave || dtype == kF32)) return hipErrorInvalidValue;
  if (wave) {
    float* xm = const_cast<float*>(x);  // not written without a residual
    if (dtype == kF32) launch_wave_rows<kF32>(out, xm, nullptr, gamma, beta, rows, width, eps, 0);
    else if (dtype == kF16) launch_wave_rows<kF16>(out, xm, nullptr, gamma, beta, rows, width, eps, tiled);
    else launch_wave_rows<kBF16>(out, xm, nullptr, gamma, beta, rows, width, eps, tiled);
    return hipGetLastError();
  }
  if (dtype == kF32) layernorm_kernel<kF32><<<rows, 256>>>(out, x, gamma, beta, width, eps);
  else if (dtype == kF16) layernorm_kernel<kF16><<<rows, 256>>>(out, x, gamma, beta, width, eps);
  else layernorm_kernel<kBF16><<<rows, 256>>>(out, x, gamma, beta, width, eps);
  return hipGetLastError();
}

hipError_t residual_layernorm(void* out, float* x, const void* y, const float* gamma,
                              const float* beta, int rows, int width, float eps, int dtype, int tiled = 0) {
  const bool wave = wave_rows(out, x, y, gamma, beta, width, dtype);
  if (tiled && (!wave || dtype == kF32)) return hipErrorInvalidValue;
  if (wave) {
    if (dtype == kF32) launch_wave_rows<kF32>(out, x, y, gamma, beta, rows, width, eps, 0);
    else if (dtype == kF16) launch_wave_rows<kF16>(out, x, y, gamma, beta, rows, width, eps, tiled);
    else launch_wave_rows<kBF16>(out, x, y, gamma, beta, rows, width, eps, tiled);
    return hipGetLastError();
  }
  if (dtype == kF32)
    residual_layernorm_kernel<kF32><<<rows, 256>>>(out, x, y, gamma, beta, width, eps);
  else if (dtype == kF16)
    residual_layernorm_kernel<kF16><<<rows, 256>>>(out, x, y, gamma, beta, width, eps);
  else
    residual_layernorm_kernel<kBF16><<<rows, 256>>>(out, x, y, gamma, beta, width, eps);
  return hipGetLastError();
}

hipError_t gelu(void* x, int64_t n, int dtype) {
  if (dtype == kF32) gelu_kernel<kF32><<<blocks_for(n), 256>>>(x, n);
  else if (dtype == kF16) gelu_kernel<kF16><<<blocks_for(n), 256>>>(x, n);
  else gelu_kernel<kBF16><<<blocks_for(n), 256>>>(x, n);
  return hipGetLastError();
}

// GEMM + bias + tanh GELU: hipBLASLt's GELU epilogue when `fused`, else the
// bias GEMM followed by gelu_kernel.
int gemm_gelu(Blas* blas, void* out, const void* a, const void* b, const void* bias, int m, int n,
              int k, int dtype, bool fused, bool tunable = false, int transb = 0) {
  if (fused) return gemm(blas, out, a, b, bias, m, n, k, transb, dtype, dtype, kEpiGelu, tunable);
  int e = gemm(blas, out, a, b, bias, m, n, k, transb, dtype, dtype, kEpiNone, tunable);
  return e ? e : gelu(out, int64_t(m) * n, dtype);
}

// Row gather with the source rows in the launch arguments: out[i, :] =
// in[i, :] for the first `head` rows, then out[head + i, :] = in[row[i], :]
// for i < count (at most kGatherRows per launch), width in 16-bit or 32-bit
// elements moved as 32-bit words.
constexpr int kGatherRows = 64;
constexpr int kGatherMaxHead = 65535 - kGatherRows;  // the grid's y extent bounds head + count
struct GatherRows {
  int head, count;
  int row[kGatherRows];
};

__global__ __launch_bounds__(256) void gather_rows_kernel(uint32_t* out, const uint32_t* in, int64_t words,
                                                          GatherRows g) {
  const int i = blockIdx.y;
  if (i >= g.head + g.count) return;
  const uint32_t* src = in + int64_t(i < g.head ? i : g.row[i - g.head]) * words;
  uint32_t* dst = out + int64_t(i) * words;
  for (int64_t w = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; w < words; w += int64_t(gridDim.x) * blockDim.x)
    dst[w] = src[w];
}

// out[i, :] = in[i, :] for i < head, then out[head + i, :] = in[rows[i], :]
// for `count` rows, rows of `row_bytes` (a multiple of 4); out and in do not
// overlap.
hipError_t gather_rows(void* out, const void* in, const int* rows, int count, size_t row_bytes, int head = 0) {
  if (row_bytes % 4 || head < 0 || head > kGatherMaxHead) return hipErrorInvalidValue;
  const int64_t words = int64_t(row_bytes / 4);
  for (int c0 = 0; c0 < count || (c0 == 0 && head > 0); c0 += kGatherRows) {
    GatherRows g{};
    g.head = c0 == 0 ? head : 0;
    g.count = count - c0 < kGatherRows ? count - c0 : kGatherRows;
    for (int i = 0; i < g.count; ++i) g.row[i] = rows[c0 + i];
    const dim3 grid(unsigned((words + 255) / 256), unsigned(g.head + g.count));
    gather_rows_kernel<<<grid, 256>>>(static_cast<uint32_t*>(out) + (c0 ? int64_t(head + c0) * words : 0),
                                      static_cast<const uint32_t*>(in), words, g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// The prompts of a ragged prefill: every request's table row and offset, the
// row of its last token (after `first` rows that precede the prompts) and the
// total token count. False when a count is not positive, the total exceeds
// INT32_MAX or the requests do not describe one pool.
struct RaggedPrompts {
  std::vector<const int*> tables;
  std::vector<int> offsets, last;
  int64_t total = 0;
};
bool ragged_prompts(const mt_prefill_attention* att, const int* tokens, int requests, int first, RaggedPrompts& rp) {
  rp.tables.resize(requests);
  rp.offsets.resize(requests);
  rp.last.resize(requests);
  rp.total = 0;
  for (int r = 0; r < requests; ++r) {
    const mt_prefill_attention& A = att[r];
    if (tokens[r] < 1 || A.slabs != att[0].slabs || A.page_size != att[0].page_size ||
        A.pages_per_slab != att[0].pages_per_slab || A.num_slabs != att[0].num_slabs ||
        A.columns != att[0].columns || A.layers != att[0].layers)
      return false;
    rp.tables[r] = A.table;
    rp.offsets[r] = A.offset;
    rp.total += tokens[r];
    if (int64_t(first) + rp.total > INT32_MAX) return false;
    rp.last[r] = int(first + rp.total - 1);
  }
  return true;
}

}  // namespace

extern "C" {

// Replaces reference mt_blas_create / mt_blas_destroy (src/cuda_runtime.cu:22-23).
int mt_blas_create(void** handle) {
  if (!handle) return hipErrorInvalidValue;
  Blas* b = new Blas();
  const char* tune = std::getenv("MT_GEMM_TUNE");
  b->tune = !(tune && tune[0] == '0');
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
  if (b->flush) hipFree(b->flush);
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

// split = 1: out [b, h, n, d] <- in [b, n, *] (rows in_stride elements
// apart, 0 = h*d); split = 0: the inverse (contiguous).
int mt_heads(void* out, const void* in, int b, int n, int h, int d, int split, int in_stride, int dtype) {
  if (!out || !in || b < 1 || n < 1 || h < 1 || d < 1 || !dtype_ok(dtype) || in_stride < 0 ||
      (in_stride != 0 && int64_t(in_stride) < int64_t(h) * d) || (split == 0 && in_stride != 0))
    return hipErrorInvalidValue;
  const int64_t total = int64_t(b) * n * h * d;
  const int64_t stride = in_stride ? in_stride : int64_t(h) * d;
  if (dtype == kF32)
    heads_kernel<float><<<blocks_for(total), 256>>>(static_cast<float*>(out), static_cast<const float*>(in), b, n, h, d, split, stride);
  else
    heads_kernel<uint16_t><<<blocks_for(total), 256>>>(static_cast<uint16_t*>(out), static_cast<const uint16_t*>(in), b, n, h, d, split, stride);
  return hipGetLastError();
}

// out[m, n] = epilogue(a[m, k] @ b[k, n] + bias[n]); epilogue 0 = none,
// 1 = tanh GELU (hipBLASLt's fused GELU when fused_gelu, else a separate
// pass of the kernel behind mt_gelu).
int mt_gemm_epilogue(void* handle, void* out, const void* a, const void* b, const void* bias, int m,
                     int n, int k, int dtype, int epilogue, int fused_gelu) {
  if (!dtype_ok(dtype) || !handle || !out || !a || !b || m < 1 || n < 1 || k < 1 ||
      (epilogue != 0 && epilogue != 1))
    return hipErrorInvalidValue;
  Blas* blas = static_cast<Blas*>(handle);
  if (epilogue == 0) return gemm(blas, out, a, b, bias, m, n, k, 0, dtype, dtype);
  return gemm_gelu(blas, out, a, b, bias, m, n, k, dtype, fused_gelu != 0);
}

// x[r, :] += y[r, :]; out[r, :] = LayerNorm(x[r, :]) in dtype.
int mt_residual_layernorm(void* out, float* x, const void* y, const float* gamma, const float* beta,
                          int rows, int width, float eps, int dtype) {
  if (!out || !x || !y || !gamma || !beta || rows < 1 || width < 1 || !dtype_ok(dtype))
    return hipErrorInvalidValue;
  return residual_layernorm(out, x, y, gamma, beta, rows, width, eps, dtype);
}

int mt_decode_projection(void* out, const void* x, const void* w, const void* bias, int m, int n, int k,
                         int splits, int epilogue, int dtype, int layout) {
  if (!projection_ok(out, x, w, bias, m, n, k, splits, epilogue, dtype, layout)) return hipErrorInvalidValue;
  return projection(out, x, w, bias, m, n, k, splits, epilogue, dtype, layout);
}

int mt_decode_projection_ln(void* out, const float* x_in, float* x_out, const float* partials, int splits,
                            const void* part_bias, const float* gamma, const float* beta, float eps, const void* w,
                            const void* bias, int m, int n, int k, int epilogue, int dtype, int layout) {
  if (!projection_ln_ok(out, x_in, x_out, partials, splits, part_bias, gamma, beta, w, bias, m, n, k, epilogue,
                        dtype, layout))
    return hipErrorInvalidValue;
  return projection_ln(out, x_in, x_out, partials, splits, part_bias, gamma, beta, eps, w, bias, m, n, k, epilogue,
                       dtype, layout);
}

int mt_residual_layernorm_partials(void* out, float* x, const float* partials, int splits, const void* bias,
                                   const float* gamma, const float* beta, int rows, int width, float eps,
                                   int dtype, int layout) {
  if (!out || !x || !partials || !gamma || !beta || rows < 1 || splits < 1 || splits > kProjMaxSplits ||
      (layout != 0 && layout != kProjOutTiled) || int64_t(splits) * rows * width > INT32_MAX ||
      !partials_ln_ok(out, x, partials, bias, gamma, beta, width, dtype))
    return hipErrorInvalidValue;
  return residual_layernorm_partials(out, x, partials, splits, bias, gamma, beta, rows, width, eps, dtype,
                                     layout == kProjOutTiled);
}

size_t mt_decoder_scratch_bytes(int rows, int d, int dtype) {
  if (rows < 1 || d < 1 || !dtype_ok(dtype)) return 0;
  const size_t e = dtype == kF32 ? 4 : 2;
  const size_t mp = (size_t(rows) + 15) / 16 * 16;  // rows of a tiled buffer
  const bool low = dtype != kF32;
  // qkv [rows, 3d] | attention [rows, d] | projection [rows, d] | mlp [mp, 4d] (room for the tiled
  // layout), then for fp16/bf16 decode batches (rows <= kProjMaxRows): fp32 split partials
  // [kProjMaxSplits, rows, d], and either (rows <= kProjFusedRows) the second residual stream
  // [rows, d] fp32 or (more rows) the tiled LayerNorm output [mp, d]; each 256-aligned
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  const size_t partials = low && rows <= kProjMaxRows ? al(size_t(kProjMaxSplits) * rows * d * 4) : 0;
  const size_t stream = low && rows <= kProjFusedRows ? al(size_t(rows) * d * 4) : 0;
  const size_t ht = low && rows > kProjFusedRows && rows <= kProjMaxRows ? al(mp * d * e) : 0;
  return al(size_t(rows) * 3 * d * e) + 2 * al(size_t(rows) * d * e) + al(mp * 4 * d * e) + partials + stream + ht;
}

int mt_decoder_layers(void* handle, const mt_decoder_layer* layers, int n_layer, float* x, void* h,
                      const float* final_gamma, const float* final_beta, const void* head_weight,
                      void* logits, int vocab, int rows, int d, int heads, float eps, int dtype,
                      int fused_gelu, void* scratch, size_t scratch_bytes,
                      const mt_decode_attention* att) {
  if (!handle || !layers || n_layer < 1 || !x || !h || !final_gamma || !final_beta ||
      (logits && (!head_weight || vocab < 1)) || rows < 1 ||
      d < 1 || heads < 1 || d % heads || !dtype_ok(dtype) || !scratch || !att ||
      scratch_bytes < mt_decoder_scratch_bytes(rows, d, dtype) || int64_t(rows) * 4 * d > INT32_MAX)
    return hipErrorInvalidValue;
  Blas* blas = static_cast<Blas*>(handle);
  const size_t e = dtype == kF32 ? 4 : 2;
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  char* base = static_cast<char*>(scratch);
  char* qkv = base;
  char* attn = qkv + al(size_t(rows) * 3 * d * e);
  char* proj = attn + al(size_t(rows) * d * e);
  char* mlp = proj + al(size_t(rows) * d * e);
  const size_t mp = (size_t(rows) + 15) / 16 * 16;
  const bool low = dtype != kF32 && rows <= kProjMaxRows;
  char* tail = mlp + al(mp * 4 * d * e);
  float* partials = low ? reinterpret_cast<float*>(tail) : nullptr;
  if (low) tail += al(size_t(kProjMaxSplits) * rows * d * 4);
  float* xb = low && rows <= kProjFusedRows ? reinterpret_cast<float*>(tail) : nullptr;
  void* ht = low && rows > kProjFusedRows ? tail : nullptr;
  const int hd = d / heads;
  const bool own = decode_projections_enabled();
  auto attention = [&](int i) -> int {
    return mt_paged_decode_split(attn, qkv, qkv + size_t(d) * e, qkv + size_t(2 * d) * e, att->slabs, att->table,
                                 att->offsets, rows, heads, hd, att->page_size, att->pages_per_slab,
                                 att->num_slabs, att->columns, i, att->layers, dtype, att->split_tokens, 0, 0,
                                 3 * d, att->work, att->work_items, att->merge_rows, att->partials,
                                 att->partial_bytes);
  };
  // A few rows: the residual add and LayerNorm run inside the QKV and fc
  // projections (LayerNorm prologue), the residual stream alternating between
  // x and xb, and the out- and proj-projections leave split partial sums:
  // five kernels per layer and one LayerNorm (the final one) per step.
  if (own && xb) {
    auto fused_splits = [&](int k) {
      for (int sp = 4; sp >= 1; sp /= 2)
        if (projection_ok(partials, attn, layers[0].w_o, nullptr, rows, d, k, sp, kProjPartials, dtype)) return sp;
      return 0;
    };
    const int so = fused_splits(d), sp = fused_splits(4 * d);
    bool ok = so > 0 && sp > 0 && partials_ln_ok(h, x, partials, layers[n_layer - 1].b_proj, final_gamma, final_beta,
                                                 d, dtype);
    for (int i = 0; i < n_layer && ok; ++i) {
      const mt_decoder_layer& L = layers[i];
      const ProjWeight wq = qkv_weight(L), wo = out_weight(L), wf = fc_weight(L), wp = proj_weight(L);
      ok = projection_ln_ok(qkv, x, xb, i ? partials : nullptr, i ? sp : 0, i ? layers[i - 1].b_proj : nullptr,
                            L.ln1_gamma, L.ln1_beta, wq.w, L.b_qkv, rows, 3 * d, d, kProjBias, dtype, wq.layout) &&
           projection_ok(partials, attn, wo.w, nullptr, rows, d, d, so, kProjPartials, dtype, wo.layout) &&
           projection_ln_ok(mlp, xb, x, partials, so, L.b_o, L.ln2_gamma, L.ln2_beta, wf.w, L.b_fc, rows, 4 * d,
                            d, kProjGelu, dtype, wf.layout) &&
           projection_ok(partials, mlp, wp.w, nullptr, rows, d, 4 * d, sp, kProjPartials, dtype, wp.layout);
    }
    if (ok) {
      int st = 0;
      for (int i = 0; i < n_layer && !st; ++i) {
        const mt_decoder_layer& L = layers[i];
        const ProjWeight wq = qkv_weight(L), wo = out_weight(L), wf = fc_weight(L), wp = proj_weight(L);
        if ((st = projection_ln(qkv, x, xb, i ? partials : nullptr, i ? sp : 0, i ? layers[i - 1].b_proj : nullptr,
                                L.ln1_gamma, L.ln1_beta, eps, wq.w, L.b_qkv, rows, 3 * d, d, kProjBias, dtype,
                                wq.layout)))
          break;
        if ((st = attention(i))) break;
        if ((st = projection(partials, attn, wo.w, nullptr, rows, d, d, so, kProjPartials, dtype, wo.layout))) break;
        if ((st = projection_ln(mlp, xb, x, partials, so, L.b_o, L.ln2_gamma, L.ln2_beta, eps, wf.w, L.b_fc, rows,
                                4 * d, d, kProjGelu, dtype, wf.layout)))
          break;
        st = projection(partials, mlp, wp.w, nullptr, rows, d, 4 * d, sp, kProjPartials, dtype, wp.layout);
      }
      if (!st)
        st = residual_layernorm_partials(h, x, partials, sp, layers[n_layer - 1].b_proj, final_gamma, final_beta,
                                         rows, d, eps, dtype);
      if (!st && logits)
        st = gemm(blas, logits, h, head_weight, nullptr, rows, vocab, d, 1, dtype, dtype, kEpiNone, true);
      return st;
    }
  }
  // More rows, up to decode_tiled_rows(): the QKV, fc and proj projections run
  // on the projection kernel with fragment-tiled activations, which the
  // LayerNorm kernels (ht) and the fc epilogue (mlp) write in that layout, and
  // proj leaves split partial sums for the next residual LayerNorm. The
  // out-projection reads attention's row-major output: split partial sums
  // (split_o) or hipBLASLt.
  if (own && ht && rows <= decode_tiled_rows()) {
    const int so = projection_splits(rows, d, d), sp = projection_splits(rows, d, 4 * d);
    // the out-projection's partial sums cost the LayerNorm a read each: own
    // kernel while they are few (GPT-2-medium at 128 rows: 4 splits, 1.80
    // against 1.81 ms with hipBLASLt; DistilGPT-2: 8 splits, 0.448 against
    // 0.439 ms)
    const bool split_o = rows <= kProjSplitRows || so <= 4;
    bool ok = wave_rows(ht, x, nullptr, layers[0].ln1_gamma, layers[0].ln1_beta, d, dtype) &&
              partials_ln_ok(h, x, partials, layers[n_layer - 1].b_proj, final_gamma, final_beta, d, dtype);
    for (int i = 0; i < n_layer && ok; ++i) {
      const mt_decoder_layer& L = layers[i];
      const ProjWeight wq = qkv_weight(L), wo = out_weight(L), wf = fc_weight(L), wp = proj_weight(L);
      const bool last = i + 1 == n_layer;
      ok = projection_ok(qkv, ht, wq.w, L.b_qkv, rows, 3 * d, d, 1, kProjBias, dtype, kProjXTiled | wq.layout) &&
           (split_o ? projection_ok(partials, attn, wo.w, nullptr, rows, d, d, so, kProjPartials, dtype, wo.layout) &&
                          partials_ln_ok(ht, x, partials, L.b_o, L.ln2_gamma, L.ln2_beta, d, dtype)
                    : wave_rows(ht, x, proj, L.ln2_gamma, L.ln2_beta, d, dtype)) &&
           projection_ok(mlp, ht, wf.w, L.b_fc, rows, 4 * d, d, 1, kProjGelu, dtype,
                         kProjXTiled | kProjOutTiled | wf.layout) &&
           projection_ok(partials, mlp, wp.w, nullptr, rows, d, 4 * d, sp, kProjPartials, dtype,
                         kProjXTiled | wp.layout) &&
           (last || partials_ln_ok(ht, x, partials, L.b_proj, layers[i + 1].ln1_gamma, layers[i + 1].ln1_beta, d,
                                   dtype));
    }
    if (ok) {
      int st = layernorm(ht, x, layers[0].ln1_gamma, layers[0].ln1_beta, rows, d, eps, dtype, 1);
      for (int i = 0; i < n_layer && !st; ++i) {
        const mt_decoder_layer& L = layers[i];
        const ProjWeight wq = qkv_weight(L), wo = out_weight(L), wf = fc_weight(L), wp = proj_weight(L);
        if ((st = projection(qkv, ht, wq.w, L.b_qkv, rows, 3 * d, d, 1, kProjBias, dtype, kProjXTiled | wq.layout)))
          break;
        if ((st = attention(i))) break;
        if (split_o) {
          if ((st = projection(partials, attn, wo.w, nullptr, rows, d, d, so, kProjPartials, dtype, wo.layout)))
            break;
          st = residual_layernorm_partials(ht, x, partials, so, L.b_o, L.ln2_gamma, L.ln2_beta, rows, d, eps, dtype, 1);
        } else {
          if ((st = gemm(blas, proj, attn, L.w_o, L.b_o, rows, d, d, 1, dtype, dtype, kEpiNone, true))) break;
          st = residual_layernorm(ht, x, proj, L.ln2_gamma, L.ln2_beta, rows, d, eps, dtype, 1);
        }
        if (st) break;
        if ((st = projection(mlp, ht, wf.w, L.b_fc, rows, 4 * d, d, 1, kProjGelu, dtype,
                             kProjXTiled | kProjOutTiled | wf.layout)))
          break;
        if ((st = projection(partials, mlp, wp.w, nullptr, rows, d, 4 * d, sp, kProjPartials, dtype,
                             kProjXTiled | wp.layout)))
          break;
        const bool last = i + 1 == n_layer;
        st = residual_layernorm_partials(last ? h : ht, x, partials, sp, L.b_proj,
                                         last ? final_gamma : layers[i + 1].ln1_gamma,
                                         last ? final_beta : layers[i + 1].ln1_beta, rows, d, eps, dtype, last ? 0 : 1);
      }
      if (!st && logits)
        st = gemm(blas, logits, h, head_weight, nullptr, rows, vocab, d, 1, dtype, dtype, kEpiNone, true);
      return st;
    }
  }
  // out = epi(in @ wt^T + b): the decode projection kernel where it takes
  // the shape, else hipBLASLt.
  auto project = [&](void* out, const void* in, const void* wt, const void* b, int n, int k, int epi,
                     ProjWeight pw) -> int {
    if (own && rows <= kProjDirectRows && projection_ok(out, in, pw.w, b, rows, n, k, 1, epi, dtype, pw.layout))
      return projection(out, in, pw.w, b, rows, n, k, 1, epi, dtype, pw.layout);
    if (epi == kProjGelu) return gemm_gelu(blas, out, in, wt, b, rows, n, k, dtype, fused_gelu != 0, true, 1);
    return gemm(blas, out, in, wt, b, rows, n, k, 1, dtype, dtype, kEpiNone, true);
  };
  // x += in @ wt^T + b, then h = LayerNorm(x): split-k partial sums that the
  // LayerNorm kernel adds up, or one projection and residual_layernorm.
  auto project_residual = [&](const void* in, const void* wt, const void* b, int k, const float* g,
                              const float* be, ProjWeight pw) -> int {
    const int s = projection_splits(rows, d, k);
    if (own && partials && rows <= kProjSplitRows &&
        projection_ok(partials, in, pw.w, nullptr, rows, d, k, s, kProjPartials, dtype, pw.layout) &&
        partials_ln_ok(h, x, partials, b, g, be, d, dtype)) {
      const int st = projection(partials, in, pw.w, nullptr, rows, d, k, s, kProjPartials, dtype, pw.layout);
      return st ? st : residual_layernorm_partials(h, x, partials, s, b, g, be, rows, d, eps, dtype);
    }
    const int st = project(proj, in, wt, b, d, k, kProjBias, pw);
    return st ? st : residual_layernorm(h, x, proj, g, be, rows, d, eps, dtype);
  };
  int st = layernorm(h, x, layers[0].ln1_gamma, layers[0].ln1_beta, rows, d, eps, dtype);
  for (int i = 0; i < n_layer && !st; ++i) {
    const mt_decoder_layer& L = layers[i];
    if ((st = project(qkv, h, L.w_qkv, L.b_qkv, 3 * d, d, kProjBias, qkv_weight(L)))) break;
    if ((st = attention(i))) break;
    if ((st = project_residual(attn, L.w_o, L.b_o, d, L.ln2_gamma, L.ln2_beta, out_weight(L)))) break;
    if ((st = project(mlp, h, L.w_fc, L.b_fc, 4 * d, d, kProjGelu, fc_weight(L)))) break;
    const bool last = i + 1 == n_layer;
    st = project_residual(mlp, L.w_proj, L.b_proj, 4 * d, last ? final_gamma : layers[i + 1].ln1_gamma,
                          last ? final_beta : layers[i + 1].ln1_beta, proj_weight(L));
  }
  // Tied head: logits [rows, vocab] = h @ head_weight^T (head_weight [vocab, d]).
  if (!st && logits)
    st = gemm(blas, logits, h, head_weight, nullptr, rows, vocab, d, 1, dtype, dtype, kEpiNone, true);
  return st;
}

int mt_prefill_layers(void* handle, const mt_decoder_layer* layers, int n_layer, float* x, void* h,
                      const float* final_gamma, const float* final_beta, const void* head_weight,
                      void* logits, int vocab, int batch, int n, int d, int heads, float eps,
                      int dtype, int fused_gelu, void* scratch, size_t scratch_bytes,
                      const mt_prefill_attention* att) {
  const int64_t rows64 = int64_t(batch) * n;
  if (!handle || !layers || n_layer < 1 || !x || !h || !final_gamma || !final_beta ||
      (logits && (!head_weight || vocab < 1)) || batch < 1 || n < 1 || rows64 > INT32_MAX ||
      d < 1 || heads < 1 || d % heads || !dtype_ok(dtype) || !scratch || !att ||
      scratch_bytes < mt_decoder_scratch_bytes(int(rows64), d, dtype) || rows64 * 4 * d > INT32_MAX)
    return hipErrorInvalidValue;
  const int rows = int(rows64);
  Blas* blas = static_cast<Blas*>(handle);
  const size_t e = dtype == kF32 ? 4 : 2;
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  char* base = static_cast<char*>(scratch);
  char* qkv = base;
  char* attn = qkv + al(size_t(rows) * 3 * d * e);
  char* proj = attn + al(size_t(rows) * d * e);
  char* mlp = proj + al(size_t(rows) * d * e);
  const int hd = d / heads;
  int st = layernorm(h, x, layers[0].ln1_gamma, layers[0].ln1_beta, rows, d, eps, dtype);
  for (int i = 0; i < n_layer && !st; ++i) {
    const mt_decoder_layer& L = layers[i];
    if ((st = gemm(blas, qkv, h, L.w_qkv, L.b_qkv, rows, 3 * d, d, 1, dtype, dtype))) break;
    if ((st = mt_paged_prefill(attn, qkv, qkv + size_t(d) * e, qkv + size_t(2 * d) * e, att->slabs,
                               att->table, batch, heads, n, hd, att->page_size, att->pages_per_slab,
                               att->num_slabs, att->columns, i, att->layers, att->offset, dtype, 3 * d,
                               d)))
      break;
    if ((st = gemm(blas, proj, attn, L.w_o, L.b_o, rows, d, d, 1, dtype, dtype))) break;
    if ((st = residual_layernorm(h, x, proj, L.ln2_gamma, L.ln2_beta, rows, d, eps, dtype))) break;
    if ((st = gemm_gelu(blas, mlp, h, L.w_fc, L.b_fc, rows, 4 * d, d, dtype, fused_gelu != 0, false, 1))) break;
    if ((st = gemm(blas, proj, mlp, L.w_proj, L.b_proj, rows, d, 4 * d, 1, dtype, dtype))) break;
    const bool last = i + 1 == n_layer;
    st = residual_layernorm(h, x, proj, last ? final_gamma : layers[i + 1].ln1_gamma,
                            last ? final_beta : layers[i + 1].ln1_beta, rows, d, eps, dtype);
  }
  // Tied head over the last position of each request: rows n - 1, 2n - 1, ...
  // of h, read with a row stride of n * d.
  if (!st && logits)
    st = gemm(blas, logits, static_cast<char*>(h) + size_t(n - 1) * d * e, head_weight, nullptr, batch,
              vocab, d, 1, dtype, dtype, kEpiNone, false, n * d);
  return st;
}

int mt_prefill_layers_ragged(void* handle, const mt_decoder_layer* layers, int n_layer, float* x,
                             void* h, const float* final_gamma, const float* final_beta,
                             const void* head_weight, void* logits, int vocab, int requests,
                             const int* tokens, int d, int heads, float eps, int dtype, int fused_gelu,
                             void* scratch, size_t scratch_bytes, const mt_prefill_attention* att) {
  if (!handle || !layers || n_layer < 1 || !x || !h || !final_gamma || !final_beta ||
      (logits && (!head_weight || vocab < 1)) || requests < 1 || !tokens || d < 1 || heads < 1 ||
      d % heads || !dtype_ok(dtype) || !scratch || !att)
    return hipErrorInvalidValue;
  RaggedPrompts rp;
  if (!ragged_prompts(att, tokens, requests, 0, rp) || rp.total * 4 * d > INT32_MAX ||
      scratch_bytes < mt_decoder_scratch_bytes(int(rp.total), d, dtype))
    return hipErrorInvalidValue;
  const int rows = int(rp.total);
  Blas* blas = static_cast<Blas*>(handle);
  const size_t e = dtype == kF32 ? 4 : 2;
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  char* qkv = static_cast<char*>(scratch);
  char* attn = qkv + al(size_t(rows) * 3 * d * e);
  char* proj = attn + al(size_t(rows) * d * e);
  char* mlp = proj + al(size_t(rows) * d * e);
  const int hd = d / heads;
  int st = layernorm(h, x, layers[0].ln1_gamma, layers[0].ln1_beta, rows, d, eps, dtype);
  for (int i = 0; i < n_layer && !st; ++i) {
    const mt_decoder_layer& L = layers[i];
    if ((st = gemm(blas, qkv, h, L.w_qkv, L.b_qkv, rows, 3 * d, d, 1, dtype, dtype))) break;
    // Every request's append and causal attention over its own pages.
    if ((st = mt_paged_prefill_ragged(attn, qkv, qkv + size_t(d) * e, qkv + size_t(2 * d) * e, att[0].slabs,
                                      rp.tables.data(), tokens, rp.offsets.data(), requests, heads, hd,
                                      att[0].page_size, att[0].pages_per_slab, att[0].num_slabs,
                                      att[0].columns, i, att[0].layers, dtype, 3 * d, d)))
      break;
    if ((st = gemm(blas, proj, attn, L.w_o, L.b_o, rows, d, d, 1, dtype, dtype))) break;
    if ((st = residual_layernorm(h, x, proj, L.ln2_gamma, L.ln2_beta, rows, d, eps, dtype))) break;
    if ((st = gemm_gelu(blas, mlp, h, L.w_fc, L.b_fc, rows, 4 * d, d, dtype, fused_gelu != 0, false, 1))) break;
    if ((st = gemm(blas, proj, mlp, L.w_proj, L.b_proj, rows, d, 4 * d, 1, dtype, dtype))) break;
    const bool last = i + 1 == n_layer;
    st = residual_layernorm(h, x, proj, last ? final_gamma : layers[i + 1].ln1_gamma,
                            last ? final_beta : layers[i + 1].ln1_beta, rows, d, eps, dtype);
  }
  // Tied head over each request's last row, gathered into the (now free)
  // attention scratch.
  if (!st && logits) {
    st = gather_rows(attn, h, rp.last.data(), requests, size_t(d) * e);
    if (!st) st = gemm(blas, logits, attn, head_weight, nullptr, requests, vocab, d, 1, dtype, dtype);
  }
  return st;
}

int mt_mixed_layers(void* handle, const mt_decoder_layer* layers, int n_layer, float* x, void* h,
                    const float* final_gamma, const float* final_beta, const void* head_weight, void* logits,
                    int vocab, int decode_rows, int requests, const int* tokens, int d, int heads, float eps,
                    int dtype, int fused_gelu, void* scratch, size_t scratch_bytes,
                    const mt_decode_attention* datt, const mt_prefill_attention* patt) {
  if (!handle || !layers || n_layer < 1 || !x || !h || !final_gamma || !final_beta ||
      (logits && (!head_weight || vocab < 1)) || decode_rows < 1 || requests < 1 || !tokens || d < 1 ||
      heads < 1 || d % heads || !dtype_ok(dtype) || !scratch || !datt || !patt)
    return hipErrorInvalidValue;
  RaggedPrompts rp;
  if (decode_rows > kGatherMaxHead || !ragged_prompts(patt, tokens, requests, decode_rows, rp))
    return hipErrorInvalidValue;
  const int64_t rows64 = decode_rows + rp.total;
  // the decode rows and the prompts share one pool
  if (rows64 * 4 * d > INT32_MAX || scratch_bytes < mt_decoder_scratch_bytes(int(rows64), d, dtype) ||
      patt[0].slabs != datt->slabs || patt[0].page_size != datt->page_size ||
      patt[0].pages_per_slab != datt->pages_per_slab || patt[0].layers != datt->layers)
    return hipErrorInvalidValue;
  const int rows = int(rows64);
  Blas* blas = static_cast<Blas*>(handle);
  const size_t e = dtype == kF32 ? 4 : 2;
  auto al = [](size_t v) { return (v + 255) / 256 * 256; };
  char* qkv = static_cast<char*>(scratch);
  char* attn = qkv + al(size_t(rows) * 3 * d * e);
  char* proj = attn + al(size_t(rows) * d * e);
  char* mlp = proj + al(size_t(rows) * d * e);
  char* pqkv = qkv + size_t(decode_rows) * 3 * d * e;   // the prompts' QKV rows
  char* pattn = attn + size_t(decode_rows) * d * e;     // and attention rows
  const int hd = d / heads;
  int st = layernorm(h, x, layers[0].ln1_gamma, layers[0].ln1_beta, rows, d, eps, dtype);
  for (int i = 0; i < n_layer && !st; ++i) {
    const mt_decoder_layer& L = layers[i];
    if ((st = gemm(blas, qkv, h, L.w_qkv, L.b_qkv, rows, 3 * d, d, 1, dtype, dtype))) break;
    if ((st = mt_paged_decode_split(attn, qkv, qkv + size_t(d) * e, qkv + size_t(2 * d) * e, datt->slabs,
                                    datt->table, datt->offsets, decode_rows, heads, hd, datt->page_size,
                                    datt->pages_per_slab, datt->num_slabs, datt->columns, i, datt->layers, dtype,
                                    datt->split_tokens, 0, 0, 3 * d, datt->work, datt->work_items,
                                    datt->merge_rows, datt->partials, datt->partial_bytes)))
      break;
    if ((st = mt_paged_prefill_ragged(pattn, pqkv, pqkv + size_t(d) * e, pqkv + size_t(2 * d) * e, patt[0].slabs,
                                      rp.tables.data(), tokens, rp.offsets.data(), requests, heads, hd,
                                      patt[0].page_size, patt[0].pages_per_slab, patt[0].num_slabs,
                                      patt[0].columns, i, patt[0].layers, dtype, 3 * d, d)))
      break;
    if ((st = gemm(blas, proj, attn, L.w_o, L.b_o, rows, d, d, 1, dtype, dtype))) break;
    if ((st = residual_layernorm(h, x, proj, L.ln2_gamma, L.ln2_beta, rows, d, eps, dtype))) break;
    if ((st = gemm_gelu(blas, mlp, h, L.w_fc, L.b_fc, rows, 4 * d, d, dtype, fused_gelu != 0, false, 1))) break;
    if ((st = gemm(blas, proj, mlp, L.w_proj, L.b_proj, rows, d, 4 * d, 1, dtype, dtype))) break;
    const bool last = i + 1 == n_layer;
    st = residual_layernorm(h, x, proj, last ? final_gamma : layers[i + 1].ln1_gamma,
                            last ? final_beta : layers[i + 1].ln1_beta, rows, d, eps, dtype);
  }
  // Tied head over the decode rows and each prompt's last row, gathered in
  // that order into the (now free) attention scratch.
  if (!st && logits) st = gather_rows(attn, h, rp.last.data(), requests, size_t(d) * e, decode_rows);
  if (!st && logits)
    st = gemm(blas, logits, attn, head_weight, nullptr, decode_rows + requests, vocab, d, 1, dtype, dtype);
  return st;
}

}  // extern "C"
