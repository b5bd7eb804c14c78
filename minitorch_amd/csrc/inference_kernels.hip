// Token I/O kernels of the decode step for gfx950: embedding gather, greedy
// argmax and last-position copy. Semantics follow the reference
// src/inference_kernels.cu (cited per kernel); the launch shapes are this
// build's own.
#include "mt_device.h"
#include <climits>

using namespace mt;

namespace {

// dst[t, :] = weights[ids[t], :]; a row whose id is non-finite, negative,
// >= vocab or not an integer becomes NaN (reference src/inference_kernels.cu:7-14).
// One thread moves 4 floats when dim % 4 == 0 and the pointers are aligned.
template <bool VEC>
__global__ __launch_bounds__(256) void embedding_gather_kernel(float* dst, const float* weights,
                                                               const float* ids, int tokens,
                                                               int vocab, int dim) {
  constexpr int E = VEC ? 4 : 1;
  const int per_row = dim / E;
  const int64_t total = int64_t(tokens) * per_row;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t t = i / per_row;
    const int col = int(i - t * per_row) * E;
    const float raw = ids[t];
    const bool bad = !isfinite(raw) || raw < 0.f || raw >= float(vocab) || raw != floorf(raw);
    float* o = dst + t * dim + col;
    if constexpr (VEC) {
      float4 val = bad ? make_float4(NAN, NAN, NAN, NAN)
                       : *reinterpret_cast<const float4*>(weights + int64_t(raw) * dim + col);
      *reinterpret_cast<float4*>(o) = val;
    } else {
      *o = bad ? NAN : weights[int64_t(raw) * dim + col];
    }
  }
}

// x[t, :] = wte[id_t, :] + wpe[pos_t, :] in one pass: the token and position
// gathers of the reference (same invalid-id rule: a NaN row) and their sum.
// id_t is ids[t], or slot_tokens[slots[t]] when slot_tokens is given (the
// sync-free decode loop's token feedback; a slot outside the table gives a
// NaN row). One thread moves 4 floats (dim % 4 == 0, 16-byte aligned rows).
__device__ __forceinline__ bool bad_id(float raw, int limit) {
  return !isfinite(raw) || raw < 0.f || raw >= float(limit) || raw != floorf(raw);
}

__global__ __launch_bounds__(256) void embed_tokens_kernel(float* x, const float* wte, const float* wpe,
                                                           const float* ids, const float* slot_tokens,
                                                           const int* slots, int num_slots,
                                                           const float* positions, int tokens,
                                                           int vocab, int n_positions, int dim) {
  const int per_row = dim / 4;
  const int64_t total = int64_t(tokens) * per_row;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t t = i / per_row;
    const int col = int(i - t * per_row) * 4;
    float id;
    if (slot_tokens) {
      const int s = slots[t];
      id = (s >= 0 && s < num_slots) ? slot_tokens[s] : NAN;
    } else {
      id = ids[t];
    }
    const float pos = positions[t];
    float4 v = make_float4(NAN, NAN, NAN, NAN);
    if (!bad_id(id, vocab) && !bad_id(pos, n_positions)) {
      const float4 a = *reinterpret_cast<const float4*>(wte + int64_t(id) * dim + col);
      const float4 b = *reinterpret_cast<const float4*>(wpe + int64_t(pos) * dim + col);
      v = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
    }
    *reinterpret_cast<float4*>(x + t * dim + col) = v;
  }
}

// Argmax with numpy.argmax's rule, as in the reference
// (src/inference_kernels.cu:37-41,47-48): a NaN beats any number, a larger
// number beats a smaller one, and on equal keys (both NaN, or equal values,
// -0 == +0) the lower index wins.
//
// Each element is mapped to an integer key with the same order: the stored
// bits' magnitude, negated for negative values (so -0 and +0 both map to 0),
// and NaN above +inf. A thread visits its elements in increasing index order,
// so "strictly greater key" keeps the first maximum; the (key, index) pairs of
// the threads are then merged with the full rule.
template <int DT>
__device__ __forceinline__ int order_key(uint32_t bits) {
  if constexpr (DT == kF32) {
    const int mag = int(bits & 0x7fffffffu);
    return mag > 0x7f800000 ? INT_MAX : ((bits >> 31) ? -mag : mag);
  } else {
    constexpr int kInf = DT == kF16 ? 0x7c00 : 0x7f80;  // exponent all ones, zero mantissa
    const int mag = int(bits & 0x7fffu);
    return mag > kInf ? INT_MAX : ((bits & 0x8000u) ? -mag : mag);
  }
}

struct Cand {
  int k;  // order key
  int i;  // index, INT_MAX for no candidate
};

__device__ __forceinline__ bool better(const Cand& b, const Cand& a) {
  return b.k > a.k || (b.k == a.k && b.i < a.i);
}

constexpr int kArgmaxThreads = 1024;
// 16-byte vectors each thread loads before comparing any: 128 KiB of a row per
// round trip, so a 16-bit row of up to 64 Ki elements (GPT-2's 50257-wide
// logits) is read in one.
constexpr int kArgmaxBatch = 8;

// One workgroup of 16 waves per row. The aligned interior of the row is read
// with 16-byte loads; the unaligned head and tail element by element, issued
// with the first batch of vectors.
template <int DT>
__global__ __launch_bounds__(kArgmaxThreads) void row_argmax_kernel(float* dst, const void* src,
                                                                    int width, float* slot_tokens,
                                                                    const int* slots, int num_slots,
                                                                    int* slot_len, int tokens) {
  using T = typename Elem<DT>::T;
  constexpr int E = per16<DT>();
  constexpr int NW = kArgmaxThreads / 64;
  __shared__ int s_k[NW];
  __shared__ int s_i[NW];
  const int row = blockIdx.x;
  const T* p = static_cast<const T*>(src) + int64_t(row) * width;
  const int tid = threadIdx.x;
  int bk = INT_MIN, bi = INT_MAX;  // below every element's key
  auto consider = [&](uint32_t bits, int j) {
    const int k = order_key<DT>(bits);
    if (k > bk) { bk = k; bi = j; }
  };
  auto raw = [&](const T& x) -> uint32_t {
    if constexpr (DT == kF32) return __float_as_uint(x);
    else return uint32_t(x);
  };
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
  // A row not aligned to its element size takes the element-by-element
  // (tail) loop for all of it.
  const bool aligned = (addr & (sizeof(T) - 1)) == 0;
  int head = aligned ? int(((16 - (addr & 15)) & 15) / sizeof(T)) : 0;
  if (head > width) head = width;
  const int nvec = aligned ? (width - head) / E : 0;
  const int tail = head + nvec * E;
  const auto* vp = global_view(reinterpret_cast<const u32x4*>(p + head));
  // The head (< E elements) and the tail (< E elements, or the whole row on
  // the scalar path) ride with the first batch; a thread's elements are
  // compared in increasing index order (head, vectors, tail), so a strictly
  // greater key keeps its first maximum.
  uint32_t hb = 0;
  const bool has_head = tid < head;
  if (has_head) hb = raw(p[tid]);
  for (int j0 = tid; j0 < nvec; j0 += kArgmaxThreads * kArgmaxBatch) {
    u32x4 x[kArgmaxBatch];
#pragma unroll
    for (int u = 0; u < kArgmaxBatch; ++u) {
      const int j = j0 + u * kArgmaxThreads;
      if (j < nvec) x[u] = vp[j];
    }
    if (j0 == tid && has_head) consider(hb, tid);
#pragma unroll
    for (int u = 0; u < kArgmaxBatch; ++u) {
      const int j = j0 + u * kArgmaxThreads;
      if (j < nvec) {
        const uint32_t w[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
        const int base = head + j * E;
        if constexpr (DT == kF32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) consider(w[e], base + e);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            consider(w[e] & 0xffffu, base + 2 * e);
            consider(w[e] >> 16, base + 2 * e + 1);
          }
        }
      }
    }
  }
  if (tid >= nvec && has_head) consider(hb, tid);  // threads without vectors
  for (int j = tail + tid; j < width; j += kArgmaxThreads) consider(raw(p[j]), j);
  Cand c{bk, bi};
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const Cand o{__shfl_xor(c.k, off), __shfl_xor(c.i, off)};
    if (better(o, c)) c = o;
  }
  const int wave = tid >> 6;
  if ((tid & 63) == 0) { s_k[wave] = c.k; s_i[wave] = c.i; }
  __syncthreads();
  if (tid < 64) {
    Cand best{tid < NW ? s_k[tid] : INT_MIN, tid < NW ? s_i[tid] : INT_MAX};
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const Cand o{__shfl_xor(best.k, off), __shfl_xor(best.i, off)};
      if (better(o, best)) best = o;
    }
    if (tid == 0) {
      dst[row] = float(best.i);
      // Token feedback: the row's cache slot keeps the chosen token for the
      // next decode step (a slot outside the table is skipped).
      if (slot_tokens) {
        const int s = slots[row];
        if (s >= 0 && s < num_slots) {
          slot_tokens[s] = float(best.i);
          // the decode step's commit: the row's committed length grows
          if (slot_len) slot_len[s] += tokens;
        }
      }
    }
  }
}

typedef short s16x2 __attribute__((ext_vector_type(2)));

// 16-bit order keys of the two halves of w (fp16 or bf16 bits), packed: a
// half's bits as a signed 16-bit integer, with the magnitude bits flipped for
// a negative value. Larger numbers get larger keys, +0 gets 0 and -0 gets -1,
// a positive NaN lies above +inf and a negative NaN below -inf.
__device__ __forceinline__ s16x2 key16x2(uint32_t w) {
  const s16x2 v = __builtin_bit_cast(s16x2, w);
  const s16x2 s = v >> (s16x2){15, 15};  // all ones for a negative half
  return v ^ (s & (s16x2){0x7fff, 0x7fff});
}

__device__ __forceinline__ int key16(uint32_t h) {
  const int v = int(short(h));
  return v < 0 ? v ^ 0x7fff : v;
}

// Wave-wide max / min over lanes.
__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = max(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ int wave_min(int x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = min(x, __shfl_xor(x, off));
  return x;
}

// row_argmax_kernel for 16-bit rows read in one round trip (at most
// kArgmaxThreads * kArgmaxBatch vectors) with element-aligned addresses, in
// two passes over the registers instead of one (key, index) update per
// element:
// 1. each thread takes the packed max and min of its elements' 16-bit keys
//    (five VALU operations per two elements); its summary is INT_MAX if it
//    holds a NaN (max above +inf's key or min below -inf's), else its max
//    key. The workgroup's max summary T is the row's winning key.
// 2. the threads whose summary is T (or -1 when T is 0: -0 equals +0) scan
//    their elements in index order for the first one that matches T (any NaN
//    when T is INT_MAX); the lowest such index wins.
// This is the rule of row_argmax_kernel: the first NaN, else the first
// element of the largest value, -0 and +0 equal.
template <int DT>
__global__ __launch_bounds__(kArgmaxThreads) void row_argmax16_kernel(float* dst, const void* src,
                                                                      int width, float* slot_tokens,
                                                                      const int* slots, int num_slots,
                                                                      int* slot_len, int tokens) {
  static_assert(DT == kF16 || DT == kBF16, "16-bit rows only");
  constexpr int kInf = DT == kF16 ? 0x7c00 : 0x7f80;  // key of +inf; -inf's is -kInf - 1
  constexpr int NW = kArgmaxThreads / 64;
  __shared__ int s_red[2][NW];
  const int row = blockIdx.x;
  const uint16_t* p = static_cast<const uint16_t*>(src) + int64_t(row) * width;
  const int tid = threadIdx.x;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p);
  int head = int(((16 - (addr & 15)) & 15) / 2);
  if (head > width) head = width;
  const int nvec = (width - head) / 8;
  const int tail = head + nvec * 8;
  const auto* vp = global_view(reinterpret_cast<const u32x4*>(p + head));
  const bool has_head = tid < head;
  const int ntail = tail + tid < width ? 1 : 0;  // width - tail < 8 <= threads
  uint32_t hb = 0, tb = 0;
  if (has_head) hb = p[tid];
  if (ntail) tb = p[tail + tid];
  u32x4 x[kArgmaxBatch];
#pragma unroll
  for (int u = 0; u < kArgmaxBatch; ++u) {
    const int j = tid + u * kArgmaxThreads;
    if (j < nvec) x[u] = vp[j];
  }
  // pass 1: packed key extremes of each vector, and of the thread's elements
  s16x2 kmax = {SHRT_MIN, SHRT_MIN}, kmin = {SHRT_MAX, SHRT_MAX};
  if (has_head) { const s16x2 k = key16x2(hb * 0x10001u); kmax = k; kmin = k; }
  if (ntail) {
    const s16x2 k = key16x2(tb * 0x10001u);
    kmax = __builtin_elementwise_max(kmax, k);
    kmin = __builtin_elementwise_min(kmin, k);
  }
  s16x2 vmax[kArgmaxBatch], vmin[kArgmaxBatch];
#pragma unroll
  for (int u = 0; u < kArgmaxBatch; ++u) {
    if (tid + u * kArgmaxThreads < nvec) {
      const s16x2 k0 = key16x2(x[u].x), k1 = key16x2(x[u].y), k2 = key16x2(x[u].z), k3 = key16x2(x[u].w);
      vmax[u] = __builtin_elementwise_max(__builtin_elementwise_max(k0, k1), __builtin_elementwise_max(k2, k3));
      vmin[u] = __builtin_elementwise_min(__builtin_elementwise_min(k0, k1), __builtin_elementwise_min(k2, k3));
      kmax = __builtin_elementwise_max(kmax, vmax[u]);
      kmin = __builtin_elementwise_min(kmin, vmin[u]);
    }
  }
  auto nan_in = [&](s16x2 hi, s16x2 lo) {
    return max(int(hi.x), int(hi.y)) > kInf || min(int(lo.x), int(lo.y)) < -kInf - 1;
  };
  const int summary = nan_in(kmax, kmin) ? INT_MAX : max(int(kmax.x), int(kmax.y));
  const int wave = tid >> 6;
  int r = wave_max(summary);
  if ((tid & 63) == 0) s_red[0][wave] = r;
  __syncthreads();
  int target = s_red[0][0];
#pragma unroll
  for (int w = 1; w < NW; ++w) target = max(target, s_red[0][w]);
  // pass 2: the first matching element of the candidate threads
  int first = INT_MAX;
  if (summary == target || (target == 0 && summary == -1)) {
    auto match = [&](uint32_t h) {
      if (target == INT_MAX) return int(h & 0x7fffu) > kInf;
      const int k = key16(h);
      return k == target || (target == 0 && k == -1);
    };
    // a vector holds a match iff its extremes do: its max key is the target
    // (or -1 when the target is 0), or it holds a NaN
    auto holds = [&](int u) {
      if (target == INT_MAX) return nan_in(vmax[u], vmin[u]);
      const int m = max(int(vmax[u].x), int(vmax[u].y));
      return m == target || (target == 0 && m == -1);
    };
    if (has_head && match(hb)) {
      first = tid;
    } else {
      int hit = -1;
#pragma unroll
      for (int u = 0; u < kArgmaxBatch; ++u)
        if (hit < 0 && tid + u * kArgmaxThreads < nvec && holds(u)) hit = u;
      if (hit >= 0) {
#pragma unroll
        for (int u = 0; u < kArgmaxBatch; ++u) {
          if (u == hit) {
            const uint32_t w[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
            int e_first = 8;
#pragma unroll
            for (int e = 7; e >= 0; --e)
              if (match((w[e >> 1] >> (16 * (e & 1))) & 0xffffu)) e_first = e;
            first = head + (tid + u * kArgmaxThreads) * 8 + e_first;
          }
        }
      } else if (ntail && match(tb)) {
        first = tail + tid;
      }
    }
  }
  r = wave_min(first);
  if ((tid & 63) == 0) s_red[1][wave] = r;
  __syncthreads();
  if (tid == 0) {
    int best = s_red[1][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) best = min(best, s_red[1][w]);
    dst[row] = float(best);
    if (slot_tokens) {
      const int s = slots[row];
      if (s >= 0 && s < num_slots) {
        slot_tokens[s] = float(best);
        if (slot_len) slot_len[s] += tokens;
      }
    }
  }
}

// ids[r] = slot_tokens[slots[r]]; a slot outside the table gives a NaN id,
// which the embedding gather turns into a NaN row.
__global__ __launch_bounds__(256) void gather_slot_tokens_kernel(float* ids, const float* slot_tokens,
                                                                 const int* slots, int rows,
                                                                 int num_slots) {
  const int r = blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const int s = slots[r];
  ids[r] = (s >= 0 && s < num_slots) ? slot_tokens[s] : NAN;
}

// dst[b, :] = src[b, n-1, :] (reference src/inference_kernels.cu:28-30).
template <class T>
__global__ __launch_bounds__(256) void last_row_kernel(T* dst, const T* src, int batch, int n,
                                                       int width) {
  const int64_t total = int64_t(batch) * width;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t b = i / width;
    dst[i] = src[(b * n + n - 1) * width + (i - b * width)];
  }
}

int blocks_for(int64_t threads) {
  const int64_t b = (threads + 255) / 256;
  return int(b < (1 << 20) ? b : (1 << 20));
}

}  // namespace

extern "C" {

int mt_embedding_gather(float* dst, const float* weights, const float* ids, int tokens, int vocab,
                        int dim) {
  if (tokens < 1 || vocab < 1 || dim < 1 || int64_t(tokens) * dim > INT32_MAX ||
      int64_t(vocab) * dim > INT32_MAX)
    return hipErrorInvalidValue;
  if (!dst || !weights || !ids) return hipErrorInvalidValue;
  const bool vec = dim % 4 == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(weights) & 15) == 0;
  const int64_t threads = int64_t(tokens) * (vec ? dim / 4 : dim);
  if (vec)
    embedding_gather_kernel<true><<<blocks_for(threads), 256>>>(dst, weights, ids, tokens, vocab, dim);
  else
    embedding_gather_kernel<false><<<blocks_for(threads), 256>>>(dst, weights, ids, tokens, vocab, dim);
  return hipGetLastError();
}

int mt_row_argmax_commit(float* dst, float* slot_tokens, const int* slots, int num_slots, int* slot_len,
                         int tokens, const void* src, int rows, int width, int dtype) {
  if (rows < 1 || width < 1 || width > 16777216 || int64_t(rows) * width > INT32_MAX)
    return hipErrorInvalidValue;
  if (!dst || !src || (slot_tokens && (!slots || num_slots < 1)) || (slot_len && !slot_tokens))
    return hipErrorInvalidValue;
  // 16-bit rows of element-aligned address that one round trip reads (the
  // head and tail are under 8 elements each) take the two-pass kernel
  const bool two_pass = (reinterpret_cast<uintptr_t>(src) & 1) == 0 &&
                        width <= kArgmaxThreads * kArgmaxBatch * 8;
#define MT_ARGMAX(K, DT) \
  K<DT><<<rows, kArgmaxThreads>>>(dst, src, width, slot_tokens, slots, num_slots, slot_len, tokens)
  if (dtype == kF32) MT_ARGMAX(row_argmax_kernel, kF32);
  else if (dtype == kF16 && two_pass) MT_ARGMAX(row_argmax16_kernel, kF16);
  else if (dtype == kBF16 && two_pass) MT_ARGMAX(row_argmax16_kernel, kBF16);
  else if (dtype == kF16) MT_ARGMAX(row_argmax_kernel, kF16);
  else if (dtype == kBF16) MT_ARGMAX(row_argmax_kernel, kBF16);
  else return hipErrorInvalidValue;
#undef MT_ARGMAX
  return hipGetLastError();
}

int mt_row_argmax_feedback(float* dst, float* slot_tokens, const int* slots, int num_slots,
                           const void* src, int rows, int width, int dtype) {
  return mt_row_argmax_commit(dst, slot_tokens, slots, num_slots, nullptr, 0, src, rows, width, dtype);
}

int mt_row_argmax(float* dst, const void* src, int rows, int width, int dtype) {
  return mt_row_argmax_commit(dst, nullptr, nullptr, 0, nullptr, 0, src, rows, width, dtype);
}

int mt_embed_tokens(float* x, const float* wte, const float* wpe, const float* ids,
                    const float* slot_tokens, const int* slots, int num_slots, const float* positions,
                    int tokens, int vocab, int n_positions, int dim) {
  auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (!x || !wte || !wpe || !positions || (slot_tokens ? (!slots || num_slots < 1) : !ids) ||
      tokens < 1 || vocab < 1 || n_positions < 1 || dim < 4 || dim % 4 || !a16(x) || !a16(wte) ||
      !a16(wpe) || int64_t(tokens) * dim > INT32_MAX || int64_t(vocab) * dim > INT32_MAX ||
      int64_t(n_positions) * dim > INT32_MAX)
    return hipErrorInvalidValue;
  const int64_t threads = int64_t(tokens) * (dim / 4);
  embed_tokens_kernel<<<blocks_for(threads), 256>>>(x, wte, wpe, ids, slot_tokens, slots, num_slots,
                                                    positions, tokens, vocab, n_positions, dim);
  return hipGetLastError();
}

int mt_gather_slot_tokens(float* ids, const float* slot_tokens, const int* slots, int num_slots,
                          int rows) {
  if (!ids || !slot_tokens || !slots || rows < 1 || num_slots < 1) return hipErrorInvalidValue;
  gather_slot_tokens_kernel<<<(rows + 255) / 256, 256>>>(ids, slot_tokens, slots, rows, num_slots);
  return hipGetLastError();
}

int mt_last_row(void* dst, const void* src, int b, int n, int w, int dtype) {
  if (b < 1 || n < 1 || w < 1 || int64_t(b) * n * w > INT32_MAX) return hipErrorInvalidValue;
  if (!dst || !src) return hipErrorInvalidValue;
  const int blocks = blocks_for(int64_t(b) * w);
  if (dtype == kF32)
    last_row_kernel<float><<<blocks, 256>>>(static_cast<float*>(dst), static_cast<const float*>(src), b, n, w);
  else if (dtype == kF16 || dtype == kBF16)
    last_row_kernel<uint16_t><<<blocks, 256>>>(static_cast<uint16_t*>(dst), static_cast<const uint16_t*>(src), b, n, w);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // extern "C"
