// Paged KV append, paged decode attention and causal paged (prefill)
// attention for gfx950 (CDNA4, wave64).
//
// Slab layout (reference src/paged_attention_kernel.cu:2,18-19 and
// minitorch/paged_kv_cache.py:30): every slab is
//   [layers][2 (K,V)][pages_per_slab][heads][page_size][head_dim]
// and physical page p lives in slab p / pages_per_slab at slot
// p % pages_per_slab; slab base addresses come from a uint64 device table.
//
// Decode attention is a GEMV over paged K/V (about one flop per byte), so it
// is bound by HBM bandwidth and uses no MFMA. The design:
//   * one workgroup (4 or 8 waves) owns one (request, head, context split);
//   * a wave covers 8 tokens per step: eight lanes per token, each lane owning
//     head_dim/8 contiguous dims, so for fp16/bf16 at D = 64 every 16-byte-per-
//     lane load instruction reads 1 KiB of one page-head block contiguously
//     (8 whole token rows), non-temporally: each K/V byte is read once;
//   * every 8-lane token group keeps its own online-softmax state (running max,
//     denominator, fp32 accumulator), so the stream needs no cross-lane
//     reduction except the 8-lane dot-product sum; groups, waves and splits are
//     merged once at the end with the log-sum-exp rule;
//   * the slab table of a small pool is staged in LDS and each lane resolves
//     the page of one of its wave's row-blocks before streaming (broadcast with
//     readlane), so the dependent table -> slab -> K/V chain is paid once;
//   * the KV append of the new token is fused: the workgroup that owns the
//     last split scores the new token from the K/V inputs and writes it into
//     its page, so append + attention is a single launch;
//   * a row longer than one split writes (max, denominator, accumulator)
//     partials to a workspace and a small reduction kernel merges them. (A
//     last-arriving-workgroup merge inside the decode kernel needs device-scope
//     release/acquire fences, which write back and invalidate the XCD's L2 per
//     workgroup; measured on MI355X that made the decode 10x slower than a
//     separate launch.)
//
// Causal attention of several queries per request (a prefill) runs on the
// matrix cores for fp16/bf16 (prefill_kernel: 64-query tiles, S^T = K Q^T and
// O^T += V^T P^T with v_mfma_f32_16x16x32); fp32 and the shapes it does not
// take use the per-query query_kernel.
#include "mt_device.h"
#include "../../include/mt_paged.h"
#include <algorithm>
#include <atomic>
#include <climits>

// The decode kernel streams every K/V byte of a launch exactly once, so its
// loads are non-temporal (streamed past the caches). Measured on MI355X
// (config 2, cold pools): 24.5 -> 21.2 us together with 8 lanes per token.
#ifndef MT_DECODE_NT_LOADS
#define MT_DECODE_NT_LOADS 1
#endif
#include <cmath>
#include <mutex>
#include <vector>

using namespace mt;

namespace {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kThreads = kWave * kWaves;
constexpr int kGroup = 4;                    // lanes per token
constexpr int kRowBlock = kWave / kGroup;    // tokens per wave step
constexpr int kMaxSplitTokens = 2048;
constexpr int kMaxSplitPages = kMaxSplitTokens / 8;
constexpr int kDefaultSplitTokens = 1024;
constexpr int kMaxSplitsPerRow = 8;
constexpr float kLog2e = 1.4426950408889634f;
#ifndef MT_STAGES
#define MT_STAGES 1
#endif
constexpr int kStages = MT_STAGES;  // register stages of the K/V stream
// Lanes per token in the decode kernel: 8 lanes of 8 dims (fp16/bf16, D 64)
// make each 16-byte-per-lane load instruction one contiguous 1 KiB of a page
// (8 whole token rows); with 4 lanes of 16 dims an instruction touches every
// row of the 2 KiB page-row block half each.
#ifndef MT_DECODE_GROUP
#define MT_DECODE_GROUP 8
#endif
constexpr int kDecodeGroup = MT_DECODE_GROUP;
constexpr bool kDecodeNT = MT_DECODE_NT_LOADS != 0;
// Pools of at most this many slabs have their slab table staged in LDS by the
// decode kernel, so that page resolution after the block-table read is an LDS
// read instead of a second dependent global load.
constexpr int kLdsSlabs = 512;

#ifdef MT_DECODE_TIMELINE
// Measurement builds only (bench.py --timeline): wall-clock stamps of each
// decode workgroup's first item, taken by thread 0 at 100 MHz
// (s_memrealtime), workgroups below kTimelineMax. Record: [start, work entry
// returned, table/query/offset returned, past the staging barrier, K/V
// stream start, end, HW_ID register, XCC_ID register]. A stamp that follows
// a load takes that load's value as an operand, so it waits for the data.
// The product build has none of this.
constexpr int kTimelineMax = 8192;
constexpr int kTimelineFields = 8;
__device__ uint64_t g_decode_timeline[kTimelineMax * kTimelineFields];
template <class T>
__device__ __forceinline__ uint64_t stamp_after(T dep) {
  uint64_t t;
  asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t) : "v"(dep) : "memory");
  return t;
}
#endif

struct Geometry {
  int heads, dim, page_size, log2_page, pps, num_slabs, columns, layer;
  int64_t kind_stride;  // elements between the K and V planes of one layer
  // p / pps for 0 <= p < 2^31 as (p * pps_magic) >> pps_shift, so that page
  // resolution needs no division: pps_magic = ceil(2^(31+s) / pps) with
  // s = ceil(log2 pps), pps_shift = 31 + s (the error n * e / 2^(31+s),
  // e < 1, stays below 1 / pps for n < 2^31 since pps <= 2^s).
  uint64_t pps_magic;
  int pps_shift;
};

__device__ __forceinline__ int slab_index(int physical, const Geometry& g) {
  return int((uint64_t(uint32_t(physical)) * g.pps_magic) >> g.pps_shift);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Address of (slot, head, row 0, col 0) in the K plane of `layer`, or nullptr
// for the cases the reference treats as a missing page
// (src/paged_attention_kernel.cu:11-16): logical column out of range, negative
// or out-of-pool physical page, or a null slab.
template <class T>
__device__ __forceinline__ const T* page_base(const uint64_t* slabs, const int* table_row,
                                              int64_t logical, const Geometry& g, int head) {
  if (logical < 0 || logical >= g.columns) return nullptr;
  const int physical = table_row[logical];
  if (physical < 0 || int64_t(physical) >= int64_t(g.num_slabs) * g.pps) return nullptr;
  const int slab = slab_index(physical, g);
  const uint64_t address = slabs[slab];
  if (!address) return nullptr;
  const int slot = physical - slab * g.pps;
  const int64_t i = ((int64_t(g.layer) * 2 * g.pps + slot) * g.heads + head) *
                    int64_t(g.page_size) * g.dim;
  return reinterpret_cast<const T*>(address) + i;
}

// Page base from an already loaded physical page ID (the table read is
// issued separately so that it overlaps other loads).
template <class T>
__device__ __forceinline__ const T* resolve_page(const uint64_t* slabs, int physical,
                                                 const Geometry& g, int head) {
  if (physical < 0 || int64_t(physical) >= int64_t(g.num_slabs) * g.pps) return nullptr;
  const int slab = slab_index(physical, g);
  const uint64_t address = slabs[slab];
  if (!address) return nullptr;
  const int slot = physical - slab * g.pps;
  const int64_t i = ((int64_t(g.layer) * 2 * g.pps + slot) * g.heads + head) *
                    int64_t(g.page_size) * g.dim;
  return reinterpret_cast<const T*>(address) + i;
}

// Page base from a physical page ID and its slab's base address (already
// looked up); nullptr for a null slab.
template <class T>
__device__ __forceinline__ const T* page_in_slab(uint64_t address, int physical, const Geometry& g,
                                                 int head) {
  if (!address) return nullptr;
  const int slot = physical - slab_index(physical, g) * g.pps;
  const int64_t i = ((int64_t(g.layer) * 2 * g.pps + slot) * g.heads + head) *
                    int64_t(g.page_size) * g.dim;
  return reinterpret_cast<const T*>(address) + i;
}

__device__ __forceinline__ bool physical_in_pool(int physical, const Geometry& g) {
  return physical >= 0 && int64_t(physical) < int64_t(g.num_slabs) * g.pps;
}

// Online-softmax state of one token group, in base-2 units (scores are
// pre-multiplied by log2(e)). A missing page contributes a NaN score, which
// fmaxf drops from the running max and which then poisons the denominator,
// matching the reference's NaN propagation (src/paged_attention_kernel.cu:53,66-69,84).
template <int N, int G = kGroup>
struct Softmax {
  float m, l, acc[N];
  __device__ __forceinline__ void init() {
    m = -INFINITY; l = 0.f;
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] = 0.f;
  }
  __device__ __forceinline__ void add(float s, const float* v) {
    const float mn = fmaxf(m, s);
    const float alpha = (m == -INFINITY) ? 0.f : fast_exp2(m - mn);
    const float p = fast_exp2(s - mn);
    l = fmaf(l, alpha, p);
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] = fmaf(p, v[i], acc[i] * alpha);
    m = mn;
  }
  // Add U tokens with one rescale: the running max moves once per call.
  template <int U, class VF>
  __device__ __forceinline__ void add_many(const float* s, const bool* valid, VF&& v_of) {
    float mx = m;
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (valid[u]) mx = fmaxf(mx, s[u]);
    const float alpha = (m == -INFINITY) ? 0.f : fast_exp2(m - mx);
    l *= alpha;
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (valid[u]) {
        const float p = fast_exp2(s[u] - mx);
        l += p;
        float v[N];
        v_of(u, v);
#pragma unroll
        for (int i = 0; i < N; ++i) acc[i] = fmaf(p, v[i], acc[i]);
      }
    }
    m = mx;
  }
  __device__ __forceinline__ void merge(float mo, float lo, const float* ao) {
    const float mn = fmaxf(m, mo);
    const float sa = (m == -INFINITY) ? 0.f : fast_exp2(m - mn);
    const float sb = (mo == -INFINITY) ? 0.f : fast_exp2(mo - mn);
    l = l * sa + lo * sb;
#pragma unroll
    for (int i = 0; i < N; ++i) acc[i] = acc[i] * sa + ao[i] * sb;
    m = mn;
  }
  // Merge with the state held `rot` lanes further along the same 16-lane row
  // (DPP row rotate; no LDS traffic).
  template <int CTRL>
  __device__ __forceinline__ void merge_dpp() {
    float ao[N];
    const float mo = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), CTRL, 0xF, 0xF, false));
    const float lo = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(l), CTRL, 0xF, 0xF, false));
#pragma unroll
    for (int i = 0; i < N; ++i)
      ao[i] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[i]), CTRL, 0xF, 0xF, false));
    merge(mo, lo, ao);
  }
  // Merge the token groups of each 16-lane row: afterwards lanes with
  // lane % 16 < G hold their row's state for chunk lane % G.
  __device__ __forceinline__ void row_merge() {
    static_assert(G == 4 || G == 8, "row_merge expects 4 or 8 lanes per token");
    if constexpr (G == 4) merge_dpp<0x124>();  // row_ror:4
    merge_dpp<0x128>();                        // row_ror:8
  }
  // Merge the states of the token groups of a wave (lanes with equal
  // lane % G): afterwards lanes 0..G-1 hold the wave's state for their chunk.
  __device__ __forceinline__ void wave_merge() {
#pragma unroll
    for (int off = G; off < kWave; off <<= 1) {
      float ao[N];
      const float mo = __shfl_xor(m, off);
      const float lo = __shfl_xor(l, off);
#pragma unroll
      for (int i = 0; i < N; ++i) ao[i] = __shfl_xor(acc[i], off);
      merge(mo, lo, ao);
    }
  }
};

__device__ __forceinline__ float finalize(float acc, float l) {
  return l > 0.f ? acc / l : (isnan(l) ? NAN : 0.f);
}

// Sum of a value over the G lanes of a token group with DPP: quad permutes
// for 4 lanes, then the half-row mirror (lane i <-> 7 - i) for 8 lanes.
template <int G = kGroup>
__device__ __forceinline__ float group_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true));
  x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true));
  if constexpr (G == 8)
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, true));
  return x;
}

// Per-lane chunk of one token row: DL values at `p` (K or V plane), converted
// to fp32. VEC uses 16-byte loads; otherwise element loads masked to `dim`.
template <int DT, int DL, bool VEC>
struct Chunk {
  using T = typename Elem<DT>::T;
  static constexpr int NV = VEC ? DL * elem_bytes<DT>() / 16 : 1;
  u32x4 raw[VEC ? NV : 1];
  float val[VEC ? 1 : DL];
  // NTL: non-temporal loads (data read once, not kept in the caches).
  template <bool NTL = false>
  __device__ __forceinline__ void load(const T* p, int col0, int dim) {
    if constexpr (VEC) {
      const auto* v = global_view(reinterpret_cast<const u32x4*>(p));
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        if constexpr (NTL) raw[i] = __builtin_nontemporal_load(v + i);
        else raw[i] = v[i];
      }
    } else {
      const auto* g = global_view(p);
#pragma unroll
      for (int i = 0; i < DL; ++i) val[i] = (col0 + i < dim) ? to_f32<DT>(g[i]) : 0.f;
    }
  }
  // Same chunk from an LDS copy of the row (p points at column col0).
  __device__ __forceinline__ void load_lds(const T* p, int col0, int dim) {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < NV; ++i) raw[i] = reinterpret_cast<const u32x4*>(p)[i];
    } else {
#pragma unroll
      for (int i = 0; i < DL; ++i) val[i] = (col0 + i < dim) ? to_f32<DT>(p[i]) : 0.f;
    }
  }
  __device__ __forceinline__ void nan_fill() {
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < NV; ++i) raw[i] = u32x4{~0u, ~0u, ~0u, ~0u};
    } else {
#pragma unroll
      for (int i = 0; i < DL; ++i) val[i] = NAN;
    }
  }
  __device__ __forceinline__ void to_float(float* o) const {
    if constexpr (VEC) {
      constexpr int E = per16<DT>();
#pragma unroll
      for (int i = 0; i < NV; ++i) unpack16<DT>(raw[i], o + i * E);
    } else {
#pragma unroll
      for (int i = 0; i < DL; ++i) o[i] = val[i];
    }
  }
};

// One query vector split over the 4 lanes of a token group. For fp16/bf16
// with 16-byte access the query stays packed in its input type and q.k uses
// the fp32-accumulating dot2 instructions (v_dot2c_f32_f16 / _bf16), so no
// K conversion is needed and the query takes DL/2 registers; the 1/sqrt(D)
// and log2(e) factors are applied to the summed score. fp32 and the masked
// path keep a pre-scaled fp32 query.
template <int DT, int D, bool VEC, int G = kGroup>
struct Query {
  using T = typename Elem<DT>::T;
  static constexpr int DL = D / G;
  static constexpr bool PACKED = VEC && DT != kF32;
  uint32_t qp[PACKED ? DL / 2 : 1];
  float qf[PACKED ? 1 : DL];
  float post_scale;
  __device__ __forceinline__ void load(const T* q, int col0, int dim, float scale) {
    Chunk<DT, DL, VEC> c;
    c.load(q + col0, col0, dim);
    if constexpr (PACKED) {
#pragma unroll
      for (int w = 0; w < DL / 2; ++w) qp[w] = c.raw[w / 4][w % 4];
      post_scale = scale;
    } else {
      c.to_float(qf);
#pragma unroll
      for (int i = 0; i < DL; ++i) qf[i] *= scale;
      post_scale = 1.f;
    }
  }
  // This lane's part of q.k (before the group sum and post_scale).
  __device__ __forceinline__ float partial(const Chunk<DT, DL, VEC>& k) const {
    float s = 0.f;
    if constexpr (PACKED) {
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      typedef __bf16 b2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int w = 0; w < DL / 2; ++w) {
        const uint32_t kw = k.raw[w / 4][w % 4];
        if constexpr (DT == kF16)
          s = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, qp[w]), __builtin_bit_cast(h2, kw), s, false);
        else
          s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, qp[w]), __builtin_bit_cast(b2, kw), s, false);
      }
    } else {
      float kf[DL];
      k.to_float(kf);
#pragma unroll
      for (int i = 0; i < DL; ++i) s = fmaf(qf[i], kf[i], s);
    }
    return s;
  }
  __device__ __forceinline__ float score(const Chunk<DT, DL, VEC>& k) const {
    return group_sum<G>(partial(k)) * post_scale;
  }
};

// Stream the tokens [t0, t0 + ntok) of one (request, head) whose page bases
// (K plane) are in s_page (entry j covers tokens t0 + j*P ...). Row-blocks
// rb = rb_first, rb_first + rb_step, ... are processed U at a time; with
// STAGES = 2 the loads of the next U row-blocks are in flight while the
// current ones are scored and accumulated.
template <int DT, int D, bool VEC, int U, int STAGES>
__device__ __forceinline__ void stream_rows(Softmax<D / kGroup>& st, const Query<DT, D, VEC>& q,
                                            typename Elem<DT>::T const* const* s_page,
                                            int ntok, int rb_first, int rb_step,
                                            const Geometry& g, int dim) {
  using T = typename Elem<DT>::T;
  constexpr int DL = D / kGroup;
  const int lane = threadIdx.x & (kWave - 1);
  const int tok = lane >> 2;
  const int col0 = (lane & 3) * DL;
  const int nrb = (ntok + kRowBlock - 1) / kRowBlock;
  const int pmask = g.page_size - 1;
  using C = Chunk<DT, DL, VEC>;
  auto issue = [&](int rb0, C* kc, C* vc, bool* valid) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int rel = (rb0 + u * rb_step) * kRowBlock + tok;
      valid[u] = rel < ntok;
      const T* base = valid[u] ? s_page[rel >> g.log2_page] : nullptr;
      if (base) {
        const T* kp = base + (rel & pmask) * dim + col0;
        kc[u].load(kp, col0, dim);
        vc[u].load(kp + g.kind_stride, col0, dim);
      } else {
        kc[u].nan_fill();
        vc[u].nan_fill();
      }
    }
  };
  auto consume = [&](const C* kc, const C* vc, const bool* valid) {
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) s[u] = q.score(kc[u]);
    st.template add_many<U>(s, valid, [&](int u, float* vf) { vc[u].to_float(vf); });
  };
  if constexpr (STAGES == 1) {
    for (int rb0 = rb_first; rb0 < nrb; rb0 += rb_step * U) {
      C kc[U], vc[U];
      bool valid[U];
      issue(rb0, kc, vc, valid);
      consume(kc, vc, valid);
    }
  } else {
    C kc[U], vc[U];
    bool valid[U];
    int rb0 = rb_first;
    if (rb0 < nrb) issue(rb0, kc, vc, valid);
    while (rb0 < nrb) {
      const int nxt = rb0 + rb_step * U;
      C nk[U], nv[U];
      bool nvalid[U];
      if (nxt < nrb) issue(nxt, nk, nv, nvalid);
      consume(kc, vc, valid);
#pragma unroll
      for (int u = 0; u < U; ++u) { kc[u] = nk[u]; vc[u] = nv[u]; valid[u] = nvalid[u]; }
      rb0 = nxt;
    }
  }
}

struct DecodeArgs {
  void* out;
  const void* q;
  const void* k;
  const void* v;
  const uint64_t* slabs;
  const int* table;
  const int* offsets;
  int batch;
  int split_tokens;
  int nsplit_max;
  float qscale;
  int64_t items;
  Geometry g;
  float* partials;
  // Optional work list: work_items (row, split) pairs in visiting order,
  // then merge_rows row indices whose splits need the reduction. Without it
  // every (split, row, head) is an item and every row is a merge candidate.
  const int* work;
  int work_items;
  int merge_rows;
  int64_t qkv_stride;  // elements between the rows of q, k and v (h * d when contiguous)
  // Without a work list and with one split per row: when rank_rows is set,
  // every workgroup ranks the batch's rows by context length from `offsets`
  // (longest first, ties by row) into dynamic LDS and visits them in the
  // order a host work list would give -- passes of rank_per rows, every
  // other pass reversed. Needs 2 * (batch rounded up to 4) ints of dynamic LDS.
  int rank_rows;
  int rank_per;
  // Work list built on the device (order_kernel) for a batch whose rows may
  // split: work_count[0] (row, split) pairs at `work`, then work_count[1]
  // merge rows. `items` is then only the capacity (batch * nsplit_max *
  // heads) and the grid one residency round that strides over the list.
  const int* work_count;
};

// How decode_kernel finds its items, a template parameter so that each
// instantiation carries only its own prologue (the kernel's start is
// latency-bound, and measured slower when unused prologue code grew):
// from a work list (host- or device-built), by ranking the rows in every
// workgroup, or as the plain (split, row, head) grid.
constexpr int kVisitList = 0, kVisitRank = 1, kVisitGrid = 2;

// Rows a decode workgroup ranks on its own (the ranking costs each thread
// batch / threads * batch LDS reads).
constexpr int kRankRows = 256;
// Rows order_kernel orders in its one workgroup; larger batches are visited
// in batch order.
constexpr int kOrderRows = 2048;
constexpr int kOrderThreads = 1024;

// Stream one wave's share of a split: row-blocks j = wave + waves * i
// (16 tokens each) of tokens [t0, t0 + ntok). Lane s of the wave holds in
// `base` the page base (K plane) of page slot s, resolved in the prologue:
// slot i for page sizes >= 16 (one page per row-block), slots 2i and 2i + 1
// for page size 8. Page bases are broadcast with readlane (scalar registers)
// or, for page size 8, a lane shuffle; no LDS and no barrier are involved.
template <int DT, int D, bool VEC, int U, int STAGES, int G>
__device__ __forceinline__ void stream_wave(Softmax<D / G, G>& st, const Query<DT, D, VEC, G>& q,
                                            uint64_t base, int ntok, int wave, int waves,
                                            const Geometry& g, int dim) {
  using T = typename Elem<DT>::T;
  constexpr int DL = D / G;
  constexpr int RB = kWave / G;  // tokens per wave step
  using C = Chunk<DT, DL, VEC>;
  const int lane = threadIdx.x & (kWave - 1);
  const int tok = lane / G;
  const int col0 = (lane % G) * DL;
  const int pmask = g.page_size - 1;
  const bool two_pages = g.page_size < RB;
  const int nrb = (ntok + RB - 1) / RB;
  const int mine = nrb > wave ? (nrb - wave + waves - 1) / waves : 0;
  const uint32_t base_lo = uint32_t(base), base_hi = uint32_t(base >> 32);
  auto issue = [&](int i0, C* kc, C* vc, bool* valid) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u;
      const int rel = (wave + waves * i) * RB + tok;
      valid[u] = i < mine && rel < ntok;
      uint64_t pb;
      if (two_pages) {
        const int slot = 2 * i + (tok >> 3);
        pb = (uint64_t(uint32_t(__shfl(int(base_hi), slot))) << 32) | uint32_t(__shfl(int(base_lo), slot));
      } else {
        const int slot = i < kWave ? i : kWave - 1;
        pb = (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(base_hi), slot))) << 32) |
             uint32_t(__builtin_amdgcn_readlane(int(base_lo), slot));
      }
      const T* page = reinterpret_cast<const T*>(pb);
      if (valid[u] && page) {
        const T* kp = page + (rel & pmask) * dim + col0;
        kc[u].template load<kDecodeNT>(kp, col0, dim);
        vc[u].template load<kDecodeNT>(kp + g.kind_stride, col0, dim);
      } else {
        kc[u].nan_fill();
        vc[u].nan_fill();
      }
    }
  };
  auto consume = [&](const C* kc, const C* vc, const bool* valid) {
    float s[U];
#pragma unroll
    for (int u = 0; u < U; ++u) s[u] = q.score(kc[u]);
    st.template add_many<U>(s, valid, [&](int u, float* vf) { vc[u].to_float(vf); });
  };
  if constexpr (STAGES == 1) {
    for (int i0 = 0; i0 < mine; i0 += U) {
      C kc[U], vc[U];
      bool valid[U];
      issue(i0, kc, vc, valid);
      consume(kc, vc, valid);
    }
  } else {
    C kc[U], vc[U];
    bool valid[U];
    if (mine > 0) issue(0, kc, vc, valid);
    for (int i0 = 0; i0 < mine; i0 += U) {
      C nk[U], nv[U];
      bool nvalid[U];
      if (i0 + U < mine) issue(i0 + U, nk, nv, nvalid);
      consume(kc, vc, valid);
#pragma unroll
      for (int u = 0; u < U; ++u) { kc[u] = nk[u]; vc[u] = nv[u]; valid[u] = nvalid[u]; }
    }
  }
}

// Fused KV append + decode attention over (request, head, split) items.
// Items come from the work list when one is given (visiting order chosen by
// the caller, e.g. longest first), else from the full (split, row, head) grid.
// 8-wave fp16/bf16 workgroups at D = 64 (config 2's shape) are meant to be
// resident three per compute unit, i.e. six waves per SIMD and at most 80
// VGPRs: one VGPR more drops a whole workgroup per compute unit (and the
// launcher then picks 4-wave workgroups), so the bound is stated. Other
// shapes need more registers and keep the compiler's choice.
template <int DT, int D, bool VEC, int U, int STAGES, int WAVES, int G, int MODE>
__global__ __launch_bounds__(WAVES * kWave)
__attribute__((amdgpu_waves_per_eu(WAVES == 8 && D == 64 && VEC && DT != kF32 && U <= 2 ? 6 : 1)))
void decode_kernel(DecodeArgs a) {
  using T = typename Elem<DT>::T;
  constexpr int DL = D / G;
  constexpr int RB = kWave / G;
  constexpr int PSTRIDE = D + 2;
  constexpr int NT = WAVES * kWave;
  constexpr int NS = WAVES * 4;  // partial states per item: one per 16-lane row
  constexpr int SLABS_PER_THREAD = (kLdsSlabs + NT - 1) / NT;
  constexpr int GROUPS = NT / D;    // thread groups of the first merge level
  constexpr int PER = NS / GROUPS;  // row states each group merges
  static_assert(NT % D == 0 && NS % GROUPS == 0, "merge partition");
  __shared__ float s_m[NS], s_l[NS];
  __shared__ float s_acc[NS][D];
  __shared__ float s2_m[GROUPS], s2_l[GROUPS];
  __shared__ float s2_acc[GROUPS][D];
  __shared__ uint64_t s_slabs[kLdsSlabs];
  __shared__ __align__(16) T s_new[2][D];  // the new token's K and V rows

#ifdef MT_DECODE_TIMELINE
  const uint64_t tl_start = wall_clock64();
  uint64_t tl_entry = 0, tl_loads = 0, tl_barrier = 0, tl_stream = 0;
#endif
  const Geometry& g = a.g;
  const int dim = VEC ? D : g.dim;
  const int tid = threadIdx.x;
  const int64_t bh_count = int64_t(a.batch) * g.heads;
  // The slab table of a small pool is staged in LDS. A workgroup whose first
  // item is certain to have work (every work-list item; split 0 of the full
  // grid) reads it before anything else, so that it arrives while the
  // item's own loads are in flight; others read it once an item has work.
  const bool lds_slabs = g.num_slabs <= kLdsSlabs;
  bool slabs_staged = !lds_slabs;
  bool slabs_loaded = false;
  uint64_t slab_reg[SLABS_PER_THREAD];
  auto load_slabs = [&]() {
#pragma unroll
    for (int j = 0; j < SLABS_PER_THREAD; ++j) {
      const int i = tid + j * NT;
      slab_reg[j] = i < g.num_slabs ? a.slabs[i] : 0;
    }
    slabs_loaded = true;
  };
  if (lds_slabs && (MODE != kVisitGrid || blockIdx.x < bh_count)) load_slabs();
  // In-kernel longest-first order (see DecodeArgs::rank_rows): s_len holds
  // the offsets, s_order[k] the row of rank k; (length desc, row asc) is a
  // strict order, so the ranks are a permutation whatever the offsets hold.
  // s_len is padded to a multiple of 4 rows with INT_MIN, which no row
  // ranks behind, and read 4 rows per LDS load. Each row's rank is counted
  // by tpr consecutive lanes (the largest power of two up to 64 with
  // tpr * batch <= threads), each over its own slice of the candidates, and
  // summed with lane shuffles: the count runs on every wave, not one.
  extern __shared__ __align__(16) int s_rank[];
  const int len4 = (a.batch + 3) & ~3;
  int* const s_len = s_rank;
  int* const s_order = s_rank + len4;
  if constexpr (MODE == kVisitRank) {
    for (int r = tid; r < len4; r += NT) s_len[r] = r < a.batch ? a.offsets[r] : INT_MIN;
    __syncthreads();
    const int4* len_v = reinterpret_cast<const int4*>(s_len);
    int tpr = 1;
    while (tpr < kWave && 2 * tpr * a.batch <= NT) tpr *= 2;
    const int n4 = len4 / 4;
    const int per_part = (n4 + tpr - 1) / tpr;  // int4 candidates per lane
    for (int t0 = 0; t0 < a.batch * tpr; t0 += NT) {
      const int t = t0 + tid;
      const int r = t / tpr, part = t - r * tpr;
      int rank = 0;
      if (r < a.batch) {
        const int lr = s_len[r];
        const int c1 = min(n4, (part + 1) * per_part);
        for (int q4 = part * per_part; q4 < c1; ++q4) {
          const int4 l = len_v[q4];
          const int q = 4 * q4;
          rank += (l.x > lr) | ((l.x == lr) & (q < r));
          rank += (l.y > lr) | ((l.y == lr) & (q + 1 < r));
          rank += (l.z > lr) | ((l.z == lr) & (q + 2 < r));
          rank += (l.w > lr) | ((l.w == lr) & (q + 3 < r));
        }
      }
      for (int o = 1; o < tpr; o <<= 1) rank += __shfl_xor(rank, o);
      if (r < a.batch && part == 0) s_order[rank] = r;
    }
    __syncthreads();
  }
  const int wave = tid >> 6;
  const int lane = tid & (kWave - 1);
  const int col0 = (lane % G) * DL;
  const int64_t cap = int64_t(g.columns) * g.page_size;
  const int sub_shift = g.page_size < RB ? 1 : 0;
  const int rb_per_wave = a.split_tokens / RB / WAVES;
  const T* qp = static_cast<const T*>(a.q);
  const T* kin = static_cast<const T*>(a.k);
  const T* vin = static_cast<const T*>(a.v);
  T* out = static_cast<T*>(a.out);
  const uint64_t* work64 = reinterpret_cast<const uint64_t*>(a.work);

  // A device-built list's length is read together with the workgroup's first
  // entry (within the list's capacity, which bounds the grid), so the count
  // adds no round trip before the first item.
  int64_t items = a.items;
  uint64_t first_entry = 0;
  if (MODE == kVisitList && a.work_count) {
    first_entry = work64[blockIdx.x / unsigned(g.heads)];
    items = std::min(int64_t(a.work_count[0]) * g.heads, a.items);  // never past the list
  }

  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    int split, b, head;
    if constexpr (MODE == kVisitList) {
      // (row, split) read as one 8-byte load: the workgroup's first dependent
      // round trip.
      const int w = int(unsigned(item) / unsigned(g.heads));
      head = int(item) - w * g.heads;
      const uint64_t e = (a.work_count && item == blockIdx.x) ? first_entry : work64[w];
      b = int(uint32_t(e));
      split = int(uint32_t(e >> 32));
#ifdef MT_DECODE_TIMELINE
      if (item == blockIdx.x) tl_entry = stamp_after(b);
#endif
      if (!((unsigned(b) < unsigned(a.batch)) & (unsigned(split) < unsigned(a.nsplit_max)))) continue;
    } else if constexpr (MODE == kVisitRank) {
      // item = (visiting position, head); one split per row
      const int pos = int(unsigned(item) / unsigned(g.heads));
      head = int(item) - pos * g.heads;
      const int pass = pos / a.rank_per, within = pos - pass * a.rank_per;
      const int width = min(a.rank_per, a.batch - pass * a.rank_per);
      b = s_order[pass * a.rank_per + ((pass & 1) ? width - 1 - within : within)];
      split = 0;
    } else {
      split = int(unsigned(item) / unsigned(bh_count));
      const int bhi = int(item) - split * int(bh_count);
      b = int(unsigned(bhi) / unsigned(g.heads));
      head = bhi - b * g.heads;
    }
    const int64_t bh = int64_t(b) * g.heads + head;

    // Loads that do not depend on the context length are issued first, all
    // in one round trip: the table entry of each of this wave's page slots
    // (the next link of the chain to the K/V loads), the query, the new
    // token's K/V (wave 0) and the offset.
    const int* table_row = a.table + int64_t(b) * g.columns;
    const int t0i = split * a.split_tokens;
    const int slot_i = lane >> sub_shift;
    const int slot_tok = (wave + WAVES * slot_i) * RB + ((lane & sub_shift) << 3);
    const int64_t slot_logical = (int64_t(t0i) + slot_tok) >> g.log2_page;
    int physical = -1;
    if (slot_i < rb_per_wave && slot_logical < g.columns) physical = table_row[slot_logical];
    Query<DT, D, VEC, G> qv;
    const int64_t qrow = int64_t(b) * a.qkv_stride + int64_t(head) * dim;  // q, k, v row
    qv.load(qp + qrow, col0, dim, a.qscale);
    T new_k{}, new_v{};
    if (tid < dim) { new_k = kin[qrow + tid]; new_v = vin[qrow + tid]; }
    const int offset = MODE == kVisitRank ? s_len[b] : a.offsets[b];
#ifdef MT_DECODE_TIMELINE
    if (item == blockIdx.x) tl_loads = stamp_after(offset + physical);
#endif

    const int64_t L = offset < 0 ? 0 : int64_t(offset) + 1;
    T* orow = out + bh * dim;
    if (L > cap) {
      // A token beyond the table's columns reads as a missing page: NaN row.
      if (split == 0)
        for (int t = tid; t < dim; t += NT) orow[t] = from_f32<DT>(NAN);
      continue;
    }
    const int nsplit = L == 0 ? 1 : int((uint32_t(L) + uint32_t(a.split_tokens) - 1) / uint32_t(a.split_tokens));
    if (split >= nsplit) continue;
    const int64_t t0 = t0i;
    const int64_t t1 = L < t0 + a.split_tokens ? L : t0 + a.split_tokens;
    const bool owns_new = L > 0 && split == nsplit - 1;
    const int ntok_paged = int((owns_new ? t1 - 1 : t1) - t0);  // tokens read from pages
    // Staged in LDS once the loads above are in flight: the slab table (first
    // item only) and the new token's K/V row, which is needed only after the
    // stream and so holds no registers during it.
    if (!slabs_staged) {
      if (!slabs_loaded) load_slabs();
#pragma unroll
      for (int j = 0; j < SLABS_PER_THREAD; ++j)
        if (tid + j * NT < kLdsSlabs) s_slabs[tid + j * NT] = slab_reg[j];
    }
    if (tid < dim) { s_new[0][tid] = new_k; s_new[1][tid] = new_v; }
    __syncthreads();
    slabs_staged = true;
#ifdef MT_DECODE_TIMELINE
    if (item == blockIdx.x) tl_barrier = wall_clock64();
#endif
    auto slab_of = [&](int physical) -> uint64_t {
      return lds_slabs ? s_slabs[slab_index(physical, g)] : a.slabs[slab_index(physical, g)];
    };
    auto resolve = [&](int physical) -> const T* {
      return physical_in_pool(physical, g) ? page_in_slab<T>(slab_of(physical), physical, g, head)
                                           : nullptr;
    };

    const T* my_page = (slot_i < rb_per_wave && t0 + slot_tok < t1) ? resolve(physical) : nullptr;
    // The new token's page (wave 0, scalar loads; needed only after the stream).
    const T* new_page = nullptr;
    if (owns_new && wave == 0) {
      const int64_t logical = (L - 1) >> g.log2_page;
      new_page = logical < g.columns ? resolve(table_row[logical]) : nullptr;
    }

    Softmax<DL, G> st;
    st.init();
#ifdef MT_DECODE_TIMELINE
    if (item == blockIdx.x) tl_stream = wall_clock64();
#endif
    stream_wave<DT, D, VEC, U, STAGES, G>(st, qv, reinterpret_cast<uint64_t>(my_page), ntok_paged,
                                           wave, WAVES, g, dim);

    if (owns_new && wave == 0) {
      // The new token: read from the K/V inputs, scored by group 0 of wave 0,
      // and written into its page when the page exists (reference append,
      // src/paged_attention_kernel.cu:23-33). A missing page reads as NaN.
      const int64_t pos = L - 1;
      Chunk<DT, DL, VEC> kn, vn;
      kn.load_lds(&s_new[0][col0], col0, dim);
      vn.load_lds(&s_new[1][col0], col0, dim);
      if (lane < G && new_page) {
        T* kp = const_cast<T*>(new_page) + (pos & (g.page_size - 1)) * dim + col0;
        T* vp = kp + g.kind_stride;
        if constexpr (VEC) {
#pragma unroll
          for (int i = 0; i < Chunk<DT, DL, VEC>::NV; ++i) {
            global_view(reinterpret_cast<u32x4*>(kp))[i] = kn.raw[i];
            global_view(reinterpret_cast<u32x4*>(vp))[i] = vn.raw[i];
          }
        } else {
          for (int i = 0; i < DL && col0 + i < dim; ++i) {
            kp[i] = kin[qrow + col0 + i];
            vp[i] = vin[qrow + col0 + i];
          }
        }
      }
      if (!new_page) { kn.nan_fill(); vn.nan_fill(); }
      const float sc = qv.score(kn);
      if (lane < G) {
        float vf[DL];
        vn.to_float(vf);
        st.add(sc, vf);
      }
    }

    // Row merges by DPP, then the WAVES * 4 row states meet in LDS.
    st.row_merge();
    const int row = lane >> 4;
    if ((lane & 15) < G) {
      const int si = wave * 4 + row;
#pragma unroll
      for (int i = 0; i < DL; ++i) s_acc[si][col0 + i] = st.acc[i];
      if ((lane & 15) == 0) { s_m[si] = st.m; s_l[si] = st.l; }
    }
    __syncthreads();

    // Two-level merge with every thread busy: group q of D threads merges
    // row states [q*PER, (q+1)*PER) per dim, then D threads merge the groups.
    {
      const int d = tid % D, q = tid / D;
      float M = -INFINITY;
#pragma unroll
      for (int j = 0; j < PER; ++j) M = fmaxf(M, s_m[q * PER + j]);
      float lq = 0.f, aq = 0.f;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const int w = q * PER + j;
        const float mw = s_m[w];
        const float sc = (mw == -INFINITY) ? 0.f : fast_exp2(mw - M);
        lq = fmaf(s_l[w], sc, lq);
        aq = fmaf(s_acc[w][d], sc, aq);
      }
      s2_acc[q][d] = aq;
      if (d == 0) { s2_m[q] = M; s2_l[q] = lq; }
    }
    __syncthreads();

    const int t = tid;
    if (t < dim) {
      float M = -INFINITY;
#pragma unroll
      for (int q = 0; q < GROUPS; ++q) M = fmaxf(M, s2_m[q]);
      float lsum = 0.f, asum = 0.f;
#pragma unroll
      for (int q = 0; q < GROUPS; ++q) {
        const float mq = s2_m[q];
        const float sc = (mq == -INFINITY) ? 0.f : fast_exp2(mq - M);
        lsum = fmaf(s2_l[q], sc, lsum);
        asum = fmaf(s2_acc[q][t], sc, asum);
      }
      if (nsplit == 1) {
        orow[t] = from_f32<DT>(finalize(asum, lsum));
      } else {
        float* part = a.partials + (bh * a.nsplit_max + split) * PSTRIDE;
        part[2 + t] = asum;
        if (t == 0) { part[0] = M; part[1] = lsum; }
      }
    }
    __syncthreads();  // LDS is reused by the next item
  }
#ifdef MT_DECODE_TIMELINE
  if (tid == 0 && blockIdx.x < unsigned(kTimelineMax)) {
    uint64_t* rec = g_decode_timeline + kTimelineFields * blockIdx.x;
    rec[0] = tl_start;
    rec[1] = tl_entry;
    rec[2] = tl_loads;
    rec[3] = tl_barrier;
    rec[4] = tl_stream;
    rec[5] = wall_clock64();
    rec[6] = __builtin_amdgcn_s_getreg(4 | (31 << 11));   // HW_ID: wave, SIMD, CU, SH, SE
    rec[7] = __builtin_amdgcn_s_getreg(20 | (15 << 11));  // XCC_ID
  }
#endif
}

// Split-context reduction: for every (request, head) whose context spans more
// than one split, merge the per-split (max, denominator, accumulator) partials
// with the log-sum-exp rule and write the output row. Rows with a single split
// were written by decode_kernel. The kernel boundary orders it after the
// partial writes, so no device-scope fences are needed.
template <int DT, int D>
__global__ __launch_bounds__(128) void merge_kernel(DecodeArgs a) {
  using T = typename Elem<DT>::T;
  constexpr int PSTRIDE = D + 2;
  const Geometry& g = a.g;
  const int dim = g.dim;
  // a device-built list's counts, bounded by its capacity
  const int64_t work_items = a.work_count ? std::min(int64_t(a.work_count[0]), a.items / g.heads) : a.work_items;
  const int64_t rows = a.work_count ? std::min(a.work_count[1], a.batch) : a.work ? a.merge_rows : a.batch;
  const int64_t count = rows * g.heads;
  const int64_t cap = int64_t(g.columns) * g.page_size;
  T* out = static_cast<T*>(a.out);
  for (int64_t i = blockIdx.x; i < count; i += gridDim.x) {
    const int64_t m = i / g.heads;
    const int head = int(i - m * g.heads);
    const int b = a.work ? a.work[2 * work_items + m] : int(m);
    if (b < 0 || b >= a.batch) continue;
    const int64_t bh = int64_t(b) * g.heads + head;
    const float* base = a.partials + bh * a.nsplit_max * PSTRIDE;
    const int t = threadIdx.x;
    // Partials of up to kChunk splits are loaded per pass; the first pass is
    // issued together with the context-length read that says how many exist.
    constexpr int kChunk = 8;
    float pm[kChunk], pl[kChunk], pa[kChunk];
    auto load_chunk = [&](int s0) {
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        const int sj = s0 + j < a.nsplit_max ? s0 + j : a.nsplit_max - 1;
        pm[j] = base[sj * PSTRIDE];
        pl[j] = base[sj * PSTRIDE + 1];
        pa[j] = t < dim ? base[sj * PSTRIDE + 2 + t] : 0.f;
      }
    };
    load_chunk(0);
    const int offset = a.offsets[b];
    const int64_t L = offset < 0 ? 0 : int64_t(offset) + 1;
    if (L > cap) continue;
    const int nsplit = L == 0 ? 1 : int((L + a.split_tokens - 1) / a.split_tokens);
    if (nsplit == 1) continue;
    // Online log-sum-exp merge over the chunks.
    float M = -INFINITY, lsum = 0.f, asum = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += kChunk) {
      if (s0 > 0) load_chunk(s0);
      float cm = M;
#pragma unroll
      for (int j = 0; j < kChunk; ++j)
        if (s0 + j < nsplit) cm = fmaxf(cm, pm[j]);
      const float rescale = (M == -INFINITY) ? 0.f : fast_exp2(M - cm);
      lsum *= rescale;
      asum *= rescale;
#pragma unroll
      for (int j = 0; j < kChunk; ++j) {
        if (s0 + j < nsplit) {
          const float sc = (pm[j] == -INFINITY) ? 0.f : fast_exp2(pm[j] - cm);
          lsum = fmaf(pl[j], sc, lsum);
          asum = fmaf(pa[j], sc, asum);
        }
      }
      M = cm;
    }
    if (t < dim) out[bh * dim + t] = from_f32<DT>(finalize(asum, lsum));
  }
}

// Work list of a decode launch built on the device from offsets[], for the
// reference entry, which has no work-list argument: the list a host caller
// builds from the lengths it knows (paged_ops.decode_work_list), bit for bit.
// Row r attends L = offsets[r] + 1 keys (0 for a negative offset) in
// n = max(1, ceil(L / S)) splits: splits 0 .. n-2 of S tokens and a last one
// of t = L - (n-1) S (a row past its table: one entry, t = 0, which the
// decode turns into a NaN row). Entries are ordered by tokens descending,
// then row, then split; position p of that order goes to slot f(p) of
// passes of `per` entries with every other pass reversed. The S-token
// entries form the first run, in (row, split) order, so entry (r, s) of it
// sits at the count of S-token entries of rows before r, plus s (a prefix
// sum). The last splits of fewer than S tokens follow, sorted by (tokens
// descending, row): a stable LDS radix sort of the rows on S - 1 - t, rows
// whose last split is full keyed past every other. The rows with more than
// one split follow the list, ascending: list[2W + m]. count = (W, M).
struct OrderArgs {
  const int* offsets;
  int* list;   // 2 * capacity + batch ints
  int* count;  // [2]
  int batch, split_tokens, per;
  int capacity;  // (row, split) pairs the list holds: batch * nsplit_max
  int64_t cap;   // tokens a table holds
};

constexpr int kOrderWaves = kOrderThreads / 64;
constexpr int kRadixBits = 6;
constexpr int kRadixDigits = 1 << kRadixBits;  // one digit per lane
constexpr int kOrderBlocks = kOrderRows / kOrderThreads;  // rows per thread (striped)
constexpr int kRadixCounts = kRadixDigits * kOrderBlocks * kOrderWaves;
static_assert(kRadixDigits == 64 && kRadixCounts % kOrderThreads == 0, "order_kernel layout");

// Exclusive prefix sums of V per-thread values over a workgroup of
// kOrderThreads, in thread order; totals in tot[].
template <int V>
__device__ __forceinline__ void order_scan(int (&v)[V], int (&tot)[V], int (*s_wave)[kOrderWaves]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) inc[j] = wave_inclusive_add(v[j]);
  if (lane == 63) {
#pragma unroll
    for (int j = 0; j < V; ++j) s_wave[j][wave] = inc[j];
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < V; ++j) {
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kOrderWaves; ++w) {
      const int x = s_wave[j][w];
      before += w < wave ? x : 0;
      all += x;
    }
    v[j] = before + inc[j] - v[j];
    tot[j] = all;
  }
  __syncthreads();
}

__global__ __launch_bounds__(kOrderThreads) void order_kernel(OrderArgs o) {
  __shared__ int s_full[kOrderRows];   // S-token entries of the rows before
  __shared__ int s_merge[kOrderRows];  // merge rows before
  __shared__ int s_key[2][kOrderRows];  // radix sort: keys, ping-pong
  __shared__ short s_row[2][kOrderRows];
  // per (digit, block, wave) counts of one radix pass, scanned in that order
  __shared__ int s_cnt[kRadixCounts];
  __shared__ int s_wave[2 * kOrderBlocks + kOrderBlocks][kOrderWaves];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = o.batch;
  const uint32_t S = uint32_t(o.split_tokens);
  const int blocks = (b + kOrderThreads - 1) / kOrderThreads;
  // Striped rows: thread tid holds rows tid + j * kOrderThreads.
  int n[kOrderBlocks], t[kOrderBlocks];
#pragma unroll
  for (int j = 0; j < kOrderBlocks; ++j) {
    const int r = tid + j * kOrderThreads;
    n[j] = 0; t[j] = 0;
    if (r < b) {
      const int off = o.offsets[r];
      const uint32_t L = off < 0 ? 0u : uint32_t(off) + 1u;
      if (int64_t(L) > o.cap) {
        n[j] = 1;
      } else {
        const uint32_t nn = L == 0 ? 1u : (L + S - 1) / S;
        n[j] = int(nn);
        t[j] = int(L - (nn - 1) * S);
      }
    }
    // sort key: S - 1 - t ascending is tokens descending; a full last split
    // (not sorted here) and padding rows go behind every other
    s_key[0][r] = (r < b && t[j] < int(S)) ? int(S) - 1 - t[j] : 4095;
    s_row[0][r] = short(r);
  }
  // Prefix sums in row order of the S-token entries, the last splits below
  // S and the merge rows: block j's sums follow block j - 1's.
  int v[3 * kOrderBlocks], tot[3 * kOrderBlocks];
#pragma unroll
  for (int j = 0; j < kOrderBlocks; ++j) {
    const bool in = tid + j * kOrderThreads < b;
    v[3 * j] = in ? n[j] - 1 + (t[j] == int(S)) : 0;
    v[3 * j + 1] = in ? int(t[j] < int(S)) : 0;
    v[3 * j + 2] = in ? int(n[j] > 1) : 0;
  }
  order_scan<3 * kOrderBlocks>(v, tot, s_wave);
  int full_total = 0, last_count = 0, M = 0;
#pragma unroll
  for (int j = 0; j < kOrderBlocks; ++j) {
    const int r = tid + j * kOrderThreads;
    if (r < b) { s_full[r] = full_total + v[3 * j]; s_merge[r] = M + v[3 * j + 2]; }
    full_total += tot[3 * j];
    last_count += tot[3 * j + 1];
    M += tot[3 * j + 2];
  }
  const int W = full_total + last_count;
  // Stable LSD radix sort of (key, row) over 12 bits, 6 per pass. Six
  // ballots give every lane the lanes of its wave with the same digit, and
  // lane d the count of digit d in its wave; a position is the scanned count
  // of (digit, block, wave) plus the same-digit lanes below it.
  const uint64_t lt = (uint64_t(1) << lane) - 1;
  int src = 0;
  for (int shift = 0; shift < 12; shift += kRadixBits, src ^= 1) {
    int digit[kOrderBlocks], within[kOrderBlocks];
#pragma unroll
    for (int j = 0; j < kOrderBlocks; ++j) {
      digit[j] = 0; within[j] = 0;
      int count = 0;
      if (j < blocks) {
        const int d = (s_key[src][tid + j * kOrderThreads] >> shift) & (kRadixDigits - 1);
        uint64_t peers = ~uint64_t(0), mine = ~uint64_t(0);
#pragma unroll
        for (int bit = 0; bit < kRadixBits; ++bit) {
          const uint64_t m = __ballot((d >> bit) & 1);
          peers &= ((d >> bit) & 1) ? m : ~m;
          mine &= ((lane >> bit) & 1) ? m : ~m;
        }
        digit[j] = d;
        within[j] = __popcll(peers & lt);
        count = __popcll(mine);
      }
      s_cnt[(lane * kOrderBlocks + j) * kOrderWaves + wave] = count;
    }
    __syncthreads();
    {
      constexpr int PER = kRadixCounts / kOrderThreads;
      int c[PER], sv[1] = {0}, st[1];
#pragma unroll
      for (int i = 0; i < PER; ++i) { c[i] = s_cnt[tid * PER + i]; sv[0] += c[i]; }
      order_scan<1>(sv, st, s_wave);
      int run = sv[0];
#pragma unroll
      for (int i = 0; i < PER; ++i) { s_cnt[tid * PER + i] = run; run += c[i]; }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kOrderBlocks; ++j) {
      if (j < blocks) {
        const int i = tid + j * kOrderThreads;
        const int pos = s_cnt[(digit[j] * kOrderBlocks + j) * kOrderWaves + wave] + within[j];
        if (unsigned(pos) < unsigned(kOrderRows)) {
          s_key[src ^ 1][pos] = s_key[src][i];
          s_row[src ^ 1][pos] = s_row[src][i];
        }
      }
    }
    __syncthreads();
  }
  const int per = o.per;
  auto place = [&](int p, int r, int s) {
    const int pass = p / per, within = p - pass * per;
    const int width = min(per, W - pass * per);
    const int f = pass * per + ((pass & 1) ? width - 1 - within : within);
    if (unsigned(f) < unsigned(min(W, o.capacity))) {
      o.list[2 * f] = r;
      o.list[2 * f + 1] = s;
    }
  };
  // The sorted last splits below S.
  for (int p = tid; p < last_count; p += kOrderThreads) {
    const int r = s_row[src][p];
    if (unsigned(r) >= unsigned(b)) continue;
    const int full = (r + 1 < b ? s_full[r + 1] : full_total) - s_full[r];
    place(full_total + p, r, full);
  }
  // Each row's S-token splits and its merge entry.
#pragma unroll
  for (int j = 0; j < kOrderBlocks; ++j) {
    const int r = tid + j * kOrderThreads;
    if (r < b) {
      const int full = n[j] - 1 + (t[j] == int(S));
      for (int s = 0; s < full; ++s) place(s_full[r] + s, r, s);
      const int m = s_merge[r];
      if (n[j] > 1 && W <= o.capacity && unsigned(m) < unsigned(b)) o.list[2 * W + m] = r;
    }
  }
  if (tid == 0) { o.count[0] = W; o.count[1] = M; }
}

struct QueryArgs {
  void* out;
  const void* q;
  const uint64_t* slabs;
  const int* table;
  int batch, nq, nk, offset;
  float qscale;
  int64_t items;
  Geometry g;
  // Element strides of q and out per request, head and query: [b, h, nq, d]
  // by default, [b, nq, row] for head-interleaved token rows.
  int64_t q_b, q_h, q_r, o_b, o_h, o_r;
  // The prompt's own K/V rows (strides of q), or null. When set (prefill
  // kernel only), keys at or past the offset are read from these rows and the
  // workgroup of each query tile writes its tokens' K/V to their pages, which
  // replaces a separate append.
  const void* k;
  const void* v;
  // Key-split prefill: per (slot, head, query of the tile) D accumulators,
  // max and denominator of one split's keys, merged by prefill_merge_kernel.
  float* partials;
};

// Floats per query in the key-split partials: D accumulators, then max and
// denominator, padded so every row starts 16-byte aligned.
template <int D>
constexpr int pf_part_row() { return D + 4; }

// Causal paged attention for nq >= 1 queries per (request, head)
// (reference paged_forward with offsets == nullptr, src/paged_attention_kernel.cu:35-85):
// query qi attends keys kj < nk with kj <= offset + qi. One wave per query,
// four queries per workgroup; page bases are resolved per 2048-token chunk.
template <int DT, int D, bool VEC, int U>
__global__ __launch_bounds__(kThreads) void query_kernel(QueryArgs a) {
  using T = typename Elem<DT>::T;
  constexpr int DL = D / kGroup;
  __shared__ const T* s_page[kMaxSplitPages];
  const Geometry& g = a.g;
  const int dim = VEC ? D : g.dim;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & (kWave - 1);
  const int col0 = (lane & 3) * DL;
  const int qblocks = (a.nq + kWaves - 1) / kWaves;
  const T* qp = static_cast<const T*>(a.q);
  T* out = static_cast<T*>(a.out);
  for (int64_t item = blockIdx.x; item < a.items; item += gridDim.x) {
    const int64_t bh = item / qblocks;
    const int qb = int(item - bh * qblocks);
    const int b = int(bh / g.heads), head = int(bh - int64_t(b) * g.heads);
    const int qi = qb * kWaves + wave;
    const bool has_q = qi < a.nq;
    const int64_t klen = has_q ? (int64_t(a.offset) + qi + 1 < a.nk ? int64_t(a.offset) + qi + 1 : a.nk) : 0;
    const int qlast = (qb * kWaves + kWaves - 1 < a.nq ? qb * kWaves + kWaves - 1 : a.nq - 1);
    const int64_t kmax = int64_t(a.offset) + qlast + 1 < a.nk ? int64_t(a.offset) + qlast + 1 : a.nk;
    const int* table_row = a.table + int64_t(b) * g.columns;
    Query<DT, D, VEC> qv;
    qv.load(qp + b * a.q_b + head * a.q_h + (has_q ? qi : 0) * a.q_r, col0, dim, a.qscale);
    Softmax<DL> st;
    st.init();
    for (int64_t c0 = 0; c0 < kmax; c0 += kMaxSplitTokens) {
      const int64_t c1 = c0 + kMaxSplitTokens < kmax ? c0 + kMaxSplitTokens : kmax;
      const int npg = int((c1 - c0 + g.page_size - 1) >> g.log2_page);
      __syncthreads();
      for (int j = tid; j < npg; j += kThreads)
        s_page[j] = page_base<T>(a.slabs, table_row, (c0 >> g.log2_page) + j, g, head);
      __syncthreads();
      const int64_t mine = klen - c0 < c1 - c0 ? klen - c0 : c1 - c0;
      if (mine > 0) stream_rows<DT, D, VEC, U, 2>(st, qv, s_page, int(mine), 0, 1, g, dim);
    }
    st.wave_merge();
    if (has_q && lane < kGroup) {
      T* orow = out + b * a.o_b + head * a.o_h + qi * a.o_r;
      for (int i = 0; i < DL; ++i)
        if (col0 + i < dim) orow[col0 + i] = from_f32<DT>(finalize(st.acc[i], st.l));
    }
    __syncthreads();
  }
}

struct AppendArgs {
  const void* k;
  const void* v;
  const uint64_t* slabs;
  const int* table;
  int batch, n, offset;
  int64_t vectors;  // number of per-thread units
  Geometry g;
  int64_t src_b, src_h, src_r;  // element strides of k/v per request, head and token
};


// ---------------------------------------------------------------------------
// Causal paged prefill attention on the matrix cores (fp16/bf16, head_dim 64
// or 128), same semantics as query_kernel: query qi attends keys
// kj < nk with kj <= offset + qi, and a query whose keys touch a missing page
// reads NaN. One workgroup of 4 waves per (request, head, 64-query tile),
// each wave owning 16 queries; keys stream in blocks of 64 staged in LDS from
// the pages (K row-major, V transposed). Per block a wave computes
// S^T = K Q^T with v_mfma_f32_16x16x32 (keys x queries, so each lane holds 16
// scores of one query), updates that query's online softmax in registers and
// accumulates O^T += V^T P^T, feeding the scores' own register layout as the
// B operand (the MFMA sums over its k index in any order, so A's key order is
// chosen to match). The MFMA takes P in the input type, so P is split into a
// high and a low part of that type (two MFMAs): the weights keep about 16
// (bf16) or 22 (fp16) significant bits instead of 8 or 11, which holds the
// output to the fp32 path's accuracy when |V| is large.
constexpr int kPfQueries = 64;     // queries per workgroup
constexpr int kPfKeys = 64;        // keys per staged block
constexpr int kPfWindowPages = 512;  // page bases resolved into LDS at a time
#ifndef MT_PREFILL_MIN_QUERIES
#define MT_PREFILL_MIN_QUERIES 16
#endif
constexpr int kPfMinQueries = MT_PREFILL_MIN_QUERIES;  // fewer queries use query_kernel

// x of lane l ^ 16 and of lane l ^ 32, combined with x by the caller: the
// permlane swaps exchange rows of 16 (32) lanes between two registers, so
// after swapping two copies of x, lane l holds x[l] in one and x[l ^ 16]
// (x[l ^ 32]) in the other.
__device__ __forceinline__ float lane_swap16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return (threadIdx.x & 16) ? a : b;
}
__device__ __forceinline__ float lane_swap32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return (threadIdx.x & 32) ? a : b;
}

// Two probabilities rounded to the input type, packed as the MFMA operand;
// r0/r1 receive the rounded values as floats (for the low part of the split).
// fp16 rounds toward zero (one packed conversion; the low part carries the
// remainder), bf16 to nearest even.
template <int DT>
struct PackP;
template <>
struct PackP<kF16> {
  static __device__ __forceinline__ uint32_t pack(float p0, float p1, float& r0, float& r1) {
    const auto h = __builtin_amdgcn_cvt_pkrtz(p0, p1);
    r0 = float(h[0]);
    r1 = float(h[1]);
    return __builtin_bit_cast(uint32_t, h);
  }
};
template <>
struct PackP<kBF16> {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ uint32_t pack(float p0, float p1, float& r0, float& r1) {
    const bf2 h = {static_cast<__bf16>(p0), static_cast<__bf16>(p1)};
    const uint32_t u = __builtin_bit_cast(uint32_t, h);
    r0 = __uint_as_float(u << 16);
    r1 = __uint_as_float(u & 0xffff0000u);
    return u;
  }
};

// What one prefill workgroup works on: query tile `tile` of `head` of a
// request whose queries start at element q0 of q (o0 of out), nq queries at
// key offset `offset` over the pages of table_row.
struct PfItem {
  int tile, head, nq, offset;
  int64_t q0, o0;
  const int* table_row;
  int kb0, kb1;  // key blocks [kb0, kb1) of the tile's keys that this item attends
  int slot;      // partials slot of a split tile, -1: the item writes the output rows
};

constexpr int kAllKeyBlocks = 1 << 24;

// The uniform batch of QueryArgs (b requests of nq queries at one offset):
// items ordered by tile, last (longest) tiles first.
struct UniformItems {
  __device__ __forceinline__ int64_t count(const QueryArgs& a) const { return a.items; }
  __device__ __forceinline__ PfItem get(int64_t item, const QueryArgs& a) const {
    const int tiles = (a.nq + kPfQueries - 1) / kPfQueries;
    const int64_t bh_count = a.items / tiles;
    PfItem it;
    it.tile = tiles - 1 - int(item / bh_count);
    const int64_t bh = item - int64_t(tiles - 1 - it.tile) * bh_count;
    const int b = int(bh / a.g.heads);
    it.head = int(bh - int64_t(b) * a.g.heads);
    it.nq = a.nq;
    it.offset = a.offset;
    it.q0 = b * a.q_b + it.head * a.q_h;
    it.o0 = b * a.o_b + it.head * a.o_h;
    it.table_row = a.table + int64_t(b) * a.g.columns;
    it.kb0 = 0; it.kb1 = kAllKeyBlocks; it.slot = -1;
    return it;
  }
};

// Prompts of different lengths in one launch (token-major rows, prompt r at
// rows [first_row[r], first_row[r] + n[r]) of q/k/v/out, with its own table
// row and key offset), passed by value: every (prompt, tile) pair in the
// order of pair_prompt / pair_tile (heaviest first), times the heads.
#ifndef MT_RAGGED_SHARE
#define MT_RAGGED_SHARE 2  // workgroups per compute unit that a ragged launch's key blocks are shared over
#endif
#ifndef MT_RAGGED_KEY_SPLIT
#define MT_RAGGED_KEY_SPLIT 1
#endif
constexpr int kRaggedPrompts = 16;
constexpr int kRaggedTiles = 256;
struct RaggedItems {
  int prompts, pairs;
  int first_row[kRaggedPrompts], n[kRaggedPrompts], offset[kRaggedPrompts];
  const int* table[kRaggedPrompts];
  unsigned char pair_prompt[kRaggedTiles];
  unsigned short pair_tile[kRaggedTiles];
  // Key blocks [kb0, kb1) of the pair's tile and its partials slot (-1: the
  // pair covers all of the tile's keys and writes the output rows).
  unsigned short pair_kb0[kRaggedTiles], pair_kb1[kRaggedTiles];
  short pair_slot[kRaggedTiles];
  __device__ __forceinline__ int64_t count(const QueryArgs& a) const { return int64_t(pairs) * a.g.heads; }
  __device__ __forceinline__ PfItem get(int64_t item, const QueryArgs& a) const {
    const int p = int(item / a.g.heads);
    const int r = pair_prompt[p];
    PfItem it;
    it.tile = pair_tile[p];
    it.head = int(item - int64_t(p) * a.g.heads);
    it.nq = n[r];
    it.offset = offset[r];
    it.q0 = int64_t(first_row[r]) * a.q_r + it.head * a.q_h;
    it.o0 = int64_t(first_row[r]) * a.o_r + it.head * a.o_h;
    it.table_row = table[r];
    it.slot = pair_slot[p];
    it.kb0 = it.slot >= 0 ? pair_kb0[p] : 0;
    it.kb1 = it.slot >= 0 ? pair_kb1[p] : kAllKeyBlocks;
    return it;
  }
};

// One request (QueryArgs with batch 1) whose long query tiles have their
// keys split over several workgroups: (tile, key blocks [kb0, kb1), slot)
// per pair, heaviest first, times the heads. A tile with one split writes its
// output; the splits of the others write partials for prefill_merge_kernel.
constexpr int kSplitPairs = 256;
struct SplitItems {
  int pairs;
  unsigned short tile[kSplitPairs], kb0[kSplitPairs], kb1[kSplitPairs];
  short slot[kSplitPairs];
  __device__ __forceinline__ int64_t count(const QueryArgs& a) const { return int64_t(pairs) * a.g.heads; }
  __device__ __forceinline__ PfItem get(int64_t item, const QueryArgs& a) const {
    const int p = int(item / a.g.heads);
    PfItem it;
    it.tile = tile[p];
    it.head = int(item - int64_t(p) * a.g.heads);
    it.nq = a.nq;
    it.offset = a.offset;
    it.q0 = it.head * a.q_h;
    it.o0 = it.head * a.o_h;
    it.table_row = a.table;
    it.kb0 = kb0[p]; it.kb1 = kb1[p]; it.slot = slot[p];
    return it;
  }
};

template <int DT, int D, class Items, bool FUSED>
__global__ __launch_bounds__(kThreads) void prefill_kernel(QueryArgs a, Items items) {
  using T = typename Elem<DT>::T;
  using V8 = typename Mfma<DT>::v8;
  constexpr int KS = kPfKeys;
  constexpr int KP = D + 8;     // LDS row of K, padded (elements)
  constexpr int VP = KS + 8;    // LDS row of V^T, padded
  constexpr int DT16 = D / 16;  // 16-dim tiles of the output
  constexpr int DS = D / 32;    // 32-dim steps of q.k
  constexpr int CPR = D / 8;    // 16-byte chunks per key row
  constexpr int NC = KS * CPR / kThreads;  // chunks per thread and plane
  static_assert(NC * kThreads == KS * CPR, "block staging must divide over the workgroup");
  __shared__ const T* s_page[kPfWindowPages];
  __shared__ __align__(16) T s_k[KS][KP];
  __shared__ __align__(16) T s_vt[D][VP];

  const Geometry& g = a.g;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & (kWave - 1);
  const int grp = lane >> 4;  // 0..3
  const int col = lane & 15;  // this lane's query within its wave's 16
  const T* qp = static_cast<const T*>(a.q);
  T* out = static_cast<T*>(a.out);
  const int win_keys = kPfWindowPages << g.log2_page;

  const int64_t n_items = items.count(a);
  for (int64_t item = blockIdx.x; item < n_items; item += gridDim.x) {
    const PfItem it = items.get(item, a);
    const int tile = it.tile, head = it.head;
    const int* table_row = it.table_row;
    const int nq = it.nq, offset = it.offset, nk = it.offset + it.nq;

    // B operand of S^T = K Q^T: dims [32*ds + 8*grp, +8) of query q0 + col.
    const int q0 = tile * kPfQueries + wave * 16;
    const int qi = q0 + col;
    const bool q_ok = qi < nq;
    V8 qv[DS];
    {
      const T* row = qp + it.q0 + (q_ok ? qi : 0) * a.q_r;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        qv[ds] = __builtin_bit_cast(V8, *global_view(reinterpret_cast<const u32x4*>(row + 32 * ds + 8 * grp)));
    }
    const int qpos = offset + qi;
    const bool wave_live = q0 < nq;
    const int wave_last = offset + (q0 + 15 < nq ? q0 + 15 : nq - 1);
    const int tile_q = (tile + 1) * kPfQueries - 1 < nq ? (tile + 1) * kPfQueries - 1 : nq - 1;
    const int kend = offset + tile_q + 1 < nk ? offset + tile_q + 1 : nk;

    float m = -INFINITY, l = 0.f;
    floatx4 o[DT16];
#pragma unroll
    for (int dt = 0; dt < DT16; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Staging of a 64-key block: K row-major, V transposed. Keys past the
    // window are zero; a missing page is NaN in K (so its score is NaN) and
    // zero in V (so a query that does not attend it is unaffected). The loads
    // are issued unconditionally (from this lane's query row when the key has
    // no page) and the substitution happens at the LDS store, so that no
    // branch waits for them before the block in between is computed.
    u32x4 kx[NC], vx[NC];
    int kstate[NC];  // 0 = loaded, 1 = missing page, 2 = past the window
    T* wpage[NC];    // page address a staged key of this tile is also written to, or null
    const T* dummy = qp + it.q0 + (q_ok ? qi : 0) * a.q_r;
    // FUSED: keys [offset, nk) come from the prompt's own K/V rows, and this
    // workgroup writes the keys of its own queries, [own0, kend), to the pages.
    const T* krows = FUSED ? static_cast<const T*>(a.k) + it.q0 : nullptr;
    const T* vrows = FUSED ? static_cast<const T*>(a.v) + it.q0 : nullptr;
    const int own0 = offset + tile * kPfQueries;
    auto stage_load = [&](int k0, int w0, int w1) {
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        const int c = tid + n * kThreads;
        const int kr = c / CPR, part = c - kr * CPR;
        const int key = k0 + kr;
        const T* page = key < w1 ? s_page[(key - w0) >> g.log2_page] : nullptr;
        kstate[n] = key >= w1 ? 2 : (page ? 0 : 1);
        const T* pk = page ? page + (key & (g.page_size - 1)) * D + part * 8 : nullptr;
        if constexpr (FUSED) {
          const bool fresh = key >= offset && key < w1;
          const T* kp = fresh ? krows + int64_t(key - offset) * a.q_r + part * 8 : (pk ? pk : dummy);
          const T* vp = fresh ? vrows + int64_t(key - offset) * a.q_r + part * 8 : (pk ? pk + g.kind_stride : dummy);
          wpage[n] = fresh && pk && key >= own0 ? const_cast<T*>(pk) : nullptr;
          kx[n] = *global_view(reinterpret_cast<const u32x4*>(kp));
          vx[n] = *global_view(reinterpret_cast<const u32x4*>(vp));
        } else {
          const T* kp = pk ? pk : dummy;
          const int64_t vstep = pk ? g.kind_stride : 0;
          kx[n] = *global_view(reinterpret_cast<const u32x4*>(kp));
          vx[n] = *global_view(reinterpret_cast<const u32x4*>(kp + vstep));
        }
      }
    };
    auto stage_store = [&]() {
#pragma unroll
      for (int n = 0; n < NC; ++n) {
        const int c = tid + n * kThreads;
        const int kr = c / CPR, part = c - kr * CPR;
        const uint32_t kfill = kstate[n] == 1 ? ~0u : 0u;
        const bool ok = kstate[n] == 0;
        const u32x4 kk = ok ? kx[n] : u32x4{kfill, kfill, kfill, kfill};
        *reinterpret_cast<u32x4*>(&s_k[kr][part * 8]) = kk;
        const uint32_t vw[4] = {ok ? vx[n].x : 0u, ok ? vx[n].y : 0u, ok ? vx[n].z : 0u, ok ? vx[n].w : 0u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          s_vt[part * 8 + 2 * j][kr] = static_cast<T>(vw[j] & 0xffffu);
          s_vt[part * 8 + 2 * j + 1][kr] = static_cast<T>(vw[j] >> 16);
        }
        if constexpr (FUSED) {
          if (wpage[n]) {  // a key of this tile's own tokens: its page copy
            *global_view(reinterpret_cast<u32x4*>(wpage[n])) = kx[n];
            *global_view(reinterpret_cast<u32x4*>(wpage[n] + g.kind_stride)) = vx[n];
          }
        }
      }
    };
    // This item's keys: blocks [kb0, kb1) of [0, kend).
    const int kstart = it.kb0 * KS;
    const int kstop = it.kb1 >= (kend + KS - 1) / KS ? kend : it.kb1 * KS;
    for (int w0 = kstart; w0 < kstop; w0 += win_keys) {
      const int w1 = w0 + win_keys < kstop ? w0 + win_keys : kstop;
      const int npg = (w1 - w0 + g.page_size - 1) >> g.log2_page;
      __syncthreads();
      for (int j = tid; j < npg; j += kThreads)
        s_page[j] = page_base<T>(a.slabs, table_row, (w0 >> g.log2_page) + j, g, head);
      __syncthreads();
      stage_load(w0, w0, w1);
      for (int k0 = w0; k0 < w1; k0 += KS) {
        if (k0 > w0) __syncthreads();  // every wave is done with the previous block
        stage_store();
        __syncthreads();
        // The next block's loads are in flight while this one is computed.
        if (k0 + KS < w1) stage_load(k0 + KS, w0, w1);
        if (!wave_live || k0 > wave_last) continue;

        // Scores: lane holds keys k0 + 16*kt + 4*grp + i of query qi.
        floatx4 sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          sc[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ds = 0; ds < DS; ++ds) {
            const V8 kk = __builtin_bit_cast(V8, *reinterpret_cast<const u32x4*>(&s_k[16 * kt + col][32 * ds + 8 * grp]));
            sc[kt] = Mfma<DT>::run(kk, qv[ds], sc[kt]);
          }
        }
        // Causal / length mask, only for blocks that reach past the wave's
        // first query or past kend (a wave-uniform test).
        if (k0 + KS - 1 > offset + q0 || k0 + KS > kend) {
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = k0 + 16 * kt + 4 * grp + i;
              if (key > qpos || key >= kend) sc[kt][i] = -INFINITY;
            }
          }
        }
        // Block max of the raw scores (qscale > 0 commutes with the max; NaN
        // scores are dropped by fmaxf), shared by the four lanes of a query.
        float bmax = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          bmax = fmaxf(fmaxf(bmax, fmaxf(sc[kt][0], sc[kt][1])), fmaxf(sc[kt][2], sc[kt][3]));
        bmax = fmaxf(bmax, lane_swap16(bmax));
        bmax = fmaxf(bmax, lane_swap32(bmax));
        const float mn = fmaxf(m, bmax * a.qscale);
        const float alpha = (m == -INFINITY) ? 0.f : fast_exp2(m - mn);
        const float mref = (mn == -INFINITY) ? 0.f : mn;  // masked scores give exp2(-inf) = 0
        // B operand of the PV step: k slot j of 32-key step ks holds key
        // 32*ks + 4*grp + j (j < 4) or 32*ks + 16 + 4*grp + (j - 4). The
        // denominator stays per lane (this lane's 16 keys) until the end.
        uint32_t phi[2][4], plo[2][4];
        float psum = 0.f;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
          for (int i = 0; i < 4; i += 2) {
            const float p0 = fast_exp2(fmaf(sc[kt][i], a.qscale, -mref));
            const float p1 = fast_exp2(fmaf(sc[kt][i + 1], a.qscale, -mref));
            psum += p0 + p1;
            const int ks = kt >> 1, w = (kt & 1) * 2 + (i >> 1);
            float r0, r1;
            phi[ks][w] = PackP<DT>::pack(p0, p1, r0, r1);
            plo[ks][w] = PackP<DT>::pack(p0 - r0, p1 - r1, r0, r1);
          }
        }
        l = l * alpha + psum;
        m = mn;
        V8 pv[2], pl[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          pv[ks] = __builtin_bit_cast(V8, u32x4{phi[ks][0], phi[ks][1], phi[ks][2], phi[ks][3]});
          pl[ks] = __builtin_bit_cast(V8, u32x4{plo[ks][0], plo[ks][1], plo[ks][2], plo[ks][3]});
        }
#pragma unroll
        for (int dt = 0; dt < DT16; ++dt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) o[dt][i] *= alpha;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            // A = V^T rows dt*16 + col, keys in pv's k-slot order.
            const T* vrow = &s_vt[dt * 16 + col][32 * ks + 4 * grp];
            const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
            const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16);
            const V8 va = __builtin_bit_cast(V8, u32x4{lo.x, lo.y, hi.x, hi.y});
            o[dt] = Mfma<DT>::run(va, pv[ks], o[dt]);
            o[dt] = Mfma<DT>::run(va, pl[ks], o[dt]);
          }
        }
      }
    }

    // The query's denominator is the sum over its four lanes.
    l += lane_swap16(l);
    l += lane_swap32(l);
    if (q_ok && it.slot >= 0) {
      // A split of the tile's keys: (max, denominator, accumulators) in
      // base-2 units for prefill_merge_kernel.
      float* part = a.partials + ((int64_t(it.slot) * g.heads + head) * kPfQueries + wave * 16 + col) * pf_part_row<D>();
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt)
        *reinterpret_cast<float4*>(part + dt * 16 + 4 * grp) = float4{o[dt][0], o[dt][1], o[dt][2], o[dt][3]};
      if (grp == 0) *reinterpret_cast<float2*>(part + D) = float2{m, l};
    }
    // O^T lane layout: dims dt*16 + 4*grp + i of query qi.
    if (q_ok && it.slot < 0) {
      T* orow = out + it.o0 + qi * a.o_r;
#pragma unroll
      for (int dt = 0; dt < DT16; ++dt) {
        const T r0 = from_f32<DT>(finalize(o[dt][0], l)), r1 = from_f32<DT>(finalize(o[dt][1], l));
        const T r2 = from_f32<DT>(finalize(o[dt][2], l)), r3 = from_f32<DT>(finalize(o[dt][3], l));
        *reinterpret_cast<uint2*>(orow + dt * 16 + 4 * grp) =
            uint2{uint32_t(r0) | (uint32_t(r1) << 16), uint32_t(r2) | (uint32_t(r3) << 16)};
      }
    }
  }
}

// Merge of a split prefill (one request): for each split tile, every query's
// outputs from its splits' (max, denominator, accumulators) by the log-sum-exp
// rule, with the finalize rule of the unsplit kernel (a NaN denominator stays
// NaN, a zero one gives 0). One workgroup per (tile, head), four threads per
// query, each taking every fourth 16-byte chunk of the row; one online pass
// over the splits, unrolled so that several splits' loads are in flight.
struct PrefillMerge {
  int tiles;
  unsigned short tile[kSplitPairs], first_slot[kSplitPairs];
  unsigned char splits[kSplitPairs];
};

// Key splits of ragged prompts: per split tile, its first output row (in the
// launch's rows), its valid queries, first partials slot and split count.
struct RaggedMerge {
  int tiles;
  int row0[kSplitPairs];
  unsigned short nq[kSplitPairs], first_slot[kSplitPairs];
  unsigned char splits[kSplitPairs];
};

// Query q of a split tile: log-sum-exp merge of the n partials from slot
// first_slot on, written to orow (256 threads: 64 queries x 4 column groups).
template <int DT, int D>
__device__ __forceinline__ void merge_query(const QueryArgs& a, int head, int q, int sub, int first_slot, int n,
                                            typename Elem<DT>::T* orow) {
  using T = typename Elem<DT>::T;
  constexpr int R = pf_part_row<D>(), C = D / 16;
  const float* base = a.partials + ((int64_t(first_slot) * a.g.heads + head) * kPfQueries + q) * R;
  const int64_t step = int64_t(a.g.heads) * kPfQueries * R;
  float M = -INFINITY, L = 0.f;
  float4 acc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) acc[c] = float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int s = 0; s < n; ++s) {
    const float* p = base + s * step;
    const float2 ml = *reinterpret_cast<const float2*>(p + D);
    float4 x[C];
#pragma unroll
    for (int c = 0; c < C; ++c) x[c] = *reinterpret_cast<const float4*>(p + 4 * (sub + 4 * c));
    const float Mn = fmaxf(M, ml.x);
    const float wo = M == -INFINITY ? 0.f : fast_exp2(M - Mn);
    const float wn = ml.x == -INFINITY ? 0.f : fast_exp2(ml.x - Mn);
    L = fmaf(L, wo, ml.y * wn);  // a NaN denominator (missing page) poisons the sum
#pragma unroll
    for (int c = 0; c < C; ++c) {
      acc[c].x = fmaf(acc[c].x, wo, x[c].x * wn);
      acc[c].y = fmaf(acc[c].y, wo, x[c].y * wn);
      acc[c].z = fmaf(acc[c].z, wo, x[c].z * wn);
      acc[c].w = fmaf(acc[c].w, wo, x[c].w * wn);
    }
    M = Mn;
  }
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const T r0 = from_f32<DT>(finalize(acc[c].x, L)), r1 = from_f32<DT>(finalize(acc[c].y, L));
    const T r2 = from_f32<DT>(finalize(acc[c].z, L)), r3 = from_f32<DT>(finalize(acc[c].w, L));
    *reinterpret_cast<uint2*>(orow + 4 * (sub + 4 * c)) =
        uint2{uint32_t(r0) | (uint32_t(r1) << 16), uint32_t(r2) | (uint32_t(r3) << 16)};
  }
}

template <int DT, int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(QueryArgs a, PrefillMerge mg) {
  using T = typename Elem<DT>::T;
  const int t = int(blockIdx.x / unsigned(a.g.heads));
  const int head = int(blockIdx.x - unsigned(t) * a.g.heads);
  if (t >= mg.tiles) return;
  const int q = threadIdx.x >> 2, sub = threadIdx.x & 3;
  const int qi = mg.tile[t] * kPfQueries + q;
  if (qi >= a.nq) return;
  T* orow = static_cast<T*>(a.out) + head * a.o_h + int64_t(qi) * a.o_r;
  merge_query<DT, D>(a, head, q, sub, mg.first_slot[t], mg.splits[t], orow);
}

// Kernel arguments stay within the 4 KiB kernarg limit.
static_assert(sizeof(QueryArgs) + sizeof(RaggedItems) <= 4096, "ragged prefill arguments");
static_assert(sizeof(QueryArgs) + sizeof(RaggedMerge) <= 4096, "ragged merge arguments");

template <int DT, int D>
__global__ __launch_bounds__(256) void ragged_merge_kernel(QueryArgs a, RaggedMerge mg) {
  using T = typename Elem<DT>::T;
  const int t = int(blockIdx.x / unsigned(a.g.heads));
  const int head = int(blockIdx.x - unsigned(t) * a.g.heads);
  if (t >= mg.tiles) return;
  const int q = threadIdx.x >> 2, sub = threadIdx.x & 3;
  if (q >= mg.nq[t]) return;
  T* orow = static_cast<T*>(a.out) + head * a.o_h + (int64_t(mg.row0[t]) + q) * a.o_r;
  merge_query<DT, D>(a, head, q, sub, mg.first_slot[t], mg.splits[t], orow);
}

// Multi-token append at a common offset (reference paged_append with
// offsets == nullptr, src/paged_attention_kernel.cu:23-33): K/V[b,h,pos,:]
// goes to token offset + pos of request b; rows whose page is missing are
// skipped. VEC moves 16 bytes per thread.
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
  using T = typename Elem<DT>::T;
  constexpr int E = VEC ? per16<DT>() : 1;
  const Geometry& g = a.g;
  const int dim = g.dim;
  const int per_row = dim / E;
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < a.vectors;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t row = i / per_row;  // (b*h + head)*n + pos
    const int col = int(i - row * per_row) * E;
    const int64_t bhh = row / a.n;
    const int pos_in = int(row - bhh * a.n);
    const int b = int(bhh / g.heads), head = int(bhh - int64_t(b) * g.heads);
    const int64_t pos = int64_t(a.offset) + pos_in;
    const T* base = page_base<T>(a.slabs, a.table + int64_t(b) * g.columns, pos >> g.log2_page, g, head);
    if (!base) continue;
    T* kp = const_cast<T*>(base) + (pos & (g.page_size - 1)) * dim + col;
    T* vp = kp + g.kind_stride;
    const int64_t src = b * a.src_b + head * a.src_h + pos_in * a.src_r + col;
    if constexpr (VEC) {
      *global_view(reinterpret_cast<u32x4*>(kp)) = *global_view(reinterpret_cast<const u32x4*>(static_cast<const T*>(a.k) + src));
      *global_view(reinterpret_cast<u32x4*>(vp)) = *global_view(reinterpret_cast<const u32x4*>(static_cast<const T*>(a.v) + src));
    } else {
      *kp = static_cast<const T*>(a.k)[src];
      *vp = static_cast<const T*>(a.v)[src];
    }
  }
}

// Shape guard of the reference (src/paged_attention_kernel.cu:87-94 and
// src/includes/flash_common.cuh:17-20): the same inputs are rejected.
bool paged_shape(int b, int h, int nq, int nk, int d, int page_size, int pps, int num_slabs,
                 int columns, int layer, int layers, int offset) {
  return b > 0 && h > 0 && nq > 0 && nk > 0 && d > 0 && d <= 128 &&
         int64_t(b) * h * nq * d <= INT32_MAX && int64_t(b) * h * nk * d <= INT32_MAX &&
         int64_t(b) * h <= 65535 && (page_size == 8 || page_size == 16 || page_size == 32) &&
         pps > 0 && num_slabs > 0 && int64_t(pps) * num_slabs <= INT32_MAX && columns > 0 &&
         int64_t(b) * columns <= INT32_MAX && nk <= int64_t(columns) * page_size && layers > 0 &&
         layer >= 0 && layer < layers && offset >= 0 && int64_t(offset) + nq == nk;
}

Geometry make_geometry(int h, int d, int page_size, int pps, int num_slabs, int columns, int layer) {
  Geometry g{};
  g.heads = h; g.dim = d; g.page_size = page_size;
  g.log2_page = page_size == 8 ? 3 : page_size == 16 ? 4 : 5;
  g.pps = pps; g.num_slabs = num_slabs; g.columns = columns; g.layer = layer;
  int sh = 0;
  while ((int64_t(1) << sh) < pps) ++sh;
  g.pps_shift = 31 + sh;
  g.pps_magic = ((uint64_t(1) << (31 + sh)) + uint64_t(pps) - 1) / uint64_t(pps);
  g.kind_stride = int64_t(pps) * h * page_size * d;
  return g;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int64_t kMaxGrid = int64_t(1) << 30;

int grid_for(int64_t items) { return int(items < kMaxGrid ? items : kMaxGrid); }

// Split length for a decode launch: kDefaultSplitTokens unless the longest
// possible context (columns * page_size) would need more than
// kMaxSplitsPerRow splits, then longer splits (multiple of 64, at most 2048).
int choose_split(int64_t cap, int requested) {
  if (requested > 0) return requested;
  int64_t s = kDefaultSplitTokens;
  if ((cap + s - 1) / s > kMaxSplitsPerRow) {
    s = (cap + kMaxSplitsPerRow - 1) / kMaxSplitsPerRow;
    s = (s + 63) / 64 * 64;
    if (s > kMaxSplitTokens) s = kMaxSplitTokens;
  }
  return int(s);
}

size_t workspace_bytes_for(int64_t bh, int nsplit_max) {
  // (max, denominator, accumulator[128]) per (row, head, split)
  return size_t(bh) * nsplit_max * (128 + 2) * sizeof(float);
}

// Whether the decode runs its 16-byte-load kernel for these operands.
bool decode_vec(int d, int dtype, const void* out, const void* q, const void* k, const void* v,
                int64_t qkv_stride) {
  return (d == 64 || d == 128) && aligned16(out) && aligned16(q) && aligned16(k) && aligned16(v) &&
         (qkv_stride * (dtype == kF32 ? 4 : 2)) % 16 == 0;
}

// Bytes of split partials a decode launch writes: (max, denominator,
// accumulator[D]) per (row, head, split), D being the kernel's head-dim
// template (64 for the 16-byte kernel at d = 64, else 128).
size_t partial_bytes(int64_t bh, int64_t nsplit_max, bool vec, int d) {
  const int dt = (vec && d == 64) ? 64 : 128;
  return size_t(bh) * size_t(nsplit_max) * size_t(dt + 2) * sizeof(float);
}

// Compute units of the current device (cached per device).
int device_compute_units() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

// A wave resolves the page of each of its steps into one lane, so a split
// may give a wave at most 64 steps (32 when a step spans two pages): 2-wave
// workgroups take splits of at most 1024 tokens (512 for pages below 8).
bool two_wave_split_ok(const DecodeArgs& a) {
  constexpr int RB = kWave / kDecodeGroup;  // tokens per wave step
  const int steps = a.split_tokens / RB / 2;
  return a.split_tokens % (2 * RB) == 0 && steps * (a.g.page_size < RB ? 2 : 1) <= kWave;
}

// Workgroups of decode_kernel<DT, D, VEC, U, kStages, WAVES, G> resident per
// compute unit (0 if the query fails), looked up once per instantiation.
template <int DT, int D, bool VEC, int U, int WAVES, int G>
int decode_occupancy() {
  static const int per_cu = [] {
    int n = 0;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_kernel<DT, D, VEC, U, kStages, WAVES, G, kVisitList>,
                                                        WAVES * kWave, 0) == hipSuccess ? n : 0;
  }();
  return per_cu;
}

// The instantiation of the launch's visiting mode.
template <int DT, int D, bool VEC, int U, int WAVES, int G>
void launch_decode_mode(const DecodeArgs& a, int64_t blocks, size_t lds) {
  constexpr int NT = WAVES * kWave;
  if (a.work) decode_kernel<DT, D, VEC, U, kStages, WAVES, G, kVisitList><<<grid_for(blocks), NT, lds>>>(a);
  else if (a.rank_rows) decode_kernel<DT, D, VEC, U, kStages, WAVES, G, kVisitRank><<<grid_for(blocks), NT, lds>>>(a);
  else decode_kernel<DT, D, VEC, U, kStages, WAVES, G, kVisitGrid><<<grid_for(blocks), NT, lds>>>(a);
}

template <int DT, int D, bool VEC, int WAVES, int G>
hipError_t launch_decode_w(const DecodeArgs& a, int64_t blocks, int unroll) {
  // Row bytes per lane bound the useful unroll: register stages beyond it spill.
  constexpr int kMaxUnroll = !VEC ? 1 : (D * elem_bytes<DT>() >= 256 ? 2 : 4);
  constexpr int NT = WAVES * kWave;
  if (unroll == 0) {
    if constexpr (G == 8) {
      // Two row-blocks per register stage: measured best or within 1 % of
      // the best at every decode shape of configs 2, 4 and 5.
      unroll = 2;
    } else if constexpr (kMaxUnroll >= 4) {
      // The deepest unroll when the whole grid is resident at its
      // occupancy (more loads in flight per wave), else unroll 1, whose
      // lower register count keeps the most workgroups per compute unit.
      unroll = blocks <= int64_t(decode_occupancy<DT, D, VEC, 4, WAVES, G>()) * device_compute_units() ? 4 : 1;
    } else {
      unroll = 1;
    }
  }
  // Requests between the supported values round down (3 -> 2, 5+ -> 4).
  unroll = unroll >= 4 ? 4 : unroll >= 2 ? 2 : 1;
  const size_t rank_lds = a.rank_rows ? size_t(2) * ((a.batch + 3) & ~3) * sizeof(int) : 0;
  if (unroll > kMaxUnroll) unroll = kMaxUnroll;
  if (a.work_count) {
    // A device-built list of unknown length: one residency round of
    // workgroups strides over it.
    int occ = 0;
    if (unroll == 4) occ = decode_occupancy<DT, D, VEC, (kMaxUnroll >= 4 ? 4 : 1), WAVES, G>();
    else if (unroll == 2) occ = decode_occupancy<DT, D, VEC, (kMaxUnroll >= 2 ? 2 : 1), WAVES, G>();
    else occ = decode_occupancy<DT, D, VEC, 1, WAVES, G>();
    const int64_t resident = int64_t(occ > 0 ? occ : 1) * std::max(1, device_compute_units());
    blocks = std::min(blocks, resident);
  }
  if constexpr (kMaxUnroll >= 4) {
    if (unroll == 4) launch_decode_mode<DT, D, VEC, 4, WAVES, G>(a, blocks, rank_lds);
  }
  if constexpr (kMaxUnroll >= 2) {
    if (unroll == 2) launch_decode_mode<DT, D, VEC, 2, WAVES, G>(a, blocks, rank_lds);
  }
  if (unroll == 1) launch_decode_mode<DT, D, VEC, 1, WAVES, G>(a, blocks, rank_lds);
  hipError_t e = hipGetLastError();
  const int64_t merge_rows = a.work && !a.work_count ? a.merge_rows : a.batch;
  if (e != hipSuccess || a.nsplit_max == 1 || merge_rows == 0) return e;
  int64_t merge_blocks = merge_rows * a.g.heads;
  // Device-built list: the merge rows' count is on the device; a grid of
  // four workgroups per compute unit strides over them.
  if (a.work_count) merge_blocks = std::min(merge_blocks, 4 * int64_t(std::max(1, device_compute_units())));
  merge_kernel<DT, (D > 64 ? 128 : 64)><<<grid_for(merge_blocks), 128>>>(a);
  return hipGetLastError();
}

// waves 0 = automatic: 8-wave workgroups when the whole grid is resident at
// their occupancy (a (row, head) streamed by 8 waves finishes its longest
// rows sooner; config 2: 21.0 us vs 21.9 us with 4), else 4 (more
// workgroups per compute unit for grids of several residency rounds;
// config 5: 256 us vs 267 us with 8), and 2 when even 2-wave workgroups take
// more than two residency rounds (finer-grained hand-out of the tail; config
// 5: 261-263 us vs 267 us with 4; config 4's layer, 2048 workgroups that 2
// waves would make resident at once, took 9 % longer per step with 2).
template <int DT, int D, bool VEC>
hipError_t launch_decode_t(const DecodeArgs& a, int64_t blocks, int unroll, int waves) {
  constexpr int G = kDecodeGroup;
  constexpr int U8 = VEC && G == 8 ? 2 : 1;
  if (waves == 0) {
    const int64_t cus = device_compute_units();
    waves = blocks <= int64_t(decode_occupancy<DT, D, VEC, U8, 8, G>()) * cus ? 8 : 4;
    if (waves == 4 && two_wave_split_ok(a) && blocks > 2 * int64_t(decode_occupancy<DT, D, VEC, U8, 2, G>()) * cus)
      waves = 2;
  }
  if (a.split_tokens % ((kWave / G) * waves) != 0 || (waves == 2 && !two_wave_split_ok(a))) waves = 4;
  if (waves == 8) return launch_decode_w<DT, D, VEC, 8, G>(a, blocks, unroll);
  if (waves == 2) return launch_decode_w<DT, D, VEC, 2, G>(a, blocks, unroll);
  return launch_decode_w<DT, D, VEC, 4, G>(a, blocks, unroll);
}

template <int DT>
hipError_t launch_decode_dt(const DecodeArgs& a, int64_t blocks, bool vec, int d, int unroll, int waves) {
  if (vec && d == 64) return launch_decode_t<DT, 64, true>(a, blocks, unroll, waves);
  if (vec && d == 128) return launch_decode_t<DT, 128, true>(a, blocks, unroll, waves);
  return launch_decode_t<DT, 128, false>(a, blocks, 1, waves);
}

int decode_common(void* out, const void* q, const void* k, const void* v, const uint64_t* slabs,
                  const int* table, const int* offsets, int b, int h, int d, int page_size,
                  int pps, int num_slabs, int columns, int layer, int layers, int dtype,
                  int split_tokens, int unroll, int waves, int qkv_stride, const int* work,
                  int work_items, int merge_rows, void* workspace, size_t workspace_bytes,
                  bool rank_order = false, int* order = nullptr) {
  const int64_t cap = int64_t(columns) * page_size;
  // A work list is built for one split length, so it must be given.
  if (work && split_tokens <= 0) return hipErrorInvalidValue;
  const int S = choose_split(cap, split_tokens);
  if (S < 64 || S % 64 != 0 || S > kMaxSplitTokens) return hipErrorInvalidValue;
  if (waves != 0 && waves != 2 && waves != 4 && waves != 8) return hipErrorInvalidValue;
  const int64_t nsplit_max = (cap + S - 1) / S;
  const int64_t bh = int64_t(b) * h;
  if (nsplit_max > INT_MAX) return hipErrorInvalidValue;
  if (work && (work_items < 0 || merge_rows < 0 || merge_rows > b ||
               work_items > int64_t(b) * nsplit_max || (reinterpret_cast<uintptr_t>(work) & 7u)))
    return hipErrorInvalidValue;
  if (work && work_items == 0) return hipSuccess;
  const int64_t stride = qkv_stride ? qkv_stride : int64_t(h) * d;
  const bool vec = decode_vec(d, dtype, out, q, k, v, stride);
  if (nsplit_max > 1 && (!workspace || workspace_bytes < partial_bytes(bh, nsplit_max, vec, d)))
    return hipErrorInvalidValue;
  DecodeArgs a{};
  a.out = out; a.q = q; a.k = k; a.v = v; a.slabs = slabs; a.table = table; a.offsets = offsets;
  a.batch = b; a.split_tokens = S; a.nsplit_max = int(nsplit_max);
  a.qscale = (1.0f / std::sqrt(float(d))) * kLog2e;
  a.items = work ? int64_t(work_items) * h : bh * nsplit_max;
  // The kernels index items with 32-bit arithmetic.
  if (a.items > INT32_MAX) return hipErrorInvalidValue;
  a.g = make_geometry(h, d, page_size, pps, num_slabs, columns, layer);
  a.partials = static_cast<float*>(workspace);
  a.qkv_stride = stride;
  a.work = work;
  a.work_items = work ? work_items : 0;
  a.merge_rows = work ? merge_rows : 0;
  // Entries without a work list visit rows longest first when every row has
  // one split and the batch is small enough to rank in each workgroup.
  if (rank_order && !work && nsplit_max == 1 && b <= kRankRows) {
    a.rank_rows = 1;
    a.rank_per = std::max(1, device_compute_units() / h);
  } else if (rank_order && !work && order) {
    // Larger batches, and rows that may split: order_kernel writes the work
    // list a host caller would build (count, then the list) into `order`.
    OrderArgs oa{};
    oa.offsets = offsets; oa.count = order; oa.list = order + 2;
    oa.batch = b; oa.split_tokens = S; oa.cap = cap; oa.capacity = int(int64_t(b) * nsplit_max);
    oa.per = std::max(1, device_compute_units() / h);
    order_kernel<<<1, kOrderThreads>>>(oa);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    a.work = order + 2;
    if (nsplit_max > 1) {
      a.work_count = order;  // a.items stays the capacity, bh * nsplit_max
    } else {
      a.work_items = b;      // one entry per row
      a.items = bh;
    }
  }
  if (dtype == kF32) return launch_decode_dt<kF32>(a, a.items, vec, d, unroll, waves);
  if (dtype == kF16) return launch_decode_dt<kF16>(a, a.items, vec, d, unroll, waves);
  if (dtype == kBF16) return launch_decode_dt<kBF16>(a, a.items, vec, d, unroll, waves);
  return hipErrorInvalidValue;
}

// Whether the reference entries have order_kernel build their visiting
// order (batches past the in-workgroup ranking, or rows that may split, up to
// kOrderRows rows), and the bytes it writes: the count pair, the (row, split)
// list and the merge rows.
bool device_order(int b, int64_t nsplit_max) {
  return b <= kOrderRows && (nsplit_max > 1 || b > kRankRows) && int64_t(b) * nsplit_max <= INT32_MAX / 2;
}
size_t order_bytes(int b, int64_t nsplit_max) {
  return size_t(2 + 2 * int64_t(b) * nsplit_max + b) * sizeof(int);
}
size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Library-owned split workspace of the reference entry points, which have no
// workspace argument (mt_paged_decode_batch for tables longer than one split,
// the key-split prefill of mt_paged_attention / mt_paged_prefill). One buffer
// per (host thread, device): every launch of these libraries goes to the
// calling thread's default stream (they are built with per-thread default
// streams), so a buffer private to the thread is private to the stream its
// kernels run on, and calls from several host threads never share one. It
// grows stream-ordered on that stream: hipMallocAsync for the larger buffer
// and hipFreeAsync for the old one, which is released only after the work
// queued before it, so growing neither synchronizes the device nor blocks the
// host. A thread's buffers are released (stream-ordered) when it exits.
// Callers that cannot allocate use mt_paged_decode_split with their own
// workspace, or mt_paged_decode_batch_noalloc.
struct ThreadWorkspaces {
  std::vector<std::pair<void*, size_t>> per_device;
  ~ThreadWorkspaces() {
    int current = 0;
    if (hipGetDevice(&current) != hipSuccess) return;
    for (size_t dev = 0; dev < per_device.size(); ++dev) {
      if (!per_device[dev].first || hipSetDevice(int(dev)) != hipSuccess) continue;
      (void)hipFreeAsync(per_device[dev].first, hipStreamPerThread);
    }
    (void)hipSetDevice(current);
  }
};
thread_local ThreadWorkspaces t_workspaces;

int library_workspace(size_t bytes, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  auto& ws = t_workspaces.per_device;
  if (ws.size() <= size_t(dev)) ws.resize(dev + 1, {nullptr, 0});
  auto& slot = ws[dev];
  if (slot.second < bytes) {
    void* p = nullptr;
    e = hipMallocAsync(&p, bytes, hipStreamPerThread);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // the caller reports the status; keep it off the next launch
      return e;
    }
    if (slot.first) {
      e = hipFreeAsync(slot.first, hipStreamPerThread);
      if (e != hipSuccess) return e;
    }
    slot = {p, bytes};
  }
  *out = slot.first;
  return hipSuccess;
}

// Split partials of mt_paged_decode_batch_noalloc: a fixed device array, so
// that entry point allocates nothing. Every call on a device shares that
// device's copy. The decode writes every partial of a split row before the
// merge reads it, so nothing carries over between calls and nothing needs
// clearing; calls that overlap on one device (other streams) would race.
}  // namespace

static __device__ __align__(256) float scratch[MT_PAGED_NOALLOC_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr size_t kNoAllocScratchBytes = MT_PAGED_NOALLOC_SCRATCH_BYTES;

// Device address of `scratch` on the current device, looked up once per
// device (the host-side name of the array is not a device address).
int scratch_address(void** out) {
  static std::mutex mutex;
  static std::vector<void*> addresses;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mutex);
  if (addresses.size() <= size_t(dev)) addresses.resize(dev + 1, nullptr);
  if (!addresses[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    addresses[dev] = p;
  }
  *out = addresses[dev];
  return hipSuccess;
}

// Launch of the append kernel for any source strides; the 16-byte path needs
// 16-byte aligned rows.
hipError_t launch_append(AppendArgs& a, int dtype) {
  const int d = a.g.dim;
  const int esize = dtype == kF32 ? 4 : 2;
  const int E = 16 / esize;
  const bool vec = d % E == 0 && aligned16(a.k) && aligned16(a.v) &&
                   (a.src_b * esize) % 16 == 0 && (a.src_h * esize) % 16 == 0 &&
                   (a.src_r * esize) % 16 == 0;
  a.vectors = int64_t(a.batch) * a.g.heads * a.n * (vec ? d / E : d);
  const int blocks = int((a.vectors + 255) / 256 < 65536 * 16 ? (a.vectors + 255) / 256 : 65536 * 16);
#define MT_APPEND(DT)                                                        \
  if (vec) append_kernel<DT, true><<<blocks, 256>>>(a);                      \
  else append_kernel<DT, false><<<blocks, 256>>>(a);
  if (dtype == kF32) { MT_APPEND(kF32) }
  else if (dtype == kF16) { MT_APPEND(kF16) }
  else { MT_APPEND(kBF16) }
#undef MT_APPEND
  return hipGetLastError();
}

// Whether launch_query runs the matrix-core prefill kernel: fp16/bf16,
// head_dim 64/128, 16-byte aligned rows and at least kPfMinQueries queries.
bool prefill_kernel_takes(const QueryArgs& a, int dtype) {
  const int d = a.g.dim;
  const int esize = dtype == kF32 ? 4 : 2;
  auto rows16 = [&](int64_t x) { return (x * esize) % 16 == 0; };
  return (d == 64 || d == 128) && dtype != kF32 && a.nq >= kPfMinQueries && aligned16(a.out) &&
         aligned16(a.q) && rows16(a.q_b) && rows16(a.q_h) && rows16(a.q_r) && rows16(a.o_b) &&
         rows16(a.o_h) && rows16(a.o_r);
}

// Launches that took the key-split prefill path (a diagnostic for tests).
std::atomic<long long> g_key_split_launches{0};

// Key-split prefill of one request whose query tiles give at most one
// workgroup per compute unit and whose last tile walks many key blocks: each tile's keys are cut
// into splits of B blocks (B chosen for about two workgroups per compute
// unit), every split a workgroup, the splits then merged. Returns
// hipErrorNotSupported when the shape is better served unsplit.
hipError_t launch_split_prefill(QueryArgs& a, int dtype) {
  const int h = a.g.heads, d = a.g.dim;
  const int tiles = (a.nq + kPfQueries - 1) / kPfQueries;
  const int cus = device_compute_units();
  auto blocks_of = [&](int t) {
    const int64_t last = int64_t(a.offset) + std::min(int64_t(t + 1) * kPfQueries, int64_t(a.nq));
    return int((std::min<int64_t>(last, a.nk) + kPfKeys - 1) / kPfKeys);
  };
  if (a.batch != 1 || cus < 1 || int64_t(tiles) * h > cus || blocks_of(tiles - 1) < 6)
    return hipErrorNotSupported;
  int64_t total = 0;
  for (int t = 0; t < tiles; ++t) total += blocks_of(t);
  const int B = std::max<int>(2, int((total * h + 2 * cus - 1) / (2 * cus)));
  SplitItems it{};
  PrefillMerge mg{};
  int pairs = 0, slots = 0;
  for (int t = tiles - 1; t >= 0; --t) {  // heaviest tiles first
    const int nb = blocks_of(t), n = (nb + B - 1) / B;
    if (pairs + n > kSplitPairs || n > 255 || nb > 65535) return hipErrorNotSupported;
    if (n > 1) {
      mg.tile[mg.tiles] = static_cast<unsigned short>(t);
      mg.first_slot[mg.tiles] = static_cast<unsigned short>(slots);
      mg.splits[mg.tiles] = static_cast<unsigned char>(n);
      ++mg.tiles;
    }
    for (int s = 0; s < n; ++s) {
      it.tile[pairs] = static_cast<unsigned short>(t);
      it.kb0[pairs] = static_cast<unsigned short>(s * B);
      it.kb1[pairs] = static_cast<unsigned short>(std::min(nb, (s + 1) * B));
      it.slot[pairs] = static_cast<short>(n > 1 ? slots++ : -1);
      ++pairs;
    }
  }
  if (mg.tiles == 0) return hipErrorNotSupported;
  it.pairs = pairs;
  void* ws = nullptr;
  // Without room for the partials the prompt runs unsplit.
  if (library_workspace(size_t(slots) * h * kPfQueries * (d + 4) * sizeof(float), &ws) != hipSuccess)
    return hipErrorNotSupported;
  a.partials = static_cast<float*>(ws);
  const int blocks = grid_for(int64_t(pairs) * h);
#define MT_SPLIT(DT, D)                                                                        \
  if (a.k) prefill_kernel<DT, D, SplitItems, true><<<blocks, kThreads>>>(a, it);              \
  else prefill_kernel<DT, D, SplitItems, false><<<blocks, kThreads>>>(a, it);                 \
  prefill_merge_kernel<DT, D><<<unsigned(mg.tiles * h), 256>>>(a, mg);
  if (dtype == kF16) {
    if (d == 64) { MT_SPLIT(kF16, 64) }
    else { MT_SPLIT(kF16, 128) }
  } else {
    if (d == 64) { MT_SPLIT(kBF16, 64) }
    else { MT_SPLIT(kBF16, 128) }
  }
#undef MT_SPLIT
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) g_key_split_launches.fetch_add(1, std::memory_order_relaxed);
  return e;
}

// Causal attention launch for any q/out strides: the matrix-core prefill
// kernel where prefill_kernel_takes, the per-query kernel otherwise (which
// reads every key from the pages: a.k must then be null).
hipError_t launch_query(QueryArgs& a, int dtype) {
  const int d = a.g.dim;
  const int esize = dtype == kF32 ? 4 : 2;
  auto rows16 = [&](int64_t x) { return (x * esize) % 16 == 0; };
  const bool vec = (d == 64 || d == 128) && aligned16(a.out) && aligned16(a.q) && rows16(a.q_b) &&
                   rows16(a.q_h) && rows16(a.q_r) && rows16(a.o_b) && rows16(a.o_h) && rows16(a.o_r);
  a.qscale = (1.0f / std::sqrt(float(d))) * kLog2e;
  const int h = a.g.heads;
  if (prefill_kernel_takes(a, dtype)) {
    const hipError_t split = launch_split_prefill(a, dtype);
    if (split != hipErrorNotSupported) return split;
    a.items = int64_t(a.batch) * h * ((a.nq + kPfQueries - 1) / kPfQueries);
    const int blocks = grid_for(a.items);
#define MT_PREFILL(DT, D)                                                                   \
  if (a.k) prefill_kernel<DT, D, UniformItems, true><<<blocks, kThreads>>>(a, UniformItems{});   \
  else prefill_kernel<DT, D, UniformItems, false><<<blocks, kThreads>>>(a, UniformItems{});
    if (dtype == kF16) {
      if (d == 64) { MT_PREFILL(kF16, 64) }
      else { MT_PREFILL(kF16, 128) }
    } else {
      if (d == 64) { MT_PREFILL(kBF16, 64) }
      else { MT_PREFILL(kBF16, 128) }
    }
#undef MT_PREFILL
    return hipGetLastError();
  }
  if (a.k) return hipErrorInvalidValue;
  a.items = int64_t(a.batch) * h * ((a.nq + kWaves - 1) / kWaves);
  const int blocks = grid_for(a.items);
#define MT_QUERY(DT)                                                                   \
  if (vec && d == 64) query_kernel<DT, 64, true, 2><<<blocks, kThreads>>>(a);          \
  else if (vec && d == 128) query_kernel<DT, 128, true, 2><<<blocks, kThreads>>>(a);   \
  else query_kernel<DT, 128, false, 1><<<blocks, kThreads>>>(a);
  if (dtype == kF32) { MT_QUERY(kF32) }
  else if (dtype == kF16) { MT_QUERY(kF16) }
  else { MT_QUERY(kBF16) }
#undef MT_QUERY
  return hipGetLastError();
}

}  // namespace

extern "C" {

int mt_paged_append(const void* k, const void* v, const uint64_t* slabs, const int* table, int b,
                    int h, int n, int d, int page_size, int pages_per_slab, int num_slabs,
                    int columns, int layer, int layers, int offset, int dtype) {
  if (!k || !v || !slabs || !table) return hipErrorInvalidValue;
  if (int64_t(offset) + n > INT32_MAX ||
      !paged_shape(b, h, n, offset + n, d, page_size, pages_per_slab, num_slabs, columns, layer,
                   layers, offset))
    return hipErrorInvalidValue;
  if (dtype < 0 || dtype > 2) return hipErrorInvalidValue;
  AppendArgs a{};
  a.k = k; a.v = v; a.slabs = slabs; a.table = table; a.batch = b; a.n = n; a.offset = offset;
  a.g = make_geometry(h, d, page_size, pages_per_slab, num_slabs, columns, layer);
  a.src_b = int64_t(h) * n * d; a.src_h = int64_t(n) * d; a.src_r = d;
  return launch_append(a, dtype);
}

int mt_paged_attention(void* out, const void* q, const uint64_t* slabs, const int* table, int b,
                       int h, int nq, int nk, int d, int page_size, int pages_per_slab,
                       int num_slabs, int columns, int layer, int layers, int offset, int dtype) {
  if (!out || !q || !slabs || !table) return hipErrorInvalidValue;
  if (!paged_shape(b, h, nq, nk, d, page_size, pages_per_slab, num_slabs, columns, layer, layers,
                   offset))
    return hipErrorInvalidValue;
  if (dtype < 0 || dtype > 2) return hipErrorInvalidValue;
  QueryArgs a{};
  a.out = out; a.q = q; a.slabs = slabs; a.table = table;
  a.batch = b; a.nq = nq; a.nk = nk; a.offset = offset;
  a.g = make_geometry(h, d, page_size, pages_per_slab, num_slabs, columns, layer);
  a.q_b = a.o_b = int64_t(h) * nq * d;
  a.q_h = a.o_h = int64_t(nq) * d;
  a.q_r = a.o_r = d;
  return launch_query(a, dtype);
}

int mt_paged_prefill(void* out, const void* q, const void* k, const void* v, const uint64_t* slabs,
                     const int* table, int b, int h, int n, int d, int page_size,
                     int pages_per_slab, int num_slabs, int columns, int layer, int layers,
                     int offset, int dtype, int qkv_stride, int out_stride) {
  if (!out || !q || !k || !v || !slabs || !table) return hipErrorInvalidValue;
  const int64_t hd = int64_t(h) * d;
  if (qkv_stride == 0) qkv_stride = int(hd);
  if (out_stride == 0) out_stride = int(hd);
  if (int64_t(offset) + n > INT32_MAX || qkv_stride < hd || out_stride < hd ||
      int64_t(b) * n * qkv_stride > INT32_MAX || int64_t(b) * n * out_stride > INT32_MAX ||
      !paged_shape(b, h, n, offset + n, d, page_size, pages_per_slab, num_slabs, columns, layer,
                   layers, offset))
    return hipErrorInvalidValue;
  if (dtype < 0 || dtype > 2) return hipErrorInvalidValue;
  QueryArgs a{};
  a.out = out; a.q = q; a.slabs = slabs; a.table = table;
  a.batch = b; a.nq = n; a.nk = offset + n; a.offset = offset;
  a.g = make_geometry(h, d, page_size, pages_per_slab, num_slabs, columns, layer);
  a.q_b = int64_t(n) * qkv_stride; a.q_h = d; a.q_r = qkv_stride;
  a.o_b = int64_t(n) * out_stride; a.o_h = d; a.o_r = out_stride;
  if (prefill_kernel_takes(a, dtype) && aligned16(k) && aligned16(v)) {
    // The prefill kernel reads the new keys from k/v and writes them to
    // their pages itself: no separate append.
    a.k = k; a.v = v;
    return launch_query(a, dtype);
  }
  AppendArgs ap{};
  ap.k = k; ap.v = v; ap.slabs = slabs; ap.table = table; ap.batch = b; ap.n = n; ap.offset = offset;
  ap.g = a.g;
  ap.src_b = int64_t(n) * qkv_stride; ap.src_h = d; ap.src_r = qkv_stride;
  hipError_t e = launch_append(ap, dtype);
  if (e != hipSuccess) return e;
  return launch_query(a, dtype);
}

int mt_paged_prefill_ragged(void* out, const void* q, const void* k, const void* v,
                            const uint64_t* slabs, const int* const* tables, const int* tokens,
                            const int* offsets, int requests, int h, int d, int page_size,
                            int pages_per_slab, int num_slabs, int columns, int layer, int layers,
                            int dtype, int qkv_stride, int out_stride) {
  if (!out || !q || !k || !v || !slabs || !tables || !tokens || !offsets || requests < 1 || h < 1 ||
      d < 1 || dtype < 0 || dtype > 2)
    return hipErrorInvalidValue;
  const int64_t hd = int64_t(h) * d;
  if (qkv_stride == 0) qkv_stride = int(hd);
  if (out_stride == 0) out_stride = int(hd);
  if (qkv_stride < hd || out_stride < hd) return hipErrorInvalidValue;
  int64_t total = 0;
  for (int r = 0; r < requests; ++r) {
    if (!tables[r] || tokens[r] < 1 || offsets[r] < 0 || int64_t(offsets[r]) + tokens[r] > INT32_MAX ||
        !paged_shape(1, h, tokens[r], offsets[r] + tokens[r], d, page_size, pages_per_slab, num_slabs,
                     columns, layer, layers, offsets[r]))
      return hipErrorInvalidValue;
    total += tokens[r];
  }
  if (total * qkv_stride > INT32_MAX || total * out_stride > INT32_MAX) return hipErrorInvalidValue;
  const size_t e = dtype == kF32 ? 4 : 2;
  auto rows16 = [&](int64_t x) { return (x * int64_t(e)) % 16 == 0; };
  const bool mfma = dtype != kF32 && (d == 64 || d == 128) && aligned16(out) && aligned16(q) &&
                    aligned16(k) && aligned16(v) && rows16(qkv_stride) && rows16(out_stride) && rows16(d);
  if (!mfma) {
    // Shapes the matrix-core kernel does not take: one call per prompt.
    int64_t first = 0;
    for (int r = 0; r < requests; ++r) {
      const int st = mt_paged_prefill(static_cast<char*>(out) + size_t(first) * out_stride * e,
                                      static_cast<const char*>(q) + size_t(first) * qkv_stride * e,
                                      static_cast<const char*>(k) + size_t(first) * qkv_stride * e,
                                      static_cast<const char*>(v) + size_t(first) * qkv_stride * e, slabs,
                                      tables[r], 1, h, tokens[r], d, page_size, pages_per_slab, num_slabs,
                                      columns, layer, layers, offsets[r], dtype, qkv_stride, out_stride);
      if (st) return st;
      first += tokens[r];
    }
    return hipSuccess;
  }
  const Geometry g = make_geometry(h, d, page_size, pages_per_slab, num_slabs, columns, layer);
  // Chunks of at most kRaggedPrompts prompts and kRaggedTiles query tiles.
  int r0 = 0;
  int64_t row0 = 0;
  while (r0 < requests) {
    RaggedItems it{};
    int r1 = r0, pairs = 0;
    int64_t rows = 0;
    while (r1 < requests && r1 - r0 < kRaggedPrompts &&
           pairs + (tokens[r1] + kPfQueries - 1) / kPfQueries <= kRaggedTiles) {
      const int p = r1 - r0;
      it.first_row[p] = int(rows);
      it.n[p] = tokens[r1];
      it.offset[p] = offsets[r1];
      it.table[p] = tables[r1];
      pairs += (tokens[r1] + kPfQueries - 1) / kPfQueries;
      rows += tokens[r1];
      ++r1;
    }
    if (r1 == r0) {
      // One prompt with more query tiles than a launch describes: on its own.
      const size_t qo = size_t(row0) * qkv_stride * e;
      const int st = mt_paged_prefill(static_cast<char*>(out) + size_t(row0) * out_stride * e,
                                      static_cast<const char*>(q) + qo, static_cast<const char*>(k) + qo,
                                      static_cast<const char*>(v) + qo, slabs, tables[r0], 1, h, tokens[r0], d,
                                      page_size, pages_per_slab, num_slabs, columns, layer, layers,
                                      offsets[r0], dtype, qkv_stride, out_stride);
      if (st) return st;
      row0 += tokens[r0];
      ++r0;
      continue;
    }
    it.prompts = r1 - r0;
    it.pairs = pairs;
    // (prompt, tile) pairs, the tiles that attend the most keys first.
    std::vector<std::pair<int, int>> order;
    for (int p = 0; p < it.prompts; ++p)
      for (int t = 0; t * kPfQueries < it.n[p]; ++t) order.push_back({p, t});
    std::stable_sort(order.begin(), order.end(), [&](const std::pair<int, int>& x, const std::pair<int, int>& y) {
      auto keys = [&](const std::pair<int, int>& z) {
        const int last = (z.second + 1) * kPfQueries < it.n[z.first] ? (z.second + 1) * kPfQueries : it.n[z.first];
        return it.offset[z.first] + last;
      };
      return keys(x) > keys(y);
    });
    // Key splits: a tile whose keys span more blocks than its share of the
    // launch (all pairs' key blocks times the heads over two workgroups per
    // compute unit, at least 2) is cut into pieces of at most that many
    // blocks, merged afterwards by ragged_merge_kernel. Only when the longest
    // tile has at least 6 blocks, as for one prompt (launch_split_prefill).
    auto blocks_of = [&](const std::pair<int, int>& z) {
      const int last = (z.second + 1) * kPfQueries < it.n[z.first] ? (z.second + 1) * kPfQueries : it.n[z.first];
      return (it.offset[z.first] + last + kPfKeys - 1) / kPfKeys;
    };
    int64_t total_blocks = 0;
    int max_blocks = 0;
    for (const auto& z : order) {
      total_blocks += blocks_of(z);
      max_blocks = std::max(max_blocks, blocks_of(z));
    }
    const int cus = device_compute_units();
    const int share = MT_RAGGED_SHARE * std::max(cus, 1);
    int B = std::max<int>(2, int((total_blocks * h + share - 1) / share));
    auto pieces = [&](int B) {
      int64_t c = 0;
      for (const auto& z : order) c += (blocks_of(z) + B - 1) / B;
      return c;
    };
    while (pieces(B) > kRaggedTiles) ++B;
    bool split = MT_RAGGED_KEY_SPLIT && cus > 0 && max_blocks >= 6 && max_blocks > B && max_blocks <= 65535;
    struct Piece { int p, t, kb0, kb1, slot; };
    std::vector<Piece> list;
    RaggedMerge mg{};
    int slots = 0;
    if (split) {
      for (const auto& z : order) {
        const int nb = blocks_of(z), n = (nb + B - 1) / B;
        if (n > 1) {
          mg.row0[mg.tiles] = it.first_row[z.first] + z.second * kPfQueries;
          mg.nq[mg.tiles] = static_cast<unsigned short>(std::min(kPfQueries, it.n[z.first] - z.second * kPfQueries));
          mg.first_slot[mg.tiles] = static_cast<unsigned short>(slots);
          mg.splits[mg.tiles] = static_cast<unsigned char>(n);
          ++mg.tiles;
        }
        for (int j = 0; j < n; ++j)
          list.push_back({z.first, z.second, j * B, std::min(nb, (j + 1) * B), n > 1 ? slots++ : -1});
      }
      // Heaviest pieces first.
      std::stable_sort(list.begin(), list.end(),
                       [](const Piece& x, const Piece& y) { return x.kb1 - x.kb0 > y.kb1 - y.kb0; });
    } else {
      for (const auto& z : order) list.push_back({z.first, z.second, 0, blocks_of(z), -1});
    }
    void* ws = nullptr;
    // Without room for the partials the launch runs unsplit.
    if (split && (mg.tiles > kSplitPairs || slots > 32767 ||
                  library_workspace(size_t(slots) * h * kPfQueries * (d + 4) * sizeof(float), &ws) != hipSuccess)) {
      split = false;
      list.clear();
      mg = RaggedMerge{};
      for (const auto& z : order) list.push_back({z.first, z.second, 0, blocks_of(z), -1});
    }
    pairs = int(list.size());
    it.pairs = pairs;
    for (int i = 0; i < pairs; ++i) {
      it.pair_prompt[i] = static_cast<unsigned char>(list[i].p);
      it.pair_tile[i] = static_cast<unsigned short>(list[i].t);
      it.pair_kb0[i] = static_cast<unsigned short>(list[i].kb0);
      it.pair_kb1[i] = static_cast<unsigned short>(list[i].kb1);
      it.pair_slot[i] = static_cast<short>(list[i].slot);
    }
    const size_t qoff = size_t(row0) * qkv_stride * e, ooff = size_t(row0) * out_stride * e;
    QueryArgs a{};
    a.out = static_cast<char*>(out) + ooff;
    a.q = static_cast<const char*>(q) + qoff;
    a.k = static_cast<const char*>(k) + qoff;  // the kernel appends the prompts' K/V itself
    a.v = static_cast<const char*>(v) + qoff;
    a.slabs = slabs;
    a.g = g;
    a.qscale = (1.0f / std::sqrt(float(d))) * kLog2e;
    a.q_h = d; a.q_r = qkv_stride;
    a.o_h = d; a.o_r = out_stride;
    a.partials = static_cast<float*>(ws);
    const int blocks = grid_for(int64_t(pairs) * h);
    if (dtype == kF16) {
      if (d == 64) prefill_kernel<kF16, 64, RaggedItems, true><<<blocks, kThreads>>>(a, it);
      else prefill_kernel<kF16, 128, RaggedItems, true><<<blocks, kThreads>>>(a, it);
    } else {
      if (d == 64) prefill_kernel<kBF16, 64, RaggedItems, true><<<blocks, kThreads>>>(a, it);
      else prefill_kernel<kBF16, 128, RaggedItems, true><<<blocks, kThreads>>>(a, it);
    }
    if (split) {
      const unsigned mblocks = unsigned(mg.tiles * h);
      if (dtype == kF16) {
        if (d == 64) ragged_merge_kernel<kF16, 64><<<mblocks, 256>>>(a, mg);
        else ragged_merge_kernel<kF16, 128><<<mblocks, 256>>>(a, mg);
      } else {
        if (d == 64) ragged_merge_kernel<kBF16, 64><<<mblocks, 256>>>(a, mg);
        else ragged_merge_kernel<kBF16, 128><<<mblocks, 256>>>(a, mg);
      }
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (split) g_key_split_launches.fetch_add(1, std::memory_order_relaxed);
    r0 = r1;
    row0 += rows;
  }
  return hipSuccess;
}

int mt_paged_decode_batch(void* out, const void* q, const void* k, const void* v,
                          const uint64_t* slabs, const int* table, const int* offsets, int b,
                          int h, int d, int page_size, int pages_per_slab, int num_slabs,
                          int columns, int layer, int layers, int dtype) {
  if (!out || !q || !k || !v || !slabs || !table || !offsets ||
      !paged_shape(b, h, 1, 1, d, page_size, pages_per_slab, num_slabs, columns, layer, layers, 0) ||
      int64_t(columns) * page_size > INT32_MAX)
    return hipErrorInvalidValue;
  if (dtype < 0 || dtype > 2) return hipErrorInvalidValue;
  const int64_t cap = int64_t(columns) * page_size;
  const int S = choose_split(cap, 0);
  const int64_t nsplit_max = (cap + S - 1) / S;
  const bool ordered = device_order(b, nsplit_max);
  // Workspace: split partials, then the device-built visiting order.
  const size_t part = nsplit_max > 1 ? align256(workspace_bytes_for(int64_t(b) * h, int(nsplit_max))) : 0;
  const size_t ws_bytes = part + (ordered ? order_bytes(b, nsplit_max) : 0);
  void* ws = nullptr;
  if (ws_bytes) {
    const int e = library_workspace(ws_bytes, &ws);
    if (e != hipSuccess) return e;
  }
  int* order = ordered ? reinterpret_cast<int*>(static_cast<char*>(ws) + part) : nullptr;
  return decode_common(out, q, k, v, slabs, table, offsets, b, h, d, page_size, pages_per_slab,
                       num_slabs, columns, layer, layers, dtype, S, 0, 0, 0,
                       nullptr, 0, 0, part ? ws : nullptr, part, true, order);
}

int mt_paged_decode_batch_noalloc(void* out, const void* q, const void* k, const void* v,
                                  const uint64_t* slabs, const int* table, const int* offsets,
                                  int b, int h, int d, int page_size, int pages_per_slab,
                                  int num_slabs, int columns, int layer, int layers, int dtype) {
  if (!out || !q || !k || !v || !slabs || !table || !offsets ||
      !paged_shape(b, h, 1, 1, d, page_size, pages_per_slab, num_slabs, columns, layer, layers, 0) ||
      int64_t(columns) * page_size > INT32_MAX)
    return hipErrorInvalidValue;
  if (dtype < 0 || dtype > 2) return hipErrorInvalidValue;
  const int64_t cap = int64_t(columns) * page_size;
  const int S = choose_split(cap, 0);
  const int64_t nsplit_max = (cap + S - 1) / S;
  const bool ordered = device_order(b, nsplit_max);
  // The fixed array holds the split partials, then the device-built visiting
  // order; a shape that needs more is refused before any launch.
  const bool vec = decode_vec(d, dtype, out, q, k, v, int64_t(h) * d);
  const size_t part = nsplit_max > 1 ? align256(partial_bytes(int64_t(b) * h, nsplit_max, vec, d)) : 0;
  const size_t need = part + (ordered ? order_bytes(b, nsplit_max) : 0);
  if (need > kNoAllocScratchBytes) return hipErrorInvalidValue;
  void* ws = nullptr;
  if (need) {
    const int e = scratch_address(&ws);
    if (e != hipSuccess) return e;
  }
  int* order = ordered ? reinterpret_cast<int*>(static_cast<char*>(ws) + part) : nullptr;
  return decode_common(out, q, k, v, slabs, table, offsets, b, h, d, page_size, pages_per_slab,
                       num_slabs, columns, layer, layers, dtype, S, 0, 0, 0,
                       nullptr, 0, 0, part ? ws : nullptr, part, true, order);
}

int mt_paged_prefill_key_splits(long long* launches) {
  if (!launches) return hipErrorInvalidValue;
  *launches = g_key_split_launches.load(std::memory_order_relaxed);
  return hipSuccess;
}

int mt_paged_decode_workspace_bytes(int b, int h, int page_size, int columns, int split_tokens,
                                    size_t* bytes) {
  if (!bytes || b < 1 || h < 1 || columns < 1 ||
      !(page_size == 8 || page_size == 16 || page_size == 32))
    return hipErrorInvalidValue;
  const int64_t cap = int64_t(columns) * page_size;
  const int S = choose_split(cap, split_tokens);
  if (S < 64 || S % 64 != 0 || S > kMaxSplitTokens) return hipErrorInvalidValue;
  const int64_t nsplit_max = (cap + S - 1) / S;
  *bytes = nsplit_max > 1 ? workspace_bytes_for(int64_t(b) * h, int(nsplit_max)) : 0;
  return hipSuccess;
}

#ifdef MT_DECODE_TIMELINE
// Measurement builds only: copies the first `count` workgroups' records
// (kTimelineFields x uint64 each, see g_decode_timeline) of the last decode
// launch to host memory `dst`, after the calling thread's stream has drained.
int mt_decode_timeline(unsigned long long* dst, int count) {
  if (!dst || count < 1 || count > kTimelineMax) return hipErrorInvalidValue;
  hipError_t e = hipStreamSynchronize(hipStreamPerThread);
  if (e == hipSuccess)
    e = hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_decode_timeline), size_t(count) * kTimelineFields * 8);
  return e;
}
#endif

int mt_paged_decode_split_tokens(int page_size, int columns, int requested, int* split_tokens) {
  if (!split_tokens || columns < 1 || requested < 0 ||
      !(page_size == 8 || page_size == 16 || page_size == 32))
    return hipErrorInvalidValue;
  const int S = choose_split(int64_t(columns) * page_size, requested);
  if (S < 64 || S % 64 != 0 || S > kMaxSplitTokens) return hipErrorInvalidValue;
  *split_tokens = S;
  return hipSuccess;
}

int mt_paged_decode_order(const int* offsets, int b, int h, int page_size, int columns,
                          int split_tokens, int compute_units, int* list, int* count) {
  if (!offsets || !list || !count || b < 1 || b > kOrderRows || h < 1 || columns < 1 ||
      split_tokens < 0 || compute_units < 0 || !(page_size == 8 || page_size == 16 || page_size == 32) ||
      int64_t(columns) * page_size > INT32_MAX)
    return hipErrorInvalidValue;
  const int64_t cap = int64_t(columns) * page_size;
  const int S = choose_split(cap, split_tokens);
  if (S < 64 || S % 64 != 0 || S > kMaxSplitTokens) return hipErrorInvalidValue;
  OrderArgs oa{};
  oa.offsets = offsets; oa.count = count; oa.list = list;
  oa.batch = b; oa.split_tokens = S; oa.cap = cap;
  const int64_t nsplit_max = (cap + S - 1) / S;
  if (int64_t(b) * nsplit_max > INT32_MAX / 2) return hipErrorInvalidValue;
  oa.capacity = int(int64_t(b) * nsplit_max);
  oa.per = std::max(1, (compute_units ? compute_units : device_compute_units()) / h);
  order_kernel<<<1, kOrderThreads>>>(oa);
  return hipGetLastError();
}

int mt_paged_decode_split(void* out, const void* q, const void* k, const void* v,
                          const uint64_t* slabs, const int* table, const int* offsets, int b,
                          int h, int d, int page_size, int pages_per_slab, int num_slabs,
                          int columns, int layer, int layers, int dtype, int split_tokens,
                          int unroll, int waves, int qkv_stride, const int* work,
                          int work_items, int merge_rows, void* workspace,
                          size_t workspace_bytes) {
  if (!out || !q || !k || !v || !slabs || !table || !offsets ||
      !paged_shape(b, h, 1, 1, d, page_size, pages_per_slab, num_slabs, columns, layer, layers, 0) ||
      int64_t(columns) * page_size > INT32_MAX || split_tokens < 0 || unroll < 0 ||
      (waves != 0 && waves != 2 && waves != 4 && waves != 8) ||
      (qkv_stride != 0 && int64_t(qkv_stride) < int64_t(h) * d) || qkv_stride < 0)
    return hipErrorInvalidValue;
  if (dtype < 0 || dtype > 2) return hipErrorInvalidValue;
  return decode_common(out, q, k, v, slabs, table, offsets, b, h, d, page_size, pages_per_slab,
                       num_slabs, columns, layer, layers, dtype, split_tokens,
                       unroll, waves, qkv_stride,
                       work, work_items, merge_rows, workspace, workspace_bytes);
}

}  // extern "C"
