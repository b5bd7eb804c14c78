/* CPU restatement of the reference's paged decode step. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/ and bench.py's cpu_baseline leg load this library, as the
 * checker and as the reported CPU baseline ("port"). The product path never
 * calls it.
 *
 * oracle_paged_decode_batch() has the argument list of the reference's
 * mt_paged_decode_batch (src/paged_attention_kernel.cu:121-137), with host
 * pointers: slabs[] holds host addresses of slab images. It
 *   1. appends K/V [B,H,1,D] at position offsets[b] through the block table,
 *      skipping rows whose page is missing (src/paged_attention_kernel.cu:23-33,
 *      page validity :11-16);
 *   2. for every (b, h) attends the offsets[b] + 1 keys in the composition of
 *      MiniTorch's CPU tensor backend: gather the rows of the pages -> scores
 *      q.K^T * (1/sqrt(D)) -> max / exp / sum / divide softmax
 *      (minitorch/nn.py:136-152) -> weights . V, all in fp32. A missing page
 *      reads as NaN, which makes the row NaN (src/paged_attention_kernel.cu:53,84).
 * OpenMP parallelises over (b, h), the prange-equivalent of FastOps
 * (minitorch/fast_ops.py:33-353). Pinned against the numpy oracle in
 * tests/test_oracle.py.
 *
 * oracle_paged_attention() has the argument list of the reference's
 * mt_paged_attention (src/paged_attention_kernel.cu:108-117, paged_forward
 * with offsets == nullptr, :35-85): for every (b, h) and query qi of q
 * [B,H,nq,D], attention over keys [0, min(offset + qi + 1, nk)) of the pages,
 * in the same fp32 composition as the decode above.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float f = (float)man * (1.0f / 16777216.0f);
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static uint16_t f32_to_f16(float f) { /* round to nearest even */
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (ax < 0x38800000u) {                                  /* subnormal or zero in fp16 */
    float a;
    memcpy(&a, &ax, 4);
    const float scaled = a * 16777216.0f; /* exact: units of 2^-24 */
    float r = nearbyintf(scaled);         /* default mode: nearest even */
    return (uint16_t)(sign | (uint32_t)r);
  }
  const uint32_t e = ((ax >> 23) - 112u) << 10;
  const uint32_t m = (ax >> 13) & 0x3ffu;
  uint32_t h = e | m;
  const uint32_t rest = ax & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

static float bf16_to_f32(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static float load(const void* p, int64_t i, int dtype) {
  if (dtype == 0) return ((const float*)p)[i];
  if (dtype == 1) return f16_to_f32(((const uint16_t*)p)[i]);
  return bf16_to_f32(((const uint16_t*)p)[i]);
}

static void store(void* p, int64_t i, float v, int dtype) {
  if (dtype == 0) ((float*)p)[i] = v;
  else if (dtype == 1) ((uint16_t*)p)[i] = f32_to_f16(v);
  else ((uint16_t*)p)[i] = f32_to_bf16(v);
}

static int elem_bytes(int dtype) { return dtype == 0 ? 4 : 2; }

/* Host address of element (position, col) of kind (0 = K, 1 = V), or NULL
 * for a missing page (src/paged_attention_kernel.cu:7-21). */
static char* page_element(const uint64_t* slabs, const int* table, int b, int head, int64_t position,
                          int col, int kind, int layer, int heads, int dim, int page_size,
                          int pps, int num_slabs, int columns, int dtype) {
  const int64_t logical = position / page_size;
  if (position < 0 || logical >= columns) return NULL;
  const int physical = table[(int64_t)b * columns + logical];
  if (physical < 0 || (int64_t)physical >= (int64_t)num_slabs * pps) return NULL;
  const uint64_t address = slabs[physical / pps];
  if (!address) return NULL;
  const int slot = physical % pps;
  int64_t i = ((((int64_t)layer * 2 + kind) * pps + slot) * heads + head) * (int64_t)page_size * dim;
  i += (position % page_size) * dim + col;
  return (char*)(uintptr_t)address + i * elem_bytes(dtype);
}

int oracle_paged_decode_batch(void* out, const void* q, const void* k, const void* v,
                              const uint64_t* slabs, const int* table, const int* offsets, int b,
                              int h, int d, int page_size, int pps, int num_slabs, int columns,
                              int layer, int layers, int dtype, int threads) {
  if (!out || !q || !k || !v || !slabs || !table || !offsets || b < 1 || h < 1 || d < 1 ||
      d > 128 || layer < 0 || layer >= layers || dtype < 0 || dtype > 2)
    return 1;
  if (threads > 0) omp_set_num_threads(threads);
  const int eb = elem_bytes(dtype);
  /* 1. append */
#pragma omp parallel for schedule(static)
  for (int64_t bh = 0; bh < (int64_t)b * h; ++bh) {
    const int bi = (int)(bh / h), head = (int)(bh % h);
    const int64_t pos = offsets[bi];
    char* kp = page_element(slabs, table, bi, head, pos, 0, 0, layer, h, d, page_size, pps, num_slabs, columns, dtype);
    char* vp = page_element(slabs, table, bi, head, pos, 0, 1, layer, h, d, page_size, pps, num_slabs, columns, dtype);
    if (kp && vp) {
      memcpy(kp, (const char*)k + bh * d * eb, (size_t)d * eb);
      memcpy(vp, (const char*)v + bh * d * eb, (size_t)d * eb);
    }
  }
  /* 2. gather -> scores -> softmax -> weights . V */
  const float scale = 1.0f / sqrtf((float)d);
#pragma omp parallel
  {
    int64_t cap = 0;
    float *keys = NULL, *vals = NULL, *scores = NULL;
#pragma omp for schedule(dynamic, 4)
    for (int64_t bh = 0; bh < (int64_t)b * h; ++bh) {
      const int bi = (int)(bh / h), head = (int)(bh % h);
      const int64_t n = offsets[bi] < 0 ? 0 : (int64_t)offsets[bi] + 1;
      if (n > cap) {
        free(keys); free(vals); free(scores);
        cap = n;
        keys = (float*)malloc(sizeof(float) * cap * d);
        vals = (float*)malloc(sizeof(float) * cap * d);
        scores = (float*)malloc(sizeof(float) * cap);
      }
      for (int64_t j = 0; j < n; ++j) {
        const char* kp = page_element(slabs, table, bi, head, j, 0, 0, layer, h, d, page_size, pps, num_slabs, columns, dtype);
        const char* vp = page_element(slabs, table, bi, head, j, 0, 1, layer, h, d, page_size, pps, num_slabs, columns, dtype);
        for (int c = 0; c < d; ++c) {
          keys[j * d + c] = kp ? load(kp, c, dtype) : NAN;
          vals[j * d + c] = vp ? load(vp, c, dtype) : NAN;
        }
      }
      float qv[128];
      for (int c = 0; c < d; ++c) qv[c] = load(q, bh * d + c, dtype);
      float mx = -INFINITY;
      int poisoned = 0;
      for (int64_t j = 0; j < n; ++j) {
        float s = 0.f;
        for (int c = 0; c < d; ++c) s += qv[c] * keys[j * d + c];
        s *= scale;
        scores[j] = s;
        if (isnan(s)) poisoned = 1;
        else if (s > mx) mx = s;
      }
      float sum = 0.f;
      for (int64_t j = 0; j < n; ++j) {
        scores[j] = expf(scores[j] - mx);
        sum += scores[j];
      }
      for (int c = 0; c < d; ++c) {
        float acc = 0.f;
        for (int64_t j = 0; j < n; ++j) acc += scores[j] / sum * vals[j * d + c];
        float o = n == 0 ? 0.f : (poisoned ? NAN : acc);
        store(out, bh * d + c, o, dtype);
      }
    }
    free(keys); free(vals); free(scores);
  }
  return 0;
}

int oracle_paged_attention(void* out, const void* q, const uint64_t* slabs, const int* table, int b,
                           int h, int nq, int nk, int d, int page_size, int pps, int num_slabs,
                           int columns, int layer, int layers, int offset, int dtype, int threads) {
  if (!out || !q || !slabs || !table || b < 1 || h < 1 || nq < 1 || nk < 1 || d < 1 || d > 128 ||
      offset < 0 || layer < 0 || layer >= layers || dtype < 0 || dtype > 2)
    return 1;
  if (threads > 0) omp_set_num_threads(threads);
  const float scale = 1.0f / sqrtf((float)d);
#pragma omp parallel
  {
    float* keys = (float*)malloc(sizeof(float) * (size_t)nk * d);
    float* vals = (float*)malloc(sizeof(float) * (size_t)nk * d);
    float* scores = (float*)malloc(sizeof(float) * (size_t)nk);
#pragma omp for schedule(dynamic, 1)
    for (int64_t bh = 0; bh < (int64_t)b * h; ++bh) {
      const int bi = (int)(bh / h), head = (int)(bh % h);
      for (int64_t j = 0; j < nk; ++j) {
        const char* kp = page_element(slabs, table, bi, head, j, 0, 0, layer, h, d, page_size, pps, num_slabs, columns, dtype);
        const char* vp = page_element(slabs, table, bi, head, j, 0, 1, layer, h, d, page_size, pps, num_slabs, columns, dtype);
        for (int c = 0; c < d; ++c) {
          keys[j * d + c] = kp ? load(kp, c, dtype) : NAN;
          vals[j * d + c] = vp ? load(vp, c, dtype) : NAN;
        }
      }
      for (int qi = 0; qi < nq; ++qi) {
        const int64_t n = (int64_t)offset + qi + 1 < nk ? (int64_t)offset + qi + 1 : nk;
        const int64_t row = bh * nq + qi;
        float qv[128];
        for (int c = 0; c < d; ++c) qv[c] = load(q, row * d + c, dtype);
        float mx = -INFINITY;
        int poisoned = 0;
        for (int64_t j = 0; j < n; ++j) {
          float s = 0.f;
          for (int c = 0; c < d; ++c) s += qv[c] * keys[j * d + c];
          s *= scale;
          scores[j] = s;
          if (isnan(s)) poisoned = 1;
          else if (s > mx) mx = s;
        }
        float sum = 0.f;
        for (int64_t j = 0; j < n; ++j) {
          scores[j] = expf(scores[j] - mx);
          sum += scores[j];
        }
        for (int c = 0; c < d; ++c) {
          float acc = 0.f;
          for (int64_t j = 0; j < n; ++j) acc += scores[j] / sum * vals[j * d + c];
          store(out, row * d + c, poisoned ? NAN : acc, dtype);
        }
      }
    }
    free(keys); free(vals); free(scores);
  }
  return 0;
}

int oracle_max_threads(void) { return omp_get_max_threads(); }
