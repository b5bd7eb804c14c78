// Device helpers shared by the gfx950 kernels: element types, fp32 conversion
// and 16-byte vector access.
//
// Element codes follow the reference's dtype codes (minitorch/dtypes.py:11):
// 0 = float32, 1 = float16, 2 = bfloat16. Low-precision values are read into
// fp32 registers (src/includes/typed_io.cuh:4-6) and written back with
// round-to-nearest-even; bfloat16 NaNs stay quiet NaNs as in the reference's
// host encoder (minitorch/dtypes.py:37-46).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace mt {

enum : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// 16 bytes as a native vector, loadable from any address space.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int DT> struct Elem;
template <> struct Elem<kF32> { using T = float; };
template <> struct Elem<kF16> { using T = uint16_t; };
template <> struct Elem<kBF16> { using T = uint16_t; };

template <int DT> constexpr int elem_bytes() { return DT == kF32 ? 4 : 2; }

__device__ __forceinline__ float f16_to_f32(uint16_t x) {
  return static_cast<float>(__builtin_bit_cast(_Float16, x));
}
__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

template <int DT> __device__ __forceinline__ float to_f32(typename Elem<DT>::T x) {
  if constexpr (DT == kF32) return x;
  else if constexpr (DT == kF16) return f16_to_f32(x);
  else return bf16_to_f32(x);
}
template <int DT> __device__ __forceinline__ typename Elem<DT>::T from_f32(float x) {
  if constexpr (DT == kF32) return x;
  else if constexpr (DT == kF16) return f32_to_f16(x);
  else return f32_to_bf16(x);
}

// Unpack one 16-byte register group holding 4 (fp32) or 8 (fp16/bf16) values.
template <int DT> __device__ __forceinline__ void unpack16(const u32x4& r, float* o) {
  if constexpr (DT == kF32) {
    o[0] = __uint_as_float(r.x); o[1] = __uint_as_float(r.y);
    o[2] = __uint_as_float(r.z); o[3] = __uint_as_float(r.w);
  } else {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = to_f32<DT>(static_cast<uint16_t>(w[i] & 0xffffu));
      o[2 * i + 1] = to_f32<DT>(static_cast<uint16_t>(w[i] >> 16));
    }
  }
}

// Pack 4 (fp32) or 8 (fp16/bf16) fp32 values into one 16-byte group.
template <int DT> __device__ __forceinline__ u32x4 pack16(const float* v) {
  u32x4 r;
  if constexpr (DT == kF32) {
    r.x = __float_as_uint(v[0]); r.y = __float_as_uint(v[1]);
    r.z = __float_as_uint(v[2]); r.w = __float_as_uint(v[3]);
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(from_f32<DT>(v[2 * i])) |
             (static_cast<uint32_t>(from_f32<DT>(v[2 * i + 1])) << 16);
    r.x = w[0]; r.y = w[1]; r.z = w[2]; r.w = w[3];
  }
  return r;
}

template <int DT> constexpr int per16() { return 16 / elem_bytes<DT>(); }

// Global-address-space view of a pointer. Pointers that come from LDS or
// kernel arguments may be generic, and generic (flat) loads are also counted
// by the LDS wait counter, so an LDS read placed after them would wait for
// the HBM load to return; global loads keep the two counters independent.
template <class T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* global_view(const T* p) {
  return (const __attribute__((address_space(1))) T*)(p);
}
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* global_view(T* p) {
  return (__attribute__((address_space(1))) T*)(p);
}

// v_mfma_f32_16x16x32 (fp16/bf16 in, fp32 accumulate). Lane l (column
// c = l % 16, group g = l / 16) supplies A[c][8g .. 8g+7] and B[8g .. 8g+7][c]
// and holds C[4g + i][c], i < 4.
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int DT>
struct Mfma;
template <>
struct Mfma<kF16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ floatx4 run(const v8& a, const v8& b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<kBF16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ floatx4 run(const v8& a, const v8& b, const floatx4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// Inclusive prefix sum over a wave: Hillis-Steele shifts of 1, 2, 4 and 8
// lanes inside each row of 16 (lanes shifted in from outside the row add 0),
// then rows 1 and 3 add lane 15 of the row before and rows 2 and 3 add lane 31.
__device__ __forceinline__ int wave_inclusive_add(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
  return x;
}

// Keeps a kernel argument in scalar registers from here on: the empty asm
// reads and writes it, so the compiler loads it at this point (together with
// the other arguments pinned next to it, one round trip for all of their
// kernarg cache lines) and cannot load it again later from the kernarg
// segment, where a first touch of a line mid-kernel costs a memory round trip.
template <class T>
__device__ __forceinline__ T pin_arg(T x) {
  asm volatile("" : "+s"(x));
  return x;
}
// pin_arg for a pointer to global memory, returned in the global address
// space: the asm hides where the pointer came from, and a generic pointer
// would make every access a flat instruction, which the LDS counter also
// counts (an LDS wait would then wait for those stores to be acknowledged).
template <class T>
__device__ __forceinline__ __attribute__((address_space(1))) T* pin_global(T* p) {
  auto g = global_view(p);
  asm volatile("" : "+s"(g));
  return g;
}

}  // namespace mt
