// Shared device helpers for the gfx950 ThetaScan kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ts {

typedef __bf16 bf16;
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx8 __attribute__((ext_vector_type(8)));

// Fragment types for one 16x16 MFMA step: eight k-values per lane for a
// 32-wide contraction block, four for a 16-wide tail block.
template <typename E> struct Frag;
template <> struct Frag<bf16> {
  typedef bf16x8 f8;
  typedef bf16x4 f4;
};
template <> struct Frag<float> {
  typedef floatx8 f8;
  typedef floatx4 f4;
};

// D += A * B over a 32-wide contraction block.  Lane l supplies row l%16 of
// A and column l%16 of B; lane group g = l/16 supplies eight k-values.  Any
// k-order is valid as long as A and B use the same one, which the callers
// exploit to consume accumulator fragments without a shuffle.
__device__ __forceinline__ floatx4 mma32(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mma32(floatx8 a, floatx8 b, floatx4 c) {
#pragma unroll
  for (int j = 0; j < 8; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
  return c;
}
// D += A * B over a 16-wide contraction block (four k-values per lane).
__device__ __forceinline__ floatx4 mma16(bf16x4 a, bf16x4 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 mma16(floatx4 a, floatx4 b, floatx4 c) {
#pragma unroll
  for (int j = 0; j < 4; ++j) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], b[j], c, 0, 0, 0);
  return c;
}

template <typename E> __device__ __forceinline__ E cvt(float x);
template <> __device__ __forceinline__ bf16 cvt<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ float cvt<float>(float x) { return x; }

__device__ __forceinline__ float tof(bf16 x) { return (float)x; }
__device__ __forceinline__ float tof(float x) { return x; }

// 16-byte vector of elements.
template <typename E> struct Vec16 {
  static constexpr int N = 16 / (int)sizeof(E);
  union {
    uint4 raw;
    E e[16 / sizeof(E)];
  };
};

}  // namespace ts
