// Shared device helpers for the gfx950 ThetaScan kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "thetascan_hip.h"

namespace ts {

// Record a message for ts_last_error() and return `code` (host side).
int fail(int code, const char* fmt, ...);

// Raise a kernel's dynamic-LDS limit to `bytes` once per process (later
// launches, including launches recorded into a graph, skip the call).
hipError_t ensure_lds_limit(const void* fn, int bytes);

// Workgroups of `fn` (`threads` threads, `lds` bytes of dynamic LDS) resident
// on the current device at once: the occupancy calculator's workgroups per CU
// times the CU count, cached per (device, kernel, LDS size, threads); 0 if a
// query fails.
long resident_workgroups(const void* fn, int lds, int threads = 256);

// Segmentation and workspace layout of a scan (host side): 64-token tiles
// per segment, segments, summaries the prefix reads, floats per segment state,
// padded widths and workspace bytes (0 when the scan needs none).
struct ScanSegments {
  int seg_chunks, nseg, nsum, nelem, dkp, dvp;
  size_t ws_bytes;
};
int scan_segments(const ts_scan_desc* d, ScanSegments* out);

// One ts_sum_slots call's arguments (host side).
struct SlotSum {
  const float* a;
  int32_t na;
  const float* b;
  int32_t nb;
  int64_t n;
  void* out;
  int32_t out_dtype;
  float scale;
};
constexpr int kMaxSlotJobs = 4;

// Several independent slot sums in one launch (each result equal to its own
// ts_sum_slots call); falls back to separate calls when one cannot be batched.
int sum_slots_batch(const SlotSum* jobs, int njobs, hipStream_t stream);

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
// Issued as the 32-deep MFMA with the upper four k-values zero: a dependent
// accumulation chain then uses one MFMA opcode throughout.  Mixing the
// 16x16x16 and 16x16x32 bf16 opcodes back to back on one accumulator read a
// stale accumulator on gfx950 (compiler-inserted wait states were missing).
__device__ __forceinline__ floatx4 mma16(bf16x4 a, bf16x4 b, floatx4 c) {
  const bf16x4 z = {(bf16)0.0f, (bf16)0.0f, (bf16)0.0f, (bf16)0.0f};
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_shufflevector(a, z, 0, 1, 2, 3, 4, 5, 6, 7),
                                                 __builtin_shufflevector(b, z, 0, 1, 2, 3, 4, 5, 6, 7), c, 0, 0, 0);
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

// Fragment loads/stores for MFMA operands (LDS or global, 16-byte aligned).
template <typename E> struct LdsIO;
template <> struct LdsIO<bf16> {
  static __device__ __forceinline__ bf16x8 ld8(const bf16* p) {
    uint4 r = *(const uint4*)p;
    return __builtin_bit_cast(bf16x8, r);
  }
  static __device__ __forceinline__ bf16x4 ld4(const bf16* p) {
    uint2 r = *(const uint2*)p;
    return __builtin_bit_cast(bf16x4, r);
  }
  static __device__ __forceinline__ bf16x8 cat(bf16x4 a, bf16x4 b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  static __device__ __forceinline__ bf16x8 from_acc(floatx4 a, floatx4 b) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r[i] = (bf16)a[i];
      r[4 + i] = (bf16)b[i];
    }
    return r;
  }
  static __device__ __forceinline__ bf16x4 from_acc4(floatx4 a) {
    bf16x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (bf16)a[i];
    return r;
  }
  static __device__ __forceinline__ void st4(bf16* p, float a0, float a1, float a2, float a3) {
    bf16x4 r;
    r[0] = (bf16)a0; r[1] = (bf16)a1; r[2] = (bf16)a2; r[3] = (bf16)a3;
    *(uint2*)p = __builtin_bit_cast(uint2, r);
  }
};
template <> struct LdsIO<float> {
  static __device__ __forceinline__ floatx8 ld8(const float* p) {
    floatx4 a = *(const floatx4*)p;
    floatx4 b = *(const floatx4*)(p + 4);
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  static __device__ __forceinline__ floatx4 ld4(const float* p) { return *(const floatx4*)p; }
  static __device__ __forceinline__ floatx8 cat(floatx4 a, floatx4 b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  static __device__ __forceinline__ floatx8 from_acc(floatx4 a, floatx4 b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  static __device__ __forceinline__ floatx4 from_acc4(floatx4 a) { return a; }
  static __device__ __forceinline__ void st4(float* p, float a0, float a1, float a2, float a3) {
    floatx4 r = {a0, a1, a2, a3};
    *(floatx4*)p = r;
  }
};

}  // namespace ts
