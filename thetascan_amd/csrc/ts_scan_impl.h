// Device helpers shared by the scan kernels (ts_scan.hip: one view per call;
// ts_scan_views.hip: several retentions of the same q, k, v per call).
#pragma once

#include "ts_common.h"
#include "thetascan_hip.h"

namespace ts {

constexpr int C = 64;               // tokens per tile
constexpr int kLdsPerCU = 160 * 1024;  // LDS of one gfx950 CU

// Raw buffer addressing.  Every tensor of one (batch, head) is addressed
// through a buffer resource whose record count ends at its last valid byte:
// loads beyond it return zero and stores beyond it are dropped.  Rows past T,
// rows before 0 of a reversed scan (negative offsets wrap past 2^31) and
// padding columns (offset kOOB) therefore need no branches.
constexpr uint32_t kOOB = 0x80000000u;
constexpr int kRsrcWord3 = 0x00020000;  // 32-bit dwords, no swizzle (gfx9 family)
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
__device__ __forceinline__ uint4 bld16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ __forceinline__ uint2 bld8(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}
__device__ __forceinline__ float bldf(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ void bst8(rsrc_t r, uint32_t off, uint2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, (int)off, 0, 0);
}
__device__ __forceinline__ void bst16(rsrc_t r, uint32_t off, uint4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)off, 0, 0);
}
__device__ __forceinline__ void bstf(rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, (int)off, 0, 0);
}

struct ScanP {
  int B, H, T, dk, dv, dvp;  // dvp: padded value width of the whole scan
  int vs;                    // padded value columns per workgroup (blockIdx.z selects the slice)
  int states_t;              // segment states read transposed (those of the swapped scan)
  int has_init;              // segment 0 also starts from a given state (the prefix wrote it)
  int nchunks, seg_chunks, nseg, nsum, nelem;
  int ret, reverse;
  int q_ext, k_ext, v_ext;
  int out_mode;
  float out_scale;
  ts_strided q, k, v, qe, ke, ve, decay, out, oe;
  // bytes spanned by one (batch, head) slice of each tensor
  uint32_t q_rec, k_rec, v_rec, qe_rec, ke_rec, ve_rec, dec_rec, out_rec, oe_rec;
  const float* log_alpha;
  float* seg;     // [BH][nseg][nelem]: S [DK][dvp], u [dvp], D [DK] (every slice's columns)
  float* segdec;  // [BH][nseg]
};

__device__ __forceinline__ const void* bh_base(const ts_strided& s, int b, int h, int es) {
  return (const char*)s.ptr + ((int64_t)b * s.sb + (int64_t)h * s.sh) * es;
}

// Byte offset of tile-local row `row` of a tile starting at t0 (uint32 wrap:
// rows before 0 of a reversed scan land past 2^31, i.e. out of range).
__device__ __forceinline__ uint32_t row_off(const ScanP& p, int t0, int row, int st_bytes) {
  const int t = t0 + row;
  const int tp = p.reverse ? p.T - 1 - t : t;
  return (uint32_t)(tp * st_bytes);
}

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

// Token-axis operand fragment of a token-major LDS tile: column c0 + (lane & 15),
// tokens {32kp+4g..+3} and {32kp+16+4g..+3} for lane group g = lane >> 4.
// This is exactly the token set the accumulator fragments of two 16x16
// score blocks 2kp, 2kp+1 hold per lane, so score fragments feed the P.V
// contraction without a shuffle.  bf16 uses the gfx950 transposing LDS read
// (ds_read_b64_tr_b16: within each 16-lane group, lane j addresses row
// r0 + j/4, column c0 + 4*(j%4), and lane i receives rows r0..r0+3 of
// column c0 + i); fp32 gathers.
template <typename E> struct Tok;
template <> struct Tok<bf16> {
  static __device__ __forceinline__ bf16x8 col8(const bf16* rows, int pitch, int c0, int kp, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const bf16* a = rows + (32 * kp + 4 * g + (j >> 2)) * pitch + c0 + 4 * (j & 3);
    shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)a);
    shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(a + 16 * pitch));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};
template <> struct Tok<float> {
  static __device__ __forceinline__ floatx8 col8(const float* rows, int pitch, int c0, int kp, int lane) {
    const int g = lane >> 4, l16 = lane & 15;
    floatx8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = rows[(32 * kp + (e < 4 ? 4 * g + e : 12 + 4 * g + e)) * pitch + c0 + l16];
    return v;
  }
};

// Feature-axis fragment of row `row` for contraction block j (32 features):
// features {32j+4g..+3} and {32j+16+4g..+3}.  Queries are loaded in the same
// order, and the state's accumulator fragments hold their rows that way.
template <typename E>
__device__ __forceinline__ typename Frag<E>::f8 frow8(const E* rows, int pitch, int row, int j, int g) {
  const E* a = rows + row * pitch + 32 * j + 4 * g;
  return LdsIO<E>::cat(LdsIO<E>::ld4(a), LdsIO<E>::ld4(a + 16));
}
template <typename E>
__device__ __forceinline__ typename Frag<E>::f4 frow4(const E* rows, int pitch, int row, int j, int g) {
  return LdsIO<E>::ld4(rows + row * pitch + 32 * j + 4 * g);
}

// A broadcast operand: eight fp32 LDS values (the same two runs of four a
// frow8 / col8 fragment covers), identical for every lane of the group.
template <typename E>
__device__ __forceinline__ typename Frag<E>::f8 bcast8(const float* vec, int base, int g, float scale = 1.0f) {
  typename Frag<E>::f8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = cvt<E>(scale * vec[base + (e < 4 ? 4 * g + e : 12 + 4 * g + e)]);
  return r;
}
template <typename E>
__device__ __forceinline__ typename Frag<E>::f4 bcast4(const float* vec, int base, int g) {
  typename Frag<E>::f4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = cvt<E>(vec[base + 4 * g + e]);
  return r;
}

// Register-staged loader of one [64 x width] tile section: each thread owns
// SLOTS 16-byte vectors (vector idx = tid + i * 256, row-major over the padded
// width).  Sections are multiples of 64 vectors, so whether a slot is in range
// is uniform per wave.  Per slot the byte offset at tile 0 and the LDS offset
// are kept; a tile adds a uniform byte offset.
template <typename E, int SLOTS>
struct TileLoader {
  static constexpr int VEC = 16 / (int)sizeof(E);
  uint32_t off0[SLOTS];
  int lds[SLOTS];
  uint4 r[SLOTS];

  __device__ __forceinline__ void setup(const ScanP& p, int per_row, int width, int pitch, int st_b, int tid) {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / per_row;
      const int c0 = (idx - row * per_row) * VEC;
      lds[i] = idx < C * per_row ? row * pitch + c0 : -1;
      off0[i] = c0 < width ? row_off(p, 0, row, st_b) + (uint32_t)(c0 * (int)sizeof(E)) : kOOB;
    }
  }
  __device__ __forceinline__ void fetch(rsrc_t data, int t0, int sgn, int st_b, int wave_first, int n) {
    const uint32_t delta = (uint32_t)(sgn * t0 * st_b);
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      if (wave_first + i * 256 >= n) break;  // uniform
      r[i] = bld16(data, off0[i] == kOOB ? kOOB : off0[i] + delta);
    }
  }
  __device__ __forceinline__ void store(E* dst, int wave_first, int n) const {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      if (wave_first + i * 256 >= n) break;  // uniform
      *(uint4*)(dst + lds[i]) = r[i];
    }
  }
};

// One segment of the prefix: the state entering the next segment.
__device__ __forceinline__ float prefix_step(float carry, float log_dec, float u) {
  return expf(log_dec) * carry + u;
}

// Exclusive scan of one element of the segment summaries of one (batch, head)
// (`base` points at that element of segment 0, summaries `nelem` apart):
// segment p receives the state entering it, sum over q < p of U_q times the
// decay of segments q+1 .. p-1 (exp of the per-segment log decays `dec`),
// plus `carry0` (the state entering segment 0) times the decay of segments
// 0 .. p-1.  Returns the state after the last summarised segment.
// Segments are taken eight at a time with all their summaries and decays
// loaded before any of their states is stored, so the loads of a block are in
// flight together instead of each waiting behind the previous store.
__device__ __forceinline__ float segment_prefix(float* base, const float* dec, int nseg, int nsum, int nelem,
                                                float carry0 = 0.0f) {
  // Loads past the last summary re-read summary nsum-1 (in bounds) and are
  // discarded, which keeps the loads free of branches.
  constexpr int K = 8;
  float carry = carry0;
  for (int s0 = 0; s0 < nseg; s0 += K) {
    float u[K], e[K];
    if (nsum > 0) {  // uniform
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int sc = min(s0 + j, nsum - 1);
        u[j] = base[(size_t)sc * nelem];
        e[j] = dec[sc];
      }
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int s = s0 + j;
      if (s < nseg) base[(size_t)s * nelem] = carry;
      if (s < nsum) carry = prefix_step(carry, e[j], u[j]);
    }
  }
  return carry;
}

// segment_prefix over four consecutive elements with 16-byte accesses
// (`base` 16-byte aligned, `nelem` a multiple of 4): per element the same
// arithmetic in the same order, so results equal four scalar calls.
__device__ __forceinline__ float4 segment_prefix4(float* base, const float* dec, int nseg, int nsum, int nelem,
                                                  float4 carry) {
  constexpr int K = 8;
  for (int s0 = 0; s0 < nseg; s0 += K) {
    float4 u[K];
    float e[K];
    if (nsum > 0) {  // uniform
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int sc = min(s0 + j, nsum - 1);
        u[j] = *(const float4*)(base + (size_t)sc * nelem);
        e[j] = dec[sc];
      }
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int s = s0 + j;
      if (s < nseg) *(float4*)(base + (size_t)s * nelem) = carry;
      if (s < nsum) {
        carry.x = prefix_step(carry.x, e[j], u[j].x);
        carry.y = prefix_step(carry.y, e[j], u[j].y);
        carry.z = prefix_step(carry.z, e[j], u[j].z);
        carry.w = prefix_step(carry.w, e[j], u[j].w);
      }
    }
  }
  return carry;
}

}  // namespace ts
