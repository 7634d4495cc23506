// Token-tile building blocks shared by the gfx950 write-side kernels
// (feature map, GN payloads): 64-token groups of one (batch, head), lane =
// token in the MFMA accumulator layout (lane l holds token l & 15 and four
// consecutive features 16b + 4(l >> 4) + i of every 16-feature block b).
#pragma once

#include "ts_common.h"

namespace ts {

// A [B,H,T,width] stream: base pointer, element strides of batch and head and
// a 32-bit element stride of time (the host checks (T + 64) * st fits).
struct Str {
  void* ptr;
  int64_t sb, sh;
  int st;
};


constexpr int TT = 64;  // tokens per group (16 per wave)

// Rows of one (batch, head) slice.
template <typename E>
struct Rows {
  E* base;
  int st;
  __device__ __forceinline__ E* at(int t) const { return base + t * st; }
};
template <typename E>
__device__ __forceinline__ Rows<E> rows_of(const Str& s, int b, int h) {
  return Rows<E>{(E*)s.ptr + b * s.sb + h * s.sh, s.st};
}

__device__ __forceinline__ float rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Values of lanes l ^ 16 and l ^ 32 by the gfx950 row-swap instructions
// v_permlane16_swap / v_permlane32_swap: swapping a VGPR with a copy of itself
// leaves lanes l and l ^ 16 (l ^ 32) in the two registers, so the per-token
// reductions over the four lane groups need no LDS round trip.  Written as
// inline asm because the compiler's builtins for these instructions return
// the same register for both halves of the swapped pair.  The s_nop covers
// the wait states between a VALU write of a VGPR and a permlane read of it.
struct LanePair {
  float a, b;
};
__device__ __forceinline__ LanePair xor16_pair(float v) {
  LanePair p{v, v};
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(p.a), "+v"(p.b));
  return p;
}
__device__ __forceinline__ LanePair xor32_pair(float v) {
  LanePair p{v, v};
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(p.a), "+v"(p.b));
  return p;
}
__device__ __forceinline__ float sum_g(float v) {  // over the 4 lane groups of a token
  LanePair p = xor16_pair(v);
  p = xor32_pair(p.a + p.b);
  return p.a + p.b;
}
__device__ __forceinline__ float max_g(float v) {
  LanePair p = xor16_pair(v);
  p = xor32_pair(fmaxf(p.a, p.b));
  return fmaxf(p.a, p.b);
}

// Orders this wave's LDS writes before its later LDS reads of rows that
// other lanes of the same wave wrote: a wave's LDS operations execute in issue
// order, so this only keeps the compiler from moving the reads above the
// writes (no workgroup barrier where each wave reads back its own rows).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Four consecutive elements <-> floats.
template <typename E>
__device__ __forceinline__ void ld4f(const E* p, float* o) {
  typename Frag<E>::f4 v = LdsIO<E>::ld4(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = tof(v[i]);
}
template <typename E>
__device__ __forceinline__ void st4f(E* p, const float* v) {
  LdsIO<E>::st4(p, v[0], v[1], v[2], v[3]);
}

// RoPE of the four-feature group starting at c (a multiple of 4) of token t:
// pairs (c, c+1) and (c+2, c+3) rotate when `on` (c < rot and t < T).
// Branch-free: other lanes read table entry 0 and rotate by the identity.
__device__ __forceinline__ void rope4(float* v, int c, int rot, const float* cs_tab, const float* sn_tab, int t,
                                      bool on, bool inverse) {
  const int idx = on ? t * (rot >> 1) + (c >> 1) : 0;
  float2 cs = *(const float2*)(cs_tab + idx);
  float2 sn = *(const float2*)(sn_tab + idx);
  if (!on) {
    cs = make_float2(1.f, 1.f);
    sn = make_float2(0.f, 0.f);
  }
  if (inverse) {
    sn.x = -sn.x;
    sn.y = -sn.y;
  }
  const float a0 = v[0], b0 = v[1], a1 = v[2], b1 = v[3];
  v[0] = a0 * cs.x - b0 * sn.x;
  v[1] = a0 * sn.x + b0 * cs.x;
  v[2] = a1 * cs.y - b1 * sn.y;
  v[3] = a1 * sn.y + b1 * cs.y;
}

// RoPE factors of one token for the four-feature groups 16 blk + 4g of its
// first NB 16-wide blocks, loaded once per token group ahead of their use:
// issued before the next group's row prefetch, a wait for them does not wait
// for the prefetch, and all blocks' loads are in flight together.  Blocks at
// or past `rot` load nothing; tokens past T read entry 0 (their rows are
// zero, so any finite factor serves); a four-feature group at or past `rot`
// inside a rotated block rotates by the identity.
template <int NB>
struct RopeRegs {
  float2 cs[NB], sn[NB];

  __device__ __forceinline__ void fetch(int rot, const float* cs_tab, const float* sn_tab, int t, bool valid, int g) {
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      if (blk * 16 < rot) {
        const int c = blk * 16 + 4 * g;
        const int idx = valid && c < rot ? t * (rot >> 1) + (c >> 1) : 0;
        cs[blk] = *(const float2*)(cs_tab + idx);
        sn[blk] = *(const float2*)(sn_tab + idx);
      }
    }
  }
  // Rotate v (features 16 blk + 4g .. +3) by the token's angles, or back.
  __device__ __forceinline__ void apply(float* v, int blk, int rot, int g, bool inverse) const {
    const bool on = blk * 16 + 4 * g < rot;
    const float cx = on ? cs[blk].x : 1.f, cy = on ? cs[blk].y : 1.f;
    float sx = on ? sn[blk].x : 0.f, sy = on ? sn[blk].y : 0.f;
    if (inverse) {
      sx = -sx;
      sy = -sy;
    }
    const float a0 = v[0], b0 = v[1], a1 = v[2], b1 = v[3];
    v[0] = a0 * cx - b0 * sx;
    v[1] = a0 * sx + b0 * cx;
    v[2] = a1 * cy - b1 * sy;
    v[3] = a1 * sy + b1 * cy;
  }
};

// Register-staged copy of one [64 x width] token tile: 16-byte vectors,
// row-major, vector idx = tid + i * 256.  Rows at or past T load as zero.
template <typename E, int MAXW>
struct RowTile {
  static constexpr int VEC = 16 / (int)sizeof(E);
  static constexpr int SLOTS = (TT * MAXW / VEC + 255) / 256;
  uint4 r[SLOTS];
  int rc[SLOTS];  // row | column << 8, or -1 for an unused slot

  __device__ __forceinline__ void init(int width, int tid) {
    const int per_row = width / VEC;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / per_row;
      rc[i] = idx < TT * per_row ? row | (((idx - row * per_row) * VEC) << 8) : -1;
    }
  }
  __device__ __forceinline__ void fetch(const Rows<E>& src, int t0, int T) {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      r[i] = make_uint4(0u, 0u, 0u, 0u);
      if (rc[i] >= 0 && t0 + (rc[i] & 255) < T) r[i] = *(const uint4*)(src.at(t0 + (rc[i] & 255)) + (rc[i] >> 8));
    }
  }
  __device__ __forceinline__ void store(E* dst, int pitch) const {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i)
      if (rc[i] >= 0) *(uint4*)(dst + (rc[i] & 255) * pitch + (rc[i] >> 8)) = r[i];
  }
  // Branch-free fetch: every slot loads, rows clamped to tmax - 1 (1 <= tmax
  // <= T) and unused slots reading column 0, so the loads issue as one
  // straight-line sequence and the compiler's wait for a load issued before
  // them need not wait for them.  store_valid() zeroes the rows at or past T.
  __device__ __forceinline__ void fetch_all(const Rows<E>& src, int t0, int tmax) {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int rcv = rc[i] < 0 ? 0 : rc[i];
      r[i] = *(const uint4*)(src.at(min(t0 + (rcv & 255), tmax - 1)) + (rcv >> 8));
    }
  }
  __device__ __forceinline__ void store_valid(E* dst, int pitch, int t0, int T) const {
    if (t0 + TT <= T) {  // a whole group (uniform): every row is valid
      store(dst, pitch);
      return;
    }
#pragma unroll
    for (int i = 0; i < SLOTS; ++i)
      if (rc[i] >= 0)
        *(uint4*)(dst + (rc[i] & 255) * pitch + (rc[i] >> 8)) =
            t0 + (rc[i] & 255) < T ? r[i] : make_uint4(0u, 0u, 0u, 0u);
  }
};

// The same for the 16 rows of a [64 x width] token tile that one wave
// computes (rows 16w .. 16w+15, vector idx = lane + i * 64), so that a wave
// that fills, reads and writes back only its own rows needs no workgroup
// barrier for them.
template <typename E, int MAXW>
struct WaveRows {
  static constexpr int VEC = 16 / (int)sizeof(E);
  static constexpr int SLOTS = (16 * MAXW / VEC + 63) / 64;
  uint4 r[SLOTS];
  int rc[SLOTS];  // row | column << 8, or -1 for an unused slot

  __device__ __forceinline__ void init(int width, int w, int lane) {
    const int per_row = width / VEC;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int idx = lane + i * 64;
      const int row = per_row ? idx / per_row : 0;
      rc[i] = idx < 16 * per_row ? (16 * w + row) | (((idx - row * per_row) * VEC) << 8) : -1;
    }
  }
  // Every slot loads (rows clamped to tmax - 1, 1 <= tmax <= T; unused slots
  // read the wave's first row), one straight-line sequence of loads.
  __device__ __forceinline__ void fetch_all(const Rows<E>& src, int t0, int tmax) {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int rcv = rc[i] < 0 ? (rc[0] & 255) : rc[i];
      r[i] = *(const uint4*)(src.at(min(t0 + (rcv & 255), tmax - 1)) + (rcv >> 8));
    }
  }
  __device__ __forceinline__ void store_valid(E* dst, int pitch, int t0, int T) const {
    const bool whole = t0 + TT <= T;  // uniform
#pragma unroll
    for (int i = 0; i < SLOTS; ++i)
      if (rc[i] >= 0)
        *(uint4*)(dst + (rc[i] & 255) * pitch + (rc[i] >> 8)) =
            whole || t0 + (rc[i] & 255) < T ? r[i] : make_uint4(0u, 0u, 0u, 0u);
  }
};

// LDS rows 16w .. 16w+15 of a [64 x width] tile -> global rows (rows past T
// dropped); one wave.
template <typename E>
__device__ __forceinline__ void write_rows_wave(const E* src, int pitch, const Rows<E>& dst, int t0, int T, int width,
                                                int w, int lane) {
  constexpr int VEC = 16 / (int)sizeof(E);
  const int per_row = width / VEC;
  for (int idx = lane; idx < 16 * per_row; idx += 64) {
    const int row = 16 * w + idx / per_row;
    const int c = (idx - (idx / per_row) * per_row) * VEC;
    if (t0 + row < T) *(uint4*)(dst.at(t0 + row) + c) = *(const uint4*)(src + row * pitch + c);
  }
}

// LDS rows of a [64 x width] tile -> global rows t0.. (rows past T dropped).
template <typename E>
__device__ __forceinline__ void write_rows(const E* src, int pitch, const Rows<E>& dst, int t0, int T, int width,
                                           int tid) {
  constexpr int VEC = 16 / (int)sizeof(E);
  const int per_row = width / VEC;
  for (int idx = tid; idx < TT * per_row; idx += 256) {
    const int row = idx / per_row;
    const int c = (idx - row * per_row) * VEC;
    if (t0 + row < T) *(uint4*)(dst.at(t0 + row) + c) = *(const uint4*)(src + row * pitch + c);
  }
}

// acc[fb] = (W1 xn^T) block fb: lane holds token l16, features 16fb+4g+i.
// W1 rows (length D) start every `wp` elements.
template <typename E, int D, int MB>
__device__ __forceinline__ void gemm_a(const E* w1, int wp, const E* xs, int xp, int l16, int g, int nfb,
                                       floatx4* acc) {
  typedef LdsIO<E> IO;
  const E* xrow = xs + l16 * xp;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb) {
    acc[fb] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (fb < nfb) {
      const E* wrow = w1 + (fb * 16 + l16) * wp;
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk)
        acc[fb] = mma32(IO::ld8(wrow + kk * 32 + 8 * g), IO::ld8(xrow + kk * 32 + 8 * g), acc[fb]);
      if (D % 32)
        acc[fb] = mma16(IO::ld4(wrow + (D / 32) * 32 + 4 * g), IO::ld4(xrow + (D / 32) * 32 + 4 * g), acc[fb]);
    }
  }
}

// out[db] = Wt x reg^T where reg holds the accumulator fragments of a
// [m x 16 tokens] tile: out lane = token, rows 16db+4g+i.  Wt is [D x m]
// with rows every `wp` elements.
template <typename E, int D, int MB>
__device__ __forceinline__ void gemm_back(const E* wt, int wp, const floatx4* reg, int l16, int g, int nfb,
                                          floatx4* out) {
  typedef LdsIO<E> IO;
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    out[db] = floatx4{0.f, 0.f, 0.f, 0.f};
    const E* wrow = wt + (db * 16 + l16) * wp;
#pragma unroll
    for (int j = 0; j < MB / 2; ++j) {
      if (2 * j + 1 < nfb)
        out[db] = mma32(IO::cat(IO::ld4(wrow + 32 * j + 4 * g), IO::ld4(wrow + 32 * j + 16 + 4 * g)),
                        IO::from_acc(reg[2 * j], reg[2 * j + 1]), out[db]);
    }
    if (nfb & 1) {
      const int j = nfb - 1;
#pragma unroll
      for (int jj = 0; jj < MB; ++jj)
        if (jj == j) out[db] = mma16(IO::ld4(wrow + 16 * jj + 4 * g), IO::from_acc4(reg[jj]), out[db]);
    }
  }
}

// Token-axis MFMA fragment of a token-major LDS tile: column c0 + (lane & 15),
// tokens {32kp+4g..+3} and {32kp+16+4g..+3} for lane group g.  bf16 uses the
// gfx950 transposing LDS read (ds_read_b64_tr_b16: within each 16-lane
// group, lane j addresses row r0 + j/4, column c0 + 4*(j%4); lane i receives
// rows r0..r0+3 of column c0 + i).
template <typename E> struct TokFrag;
template <> struct TokFrag<bf16> {
  typedef short shortx4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) shortx4 lds_shortx4;
  static __device__ __forceinline__ bf16x8 get(const bf16* rows, int pitch, int c0, int kp, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const bf16* a = rows + (32 * kp + 4 * g + (j >> 2)) * pitch + c0 + 4 * (j & 3);
    shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)a);
    shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(a + 16 * pitch));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};
template <> struct TokFrag<float> {
  static __device__ __forceinline__ floatx8 get(const float* rows, int pitch, int c0, int kp, int lane) {
    const int g = lane >> 4, l16 = lane & 15;
    floatx8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = 32 * kp + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4);
      v[e] = rows[tok * pitch + c0 + l16];
    }
    return v;
  }
};

// Copy a [rows x cols] row-major global matrix into LDS rows of pitch `pitch`.
template <typename E>
__device__ __forceinline__ void stage_matrix(const E* src, int rows, int cols, E* dst, int pitch, int tid) {
  constexpr int VEC = 16 / (int)sizeof(E);
  const int per_row = cols / VEC;
  for (int idx = tid; idx < rows * per_row; idx += 256) {
    const int r = idx / per_row, c = (idx - r * per_row) * VEC;
    *(uint4*)(dst + r * pitch + c) = *(const uint4*)(src + r * cols + c);
  }
}

// Copy a [rows x cols] row-major global matrix transposed into LDS: row c of
// the destination (pitch `pitch`) is column c of the source.
template <typename E>
__device__ __forceinline__ void stage_transposed(const E* src, int rows, int cols, E* dst, int pitch, int tid) {
  for (int idx = tid; idx < rows * cols; idx += 256) {
    const int r = idx / cols, c = idx - r * cols;
    dst[c * pitch + r] = src[idx];
  }
}

}  // namespace ts
