// Chunked exact linear-attention scan for gfx950 (MI355X).
//
// One view of the reference's chunk backend
// (src/thetascan/_core/ops/scan_chunk.py:246-339): the sequence is cut into
// 64-token tiles; inside a tile the causal score block is a bf16 (or fp32)
// MFMA contraction with fp32 accumulation, and across tiles an fp32
// [dk, dv] state carries everything already written.
//
// Work decomposition (one workgroup per (batch*head, segment)):
//   1. summary kernel : each segment of `seg_chunks` tiles folds its own
//                       writes into a local state U_p (no queries needed);
//   2. prefix kernel  : exclusive scan of U_p over segments with the decay
//                       of each segment -> the state entering every segment;
//   3. main kernel    : each segment re-walks its tiles from that incoming
//                       state and writes the outputs.
// This turns B*H sequential scans (64 at the benchmark shape) into B*H*nseg
// independent workgroups so the whole chip is busy.
//
// Inside a workgroup wave w owns value block w (16 value columns): it holds
// the state S[:, 16w:16w+16] in registers (MFMA accumulator layout) and
// produces out[:, 16w:16w+16].  The score tile is computed once and shared
// through LDS.  Orientation (O^T = S^T Q^T + V^T P^T, S += K_w^T V) is chosen
// so the register state feeds the next MFMA directly as an operand, with the
// contraction index permuted consistently in both operands.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace ts {

constexpr int C = 64;  // tokens per tile

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
  int B, H, T, dk, dv, dvp;
  int nchunks, seg_chunks, nseg, nsum;
  int ret, reverse;
  int q_ext, k_ext, v_ext;
  int out_mode;
  float out_scale;
  ts_strided q, k, v, qe, ke, ve, decay, out, oe;
  // bytes spanned by one (batch, head) slice of each tensor
  uint32_t q_rec, k_rec, v_rec, qe_rec, ke_rec, ve_rec, dec_rec, out_rec, oe_rec;
  const float* log_alpha;
  float* seg;     // [BH][nseg][DKP][dvp]
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

// Token-axis operand fragments.  Contractions over the 64 tokens of a tile
// are split into two 32-token halves kp; within a half, lane group g = lane/16
// supplies the tokens {4g..4g+3} and {16+4g..16+4g+3} (offset 32kp).  This is
// exactly the token set that the accumulator fragment of a 16x16 score block
// holds per lane (rows 4g..4g+3 of key blocks 2kp and 2kp+1), so score
// fragments feed the P.V contraction without a shuffle.
//
// bf16: tiles stay row-major in LDS and the fragment is read with the gfx950
// LDS transpose read (ds_read_b64_tr_b16): within each 16-lane group, lane j
// addresses row r0 + j/4, column c0 + 4*(j%4), and lane i receives
// M[r0 .. r0+3][c0 + i].
// fp32: tiles are additionally stored transposed ([feature][token]).
template <typename E> struct Tiles;

template <> struct Tiles<bf16> {
  static constexpr bool kTransposedCopy = false;
  // lane: column c0 + (lane & 15), the eight tokens of half kp for group lane >> 4
  static __device__ __forceinline__ bf16x8 tcol8(const bf16* rows, int pitch, int c0, int kp, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const bf16* a = rows + (32 * kp + 4 * g + (j >> 2)) * pitch + c0 + 4 * (j & 3);
    shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)a);
    shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(a + 16 * pitch));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

template <> struct Tiles<float> {
  static constexpr bool kTransposedCopy = true;
  static __device__ __forceinline__ floatx8 tcol8(const float* cols, int pitch, int c0, int kp, int lane) {
    const int g = lane >> 4, l16 = lane & 15;
    const float* a = cols + (c0 + l16) * pitch + 32 * kp + 4 * g;
    return LdsIO<float>::cat(LdsIO<float>::ld4(a), LdsIO<float>::ld4(a + 16));
  }
};

// Feature-axis fragment of row `row` for contraction block j (32 features):
// features {32j+4g..+3} and {32j+16+4g..+3}, the order in which the state's
// accumulator fragments S[2j], S[2j+1] hold them.
template <typename E>
__device__ __forceinline__ typename Frag<E>::f8 frow8(const E* rows, int pitch, int row, int j, int g) {
  const E* a = rows + row * pitch + 32 * j + 4 * g;
  return LdsIO<E>::cat(LdsIO<E>::ld4(a), LdsIO<E>::ld4(a + 16));
}
template <typename E>
__device__ __forceinline__ typename Frag<E>::f4 frow4(const E* rows, int pitch, int row, int j, int g) {
  return LdsIO<E>::ld4(rows + row * pitch + 32 * j + 4 * g);
}

// Register-staged loader (bf16) of one tile section (Q, K or V rows): each
// thread owns SLOTS 16-byte vectors, vector idx = tid + i * NT, row-major over
// the section's padded width.  Section sizes are multiples of 64 vectors, so
// whether slot i is in range is uniform per wave.  Per slot only the row and
// column (meta) and the byte offset of that row in tile 0 are kept; a tile
// adds a uniform offset.
template <typename E, int SLOTS>
struct SecLoader {
  static constexpr int VEC = 16 / (int)sizeof(E);
  uint32_t off0[SLOTS];  // data (or ext column) byte offset at tile t = 0
  int meta[SLOTS];       // row | c0 << 8 | kind << 16 ; kind 0 data, 1 ext ones, 2 ext array, 3 pad
  uint4 r[SLOTS];
  float ev[SLOTS];

  __device__ __forceinline__ static int kind_of(int c0, int width, int ext_mode) {
    return c0 < width ? 0 : (c0 == width && ext_mode != TS_EXT_NONE ? ext_mode : 3);
  }
  __device__ __forceinline__ void setup(const ScanP& p, int n, int per_row, int width, int ext_mode, int st_b,
                                        int est_b, int tid, int NT) {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int idx = tid + i * NT;
      const int row = idx / per_row;
      const int c0 = (idx - row * per_row) * VEC;
      const int kind = idx < n ? kind_of(c0, width, ext_mode) : 3;
      meta[i] = (row & 255) | (c0 << 8) | (kind << 16);
      off0[i] = kind == 0 ? row_off(p, 0, row, st_b) + (uint32_t)(c0 * sizeof(E))
                          : (kind == TS_EXT_ARRAY ? row_off(p, 0, row, est_b) : kOOB);
    }
  }
  // Registers <- rows of the tile starting at t0.
  __device__ __forceinline__ void fetch(const ScanP& p, rsrc_t data, rsrc_t ext, int ext_mode, int n, int st_b,
                                        int est_b, int t0, int sgn, int wave_first, int NT) {
    const uint32_t delta = (uint32_t)(sgn * t0 * st_b);
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      if (wave_first + i * NT >= n) break;  // uniform
      const int kind = meta[i] >> 16;
      r[i] = bld16(data, kind == 0 ? off0[i] + delta : kOOB);
      if (ext_mode == TS_EXT_ARRAY) {
        const uint32_t edelta = (uint32_t)(sgn * t0 * est_b);
        ev[i] = bldf(ext, kind == TS_EXT_ARRAY ? off0[i] + edelta : kOOB);
      } else if (ext_mode == TS_EXT_ONES) {
        ev[i] = (t0 + (meta[i] & 255) < p.T) ? 1.0f : 0.0f;
      }
    }
  }
  // LDS rows (pitch in elements) <- registers.
  __device__ __forceinline__ void store(E* dst, int pitch, int ext_mode, int n, int wave_first, int NT) {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      if (wave_first + i * NT >= n) break;  // uniform
      const int m = meta[i];
      const int row = m & 255, c0 = (m >> 8) & 255, kind = m >> 16;
      Vec16<E> val;
      val.raw = r[i];
      if (ext_mode != TS_EXT_NONE && (kind == TS_EXT_ONES || kind == TS_EXT_ARRAY)) val.e[0] = cvt<E>(ev[i]);
      *(uint4*)(dst + row * pitch + c0) = val.raw;
    }
  }
};

// Slots per thread for a section of `width` padded columns when the kernel
// runs `nt_min` or more threads.
constexpr int sec_slots(int width, int vec, int nt_min) { return (C * width / vec + nt_min - 1) / nt_min; }
constexpr int nt_min_of(int maxw) { return maxw == 4 ? 256 : (maxw == 5 ? 320 : 384); }
// V-section slots: the largest over the value widths a kernel with `maxw`
// waves serves (one wave per 16 value columns, at least four waves).
constexpr int v_slots(int maxw, int vec) {
  int best = 1;
  for (int dvp = maxw == 4 ? 16 : (maxw == 5 ? 80 : 96); dvp <= maxw * 16; dvp += 16) {
    const int nt = (dvp / 16 < 4 ? 4 : dvp / 16) * 64;
    const int s = (C * dvp / vec + nt - 1) / nt;
    if (s > best) best = s;
  }
  return best;
}

// GEN = false compiles the common case only: no retention, no ext columns,
// plain stores, no ext output (the host picks it whenever a call allows).
template <typename E, int DKP, bool MAIN, int MAXW, bool GEN>
__global__ __launch_bounds__(MAXW * 64) void scan_kernel(ScanP p) {
  typedef typename Frag<E>::f8 F8;
  typedef typename Frag<E>::f4 F4;
  typedef LdsIO<E> IO;
  typedef Tiles<E> TL;
  constexpr int ES = (int)sizeof(E);
  constexpr int VEC = 16 / ES;
  constexpr bool QREG = MAIN && ES == 2 && DKP <= 80;  // Q fragments straight from HBM to registers
  constexpr bool QLDS = MAIN && !QREG;                 // Q staged through LDS
  constexpr int STAGES = ES == 2 ? 2 : 1;
  constexpr int KP = DKP + VEC;  // row pitch of Q / K tiles (elements)
  constexpr int TP = C + VEC;    // row pitch of transposed copies (fp32)
  constexpr int NK32 = DKP / 32;
  constexpr bool KTAIL = (DKP % 32) != 0;
  constexpr int NKB = DKP / 16;
  constexpr int SLOTS_K = sec_slots(DKP, VEC, nt_min_of(MAXW));
  constexpr int SLOTS_V = v_slots(MAXW, VEC);

  const int ret = GEN ? p.ret : TS_RET_NONE;
  const int q_ext = GEN ? p.q_ext : TS_EXT_NONE;
  const int k_ext = GEN ? p.k_ext : TS_EXT_NONE;
  const int v_ext = GEN ? p.v_ext : TS_EXT_NONE;
  const int out_mode = GEN ? p.out_mode : TS_OUT_STORE;
  const bool has_oe = GEN && p.oe.ptr != nullptr;

  const int tid = threadIdx.x;
  const int NT = blockDim.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 4;
  const int l16 = lane & 15;
  const int seg = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int dvp = p.dvp;
  const int NWV = dvp >> 4;
  const bool owner = w < NWV;
  const int VP = dvp + VEC;  // row pitch of V tiles (bf16)
  const int sgn = p.reverse ? -1 : 1;

  // ---- LDS carve-up
  extern __shared__ __align__(16) unsigned char smem[];
  const int q_elems = QLDS ? C * KP : 0;
  const int k_elems = C * KP;
  const int kt_elems = TL::kTransposedCopy ? DKP * TP : 0;
  const int v_elems = TL::kTransposedCopy ? dvp * TP : C * VP;
  const int stage_elems = q_elems + k_elems + kt_elems + v_elems;
  E* stage0 = (E*)smem;
  float* s_pw = (float*)(stage0 + STAGES * stage_elems);  // alpha^d, d = 0..64 (static)
  float* s_lloc = s_pw + 68;                              // per-wave tile log-decay (stream)
  float* my_lloc = s_lloc + w * C;

  // ---- per-(b, h) addressing.  Section 0 is Q, 1 is K, 2 is V.
  auto sec_stream = [&](int sec) -> const ts_strided& { return sec == 0 ? p.q : (sec == 1 ? p.k : p.v); };
  const int nq_vec = QLDS ? C * (DKP / VEC) : 0;
  const int nk_vec = C * (DKP / VEC);
  const int nv_vec = C * (dvp / VEC);
  const int n_vec = nq_vec + nk_vec + nv_vec;
  const int64_t bh_q = (int64_t)b * p.q.sb + (int64_t)h * p.q.sh;
  const int64_t bh_k = (int64_t)b * p.k.sb + (int64_t)h * p.k.sh;
  const int64_t bh_v = (int64_t)b * p.v.sb + (int64_t)h * p.v.sh;
  // Buffer resources are rebuilt where used from these scalars, so they do
  // not stay live in scalar registers across the tile loop.
  auto data_rsrc = [&](int sec) -> rsrc_t {
    if (sec == 0) return make_rsrc((const E*)p.q.ptr + bh_q, p.q_rec);
    if (sec == 1) return make_rsrc((const E*)p.k.ptr + bh_k, p.k_rec);
    return make_rsrc((const E*)p.v.ptr + bh_v, p.v_rec);
  };
  auto ext_rsrc = [&](int sec) -> rsrc_t {
    const ts_strided& e = sec == 0 ? p.qe : (sec == 1 ? p.ke : p.ve);
    const uint32_t rec = sec == 0 ? p.qe_rec : (sec == 1 ? p.ke_rec : p.ve_rec);
    return make_rsrc(bh_base(e, b, h, 4), rec);
  };
  auto ext_mode_of = [&](int sec) -> int { return sec == 0 ? q_ext : (sec == 1 ? k_ext : v_ext); };
  auto st_bytes = [&](int sec) -> int { return (int)sec_stream(sec).st * ES; };
  auto est_bytes = [&](int sec) -> int { return (int)(sec == 0 ? p.qe.st : (sec == 1 ? p.ke.st : p.ve.st)) * 4; };
  auto width_of = [&](int sec) -> int { return sec == 2 ? p.dv : p.dk; };
  auto per_row_of = [&](int sec) -> int { return sec == 2 ? dvp / VEC : DKP / VEC; };

  // ---- retention addressing
  const int dec_st_b = (int)p.decay.st * 4;
  // a(s), the decay applied when stepping into logical position s: a reversed
  // scan steps from physical s+1 down to s and uses the decay of the physical
  // successor (logical s = 0 has none).
  auto decay_of = [&](int t0) -> float {
    const int s = t0 + lane;
    const int src = p.reverse ? p.T - s : s;
    const uint32_t off = (s < p.T && src < p.T) ? (uint32_t)(src * dec_st_b) : kOOB;
    return bldf(make_rsrc(bh_base(p.decay, b, h, 4), p.dec_rec), off);
  };

  // ---- state
  floatx4 S[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) S[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
  bool state_zero = true;
  if (MAIN && seg > 0) {
    state_zero = false;
    if (owner) {
      const float* src = p.seg + ((size_t)bh * p.nseg + seg) * (size_t)(DKP * dvp);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[kb][i] = src[(kb * 16 + 4 * g + i) * dvp + w * 16 + l16];
    }
  }
  const float la = ret == TS_RET_STATIC ? p.log_alpha[h] : 0.0f;
  if (ret == TS_RET_STATIC && w == 0) {
    s_pw[lane] = expf(la * (float)lane);
    if (lane == 0) s_pw[64] = expf(la * 64.0f);
  }

  const int c_begin = seg * p.seg_chunks;
  const int c_end = min(c_begin + p.seg_chunks, p.nchunks);
  float seg_log = 0.0f;

  // ---- tile loading --------------------------------------------------------
  const int wave_first = __builtin_amdgcn_readfirstlane(tid & ~63);
  SecLoader<E, QLDS ? SLOTS_K : 1> ldq;
  SecLoader<E, SLOTS_K> ldk;
  SecLoader<E, SLOTS_V> ldv;
  if constexpr (STAGES == 2) {
    if constexpr (QLDS)
      ldq.setup(p, nq_vec, DKP / VEC, p.dk, q_ext, st_bytes(0), est_bytes(0), tid, NT);
    ldk.setup(p, nk_vec, DKP / VEC, p.dk, k_ext, st_bytes(1), est_bytes(1), tid, NT);
    ldv.setup(p, nv_vec, dvp / VEC, p.dv, v_ext, st_bytes(2), est_bytes(2), tid, NT);
  }
  // Registers <- tile starting at t0.
  auto fetch = [&](int t0) {
    if constexpr (QLDS)
      ldq.fetch(p, data_rsrc(0), ext_rsrc(0), q_ext, nq_vec, st_bytes(0), est_bytes(0), t0, sgn, wave_first, NT);
    ldk.fetch(p, data_rsrc(1), ext_rsrc(1), k_ext, nk_vec, st_bytes(1), est_bytes(1), t0, sgn, wave_first, NT);
    ldv.fetch(p, data_rsrc(2), ext_rsrc(2), v_ext, nv_vec, st_bytes(2), est_bytes(2), t0, sgn, wave_first, NT);
  };
  // Stage `st` <- registers.
  auto store = [&](int st) {
    E* base = stage0 + st * stage_elems;
    if constexpr (QLDS) ldq.store(base, KP, q_ext, nq_vec, wave_first, NT);
    ldk.store(base + q_elems, KP, k_ext, nk_vec, wave_first, NT);
    ldv.store(base + q_elems + k_elems + kt_elems, VP, v_ext, nv_vec, wave_first, NT);
  };
  // fp32: synchronous load of tile t0 into the single stage (row-major Q, K;
  // transposed K^T, V^T).
  auto load_sync = [&](int t0) {
    E* Qs = stage0;
    E* Ks = Qs + q_elems;
    E* KTs = Ks + k_elems;
    E* VTs = KTs + kt_elems;
    for (int idx = tid; idx < n_vec; idx += NT) {
      const int sec = idx < nq_vec ? 0 : (idx < nq_vec + nk_vec ? 1 : 2);
      const int j = idx - (sec == 2 ? nq_vec + nk_vec : (sec == 1 ? nq_vec : 0));
      const int per_row = per_row_of(sec);
      const int row = j / per_row;
      const int c0 = (j - row * per_row) * VEC;
      const int kind = SecLoader<E, 1>::kind_of(c0, width_of(sec), ext_mode_of(sec));
      Vec16<E> val;
      val.raw = bld16(data_rsrc(sec), kind == 0 ? row_off(p, t0, row, st_bytes(sec)) + (uint32_t)(c0 * ES) : kOOB);
      if (kind == TS_EXT_ARRAY) val.e[0] = cvt<E>(bldf(ext_rsrc(sec), row_off(p, t0, row, est_bytes(sec))));
      if (kind == TS_EXT_ONES) val.e[0] = cvt<E>(t0 + row < p.T ? 1.0f : 0.0f);
      if (sec == 0) {
        *(uint4*)(Qs + row * KP + c0) = val.raw;
      } else if (sec == 1) {
        *(uint4*)(Ks + row * KP + c0) = val.raw;
#pragma unroll
        for (int e = 0; e < VEC; ++e) KTs[(c0 + e) * TP + row] = val.e[e];
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) VTs[(c0 + e) * TP + row] = val.e[e];
      }
    }
  };

  // ---- Q fragments in registers (bf16, narrow keys)
  constexpr int NQJ = QREG ? NK32 : 1;
  F8 qr[4][NQJ];
  F4 qt[4];
  const int q_st_b = (int)p.q.st * ES;
  auto qload = [&](int t0, int qb) {
    if constexpr (QREG) {
      const uint32_t ro = row_off(p, t0, qb * 16 + l16, q_st_b);
      float qev = 0.0f;
      if (q_ext == TS_EXT_ARRAY) qev = bldf(ext_rsrc(0), row_off(p, t0, qb * 16 + l16, est_bytes(0)));
      else if (q_ext == TS_EXT_ONES) qev = t0 + qb * 16 + l16 < p.T ? 1.0f : 0.0f;
      auto part = [&](int c) -> bf16x4 {
        uint2 raw = bld8(data_rsrc(0), c < p.dk ? ro + (uint32_t)(c * ES) : kOOB);
        bf16x4 v = __builtin_bit_cast(bf16x4, raw);
        if (q_ext != TS_EXT_NONE && c == p.dk) v[0] = (bf16)qev;
        return v;
      };
#pragma unroll
      for (int j = 0; j < NK32; ++j) qr[qb][j] = IO::cat(part(32 * j + 4 * g), part(32 * j + 16 + 4 * g));
      if (KTAIL) qt[qb] = part(32 * NK32 + 4 * g);
    }
  };

  // ---- output addressing
  const int osz = out_mode == TS_OUT_STORE ? ES : 4;
  const void* out_base = bh_base(p.out, b, h, osz);
  const int out_st_b = (int)p.out.st * osz;
  const int oe_st_b = (int)p.oe.st * 4;
  const int ocol = w * 16 + 4 * g;  // first of this lane's 4 value columns
  const uint32_t ocol_off = ocol < p.dv ? (uint32_t)(ocol * osz) : kOOB;
  const int oext_r = p.dv - ocol;   // 0..3 if this lane holds the ext column

  // ---- prologue
  float dcur = 0.0f, dnext = 0.0f;
  if constexpr (STAGES == 2) {
    fetch(c_begin * C);
    if constexpr (QREG) {
#pragma unroll
      for (int qb = 0; qb < 4; ++qb) qload(c_begin * C, qb);
    }
    if (ret == TS_RET_STREAM && owner) dnext = decay_of(c_begin * C);
    store(c_begin & 1);
    if (c_begin + 1 < c_end) fetch((c_begin + 1) * C);
    __syncthreads();
  }

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * C;
    const int len = min(C, p.T - t0);
    const E* base;
    if constexpr (STAGES == 2) {
      if (c + 1 < c_end) store((c + 1) & 1);
      if (c + 2 < c_end) fetch(t0 + 2 * C);
      base = stage0 + (c & 1) * stage_elems;
      if (ret == TS_RET_STREAM && owner) {
        dcur = dnext;
        if (c + 1 < c_end) dnext = decay_of(t0 + C);
      }
    } else {
      __syncthreads();  // the previous tile is no longer read
      load_sync(t0);
      if (ret == TS_RET_STREAM && owner) dcur = decay_of(t0);
      __syncthreads();
      base = stage0;
    }
    const E* Qs = base;
    const E* Ks = base + q_elems;
    const E* KTs = Ks + k_elems;
    const E* Vs = KTs + kt_elems;
    const E* Kt_src = TL::kTransposedCopy ? KTs : Ks;
    const int kt_pitch = TL::kTransposedCopy ? TP : KP;
    const int vt_pitch = TL::kTransposedCopy ? TP : VP;

    // ---- retention of this tile (per wave)
    float tile_log = 0.0f;
    if (ret == TS_RET_STATIC) {
      tile_log = la * (float)len;
    } else if (ret == TS_RET_STREAM && owner) {
      float x = dcur;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        float y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      my_lloc[lane] = x;
      tile_log = __shfl(x, len - 1, 64);
    }
    seg_log += tile_log;

    if (owner) {
      // value fragments of this wave's 16 columns, both token halves
      F8 av[2];
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) av[kp] = TL::tcol8(Vs, vt_pitch, w * 16, kp, lane);

      if constexpr (MAIN) {
        F8 sA[NK32 > 0 ? NK32 : 1];
        F4 sT;
        if (!state_zero) {
#pragma unroll
          for (int j = 0; j < NK32; ++j) sA[j] = IO::from_acc(S[2 * j], S[2 * j + 1]);
          if (KTAIL) sT = IO::from_acc4(S[NKB - 1]);
        }
#pragma unroll
        for (int qb = 0; qb < 4; ++qb) {
          const int query = qb * 16 + l16;
          auto qfrag = [&](int j) -> F8 {
            if constexpr (QREG) return qr[qb][j];
            else return frow8<E>(Qs, KP, query, j, g);
          };
          auto qtail = [&]() -> F4 {
            if constexpr (QREG) return qt[qb];
            else return frow4<E>(Qs, KP, query, NK32, g);
          };
          float lq = 0.0f;
          if (ret == TS_RET_STREAM) lq = my_lloc[query];
          // causal score blocks (key block kb <= qb): D[key][query]
          floatx4 sc[4];
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            sc[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (kb > qb) continue;
            const int krow = kb * 16 + l16;
#pragma unroll
            for (int j = 0; j < NK32; ++j) sc[kb] = mma32(frow8<E>(Ks, KP, krow, j, g), qfrag(j), sc[kb]);
            if (KTAIL) sc[kb] = mma16(frow4<E>(Ks, KP, krow, NK32, g), qtail(), sc[kb]);
            floatx4 lk;
            if (ret == TS_RET_STREAM) lk = *(const floatx4*)(my_lloc + kb * 16 + 4 * g);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = kb * 16 + 4 * g + i;
              float wt = 1.0f;
              if (ret == TS_RET_STATIC) wt = s_pw[max(query - key, 0)];
              else if (ret == TS_RET_STREAM) wt = expf(fminf(lq - lk[i], 0.0f));
              sc[kb][i] = (kb < qb || key <= query) ? sc[kb][i] * wt : 0.0f;
            }
          }
          // O^T = carry * S^T Q^T + V^T P^T
          floatx4 acc = {0.f, 0.f, 0.f, 0.f};
          if (!state_zero) {
#pragma unroll
            for (int j = 0; j < NK32; ++j) acc = mma32(sA[j], qfrag(j), acc);
            if (KTAIL) acc = mma16(sT, qtail(), acc);
            if (ret != TS_RET_NONE) {
              const float cw = ret == TS_RET_STATIC ? s_pw[query + 1] : expf(lq);
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[i] *= cw;
            }
          }
          acc = mma32(av[0], IO::from_acc(sc[0], sc[1]), acc);
          if (qb >= 2) acc = mma32(av[1], IO::from_acc(sc[2], sc[3]), acc);
          if constexpr (QREG) {
            if (c + 1 < c_end) qload(t0 + C, qb);  // next tile's queries of this block
          }

          // ---- output rows
          const uint32_t ro = row_off(p, t0, query, out_st_b);
          if (out_mode == TS_OUT_STORE) {
            if constexpr (ES == 2) {
              bf16x4 o;
#pragma unroll
              for (int i = 0; i < 4; ++i) o[i] = (bf16)acc[i];
              bst8(make_rsrc(out_base, p.out_rec), ro + ocol_off, __builtin_bit_cast(uint2, o));
            } else {
              bst16(make_rsrc(out_base, p.out_rec), ro + ocol_off, __builtin_bit_cast(uint4, acc));
            }
          } else {
            floatx4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = p.out_scale * acc[i];
            if (out_mode == TS_OUT_ACCUM_F32) {
              const floatx4 prev = __builtin_bit_cast(floatx4, bld16(make_rsrc(out_base, p.out_rec), ro + ocol_off));
#pragma unroll
              for (int i = 0; i < 4; ++i) o[i] += prev[i];
            }
            bst16(make_rsrc(out_base, p.out_rec), ro + ocol_off, __builtin_bit_cast(uint4, o));
          }
          if (has_oe && oext_r >= 0 && oext_r < 4) {
            float val = acc[0];
            if (oext_r == 1) val = acc[1];
            if (oext_r == 2) val = acc[2];
            if (oext_r == 3) val = acc[3];
            if (out_mode != TS_OUT_STORE) val *= p.out_scale;
            const uint32_t eo = row_off(p, t0, query, oe_st_b);
            const rsrc_t oe_rs = make_rsrc(bh_base(p.oe, b, h, 4), p.oe_rec);
            if (out_mode == TS_OUT_ACCUM_F32) val += bldf(oe_rs, eo);
            bstf(oe_rs, eo, val);
          }
        }
      }

      // ---- state update: S = decay(tile) * S + K^T diag(wk) V
      F8 avw[2] = {av[0], av[1]};
      if (ret != TS_RET_NONE) {
        const float cdec = ret == TS_RET_STATIC ? s_pw[len] : expf(tile_log);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) S[kb][i] *= cdec;
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
          floatx4 l0, l1;
          if (ret == TS_RET_STREAM) {
            l0 = *(const floatx4*)(my_lloc + 32 * kp + 4 * g);
            l1 = *(const floatx4*)(my_lloc + 32 * kp + 16 + 4 * g);
          }
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int key = 32 * kp + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4);
            float wk = 0.0f;
            if (key < len) {
              if (ret == TS_RET_STATIC) wk = s_pw[len - 1 - key];
              else wk = expf(tile_log - (e < 4 ? l0[e] : l1[e - 4]));
            }
            avw[kp][e] = cvt<E>(tof(av[kp][e]) * wk);
          }
        }
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) S[kb] = mma32(TL::tcol8(Kt_src, kt_pitch, kb * 16, kp, lane), avw[kp], S[kb]);
    }
    state_zero = false;
    if constexpr (STAGES == 2) __syncthreads();
  }

  if constexpr (!MAIN) {
    if (owner) {
      float* dst = p.seg + ((size_t)bh * p.nseg + seg) * (size_t)(DKP * dvp);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[(kb * 16 + 4 * g + i) * dvp + w * 16 + l16] = S[kb][i];
    }
    if (tid == 0) p.segdec[(size_t)bh * p.nseg + seg] = seg_log;
  }
}

// Exclusive scan of the segment summaries:  seg[p] <- state entering segment p.
__global__ void scan_prefix_kernel(float* seg, const float* segdec, float* final_state, int nseg,
                                   int nsum, int nelem) {
  const int bh = blockIdx.y;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nelem) return;
  float* base = seg + (size_t)bh * nseg * nelem + e;
  float carry = 0.0f;
  for (int s = 0; s < nseg; ++s) {
    float u = 0.0f;
    if (s < nsum) u = base[(size_t)s * nelem];
    base[(size_t)s * nelem] = carry;
    if (s < nsum) carry = expf(segdec[(size_t)bh * nseg + s]) * carry + u;
  }
  if (final_state) final_state[(size_t)bh * nelem + e] = carry;
}

}  // namespace ts

// ============================================================== host side
namespace ts {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace ts

namespace {

using ts::fail;

const int kDkPads[] = {32, 64, 80, 128, 144};

int pick_dkp(int need) {
  for (int v : kDkPads)
    if (need <= v) return v;
  return -1;
}

struct Layout {
  int dkp, dvp, nchunks, seg_chunks, nseg, nsum;
  size_t ws_bytes;
};

int compute_layout(const ts_scan_desc* d, Layout* L) {
  if (!d) return fail(TS_ERR_VALUE, "scan: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0) return fail(TS_ERR_VALUE, "scan: bad shape");
  if (d->dk < 1 || d->dv < 1) return fail(TS_ERR_VALUE, "scan: feature widths must be >= 1");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "scan: unknown dtype");
  if (d->retention < TS_RET_NONE || d->retention > TS_RET_STREAM)
    return fail(TS_ERR_VALUE, "scan: unknown retention kind");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  if (d->dk % vec || d->dv % vec)
    return fail(TS_ERR_VALUE, "scan: feature widths must be multiples of 16 bytes (dk=%d dv=%d)",
                d->dk, d->dv);
  const int dk_eff = d->dk + ((d->q_ext != TS_EXT_NONE || d->k_ext != TS_EXT_NONE) ? 1 : 0);
  L->dkp = pick_dkp(dk_eff);
  if (L->dkp < 0) return fail(TS_ERR_NOT_IMPLEMENTED, "scan: key width %d exceeds 144", dk_eff);
  L->dvp = ((d->dv + (d->v_ext != TS_EXT_NONE ? 1 : 0)) + 15) / 16 * 16;
  if (L->dvp > 144) return fail(TS_ERR_NOT_IMPLEMENTED, "scan: value width %d exceeds 144", L->dvp);
  L->nchunks = (d->T + ts::C - 1) / ts::C;
  const int bh = d->B * d->H;
  if (d->seg_chunks > 0) {
    L->seg_chunks = d->seg_chunks;
  } else {
    // Two resident workgroups per CU on 256 CUs.
    int want = 512 / (bh > 0 ? bh : 1);
    if (want < 1) want = 1;
    L->seg_chunks = (L->nchunks + want - 1) / want;
    if (L->seg_chunks < 1) L->seg_chunks = 1;
  }
  L->nseg = L->nchunks > 0 ? (L->nchunks + L->seg_chunks - 1) / L->seg_chunks : 0;
  L->nsum = d->want_final ? L->nseg : (L->nseg > 0 ? L->nseg - 1 : 0);
  L->ws_bytes = 0;
  if (L->nsum > 0)
    L->ws_bytes = (size_t)bh * L->nseg * (size_t)L->dkp * L->dvp * sizeof(float) +
                  (size_t)bh * L->nseg * sizeof(float) + 256;
  return TS_OK;
}

int max_waves(int dvp) {
  const int nw = dvp / 16;
  return nw <= 4 ? 4 : (nw <= 5 ? 5 : 9);
}

int block_threads(int dvp) {
  const int nw = dvp / 16;
  return (nw < 4 ? 4 : nw) * 64;
}

// Dynamic LDS of one workgroup; mirrors the carve-up at the top of scan_kernel.
size_t lds_bytes(int esize, int dkp, int dvp, bool main_kernel) {
  const int vec = 16 / esize;
  const bool qreg = main_kernel && esize == 2 && dkp <= 80;
  const bool qlds = main_kernel && !qreg;
  const int stages = esize == 2 ? 2 : 1;
  const int kp = dkp + vec, tp = ts::C + vec, vp = dvp + vec;
  size_t elems = (qlds ? (size_t)ts::C * kp : 0) + (size_t)ts::C * kp;
  if (esize == 2)
    elems += (size_t)ts::C * vp;
  else
    elems += (size_t)dkp * tp + (size_t)dvp * tp;
  const int nw = block_threads(dvp) / 64;
  return stages * elems * esize + (68 + (size_t)nw * ts::C) * sizeof(float);
}

typedef void (*KernelFn)(ts::ScanP);

template <typename E, int MAXW, bool GEN>
KernelFn pick_kernel_w(int dkp, bool main_kernel) {
  switch (dkp) {
#define TS_CASE(D)                                                                      \
  case D:                                                                               \
    return main_kernel ? (KernelFn)ts::scan_kernel<E, D, true, MAXW, GEN>               \
                       : (KernelFn)ts::scan_kernel<E, D, false, MAXW, GEN>;
    TS_CASE(32)
    TS_CASE(64)
    TS_CASE(80)
    TS_CASE(128)
    TS_CASE(144)
#undef TS_CASE
  }
  return nullptr;
}

// bf16 kernels are specialised by wave count (register budget per launch
// size) and, up to five waves, by whether the call needs the general
// features; the fp32 parity kernels use one general 9-wave build.
KernelFn pick_kernel(bool bf16, int dkp, int dvp, bool main_kernel, bool general) {
  if (!bf16) return pick_kernel_w<float, 9, true>(dkp, main_kernel);
  switch (max_waves(dvp)) {
    case 4:
      return general ? pick_kernel_w<ts::bf16, 4, true>(dkp, main_kernel)
                     : pick_kernel_w<ts::bf16, 4, false>(dkp, main_kernel);
    case 5:
      return general ? pick_kernel_w<ts::bf16, 5, true>(dkp, main_kernel)
                     : pick_kernel_w<ts::bf16, 5, false>(dkp, main_kernel);
    default: return pick_kernel_w<ts::bf16, 9, true>(dkp, main_kernel);
  }
}

// Bytes spanned by one (batch, head) slice of a [.., T, width] stream, or an
// error if rows up to T + one tile could not be addressed with 31-bit offsets.
int slice_bytes(const char* name, const ts_strided& s, int T, int width, int esize, uint32_t* out) {
  *out = 0;
  if (!s.ptr) return TS_OK;
  if (s.st < 0) return fail(TS_ERR_VALUE, "scan: negative time stride of %s", name);
  const int64_t last = ((int64_t)(T > 0 ? T - 1 : 0) * s.st + width) * esize;
  const int64_t reach = ((int64_t)T + 2 * ts::C) * s.st * esize + (int64_t)width * esize;
  if (reach >= ((int64_t)1 << 31))
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan: one (batch, head) slice of %s spans more than 2 GiB", name);
  *out = (uint32_t)last;
  return TS_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_stream(const char* name, const ts_strided& s, int vec, bool required) {
  if (!s.ptr) return required ? fail(TS_ERR_VALUE, "scan: missing tensor %s", name) : TS_OK;
  if (!aligned16(s.ptr)) return fail(TS_ERR_VALUE, "scan: tensor %s is not 16-byte aligned", name);
  if (s.st % vec || s.sh % vec || s.sb % vec)
    return fail(TS_ERR_VALUE, "scan: strides of %s must be multiples of 16 bytes", name);
  return TS_OK;
}

int launch(KernelFn fn, dim3 grid, dim3 block, size_t lds, hipStream_t stream, const ts::ScanP& p) {
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: LDS request failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(fn, grid, block, lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_abi_version(void) { return TS_ABI_VERSION; }

const char* ts_last_error(void) { return ts::g_err; }

int ts_scan_layout(const ts_scan_desc* desc, int32_t* dk_pad, int32_t* dv_pad, int32_t* n_segments) {
  Layout L;
  int rc = compute_layout(desc, &L);
  if (rc) return rc;
  if (dk_pad) *dk_pad = L.dkp;
  if (dv_pad) *dv_pad = L.dvp;
  if (n_segments) *n_segments = L.nseg;
  return TS_OK;
}

int ts_scan_workspace_bytes(const ts_scan_desc* desc, size_t* bytes) {
  Layout L;
  int rc = compute_layout(desc, &L);
  if (rc) return rc;
  if (bytes) *bytes = L.ws_bytes;
  return TS_OK;
}

int ts_scan_fwd(const ts_scan_desc* d, const ts_scan_io* io, void* workspace, size_t ws_bytes,
                hipStream_t stream) {
  Layout L;
  int rc = compute_layout(d, &L);
  if (rc) return rc;
  if (!io) return fail(TS_ERR_VALUE, "scan: null io");
  if (d->T == 0) return TS_OK;
  const int esize = d->dtype == TS_BF16 ? 2 : 4;
  const int vec = 16 / esize;
  if ((rc = check_stream("q", io->q, vec, true))) return rc;
  if ((rc = check_stream("k", io->k, vec, true))) return rc;
  if ((rc = check_stream("v", io->v, vec, true))) return rc;
  const int out_vec = d->out_mode == TS_OUT_STORE ? vec : 4;
  if (!io->out.ptr) return fail(TS_ERR_VALUE, "scan: missing output");
  if (((uintptr_t)io->out.ptr & (d->out_mode == TS_OUT_STORE ? 7u : 15u)) || io->out.st % out_vec ||
      io->out.sh % out_vec || io->out.sb % out_vec)
    return fail(TS_ERR_VALUE, "scan: output rows must be aligned");
  if (d->q_ext == TS_EXT_ARRAY && !io->q_ext.ptr) return fail(TS_ERR_VALUE, "scan: missing q ext column");
  if (d->k_ext == TS_EXT_ARRAY && !io->k_ext.ptr) return fail(TS_ERR_VALUE, "scan: missing k ext column");
  if (d->v_ext == TS_EXT_ARRAY && !io->v_ext.ptr) return fail(TS_ERR_VALUE, "scan: missing v ext column");
  if (d->retention == TS_RET_STATIC && !io->log_alpha) return fail(TS_ERR_VALUE, "scan: missing log_alpha");
  if (d->retention == TS_RET_STREAM && !io->decay.ptr) return fail(TS_ERR_VALUE, "scan: missing decay stream");
  if (d->want_final && !io->final_state) return fail(TS_ERR_VALUE, "scan: missing final_state buffer");
  if (L.ws_bytes > 0 && (!workspace || ws_bytes < L.ws_bytes))
    return fail(TS_ERR_VALUE, "scan: workspace too small (%lld < %lld bytes)", (long long)ws_bytes,
                (long long)L.ws_bytes);

  ts::ScanP p;
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.dk = d->dk; p.dv = d->dv; p.dvp = L.dvp;
  p.nchunks = L.nchunks; p.seg_chunks = L.seg_chunks; p.nseg = L.nseg; p.nsum = L.nsum;
  p.ret = d->retention; p.reverse = d->reverse;
  p.q_ext = d->q_ext; p.k_ext = d->k_ext; p.v_ext = d->v_ext;
  p.out_mode = d->out_mode; p.out_scale = d->out_scale;
  p.q = io->q; p.k = io->k; p.v = io->v;
  p.qe = io->q_ext; p.ke = io->k_ext; p.ve = io->v_ext;
  p.decay = io->decay; p.out = io->out; p.oe = io->out_ext;
  p.log_alpha = io->log_alpha;
  const int osz = d->out_mode == TS_OUT_STORE ? esize : 4;
  if ((rc = slice_bytes("q", p.q, d->T, d->dk, esize, &p.q_rec))) return rc;
  if ((rc = slice_bytes("k", p.k, d->T, d->dk, esize, &p.k_rec))) return rc;
  if ((rc = slice_bytes("v", p.v, d->T, d->dv, esize, &p.v_rec))) return rc;
  if ((rc = slice_bytes("q_ext", p.qe, d->T, 1, 4, &p.qe_rec))) return rc;
  if ((rc = slice_bytes("k_ext", p.ke, d->T, 1, 4, &p.ke_rec))) return rc;
  if ((rc = slice_bytes("v_ext", p.ve, d->T, 1, 4, &p.ve_rec))) return rc;
  if ((rc = slice_bytes("decay", p.decay, d->T, 1, 4, &p.dec_rec))) return rc;
  if ((rc = slice_bytes("out", p.out, d->T, d->dv, osz, &p.out_rec))) return rc;
  if ((rc = slice_bytes("out_ext", p.oe, d->T, 1, 4, &p.oe_rec))) return rc;
  if (L.ws_bytes > 0) {
    p.seg = (float*)workspace;
    p.segdec = p.seg + (size_t)d->B * d->H * L.nseg * (size_t)L.dkp * L.dvp;
  }

  const int bh = d->B * d->H;
  const dim3 block(block_threads(L.dvp));
  const bool general = d->retention != TS_RET_NONE || d->q_ext != TS_EXT_NONE || d->k_ext != TS_EXT_NONE ||
                       d->v_ext != TS_EXT_NONE || d->out_mode != TS_OUT_STORE || io->out_ext.ptr != nullptr;
  KernelFn fsum = pick_kernel(d->dtype == TS_BF16, L.dkp, L.dvp, false, general);
  KernelFn fmain = pick_kernel(d->dtype == TS_BF16, L.dkp, L.dvp, true, general);
  const size_t lds_sum = lds_bytes(esize, L.dkp, L.dvp, false);
  const size_t lds_main = lds_bytes(esize, L.dkp, L.dvp, true);
  if (lds_main > 160 * 1024)
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan: tile of %lld bytes exceeds LDS (dk_pad=%d)",
                (long long)lds_main, L.dkp);

  if (L.nsum > 0) {
    if ((rc = launch(fsum, dim3(L.nsum, bh), block, lds_sum, stream, p))) return rc;
    const int nelem = L.dkp * L.dvp;
    hipLaunchKernelGGL(ts::scan_prefix_kernel, dim3((nelem + 255) / 256, bh), dim3(256), 0, stream, p.seg,
                       p.segdec, d->want_final ? io->final_state : nullptr, L.nseg, L.nsum, nelem);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: prefix launch failed: %s", hipGetErrorString(e));
  }
  return launch(fmain, dim3(L.nseg, bh), block, lds_main, stream, p);
}

}  // extern "C"
