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

// (query block, key block) pairs of the score tile, 2 bits each: the 10
// causal 16x16 blocks, then the two upper blocks read by the 32-key
// contractions of query blocks 0 and 2 (stored as zeros).
constexpr int kScoreBlocks = 12;
constexpr unsigned pack_blocks(const int (&a)[kScoreBlocks]) {
  unsigned r = 0;
  for (int i = 0; i < kScoreBlocks; ++i) r |= (unsigned)a[i] << (2 * i);
  return r;
}
constexpr int kBq[kScoreBlocks] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3, 0, 2};
constexpr int kBk[kScoreBlocks] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3, 1, 3};
constexpr unsigned kBlockQ = pack_blocks(kBq);
constexpr unsigned kBlockK = pack_blocks(kBk);

struct ScanP {
  int B, H, T, dk, dv, dvp;
  int nchunks, seg_chunks, nseg;
  int ret, reverse;
  int q_ext, k_ext, v_ext;
  int out_mode;
  float out_scale;
  ts_strided q, k, v, qe, ke, ve, decay, out, oe;
  const float* log_alpha;
  float* seg;     // [BH][nseg][DKP][dvp]
  float* segdec;  // [BH][nseg]
  int nsum;       // segments that run the summary kernel
};

__device__ __forceinline__ int phys_t(const ScanP& p, int t) { return p.reverse ? p.T - 1 - t : t; }

// Per-tile retention tables (wave 0).  Matches scan_chunk._static_weights
// (scan_chunk.py:102-119) and _tile_weights (scan_chunk.py:122-155): phases
// are formed in fp32, exponents of the intra-tile weight are clamped to <= 0.
//   carry[i] : weight of the incoming state at local position i
//   wk[j]    : weight of key j in the state leaving the tile (after `len` steps)
//   pw[d]    : static weight alpha^d;  lloc[i] : stream tile-local cum. log
//   misc[0]  : log-decay of the whole tile (len steps)
__device__ __forceinline__ void tile_decay(const ScanP& p, int b, int h, int t0, int len, int lane,
                                          float* carry, float* wk, float* pw, float* lloc,
                                          float* misc) {
  if (p.ret == TS_RET_STATIC) {
    const float la = p.log_alpha[h];
    pw[lane] = expf(la * (float)lane);
    carry[lane] = expf(la * (float)(lane + 1));
    wk[lane] = lane < len ? expf(la * (float)(len - 1 - lane)) : 0.0f;
    if (lane == 0) misc[0] = la * (float)len;
  } else {
    // a(s): decay applied when stepping into logical position s.  Reversed
    // scans step from physical s+1 down to s, so they use the decay of the
    // physical successor.
    const int s = t0 + lane;
    float a = 0.0f;
    if (s < p.T) {
      int src = s;
      if (p.reverse) src = (p.T - 1 - s) + 1;
      if (src < p.T)
        a = ((const float*)p.decay.ptr)[(int64_t)b * p.decay.sb + (int64_t)h * p.decay.sh +
                                        (int64_t)src * p.decay.st];
    }
    float x = a;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      float y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    lloc[lane] = x;
    const float last = __shfl(x, len - 1, 64);
    carry[lane] = expf(x);
    wk[lane] = lane < len ? expf(last - x) : 0.0f;
    if (lane == 0) misc[0] = last;
  }
}

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) shortx4 lds_shortx4;

// Staging of the K / V tiles and access to their transposed fragments.
//
// bf16: tiles stay row-major in LDS ([token][feature], 16-byte writes) and
// the token-contiguous fragments that the key-axis contractions need are read
// with the gfx950 LDS transpose read (ds_read_b64_tr_b16).  Within each group
// of 16 lanes, lane j addresses row key0 + j/4, column c0 + 4*(j%4); lane i
// then receives M[key0 .. key0+3][c0 + i], i.e. one column and four
// consecutive tokens -- an MFMA operand fragment.  Two such reads give the
// eight tokens of a 32-deep contraction.
//
// fp32 (the parity path): K and V are additionally stored transposed.
template <typename E> struct Tiles;

template <> struct Tiles<bf16> {
  static constexpr bool kTransposedCopy = false;
  // lane: column c0 + (lane & 15), tokens 32kp + 8*(lane >> 4) + 0..7
  static __device__ __forceinline__ bf16x8 tcol8(const bf16* rows, int pitch, int c0, int kp, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const bf16* a = rows + (32 * kp + 8 * g + (j >> 2)) * pitch + c0 + 4 * (j & 3);
    shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)a);
    shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_shortx4*)(a + 4 * pitch));
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

template <> struct Tiles<float> {
  static constexpr bool kTransposedCopy = true;
  // rows here is the transposed copy [feature][token]
  static __device__ __forceinline__ floatx8 tcol8(const float* cols, int pitch, int c0, int kp, int lane) {
    const int g = lane >> 4, l16 = lane & 15;
    return LdsIO<float>::ld8(cols + (c0 + l16) * pitch + 32 * kp + 8 * g);
  }
};

// Register-staged tile loader.  Each thread owns MAXV 16-byte vectors of the
// next tile (Q rows for MAIN, then K rows, then V rows).  Vector counts per
// tensor are multiples of 64, so the tensor a vector belongs to is uniform
// across a wave; everything that does not change from tile to tile (tensor,
// row, column, ext role, base pointer) is resolved once before the tile loop,
// and a tile only adds its time offset.  The fetch for tile c+1 is issued
// before tile c is computed, so its latency hides behind the MFMA work.
struct LoadSlot {
  const char* base;   // (b, h) row 0 of the tensor, plus the column offset
  const float* ext;   // (b, h) base of the ext column array (or null)
  int64_t st;         // row stride in bytes
  int ext_st;         // row stride of the ext array (elements)
  int row;            // row inside the tile
  int kind;           // 0 data, 1 ext column (ones), 2 ext column (array), 3 zero padding
  int tensor;         // 0 Q, 1 K, 2 V, -1 idle
  int off;            // element offset of the vector inside its LDS row
};

template <typename E, int DKP, bool MAIN, int MAXV>
struct Loader {
  static constexpr int VEC = 16 / (int)sizeof(E);
  uint4 r[MAXV];
  LoadSlot sl[MAXV];

  __device__ __forceinline__ void setup(const ScanP& p, int b, int h, int dvp, int tid, int nt) {
    const int nq = MAIN ? C * (DKP / VEC) : 0;
    const int nk = C * (DKP / VEC);
    const int nv = C * (dvp / VEC);
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      LoadSlot& L = sl[i];
      int idx = tid + i * nt;
      int per_row, width, ext_mode;
      const ts_strided* src;
      const ts_strided* ext;
      if (idx < nq) {
        L.tensor = 0; per_row = DKP / VEC; width = p.dk; ext_mode = p.q_ext; src = &p.q; ext = &p.qe;
      } else if ((idx -= nq) < nk) {
        L.tensor = 1; per_row = DKP / VEC; width = p.dk; ext_mode = p.k_ext; src = &p.k; ext = &p.ke;
      } else if ((idx -= nk) < nv) {
        L.tensor = 2; per_row = dvp / VEC; width = p.dv; ext_mode = p.v_ext; src = &p.v; ext = &p.ve;
      } else {
        L.tensor = -1; per_row = 1; width = 0; ext_mode = 0; src = &p.v; ext = &p.ve;
      }
      L.row = idx / per_row;
      const int c0 = (idx - L.row * per_row) * VEC;
      L.off = c0;
      L.kind = c0 < width ? 0 : (c0 == width && ext_mode != TS_EXT_NONE ? ext_mode : 3);
      L.base = (const char*)src->ptr + ((int64_t)b * src->sb + (int64_t)h * src->sh + c0) * (int64_t)sizeof(E);
      L.st = src->st * (int64_t)sizeof(E);
      L.ext = ext->ptr ? (const float*)ext->ptr + (int64_t)b * ext->sb + (int64_t)h * ext->sh : nullptr;
      L.ext_st = (int)ext->st;
    }
  }

  __device__ __forceinline__ void fetch(const ScanP& p, int t0) {
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      const LoadSlot& L = sl[i];
      const int t = t0 + L.row;
      const int tp = p.reverse ? p.T - 1 - t : t;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (L.tensor >= 0 && t < p.T) {
        if (L.kind == 0) {
          v = *(const uint4*)(L.base + (int64_t)tp * L.st);
        } else if (L.kind != 3) {
          Vec16<E> e;
          e.raw = v;
          e.e[0] = cvt<E>(L.kind == TS_EXT_ARRAY ? L.ext[(int64_t)tp * L.ext_st] : 1.0f);
          v = e.raw;
        }
      }
      r[i] = v;
    }
  }

  __device__ __forceinline__ void store(E* Qs, E* Ks, E* Vs, E* KTs, E* VTs, int qp, int vp, int tp) {
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
      const LoadSlot& L = sl[i];
      Vec16<E> val;
      val.raw = r[i];
      if (L.tensor == 0) {
        *(uint4*)(Qs + L.row * qp + L.off) = val.raw;
      } else if (L.tensor == 1) {
        *(uint4*)(Ks + L.row * qp + L.off) = val.raw;
        if (Tiles<E>::kTransposedCopy) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) KTs[(L.off + e) * tp + L.row] = val.e[e];
        }
      } else if (L.tensor == 2) {
        if (Tiles<E>::kTransposedCopy) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) VTs[(L.off + e) * tp + L.row] = val.e[e];
        } else {
          *(uint4*)(Vs + L.row * vp + L.off) = val.raw;
        }
      }
    }
  }
};

template <typename E, int DKP, bool MAIN, bool WIDE>
__global__ __launch_bounds__(WIDE ? 576 : 256) void scan_kernel(ScanP p) {
  typedef typename Frag<E>::f8 F8;
  typedef LdsIO<E> IO;
  typedef Tiles<E> TL;
  constexpr int VEC = 16 / (int)sizeof(E);
  constexpr int QP = DKP + VEC;  // row pitch of Qs / Ks (elements)
  constexpr int TP = C + VEC;    // row pitch of Ps and of transposed copies
  constexpr int NKB = DKP / 16;  // 16-row key-feature blocks of the state
  constexpr int NK32 = DKP / 32; // full 32-wide contraction blocks over dk
  constexpr bool KTAIL = (DKP % 32) != 0;
  // Worst case of (Q + K + V vectors) / threads with NT = max(256, 4*dvp):
  // ((MAIN ? 2 : 1) * 64 * DKP + 64 * 64) / VEC / 256.
  constexpr int MAXV = ((MAIN ? 2 : 1) * DKP + 64 + 4 * VEC - 1) / (4 * VEC);

  const int dvp = p.dvp;
  const int NWV = dvp / 16;              // waves that own a value block
  const int NT = blockDim.x;
  const int VP = dvp + VEC;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int seg = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const bool owner = w < NWV;
  const int64_t obase = (int64_t)b * p.out.sb + (int64_t)h * p.out.sh;
  const int64_t oebase = (int64_t)b * p.oe.sb + (int64_t)h * p.oe.sh;

  extern __shared__ __align__(16) unsigned char smem[];
  E* Qs = (E*)smem;
  E* Ks = Qs + (MAIN ? C * QP : 0);
  E* Vs = Ks + C * QP;                                   // row-major V (bf16)
  E* KTs = Vs + (TL::kTransposedCopy ? 0 : C * VP);      // transposed copies (fp32)
  E* VTs = KTs + (TL::kTransposedCopy ? DKP * TP : 0);
  E* Ps = VTs + (TL::kTransposedCopy ? dvp * TP : 0);
  float* s_carry = (float*)(Ps + (MAIN ? C * TP : 0));
  float* s_wk = s_carry + C;
  float* s_pw = s_wk + C;
  float* s_lloc = s_pw + C;
  float* s_misc = s_lloc + C;
  const E* Kt_src = TL::kTransposedCopy ? KTs : Ks;
  const E* Vt_src = TL::kTransposedCopy ? VTs : Vs;
  const int kt_pitch = TL::kTransposedCopy ? TP : QP;
  const int vt_pitch = TL::kTransposedCopy ? TP : VP;

  floatx4 S[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) S[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
  bool state_zero = true;
  if (MAIN && seg > 0 && owner) {
    const float* src = p.seg + ((size_t)bh * p.nseg + seg) * (size_t)(DKP * dvp);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[kb][i] = src[(kb * 16 + 4 * g + i) * dvp + w * 16 + l16];
  }
  if (MAIN && seg > 0) state_zero = false;

  const int c_begin = seg * p.seg_chunks;
  const int c_end = min(c_begin + p.seg_chunks, p.nchunks);
  float seg_log = 0.0f;
  Loader<E, DKP, MAIN, MAXV> ld;
  ld.setup(p, b, h, dvp, tid, NT);
  ld.fetch(p, c_begin * C);

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * C;
    const int len = min(C, p.T - t0);
    __syncthreads();  // LDS of the previous tile is no longer read
    ld.store(Qs, Ks, Vs, KTs, VTs, QP, VP, TP);
    if (p.ret != TS_RET_NONE && w == 0)
      tile_decay(p, b, h, t0, len, lane, s_carry, s_wk, s_pw, s_lloc, s_misc);
    __syncthreads();
    if (c + 1 < c_end) ld.fetch(p, t0 + C);  // next tile in flight

    if (MAIN) {
      // ---- causal score tile P[query][key] = w(q,k) <q, k>, shared via LDS.
      const int nw_all = NT >> 6;
      for (int bi = w; bi < kScoreBlocks; bi += nw_all) {
        const int qb = (kBlockQ >> (2 * bi)) & 3;
        const int kb = (kBlockK >> (2 * bi)) & 3;
        const int query = qb * 16 + l16;
        const int key0 = kb * 16 + 4 * g;
        float pv[4] = {0.f, 0.f, 0.f, 0.f};
        if (bi < 10) {
          floatx4 acc = {0.f, 0.f, 0.f, 0.f};
          const E* krow = Ks + (kb * 16 + l16) * QP;
          const E* qrow = Qs + query * QP;
#pragma unroll
          for (int kk = 0; kk < NK32; ++kk)
            acc = mma32(IO::ld8(krow + kk * 32 + 8 * g), IO::ld8(qrow + kk * 32 + 8 * g), acc);
          if (KTAIL)
            acc = mma16(IO::ld4(krow + NK32 * 32 + 4 * g), IO::ld4(qrow + NK32 * 32 + 4 * g), acc);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = key0 + i;
            float wt = 1.0f;
            if (p.ret == TS_RET_STATIC)
              wt = s_pw[max(query - key, 0)];
            else if (p.ret == TS_RET_STREAM)
              wt = expf(fminf(s_lloc[query] - s_lloc[key], 0.0f));
            pv[i] = key <= query ? acc[i] * wt : 0.0f;
          }
        }
        IO::st4(Ps + query * TP + key0, pv[0], pv[1], pv[2], pv[3]);
      }
      __syncthreads();
    }

    if (owner) {
      // ---- value block of this wave
      F8 av[2];
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) av[kp] = TL::tcol8(Vt_src, vt_pitch, w * 16, kp, lane);

      if (MAIN) {
#pragma unroll
        for (int qb = 0; qb < 4; ++qb) {
          const int query = qb * 16 + l16;
          floatx4 acc = {0.f, 0.f, 0.f, 0.f};
          if (!state_zero) {
            const E* qrow = Qs + query * QP;
#pragma unroll
            for (int j = 0; j < NK32; ++j)
              acc = mma32(IO::from_acc(S[2 * j], S[2 * j + 1]),
                          IO::cat(IO::ld4(qrow + 32 * j + 4 * g), IO::ld4(qrow + 32 * j + 16 + 4 * g)), acc);
            if (KTAIL) acc = mma16(IO::from_acc4(S[NKB - 1]), IO::ld4(qrow + NK32 * 32 + 4 * g), acc);
            if (p.ret != TS_RET_NONE) {
              const float cw = s_carry[query];
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[i] *= cw;
            }
          }
#pragma unroll
          for (int kp = 0; kp <= qb / 2; ++kp)
            acc = mma32(av[kp], IO::ld8(Ps + query * TP + kp * 32 + 8 * g), acc);

          const int t = t0 + query;
          if (t < p.T) {
            const int tp = phys_t(p, t);
            const int dvb = w * 16 + 4 * g;
            const int64_t ooff = obase + (int64_t)tp * p.out.st;
            if (p.out_mode == TS_OUT_STORE) {
              E* o = (E*)p.out.ptr + ooff + dvb;
              if (dvb + 4 <= p.dv) {
                IO::st4(o, acc[0], acc[1], acc[2], acc[3]);
              } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                  if (dvb + i < p.dv) o[i] = cvt<E>(acc[i]);
              }
            } else {
              float* o = (float*)p.out.ptr + ooff + dvb;
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                if (dvb + i < p.dv) {
                  const float val = p.out_scale * acc[i];
                  o[i] = p.out_mode == TS_OUT_ACCUM_F32 ? o[i] + val : val;
                }
              }
            }
            if (p.oe.ptr && dvb <= p.dv && p.dv < dvb + 4) {
              float* oe = (float*)p.oe.ptr + oebase + (int64_t)tp * p.oe.st;
              const float val = (p.out_mode == TS_OUT_STORE ? 1.0f : p.out_scale) * acc[p.dv - dvb];
              *oe = p.out_mode == TS_OUT_ACCUM_F32 ? *oe + val : val;
            }
          }
        }
      }

      // ---- state update: S = decay(tile) * S + K_w^T V
      if (p.ret != TS_RET_NONE) {
        const float cdec = expf(s_misc[0]);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) S[kb][i] *= cdec;
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
          F8 ak = TL::tcol8(Kt_src, kt_pitch, kb * 16, kp, lane);
          if (p.ret != TS_RET_NONE) {
#pragma unroll
            for (int e = 0; e < 8; ++e) ak[e] = cvt<E>(tof(ak[e]) * s_wk[kp * 32 + 8 * g + e]);
          }
          S[kb] = mma32(ak, av[kp], S[kb]);
        }
      }
    }
    if (p.ret != TS_RET_NONE && tid == 0) seg_log += s_misc[0];
    state_zero = false;
  }

  if (!MAIN) {
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

size_t lds_bytes(int esize, int dkp, int dvp, bool main_kernel) {
  const int vec = 16 / esize;
  const int qp = dkp + vec, tp = ts::C + vec, vp = dvp + vec;
  size_t elems = (size_t)ts::C * qp;                       // K rows
  if (main_kernel) elems += (size_t)ts::C * qp + (size_t)ts::C * tp;  // Q rows, P
  if (esize == 2)
    elems += (size_t)ts::C * vp;                           // V rows
  else
    elems += (size_t)dkp * tp + (size_t)dvp * tp;          // K^T, V^T copies
  return elems * esize + 5 * ts::C * sizeof(float);
}

int block_threads(int dvp) {
  const int t = dvp / 16 * 64;
  return t < 256 ? 256 : t;
}

typedef void (*KernelFn)(ts::ScanP);

template <typename E, bool WIDE>
KernelFn pick_kernel_w(int dkp, bool main_kernel) {
  switch (dkp) {
#define TS_CASE(D)                                                                                   \
  case D:                                                                                            \
    return main_kernel ? (KernelFn)ts::scan_kernel<E, D, true, WIDE> : (KernelFn)ts::scan_kernel<E, D, false, WIDE>;
    TS_CASE(32)
    TS_CASE(64)
    TS_CASE(80)
    TS_CASE(128)
    TS_CASE(144)
#undef TS_CASE
  }
  return nullptr;
}

template <typename E>
KernelFn pick_kernel(int dkp, int dvp, bool main_kernel) {
  return dvp > 64 ? pick_kernel_w<E, true>(dkp, main_kernel) : pick_kernel_w<E, false>(dkp, main_kernel);
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
  if (((uintptr_t)io->out.ptr & 7u) || io->out.st % out_vec || io->out.sh % out_vec || io->out.sb % out_vec)
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
  if (L.ws_bytes > 0) {
    p.seg = (float*)workspace;
    p.segdec = p.seg + (size_t)d->B * d->H * L.nseg * (size_t)L.dkp * L.dvp;
  }

  const int bh = d->B * d->H;
  const dim3 block(block_threads(L.dvp));
  KernelFn fsum = d->dtype == TS_BF16 ? pick_kernel<ts::bf16>(L.dkp, L.dvp, false)
                                      : pick_kernel<float>(L.dkp, L.dvp, false);
  KernelFn fmain = d->dtype == TS_BF16 ? pick_kernel<ts::bf16>(L.dkp, L.dvp, true)
                                       : pick_kernel<float>(L.dkp, L.dvp, true);
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
