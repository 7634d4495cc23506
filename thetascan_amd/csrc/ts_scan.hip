// Chunked exact linear-attention scan for gfx950 (MI355X).
//
// One view of the reference's chunk backend
// (src/thetascan/_core/ops/scan_chunk.py:246-339): the sequence is cut into
// 64-token tiles; inside a tile the causal score block is an MFMA contraction
// (bf16 or fp32 operands, fp32 accumulation), and across tiles an fp32
// [dk, dv] state carries everything already written.
//
// Work decomposition (one workgroup of four waves per (batch*head, segment)):
//   1. summary kernel : each segment of `seg_chunks` tiles folds its own
//                       writes into a local state U_p (no queries needed);
//   2. prefix kernel  : exclusive scan of U_p over segments with the decay of
//                       each segment -> the state entering every segment;
//   3. main kernel    : each segment re-walks its tiles from that incoming
//                       state and writes the outputs.
// This turns B*H sequential scans (64 at the benchmark shape) into B*H*nseg
// independent workgroups so the whole chip is busy.
//
// Inside a tile, wave w owns query block w (16 queries) and value block(s)
// w (+4): it computes the causal scores of its own queries only (no score is
// computed twice), keeps them in MFMA accumulator registers and feeds them
// straight into the P.V contraction for every value block; the carried state
// enters through a bf16 copy of the state that each wave publishes in LDS for
// its own value block.  The fp32 state itself never leaves the owning wave's
// registers.  One barrier per tile.
//
// Extra "ext" columns (the key-mass unit column of the normalized read and
// its gradient) are rank-1 terms and never widen an MFMA tile:
//   key-side ext  (q_ext x k_ext): score += qe_t ke_i; the state gains a row
//                 u = sum_i w ke_i v_i (a [dv] vector), read as qe_t u;
//   value-side ext (v_ext):        out_ext_t = sum_i w s_ti ve_i + <q_t, D>,
//                 D = sum_i w ve_i k_i (a [dk] vector).
// Both vector states are MFMA contractions against a broadcast ext row.

#include "ts_common.h"
#include "ts_scan_impl.h"
#include "thetascan_hip.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <tuple>
#include <unordered_map>

namespace ts {

// LDS carve-up (elements of E unless noted), shared with the host.
struct ScanLayout {
  int kp, vp;        // row pitches of K / V / state tiles
  int stage;         // elements per stage: K [C][kp], V [C][vp]
  int stages;
  int st;            // state copy [dvp][kp] (MAIN), `nst` buffers
  int nst;
  int fbase;         // float offset (in floats, from the byte end of the E part)
  int bytes;
};

__host__ __device__ constexpr int scan_stages(int esize) { return esize == 2 ? 2 : 1; }

// Float region after the E tiles (per stage: ke[C], ve[C]; then u[2][dvp],
// D[2][DK], pw[68], lloc[4][C]).
__host__ __device__ inline ScanLayout scan_layout_n(int esize, int DK, int dvp, int nst) {
  const int vec = 16 / esize;
  ScanLayout L{};
  L.kp = DK + vec;
  L.vp = dvp + vec;
  L.stage = C * L.kp + C * L.vp;
  L.stages = scan_stages(esize);
  L.nst = nst;
  L.st = dvp * L.kp;
  const int e_elems = L.stages * L.stage + L.nst * L.st;
  const int e_bytes = (e_elems * esize + 15) / 16 * 16;
  L.fbase = e_bytes / 4;
  const int floats = L.stages * 2 * C + 2 * dvp + 2 * DK + 68 + 4 * C;
  L.bytes = e_bytes + floats * 4;
  return L;
}

// The main kernel double-buffers the published state (one barrier per tile)
// unless that leaves a CU room for only one workgroup while a single copy
// (one more barrier per tile) fits two: at 128-wide keys and 64 value
// columns the two copies take 92 KB, one copy 75 KB of the CU's 160 KB.
__host__ __device__ inline ScanLayout scan_layout(int esize, int DK, int dvp, bool main_kernel) {
  if (!main_kernel) return scan_layout_n(esize, DK, dvp, 0);
  ScanLayout L = scan_layout_n(esize, DK, dvp, esize == 2 ? 2 : 1);
  if (L.nst == 2 && 2 * L.bytes > kLdsPerCU) {
    const ScanLayout L1 = scan_layout_n(esize, DK, dvp, 1);
    if (2 * L1.bytes <= kLdsPerCU) L = L1;
  }
  return L;
}

// MODE selects what the kernel supports, so a call carries no code for what
// it does not use.  Bits: kStatic (static [H] retention), kKeyExt (the
// key-side ext column pair q_ext, k_ext), kValExt (the value-side ext column
// v_ext, out_ext), kF32Out (fp32 outputs, stored or accumulated); kGeneral
// alone reads every retention, ext column and output mode at run time.  The
// host picks an instantiated mode that covers the call, else kGeneral.
constexpr int kPlain = 0, kStatic = 1, kKeyExt = 2, kValExt = 4, kF32Out = 8, kGeneral = 16;

template <typename E, int DK, int NVW, bool MAIN, int MODE>
__global__ __launch_bounds__(256) void scan_kernel(ScanP p) {
  typedef typename Frag<E>::f8 F8;
  typedef typename Frag<E>::f4 F4;
  typedef LdsIO<E> IO;
  typedef Tok<E> TK;
  constexpr int ES = (int)sizeof(E);
  constexpr int VEC = 16 / ES;
  constexpr int NK32 = DK / 32;
  constexpr bool KTAIL = (DK % 32) != 0;
  constexpr int NKB = DK / 16;
  constexpr int NKO = (NKB + 3) / 4;         // key blocks of D owned per wave
  constexpr int STAGES = scan_stages(ES);
  constexpr int SLOTS_K = (C * DK / VEC + 255) / 256;
  constexpr int SLOTS_V = (C * 64 * NVW / VEC + 255) / 256;

  constexpr bool GEN = MODE == kGeneral;
  constexpr bool M_KX = (MODE & kKeyExt) != 0, M_VX = (MODE & kValExt) != 0;
  const int ret = GEN ? p.ret : ((MODE & kStatic) ? TS_RET_STATIC : TS_RET_NONE);
  const int q_ext = GEN || M_KX ? p.q_ext : TS_EXT_NONE;
  const int k_ext = GEN || M_KX ? p.k_ext : TS_EXT_NONE;
  const int v_ext = GEN || M_VX ? p.v_ext : TS_EXT_NONE;
  // key-side rank-1 term (kKeyExt: the host guarantees both columns)
  const bool kx = M_KX || (GEN && q_ext != TS_EXT_NONE && k_ext != TS_EXT_NONE);
  const bool vx = (M_VX || (GEN && v_ext != TS_EXT_NONE)) && blockIdx.z == 0;
  const int out_mode = GEN || (MODE & kF32Out) ? p.out_mode : TS_OUT_STORE;
  const bool has_oe = (GEN || M_VX) && p.oe.ptr != nullptr;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 4;
  const int l16 = lane & 15;
  const int seg = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  // value slice of this workgroup: padded columns col0 .. col0 + vs, of which
  // dvz are real.  Slices of one (segment, b, h) share the q / k tiles through
  // L2; the value-side ext column belongs to slice 0.
  const int col0 = blockIdx.z * p.vs;
  const int vs = p.vs;
  const int dvz = min(p.vs, p.dv - col0);
  const int nvb = vs >> 4;
  const int sgn = p.reverse ? -1 : 1;
  const int wave_first = __builtin_amdgcn_readfirstlane(tid & ~63);

  // ---- LDS carve-up
  const ScanLayout L = scan_layout(ES, DK, vs, MAIN);
  extern __shared__ __align__(16) unsigned char smem[];
  E* ebase = (E*)smem;
  E* st_base = ebase + STAGES * L.stage;
  float* fb = (float*)smem + L.fbase;
  float* s_ext = fb;                              // [stage][ke C | ve C]
  float* s_u = s_ext + STAGES * 2 * C;            // [2][vs]
  float* s_d = s_u + 2 * vs;                      // [2][DK]
  float* s_pw = s_d + 2 * DK;                     // alpha^d, d = 0..64 (static)
  float* my_lloc = s_pw + 68 + w * C;             // per-wave tile log-decay (stream)

  // ---- per-(b, h) addressing
  const int64_t bh_q = (int64_t)b * p.q.sb + (int64_t)h * p.q.sh;
  const int64_t bh_k = (int64_t)b * p.k.sb + (int64_t)h * p.k.sh;
  const int64_t bh_v = (int64_t)b * p.v.sb + (int64_t)h * p.v.sh + col0;
  const int q_st_b = (int)p.q.st * ES;
  const int k_st_b = (int)p.k.st * ES;
  const int v_st_b = (int)p.v.st * ES;
  const int dec_st_b = (int)p.decay.st * 4;
  auto k_rsrc = [&]() { return make_rsrc((const E*)p.k.ptr + bh_k, p.k_rec); };
  auto v_rsrc = [&]() { return make_rsrc((const E*)p.v.ptr + bh_v, p.v_rec - (uint32_t)(col0 * ES)); };
  auto q_rsrc = [&]() { return make_rsrc((const E*)p.q.ptr + bh_q, p.q_rec); };

  // a(s), the decay applied when stepping into logical position s: a reversed
  // scan steps from physical s+1 down to s and uses the decay of the physical
  // successor (logical s = 0 has none).
  auto decay_of = [&](int t0) -> float {
    const int s = t0 + lane;
    const int src = p.reverse ? p.T - s : s;
    const uint32_t off = (s < p.T && src < p.T) ? (uint32_t)(src * dec_st_b) : kOOB;
    return bldf(make_rsrc(bh_base(p.decay, b, h, 4), p.dec_rec), off);
  };
  // ext value of token t0 + row for an ext column (ones or fp32 array)
  auto ext_of = [&](int mode, const ts_strided& e, uint32_t rec, int t0, int row) -> float {
    if (mode == TS_EXT_ONES) return t0 + row < p.T ? 1.0f : 0.0f;
    return bldf(make_rsrc(bh_base(e, b, h, 4), rec), row_off(p, t0, row, (int)e.st * 4));
  };

  // ---- state: value blocks vb = w + 4r owned by this wave
  floatx4 S[NVW][NKB];
  floatx4 us[NVW];   // u for the owned value blocks (every row the same)
  floatx4 dst_[NKO]; // D for the owned key blocks kb = w + 4r (every row the same)
#pragma unroll
  for (int r = 0; r < NVW; ++r) {
    us[r] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) S[r][kb] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int r = 0; r < NKO; ++r) dst_[r] = floatx4{0.f, 0.f, 0.f, 0.f};

  const float la = ret == TS_RET_STATIC ? p.log_alpha[h] : 0.0f;
  if (ret == TS_RET_STATIC && w == 0) {
    s_pw[lane] = expf(la * (float)lane);
    if (lane == 0) s_pw[64] = expf(la * 64.0f);
  }

  const int c_begin = seg * p.seg_chunks;
  const int c_end = min(c_begin + p.seg_chunks, p.nchunks);
  float seg_log = 0.0f;
  bool state_zero = true;

  // publish the state entering a tile (bf16 / fp32 copy, u, D) into buffer `bi`
  auto publish = [&](int bi) {
    E* st = st_base + bi * L.st;
#pragma unroll
    for (int r = 0; r < NVW; ++r) {
      const int vb = w + 4 * r;
      if (vb < nvb) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
          IO::st4(st + (vb * 16 + l16) * L.kp + kb * 16 + 4 * g, S[r][kb][0], S[r][kb][1], S[r][kb][2], S[r][kb][3]);
        if (kx && g == 0) s_u[bi * vs + vb * 16 + l16] = us[r][0];
      }
    }
    if (vx && g == 0) {
#pragma unroll
      for (int r = 0; r < NKO; ++r) {
        const int kb = w + 4 * r;
        if (kb < NKB) s_d[bi * DK + kb * 16 + l16] = dst_[r][0];
      }
    }
  };

  if (MAIN && (seg > 0 || p.has_init)) {
    state_zero = false;
    const float* src = p.seg + ((size_t)bh * p.nseg + seg) * (size_t)p.nelem;
#pragma unroll
    for (int r = 0; r < NVW; ++r) {
      const int vb = w + 4 * r;
      if (vb < nvb) {
        float u;
        if (p.states_t) {
          // the swapped scan's state [value][key] is this scan's [key][value],
          // and its value-side ext state D (sum of its keys times its ext
          // value) is this scan's key-side ext row u
          const int c = col0 + vb * 16 + l16;
          const float* row = src + (size_t)c * DK;
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            const floatx4 v4 = *(const floatx4*)(row + kb * 16 + 4 * g);
            S[r][kb] = v4;
          }
          u = src[DK * DK + DK + c];
        } else {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) S[r][kb][i] = src[(kb * 16 + 4 * g + i) * p.dvp + col0 + vb * 16 + l16];
          u = src[DK * p.dvp + col0 + vb * 16 + l16];
        }
        us[r] = floatx4{u, u, u, u};
      }
    }
#pragma unroll
    for (int r = 0; r < NKO; ++r) {
      const int kb = w + 4 * r;
      if (kb < NKB) {
        const float d = src[DK * p.dvp + p.dvp + kb * 16 + l16];
        dst_[r] = floatx4{d, d, d, d};
      }
    }
  }

  // ---- tile loading
  const int nk_vec = C * (DK / VEC);
  const int nv_vec = C * (vs / VEC);
  TileLoader<E, SLOTS_K> ldk;
  TileLoader<E, SLOTS_V> ldv;
  ldk.setup(p, DK / VEC, p.dk, L.kp, k_st_b, tid);
  ldv.setup(p, vs / VEC, dvz, L.vp, v_st_b, tid);
  float ext_r = 0.0f;  // this thread's ke (wave 0) / ve (wave 1) of the fetched tile
  auto fetch = [&](int t0) {
    ldk.fetch(k_rsrc(), t0, sgn, k_st_b, wave_first, nk_vec);
    ldv.fetch(v_rsrc(), t0, sgn, v_st_b, wave_first, nv_vec);
    if (w == 0 && kx) ext_r = ext_of(k_ext, p.ke, p.ke_rec, t0, lane);
    if (w == 1 && vx) ext_r = ext_of(v_ext, p.ve, p.ve_rec, t0, lane);
  };
  auto store = [&](int stg) {
    E* base = ebase + stg * L.stage;
    ldk.store(base, wave_first, nk_vec);
    ldv.store(base + C * L.kp, wave_first, nv_vec);
    if (w < 2) s_ext[stg * 2 * C + w * C + lane] = ext_r;
  };

  // ---- queries of this wave's block (registers)
  F8 qr[NK32 > 0 ? NK32 : 1];
  F4 qt;
  float qe = 0.0f;
  auto qload = [&](int t0) {
    const int row = w * 16 + l16;
    const uint32_t ro = row_off(p, t0, row, q_st_b);
    auto part = [&](int c) -> F4 {
      const uint32_t off = c < p.dk ? ro + (uint32_t)(c * ES) : kOOB;
      if constexpr (ES == 2) {
        return __builtin_bit_cast(F4, bld8(q_rsrc(), off));
      } else {
        return __builtin_bit_cast(F4, bld16(q_rsrc(), off));
      }
    };
#pragma unroll
    for (int j = 0; j < NK32; ++j) qr[j] = IO::cat(part(32 * j + 4 * g), part(32 * j + 16 + 4 * g));
    if (KTAIL) qt = part(32 * NK32 + 4 * g);
    if (kx) qe = ext_of(q_ext, p.qe, p.qe_rec, t0, row);
  };

  // ---- output addressing
  const int osz = out_mode == TS_OUT_STORE ? ES : 4;
  const void* out_base = (const char*)bh_base(p.out, b, h, osz) + col0 * osz;
  const uint32_t out_rec = p.out_rec - (uint32_t)(col0 * osz);
  const int out_st_b = (int)p.out.st * osz;
  const int oe_st_b = (int)p.oe.st * 4;

  // ---- prologue
  float dcur = 0.0f, dnext = 0.0f;
  if constexpr (STAGES == 2) {
    fetch(c_begin * C);
    if (ret == TS_RET_STREAM) dnext = decay_of(c_begin * C);
    store(c_begin & 1);
    if (c_begin + 1 < c_end) fetch((c_begin + 1) * C);
  }
  if (MAIN) {
    qload(c_begin * C);
    if (!state_zero) publish(c_begin & (L.nst - 1));
  }
  if constexpr (STAGES == 2) __syncthreads();

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * C;
    const int len = min(C, p.T - t0);
    const E* Ks;
    const float* ext_s;
    if constexpr (STAGES == 2) {
      if (c + 1 < c_end) store((c + 1) & 1);
      if (c + 2 < c_end) fetch(t0 + 2 * C);
      Ks = ebase + (c & 1) * L.stage;
      ext_s = s_ext + (c & 1) * 2 * C;
      if (ret == TS_RET_STREAM) {
        dcur = dnext;
        if (c + 1 < c_end) dnext = decay_of(t0 + C);
      }
    } else {
      __syncthreads();  // the previous tile is no longer read
      fetch(t0);
      store(0);
      if (ret == TS_RET_STREAM) dcur = decay_of(t0);
      __syncthreads();
      Ks = ebase;
      ext_s = s_ext;
    }
    const E* Vs = Ks + C * L.kp;
    const float* ke_s = ext_s;
    const float* ve_s = ext_s + C;

    // ---- retention of this tile (per wave)
    float tile_log = 0.0f;
    if (ret == TS_RET_STATIC) {
      tile_log = la * (float)len;
    } else if (ret == TS_RET_STREAM) {
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

    if constexpr (MAIN) {
      const int query = w * 16 + l16;
      const float lq = ret == TS_RET_STREAM ? my_lloc[query] : 0.0f;
      const float cw = ret == TS_RET_STATIC ? s_pw[query + 1] : (ret == TS_RET_STREAM ? expf(lq) : 1.0f);
      // ---- causal scores of this query block: sc[kb] = D[key][query], kb <= w
      floatx4 sc[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        sc[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (kb > w) continue;
        const int krow = kb * 16 + l16;
#pragma unroll
        for (int j = 0; j < NK32; ++j) sc[kb] = mma32(frow8<E>(Ks, L.kp, krow, j, g), qr[j], sc[kb]);
        if (KTAIL) sc[kb] = mma16(frow4<E>(Ks, L.kp, krow, NK32, g), qt, sc[kb]);
        floatx4 lk;
        if (ret == TS_RET_STREAM) lk = *(const floatx4*)(my_lloc + kb * 16 + 4 * g);
        floatx4 kev;
        if (kx) kev = *(const floatx4*)(ke_s + kb * 16 + 4 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb * 16 + 4 * g + i;
          float s = sc[kb][i];
          if (kx) s += qe * kev[i];
          float wt = 1.0f;
          if (ret == TS_RET_STATIC) wt = s_pw[max(query - key, 0)];
          else if (ret == TS_RET_STREAM) wt = expf(fminf(lq - lk[i], 0.0f));
          sc[kb][i] = (kb < w || key <= query) ? s * wt : 0.0f;
        }
      }
      const F8 p0 = IO::from_acc(sc[0], sc[1]);
      const F8 p1 = IO::from_acc(sc[2], sc[3]);
      const E* st = st_base + (c & (L.nst - 1)) * L.st;
      const float* u_in = s_u + (c & (L.nst - 1)) * vs;
      const float* d_in = s_d + (c & (L.nst - 1)) * DK;

      // ---- outputs O^T[v][query] = cw (S^T Q^T)[v] + (V^T P^T)[v], every value block
      const uint32_t ro = row_off(p, t0, query, out_st_b);
      const rsrc_t out_rs = make_rsrc(out_base, out_rec);
#pragma unroll
      for (int vb = 0; vb < 4 * NVW; ++vb) {
        if (vb >= nvb) break;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        if (!state_zero) {
          const int vrow = vb * 16 + l16;
#pragma unroll
          for (int j = 0; j < NK32; ++j) acc = mma32(frow8<E>(st, L.kp, vrow, j, g), qr[j], acc);
          if (KTAIL) acc = mma16(frow4<E>(st, L.kp, vrow, NK32, g), qt, acc);
          if (kx) {
            const floatx4 u4 = *(const floatx4*)(u_in + vb * 16 + 4 * g);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] += qe * u4[i];
          }
          if (ret != TS_RET_NONE) {
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] *= cw;
          }
        }
        acc = mma32(TK::col8(Vs, L.vp, vb * 16, 0, lane), p0, acc);
        if (w >= 2) acc = mma32(TK::col8(Vs, L.vp, vb * 16, 1, lane), p1, acc);

        const int ocol = vb * 16 + 4 * g;
        const uint32_t ooff = ocol < dvz ? ro + (uint32_t)(ocol * osz) : kOOB;
        if (out_mode == TS_OUT_STORE) {
          if constexpr (ES == 2) {
            bf16x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (bf16)acc[i];
            bst8(out_rs, ooff, __builtin_bit_cast(uint2, o));
          } else {
            bst16(out_rs, ooff, __builtin_bit_cast(uint4, acc));
          }
        } else {
          floatx4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = p.out_scale * acc[i];
          if (out_mode == TS_OUT_ACCUM_F32) {
            const floatx4 prev = __builtin_bit_cast(floatx4, bld16(out_rs, ooff));
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] += prev[i];
          }
          bst16(out_rs, ooff, __builtin_bit_cast(uint4, o));
        }
      }

      // ---- value-side ext column: out_ext = cw <q, D> + sum_keys P ve
      if (vx) {
        floatx4 oacc = {0.f, 0.f, 0.f, 0.f};
        if (!state_zero) {
#pragma unroll
          for (int j = 0; j < NK32; ++j) oacc = mma32(bcast8<E>(d_in, 32 * j, g), qr[j], oacc);
          if (KTAIL) oacc = mma16(bcast4<E>(d_in, 32 * NK32, g), qt, oacc);
#pragma unroll
          for (int i = 0; i < 4; ++i) oacc[i] *= cw;
        }
        oacc = mma32(bcast8<E>(ve_s, 0, g), p0, oacc);
        if (w >= 2) oacc = mma32(bcast8<E>(ve_s, 32, g), p1, oacc);
        if (has_oe && g == 0) {
          float val = oacc[0];
          if (out_mode != TS_OUT_STORE) val *= p.out_scale;
          const uint32_t eo = row_off(p, t0, query, oe_st_b);
          const rsrc_t oe_rs = make_rsrc(bh_base(p.oe, b, h, 4), p.oe_rec);
          if (out_mode == TS_OUT_ACCUM_F32) val += bldf(oe_rs, eo);
          bstf(oe_rs, eo, val);
        }
      }
      if (c + 1 < c_end) qload(t0 + C);  // next tile's queries of this block
    }

    // ---- state update: S = decay(tile) * S + K^T diag(wk) V (owned value blocks)
    const float cdec = ret == TS_RET_STATIC ? s_pw[len] : (ret == TS_RET_STREAM ? expf(tile_log) : 1.0f);
    floatx4 wk4[2][2];  // per-key weights of this lane's keys {32kp+4g+i, 32kp+16+4g+i}
#pragma unroll
    for (int kp = 0; kp < 2; ++kp)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = 32 * kp + 16 * hf + 4 * g + i;
          float wk = 1.0f;
          if (ret == TS_RET_STATIC) wk = key < len ? s_pw[len - 1 - key] : 0.0f;
          else if (ret == TS_RET_STREAM) wk = key < len ? expf(tile_log - my_lloc[key]) : 0.0f;
          wk4[kp][hf][i] = wk;
        }
#pragma unroll
    for (int r = 0; r < NVW; ++r) {
      const int vb = w + 4 * r;
      if (vb >= nvb) break;
      F8 avw[2];
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        avw[kp] = TK::col8(Vs, L.vp, vb * 16, kp, lane);
        if (ret != TS_RET_NONE) {
#pragma unroll
          for (int e = 0; e < 8; ++e) avw[kp][e] = cvt<E>(tof(avw[kp][e]) * wk4[kp][e >> 2][e & 3]);
        }
      }
      if (ret != TS_RET_NONE && !(MAIN && state_zero)) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) S[r][kb][i] *= cdec;
#pragma unroll
        for (int i = 0; i < 4; ++i) us[r][i] *= cdec;
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) S[r][kb] = mma32(TK::col8(Ks, L.kp, kb * 16, kp, lane), avw[kp], S[r][kb]);
      if (kx) {
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) us[r] = mma32(bcast8<E>(ke_s, 32 * kp, g), avw[kp], us[r]);
      }
    }
    if (vx) {
      // D = decay * D + K^T (wk ve): a broadcast (wk ve) row against K columns
#pragma unroll
      for (int r = 0; r < NKO; ++r) {
        const int kb = w + 4 * r;
        if (kb >= NKB) break;
        if (ret != TS_RET_NONE) {
#pragma unroll
          for (int i = 0; i < 4; ++i) dst_[r][i] *= cdec;
        }
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
          F8 a;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int key = 32 * kp + (e < 4 ? 4 * g + e : 12 + 4 * g + e);
            a[e] = cvt<E>(ve_s[key] * wk4[kp][e >> 2][e & 3]);
          }
          dst_[r] = mma32(a, TK::col8(Ks, L.kp, kb * 16, kp, lane), dst_[r]);
        }
      }
    }
    state_zero = false;
    if constexpr (MAIN) {
      if (c + 1 < c_end) {
        if (STAGES == 1 || L.nst == 1) __syncthreads();  // single state copy: readers of this tile are done
        publish((c + 1) & (L.nst - 1));
      }
    }
    if constexpr (STAGES == 2) __syncthreads();
  }

  if constexpr (!MAIN) {
    float* dst = p.seg + ((size_t)bh * p.nseg + seg) * (size_t)p.nelem;
#pragma unroll
    for (int r = 0; r < NVW; ++r) {
      const int vb = w + 4 * r;
      if (vb < nvb) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[(kb * 16 + 4 * g + i) * p.dvp + col0 + vb * 16 + l16] = S[r][kb][i];
        if (g == 0) dst[DK * p.dvp + col0 + vb * 16 + l16] = us[r][0];
      }
    }
    if (g == 0 && blockIdx.z == 0) {
#pragma unroll
      for (int r = 0; r < NKO; ++r) {
        const int kb = w + 4 * r;
        if (kb < NKB) dst[DK * p.dvp + p.dvp + kb * 16 + l16] = dst_[r][0];
      }
    }
    if (tid == 0 && blockIdx.z == 0) p.segdec[(size_t)bh * p.nseg + seg] = seg_log;
  }
}

// Two plain scans that share keys and values up to a swap, in one pass:
//   A: out_a_t = sum_i <qa_t, k_i> v_i   (state S = sum_i k_i v_i^T)
//   B: out_b_t = sum_i <qb_t, v_i> k_i   (state S^T)
// with the same causal (or anti-causal) order.  These are the backward's dk
// and dv scans of a kernel memory (keys dnum, values phi(q); queries v and
// phi(k)).  K and V tiles are read once, S is updated once per tile, both
// score blocks stay in accumulators, and scan B reads the published state
// copy transposed (ds_read_b64_tr_b16) instead of carrying S^T.  Each output
// is computed in the order its own one-scan kernel uses.  bf16, dk = dv = DK;
// segment states come from scan A's summary and prefix passes.  With KX, scan
// A carries the key-side ext pair of a normalized read's backward (q_ext =
// ones, k_ext = dmass): score_a += ke_t and its state gains the row u =
// sum_t ke_t v_t; scan B is unchanged.  MODE may add kStatic (one static
// per-head retention for both scans: the same causal weights alpha^(t-i)) and
// kF32Out (fp32 outputs, stored or accumulated with out_scale, as the one-view
// kernel's fp32 output modes).
struct PairP {
  ScanP s;           // q = qa, k, v, out = out_a (and the segmentation)
  ts_strided qb, ob;
  uint32_t qb_rec, ob_rec;
};

template <int DK, bool KX, int MODE>
__global__ __launch_bounds__(256) void pair_kernel(PairP pp) {
  constexpr bool STATIC = (MODE & kStatic) != 0;
  constexpr bool F32OUT = (MODE & kF32Out) != 0;
  typedef bf16 E;
  typedef bf16x8 F8;
  typedef LdsIO<E> IO;
  typedef Tok<E> TK;
  constexpr int ES = 2;
  constexpr int VEC = 8;
  constexpr int NK32 = DK / 32;
  constexpr int NKB = DK / 16;
  constexpr int SLOTS_K = (C * DK / VEC + 255) / 256;
  const ScanP& p = pp.s;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 4;
  const int l16 = lane & 15;
  const int seg = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int sgn = p.reverse ? -1 : 1;
  const int wave_first = __builtin_amdgcn_readfirstlane(tid & ~63);
  const int nvb = DK / 16;

  const ScanLayout L = scan_layout(ES, DK, DK, true);
  extern __shared__ __align__(16) unsigned char smem[];
  E* ebase = (E*)smem;
  E* st_base = ebase + L.stages * L.stage;
  float* s_ext = (float*)smem + L.fbase;          // [stage][ke C | (unused) C]
  float* s_u = s_ext + L.stages * 2 * C;          // [2][DK]
  float* s_pw = s_u + 2 * DK + 2 * DK;            // alpha^d, d = 0..64 (static)
  if (STATIC && w == 0) {
    const float la = p.log_alpha[h];
    s_pw[lane] = expf(la * (float)lane);
    if (lane == 0) s_pw[64] = expf(la * 64.0f);
  }

  const int64_t bh_q = (int64_t)b * p.q.sb + (int64_t)h * p.q.sh;
  const int64_t bh_b = (int64_t)b * pp.qb.sb + (int64_t)h * pp.qb.sh;
  const int64_t bh_k = (int64_t)b * p.k.sb + (int64_t)h * p.k.sh;
  const int64_t bh_v = (int64_t)b * p.v.sb + (int64_t)h * p.v.sh;
  const int q_st_b = (int)p.q.st * ES;
  const int b_st_b = (int)pp.qb.st * ES;
  const int k_st_b = (int)p.k.st * ES;
  const int v_st_b = (int)p.v.st * ES;
  auto k_rsrc = [&]() { return make_rsrc((const E*)p.k.ptr + bh_k, p.k_rec); };
  auto v_rsrc = [&]() { return make_rsrc((const E*)p.v.ptr + bh_v, p.v_rec); };

  // state: value block w of S, every key block (and u over its columns)
  floatx4 S[NKB];
  floatx4 us = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) S[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
  const int c_begin = seg * p.seg_chunks;
  const int c_end = min(c_begin + p.seg_chunks, p.nchunks);
  bool state_zero = true;
  if (seg > 0) {
    state_zero = false;
    const float* src = p.seg + ((size_t)bh * p.nseg + seg) * (size_t)p.nelem;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[kb][i] = src[(kb * 16 + 4 * g + i) * p.dvp + w * 16 + l16];
    if (KX) {
      const float u = src[DK * p.dvp + w * 16 + l16];
      us = floatx4{u, u, u, u};
    }
  }
  auto publish = [&](int bi) {
    E* st = st_base + bi * L.st;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      IO::st4(st + (w * 16 + l16) * L.kp + kb * 16 + 4 * g, S[kb][0], S[kb][1], S[kb][2], S[kb][3]);
    if (KX && g == 0) s_u[bi * DK + w * 16 + l16] = us[0];
  };

  const int nk_vec = C * (DK / VEC);
  TileLoader<E, SLOTS_K> ldk;
  TileLoader<E, SLOTS_K> ldv;
  ldk.setup(p, DK / VEC, p.dk, L.kp, k_st_b, tid);
  ldv.setup(p, DK / VEC, p.dv, L.vp, v_st_b, tid);
  float ke_r = 0.0f;  // this thread's ke of the fetched tile (wave 0)
  auto fetch = [&](int t0) {
    ldk.fetch(k_rsrc(), t0, sgn, k_st_b, wave_first, nk_vec);
    ldv.fetch(v_rsrc(), t0, sgn, v_st_b, wave_first, nk_vec);
    if (KX && w == 0)
      ke_r = bldf(make_rsrc(bh_base(p.ke, b, h, 4), p.ke_rec), row_off(p, t0, lane, (int)p.ke.st * 4));
  };
  auto store = [&](int stg) {
    E* base = ebase + stg * L.stage;
    ldk.store(base, wave_first, nk_vec);
    ldv.store(base + C * L.kp, wave_first, nk_vec);
    if (KX && w == 0) s_ext[stg * 2 * C + lane] = ke_r;
  };

  // queries of this wave's block, for both scans
  F8 qa[NK32], qb[NK32];
  auto qload = [&](int t0) {
    const int row = w * 16 + l16;
    const rsrc_t ra = make_rsrc((const E*)p.q.ptr + bh_q, p.q_rec);
    const rsrc_t rb = make_rsrc((const E*)pp.qb.ptr + bh_b, pp.qb_rec);
    const uint32_t oa = row_off(p, t0, row, q_st_b), ob = row_off(p, t0, row, b_st_b);
    auto part = [&](rsrc_t r, uint32_t ro, int c) -> bf16x4 {
      return __builtin_bit_cast(bf16x4, bld8(r, ro + (uint32_t)(c * ES)));
    };
#pragma unroll
    for (int j = 0; j < NK32; ++j) {
      qa[j] = IO::cat(part(ra, oa, 32 * j + 4 * g), part(ra, oa, 32 * j + 16 + 4 * g));
      qb[j] = IO::cat(part(rb, ob, 32 * j + 4 * g), part(rb, ob, 32 * j + 16 + 4 * g));
    }
  };

  constexpr int OSZ = F32OUT ? 4 : ES;
  const int out_mode = F32OUT ? p.out_mode : TS_OUT_STORE;
  const void* oa_base = bh_base(p.out, b, h, OSZ);
  const void* ob_base = bh_base(pp.ob, b, h, OSZ);
  const int oa_st_b = (int)p.out.st * OSZ;
  const int ob_st_b = (int)pp.ob.st * OSZ;

  fetch(c_begin * C);
  store(c_begin & 1);
  if (c_begin + 1 < c_end) fetch((c_begin + 1) * C);
  qload(c_begin * C);
  if (!state_zero) publish(c_begin & 1);
  __syncthreads();

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * C;
    if (c + 1 < c_end) store((c + 1) & 1);
    if (c + 2 < c_end) fetch(t0 + 2 * C);
    const E* Ks = ebase + (c & 1) * L.stage;
    const E* Vs = Ks + C * L.kp;
    const E* st = st_base + (c & 1) * L.st;
    const float* ke_s = s_ext + (c & 1) * 2 * C;
    const float* u_in = s_u + (c & 1) * DK;
    const int query = w * 16 + l16;
    const float qe = t0 + query < p.T ? 1.0f : 0.0f;  // the ones column of scan A's queries
    const int len = min(C, p.T - t0);
    const float cw = STATIC ? s_pw[query + 1] : 1.0f;

    // causal score blocks of this wave's queries against keys k (A) and v (B)
    floatx4 sa[4], sb[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      sa[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
      sb[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (kb > w) continue;
      const int krow = kb * 16 + l16;
#pragma unroll
      for (int j = 0; j < NK32; ++j) sa[kb] = mma32(frow8<E>(Ks, L.kp, krow, j, g), qa[j], sa[kb]);
#pragma unroll
      for (int j = 0; j < NK32; ++j) sb[kb] = mma32(frow8<E>(Vs, L.vp, krow, j, g), qb[j], sb[kb]);
      floatx4 kev;
      if (KX) kev = *(const floatx4*)(ke_s + kb * 16 + 4 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb * 16 + 4 * g + i;
        const bool keep = kb < w || key <= query;
        float sv = sa[kb][i];
        if (KX) sv += qe * kev[i];
        if (STATIC) {
          const float wt = s_pw[max(query - key, 0)];
          sa[kb][i] = keep ? sv * wt : 0.0f;
          sb[kb][i] = keep ? sb[kb][i] * wt : 0.0f;
        } else {
          sa[kb][i] = keep ? sv : 0.0f;
          sb[kb][i] = keep ? sb[kb][i] : 0.0f;
        }
      }
    }
    const F8 pa0 = IO::from_acc(sa[0], sa[1]), pa1 = IO::from_acc(sa[2], sa[3]);
    const F8 pb0 = IO::from_acc(sb[0], sb[1]), pb1 = IO::from_acc(sb[2], sb[3]);

    const uint32_t roa = row_off(p, t0, query, oa_st_b);
    const uint32_t rob = row_off(p, t0, query, ob_st_b);
    const rsrc_t oa_rs = make_rsrc(oa_base, p.out_rec);
    const rsrc_t ob_rs = make_rsrc(ob_base, pp.ob_rec);
#pragma unroll
    for (int vb = 0; vb < nvb; ++vb) {
      // A: O^T[v][query] = (S^T qa^T)[v] + (V^T Pa^T)[v]
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      if (!state_zero) {
#pragma unroll
        for (int j = 0; j < NK32; ++j) acc = mma32(frow8<E>(st, L.kp, vb * 16 + l16, j, g), qa[j], acc);
        if (KX) {
          const floatx4 u4 = *(const floatx4*)(u_in + vb * 16 + 4 * g);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] += qe * u4[i];
        }
        if (STATIC) {
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] *= cw;
        }
      }
      acc = mma32(TK::col8(Vs, L.vp, vb * 16, 0, lane), pa0, acc);
      if (w >= 2) acc = mma32(TK::col8(Vs, L.vp, vb * 16, 1, lane), pa1, acc);
      // B: O^T[k][query] = (S qb^T)[k] (state copy read transposed) + (K^T Pb^T)[k]
      floatx4 accb = {0.f, 0.f, 0.f, 0.f};
      if (!state_zero) {
#pragma unroll
        for (int j = 0; j < NK32; ++j) accb = mma32(TK::col8(st, L.kp, vb * 16, j, lane), qb[j], accb);
        if (STATIC) {
#pragma unroll
          for (int i = 0; i < 4; ++i) accb[i] *= cw;
        }
      }
      accb = mma32(TK::col8(Ks, L.kp, vb * 16, 0, lane), pb0, accb);
      if (w >= 2) accb = mma32(TK::col8(Ks, L.kp, vb * 16, 1, lane), pb1, accb);
      const int ocol = vb * 16 + 4 * g;
      const uint32_t offa = ocol < p.dv ? roa + (uint32_t)(ocol * OSZ) : kOOB;
      const uint32_t offb = ocol < p.dk ? rob + (uint32_t)(ocol * OSZ) : kOOB;
      if (out_mode == TS_OUT_STORE) {
        bf16x4 oa, ob;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          oa[i] = (bf16)acc[i];
          ob[i] = (bf16)accb[i];
        }
        bst8(oa_rs, offa, __builtin_bit_cast(uint2, oa));
        bst8(ob_rs, offb, __builtin_bit_cast(uint2, ob));
      } else {
        floatx4 oa, ob;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          oa[i] = p.out_scale * acc[i];
          ob[i] = p.out_scale * accb[i];
        }
        if (out_mode == TS_OUT_ACCUM_F32) {
          const floatx4 pa = __builtin_bit_cast(floatx4, bld16(oa_rs, offa));
          const floatx4 pb = __builtin_bit_cast(floatx4, bld16(ob_rs, offb));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            oa[i] += pa[i];
            ob[i] += pb[i];
          }
        }
        bst16(oa_rs, offa, __builtin_bit_cast(uint4, oa));
        bst16(ob_rs, offb, __builtin_bit_cast(uint4, ob));
      }
    }
    if (c + 1 < c_end) qload(t0 + C);

    // S = decay(tile) S + K^T diag(wk) V (value block w), once for both scans
    F8 av[2];
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) av[kp] = TK::col8(Vs, L.vp, w * 16, kp, lane);
    if (STATIC) {
#pragma unroll
      for (int kp = 0; kp < 2; ++kp)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = 32 * kp + (e < 4 ? 4 * g + e : 12 + 4 * g + e);
          const float wk = key < len ? s_pw[len - 1 - key] : 0.0f;
          av[kp][e] = cvt<E>(tof(av[kp][e]) * wk);
        }
      if (!state_zero) {
        const float cdec = s_pw[len];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) S[kb][i] *= cdec;
#pragma unroll
        for (int i = 0; i < 4; ++i) us[i] *= cdec;
      }
    }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) S[kb] = mma32(TK::col8(Ks, L.kp, kb * 16, kp, lane), av[kp], S[kb]);
    if (KX) {
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) us = mma32(bcast8<E>(ke_s, 32 * kp, g), av[kp], us);
    }
    state_zero = false;
    if (c + 1 < c_end) publish((c + 1) & 1);
    __syncthreads();
  }
}

// Exclusive scan of the segment summaries:  seg[p] <- state entering segment p.
// With `fin`, the state after the last token is also written in the exact
// [dk + kx][dv + vx] layout (ext row / column last).
struct FinalP {
  float* fin;
  const float* init;  // the state entering the first token, same layout as fin (or null)
  int DK, dvp, dk, dv, kx, vx;
};

// Element e of the segment-state layout ([DK][dvp] S, [dvp] u, [DK] D) in the
// exact [dk + kx][dv + vx] layout of a final / initial state, or -1.
__device__ __forceinline__ int exact_index(const FinalP& F, int e) {
  const int cols = F.dv + F.vx;
  const int ns = F.DK * F.dvp;
  if (e < ns) {
    const int f = e / F.dvp, v = e - f * F.dvp;
    return f < F.dk && v < F.dv ? f * cols + v : -1;
  }
  if (e < ns + F.dvp) {
    const int v = e - ns;
    return F.kx && v < F.dv ? F.dk * cols + v : -1;
  }
  const int f = e - ns - F.dvp;
  return F.vx && f < F.dk ? f * cols + F.dv : -1;
}

// Short continuations (a decode step): T <= kStepMaxT tokens after a carried
// state.  One workgroup per (b, h) walks the recurrence token by token,
//   S_t = a_t S_{t-1} + k_t v_t^T,  out_t = S_t^T q_t,
//   D_t = a_t D_{t-1} + k_t,        out_ext_t = <q_t, D_t>   (the ones column),
// with the fp32 state in registers: thread (row group rg, column j) holds
// S[rg * DKP/2 .. rg * DKP/2 + DKP/2)[j] and threads below dk hold D.  One
// launch replaces the summary, prefix and main passes (and their workspace).
constexpr int kStepMaxT = 8;

struct StepP {
  int H, T, dk, dv, vx, ret, out_f32, has_init;
  float out_scale;
  ts_strided q, k, v, decay, out, oe;
  const float* log_alpha;
  const float* init;  // [B*H][dk][dv + vx] fp32 (or null)
  float* fin;         // same layout (or null)
};

template <typename E>
__device__ __forceinline__ float step_ld(const ts_strided& s, int b, int h, int t, int c) {
  return tof(*((const E*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st + c));
}

template <typename E, int DKP>
__global__ __launch_bounds__(256) void scan_step_kernel(StepP p) {
  constexpr int RPT = DKP / 2;
  // every token's rows are staged up front, so the state loads and the
  // token loads are in flight together; the per-token sums alternate
  // between two buffers (one barrier per token)
  __shared__ float sq[kStepMaxT][128], sk[kStepMaxT][128], sv[kStepMaxT][128];
  __shared__ float sa[kStepMaxT];
  __shared__ float red[2][2][128], sd[2][128];
  const int tid = threadIdx.x, j = tid & 127, rg = tid >> 7, lane = tid & 63;
  const int bh = blockIdx.x, b = bh / p.H, h = bh - b * p.H;
  const int cols = p.dv + p.vx;
  const size_t state = (size_t)bh * p.dk * cols;
  for (int e = tid; e < p.T * 128; e += 256) {
    const int t = e >> 7, c = e & 127;
    if (c < p.dk) {
      sq[t][c] = step_ld<E>(p.q, b, h, t, c);
      sk[t][c] = step_ld<E>(p.k, b, h, t, c);
    }
    if (c < p.dv) sv[t][c] = step_ld<E>(p.v, b, h, t, c);
  }
  if (tid < p.T)
    sa[tid] = p.ret == TS_RET_STREAM ? expf(step_ld<float>(p.decay, b, h, tid, 0))
                                     : (p.ret == TS_RET_STATIC ? expf(p.log_alpha[h]) : 1.f);
  float S[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg * RPT + r;
    S[r] = p.has_init && i < p.dk && j < p.dv ? p.init[state + (size_t)i * cols + j] : 0.f;
  }
  float D = p.vx && p.has_init && tid < p.dk ? p.init[state + (size_t)tid * cols + p.dv] : 0.f;
  __syncthreads();
  for (int t = 0; t < p.T; ++t) {
    const int buf = t & 1;
    const float a = sa[t];
    float part = 0.f;
    if (j < p.dv) {
      const float vj = sv[t][j];
#pragma unroll
      for (int r = 0; r < RPT; ++r) {
        const int i = rg * RPT + r;
        if (i < p.dk) {
          S[r] = a * S[r] + sk[t][i] * vj;
          part += sq[t][i] * S[r];
        }
      }
    }
    red[buf][rg][j] = part;
    if (tid < 128) {
      float md = 0.f;
      if (p.vx && tid < p.dk) {
        D = a * D + sk[t][tid];
        md = sq[t][tid] * D;
      }
      sd[buf][tid] = md;
    }
    // a slow thread still reading buffer `buf` of token t has passed this
    // barrier before any thread writes it again (token t + 2)
    __syncthreads();
    if (tid < p.dv) {
      const float o = red[buf][0][tid] + red[buf][1][tid];
      const int64_t off = (int64_t)b * p.out.sb + (int64_t)h * p.out.sh + (int64_t)t * p.out.st + tid;
      if (p.out_f32) ((float*)p.out.ptr)[off] = p.out_scale * o;
      else ((E*)p.out.ptr)[off] = cvt<E>(o);
    }
    if (p.vx && p.oe.ptr && tid >= 128 && tid < 192) {
      float m = sd[buf][lane] + sd[buf][lane + 64];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) m += __shfl_xor(m, o, 64);
      if (lane == 0)
        ((float*)p.oe.ptr)[(int64_t)b * p.oe.sb + (int64_t)h * p.oe.sh + (int64_t)t * p.oe.st] =
            p.out_f32 ? p.out_scale * m : m;
    }
  }
  if (p.fin) {
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int i = rg * RPT + r;
      if (i < p.dk && j < p.dv) p.fin[state + (size_t)i * cols + j] = S[r];
    }
    if (p.vx && tid < p.dk) p.fin[state + (size_t)tid * cols + p.dv] = D;
  }
}

// Four consecutive elements per thread (nelem is a multiple of 16).
__global__ void scan_prefix_kernel(float* seg, const float* segdec, FinalP F, int nseg, int nsum, int nelem) {
  const int bh = blockIdx.y;
  const int e0 = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (e0 >= nelem) return;
  const size_t state = (size_t)bh * (F.dk + F.kx) * (F.dv + F.vx);
  int x[4];
  float c0[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = exact_index(F, e0 + i);
    c0[i] = F.init && x[i] >= 0 ? F.init[state + x[i]] : 0.0f;
  }
  const float4 carry = segment_prefix4(seg + (size_t)bh * nseg * nelem + e0, segdec + (size_t)bh * nseg, nseg, nsum,
                                       nelem, make_float4(c0[0], c0[1], c0[2], c0[3]));
  const float c[4] = {carry.x, carry.y, carry.z, carry.w};
  if (F.fin) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (x[i] >= 0) F.fin[state + x[i]] = c[i];
  }
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

hipError_t ensure_lds_limit(const void* fn, int bytes) {
  static std::mutex mu;
  static std::unordered_map<const void*, int> limits;
  std::lock_guard<std::mutex> lock(mu);
  auto it = limits.find(fn);
  if (it != limits.end() && it->second >= bytes) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) limits[fn] = bytes;
  return e;
}

long resident_workgroups(const void* fn, int lds, int threads) {
  static std::mutex mu;
  static std::map<std::tuple<int, const void*, int, int>, long> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(dev, fn, lds, threads);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  long n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, (size_t)lds) == hipSuccess &&
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess)
    n = (long)per_cu * cus;
  cache[key] = n;
  return n;
}

}  // namespace ts

namespace {

using ts::fail;

const int kDkPads[] = {16, 32, 64, 128};

int pick_dkp(int need) {
  for (int v : kDkPads)
    if (need <= v) return v;
  return -1;
}

struct Layout {
  int dkp, dvp, vs, nvs, nvw, nchunks, seg_chunks, nseg, nsum, nelem;
  bool kx, vx;
  size_t ws_bytes;
};

int compute_layout(const ts_scan_desc* d, Layout* L) {
  if (!d) return fail(TS_ERR_VALUE, "scan: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0) return fail(TS_ERR_VALUE, "scan: bad shape");
  if (d->dk < 1 || d->dv < 1) return fail(TS_ERR_VALUE, "scan: feature widths must be >= 1");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "scan: unknown dtype");
  if (d->retention < TS_RET_NONE || d->retention > TS_RET_STREAM)
    return fail(TS_ERR_VALUE, "scan: unknown retention kind");
  for (int e : {d->q_ext, d->k_ext, d->v_ext})
    if (e < TS_EXT_NONE || e > TS_EXT_ARRAY) return fail(TS_ERR_VALUE, "scan: unknown ext column kind");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  if (d->dk % vec || d->dv % vec)
    return fail(TS_ERR_VALUE, "scan: feature widths must be multiples of 16 bytes (dk=%d dv=%d)",
                d->dk, d->dv);
  L->kx = d->q_ext != TS_EXT_NONE && d->k_ext != TS_EXT_NONE;
  L->vx = d->v_ext != TS_EXT_NONE;
  if (L->kx && L->vx)
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan: key-side and value-side ext columns together");
  L->dkp = pick_dkp(d->dk);
  if (L->dkp < 0) return fail(TS_ERR_NOT_IMPLEMENTED, "scan: key width %d exceeds 128", d->dk);
  L->dvp = (d->dv + 15) / 16 * 16;
  if (L->dvp > 128) return fail(TS_ERR_NOT_IMPLEMENTED, "scan: value width %d exceeds 128", d->dv);
  L->nchunks = (d->T + ts::C - 1) / ts::C;
  const int bh = d->B * d->H;
  // Value slices: each workgroup carries the state of `vs` value columns, so
  // B*H*nvs scans run side by side (the slices of one (b, h) re-read its q / k
  // tiles from L2).  Auto: one slice of the whole width -- at 64-wide keys and
  // values time segments beat slices (46 us against 49 us for two slices and
  // 68 us for four; a slice's 64-token steps are bound by the in-CU
  // dependency chain, not by memory) -- unless that tile leaves room for only
  // one workgroup per CU: then 64-column slices (128-wide keys and values,
  // B8 H8 T2048: 59 us against 82 us for one slice).
  if (d->value_split > 0) {
    const int v = d->value_split;
    if ((v != 16 && v != 32 && v != 64 && v != 128) || L->dvp % v)
      return fail(TS_ERR_VALUE, "scan: value_split %d must be 16, 32, 64 or 128 and divide %d", v, L->dvp);
    L->vs = v;
  } else {
    const int esize = d->dtype == TS_BF16 ? 2 : 4;
    L->vs = L->dvp;
    if (L->dvp == 128 && 2 * ts::scan_layout(esize, L->dkp, 128, true).bytes > ts::kLdsPerCU) L->vs = 64;
  }
  L->nvs = L->dvp / L->vs;
  L->nvw = L->vs <= 64 ? 1 : 2;
  if (d->seg_chunks > 0) {
    L->seg_chunks = d->seg_chunks;
  } else {
    // Segments of the time axis up to about two workgroups per CU (256 CUs).
    const int lanes = bh * L->nvs;
    int want = 512 / (lanes > 0 ? lanes : 1);
    if (want < 1) want = 1;
    L->seg_chunks = (L->nchunks + want - 1) / want;
    if (L->seg_chunks < 1) L->seg_chunks = 1;
  }
  L->nseg = L->nchunks > 0 ? (L->nchunks + L->seg_chunks - 1) / L->seg_chunks : 0;
  L->nsum = d->want_final ? L->nseg : (L->nseg > 0 ? L->nseg - 1 : 0);
  L->nelem = L->dkp * L->dvp + L->dvp + L->dkp;
  if (d->states_in < 0 || d->states_in > 3) return fail(TS_ERR_VALUE, "scan: states_in must be 0, 1, 2 or 3");
  if (d->states_in == 3) {
    if (d->want_final || L->kx || d->retention != TS_RET_NONE)
      return fail(TS_ERR_NOT_IMPLEMENTED, "scan: given segment summaries need a plain sum without a final state "
                                          "or key-side ext columns");
  } else if (d->states_in) {
    if ((L->kx && d->states_in == 1) || L->vx || d->want_final)
      return fail(TS_ERR_NOT_IMPLEMENTED, "scan: given segment states need no value-side ext column and no "
                                          "final state");
    if (d->states_in == 2 && (d->dk != d->dv || L->dkp != L->dvp))
      return fail(TS_ERR_NOT_IMPLEMENTED, "scan: transposed segment states need dk == dv (a padded width)");
  }
  if (d->init_state && d->states_in)
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan: an initial state with given segment states");
  if (d->states_in == 3 && L->nsum > 0 && !(d->value_split == 0 && L->nvs == 1))
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan: given segment summaries need one value slice");
  L->ws_bytes = 0;
  if (L->nsum > 0 || d->init_state)
    L->ws_bytes = (size_t)bh * L->nseg * (size_t)L->nelem * sizeof(float) + (size_t)bh * L->nseg * sizeof(float) + 256;
  return TS_OK;
}

}  // namespace

int ts::scan_segments(const ts_scan_desc* d, ts::ScanSegments* out) {
  Layout L;
  int rc = compute_layout(d, &L);
  if (rc) return rc;
  out->seg_chunks = L.seg_chunks; out->nseg = L.nseg; out->nsum = L.nsum; out->nelem = L.nelem;
  out->dkp = L.dkp; out->dvp = L.dvp; out->ws_bytes = L.ws_bytes;
  return TS_OK;
}

namespace {

typedef void (*KernelFn)(ts::ScanP);

template <typename E, int NVW, int MODE>
KernelFn pick_kernel_v(int dkp, bool main_kernel) {
  switch (dkp) {
#define TS_CASE(D)                                                                    \
  case D:                                                                             \
    return main_kernel ? (KernelFn)ts::scan_kernel<E, D, NVW, true, MODE>             \
                       : (KernelFn)ts::scan_kernel<E, D, NVW, false, MODE>;
    TS_CASE(16)
    TS_CASE(32)
    TS_CASE(64)
    TS_CASE(128)
#undef TS_CASE
  }
  return nullptr;
}

// The bf16 modes compiled: the kernel memory's scans (plain, key-side and
// value-side ext columns), the temporal bank's static views (with or without
// the key-mass column) and the composed backward's fp32 gradient scans (with
// or without the key-side column and a static retention).
template <typename E, int NVW>
KernelFn pick_kernel_m(int dkp, bool main_kernel, int mode) {
  using namespace ts;
  switch (mode) {
#define TS_MODE(M) \
  case M: return pick_kernel_v<E, NVW, M>(dkp, main_kernel);
    TS_MODE(kPlain)
    TS_MODE(kKeyExt)
    TS_MODE(kValExt)
    TS_MODE(kStatic)
    TS_MODE(kStatic | kValExt)
    TS_MODE(kF32Out)
    TS_MODE(kF32Out | kKeyExt)
    TS_MODE(kF32Out | kStatic)
    TS_MODE(kF32Out | kStatic | kKeyExt)
#undef TS_MODE
  }
  return pick_kernel_v<E, NVW, kGeneral>(dkp, main_kernel);
}

// bf16 kernels are specialised by mode; the fp32 parity kernels are general.
KernelFn pick_kernel(bool bf16, int dkp, int nvw, bool main_kernel, int mode) {
  if (!bf16)
    return nvw == 1 ? pick_kernel_v<float, 1, ts::kGeneral>(dkp, main_kernel)
                    : pick_kernel_v<float, 2, ts::kGeneral>(dkp, main_kernel);
  return nvw == 1 ? pick_kernel_m<ts::bf16, 1>(dkp, main_kernel, mode)
                  : pick_kernel_m<ts::bf16, 2>(dkp, main_kernel, mode);
}

// Bytes spanned by one (batch, head) slice of a [.., T, width] stream, or an
// error if rows up to T + two tiles could not be addressed with 31-bit offsets.
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

int launch(KernelFn fn, dim3 grid, size_t lds, hipStream_t stream, const ts::ScanP& p) {
  if (!fn) return fail(TS_ERR_NOT_IMPLEMENTED, "scan: no kernel for this shape");
  if (lds > 65536) {
    hipError_t e = ts::ensure_lds_limit((const void*)fn, (int)lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: LDS request failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(fn, grid, dim3(256), lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

}  // namespace

// Workspace of ts_scan_fwd_noalloc: one copy on every GPU the library runs
// on, held until the process ends (the code object's device globals are
// placed when the library's kernels are loaded on a device).  Host code never
// passes `scratch` itself to a kernel or a copy -- on the host the name is a
// stand-in, not a device address -- but the per-device address that
// hipGetSymbolAddress returns (device_scratch).
static __device__ __align__(256) unsigned char scratch[TS_SCAN_NOALLOC_MAX_WORKSPACE];

namespace {

std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices];  // per device, set on the first call made with that device current

// Device address of `scratch` on the current device, looked up once per
// device with that device current.
int device_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(TS_ERR_RUNTIME, "scan noalloc: device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(TS_ERR_RUNTIME, "scan noalloc: no device address for the scratch buffer on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
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
  if (dk_pad) *dk_pad = desc->dk + (L.kx ? 1 : 0);
  if (dv_pad) *dv_pad = desc->dv + (L.vx ? 1 : 0);
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

int ts_scan_pair_fwd(const ts_scan_desc* d, const ts_scan_pair_io* io, void* workspace, size_t ws_bytes,
                     hipStream_t stream) {
  Layout L;
  int rc = compute_layout(d, &L);
  if (rc) return rc;
  if (!io) return fail(TS_ERR_VALUE, "scan pair: null io");
  // scan A may carry the key-side ext pair of a normalized read's backward
  const bool kx = L.kx;
  if (kx && (d->q_ext != TS_EXT_ONES || d->k_ext != TS_EXT_ARRAY))
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan pair: the key-side ext pair must be q_ext ones, k_ext array");
  if (d->dtype != TS_BF16 || (d->retention != TS_RET_NONE && d->retention != TS_RET_STATIC) || L.vx ||
      d->dk != 64 || d->dv != 64 || L.nvs != 1 || d->states_in || d->want_final || d->init_state)
    return fail(TS_ERR_NOT_IMPLEMENTED,
                "scan pair: bf16 scans of 64-wide keys and values with no or a static retention only");
  if (kx && !io->k_ext.ptr) return fail(TS_ERR_VALUE, "scan pair: missing k ext column");
  const bool stat = d->retention == TS_RET_STATIC;
  if (stat && !io->log_alpha) return fail(TS_ERR_VALUE, "scan pair: missing log_alpha");
  const bool f32 = d->out_mode != TS_OUT_STORE;
  if (d->T == 0) return TS_OK;
  int rc2;
  if ((rc2 = check_stream("qa", io->qa, 8, true)) || (rc2 = check_stream("k", io->k, 8, true)) ||
      (rc2 = check_stream("v", io->v, 8, true)) || (rc2 = check_stream("qb", io->qb, 8, true)))
    return rc2;
  for (const ts_strided* o : {&io->out_a, &io->out_b})
    if (!o->ptr || ((uintptr_t)o->ptr & (f32 ? 15u : 7u)) || o->st % (f32 ? 4 : 8) || o->sh % (f32 ? 4 : 8) ||
        o->sb % (f32 ? 4 : 8))
      return fail(TS_ERR_VALUE, "scan pair: outputs must be 16-byte aligned rows");
  if (L.ws_bytes > 0 && (!workspace || ws_bytes < L.ws_bytes))
    return fail(TS_ERR_VALUE, "scan pair: workspace too small (%zu < %zu bytes)", ws_bytes, L.ws_bytes);
  if (L.ws_bytes > 0 && !aligned16(workspace)) return fail(TS_ERR_VALUE, "scan pair: workspace is not 16-byte aligned");

  ts::PairP pp;
  memset(&pp, 0, sizeof(pp));
  ts::ScanP& p = pp.s;
  p.B = d->B; p.H = d->H; p.T = d->T; p.dk = d->dk; p.dv = d->dv; p.dvp = L.dvp; p.vs = L.vs;
  p.nchunks = L.nchunks; p.seg_chunks = L.seg_chunks; p.nseg = L.nseg; p.nsum = L.nsum; p.nelem = L.nelem;
  p.ret = stat ? TS_RET_STATIC : TS_RET_NONE; p.reverse = d->reverse;
  p.log_alpha = io->log_alpha;
  p.q_ext = p.k_ext = p.v_ext = TS_EXT_NONE;
  if (kx) { p.q_ext = TS_EXT_ONES; p.k_ext = TS_EXT_ARRAY; p.ke = io->k_ext; }
  p.out_mode = d->out_mode; p.out_scale = f32 ? d->out_scale : 1.0f;
  p.q = io->qa; p.k = io->k; p.v = io->v; p.out = io->out_a;
  pp.qb = io->qb; pp.ob = io->out_b;
  if (kx && (rc = slice_bytes("k_ext", p.ke, d->T, 1, 4, &p.ke_rec))) return rc;
  if ((rc = slice_bytes("qa", p.q, d->T, d->dk, 2, &p.q_rec))) return rc;
  if ((rc = slice_bytes("k", p.k, d->T, d->dk, 2, &p.k_rec))) return rc;
  if ((rc = slice_bytes("v", p.v, d->T, d->dv, 2, &p.v_rec))) return rc;
  if ((rc = slice_bytes("qb", pp.qb, d->T, d->dv, 2, &pp.qb_rec))) return rc;
  if ((rc = slice_bytes("out_a", p.out, d->T, d->dv, f32 ? 4 : 2, &p.out_rec))) return rc;
  if ((rc = slice_bytes("out_b", pp.ob, d->T, d->dk, f32 ? 4 : 2, &pp.ob_rec))) return rc;
  if (L.ws_bytes > 0) {
    p.seg = (float*)workspace;
    p.segdec = p.seg + (size_t)d->B * d->H * L.nseg * (size_t)L.nelem;
  }
  const int bh = d->B * d->H;
  const ts::ScanLayout SL = ts::scan_layout(2, 64, 64, true);
  if (SL.nst != 2) return fail(TS_ERR_RUNTIME, "scan pair: unexpected state buffering");
  if (L.nsum > 0) {
    // The summary pass writes no outputs, so kF32Out only picks an
    // instantiation that exists for a static key-ext scan.
    const int smode = stat ? (kx ? ts::kStatic | ts::kKeyExt | ts::kF32Out : ts::kStatic)
                           : (kx ? ts::kKeyExt : ts::kPlain);
    KernelFn fsum = pick_kernel(true, 64, 1, false, smode);
    if ((rc = launch(fsum, dim3(L.nsum, bh, 1), (size_t)ts::scan_layout(2, 64, 64, false).bytes, stream, p))) return rc;
    ts::FinalP F{nullptr, nullptr, L.dkp, L.dvp, d->dk, d->dv, 0, 0};
    hipLaunchKernelGGL(ts::scan_prefix_kernel, dim3((L.nelem / 4 + 255) / 256, bh), dim3(256), 0, stream, p.seg,
                       p.segdec, F, L.nseg, L.nsum, L.nelem);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan pair: prefix launch failed: %s", hipGetErrorString(e));
  }
  typedef void (*PairFn)(ts::PairP);
  const int pm = (stat ? ts::kStatic : 0) | (f32 ? ts::kF32Out : 0);
  PairFn fn = nullptr;
  switch (pm) {
#define TS_PAIR(M) \
  case M: fn = kx ? (PairFn)ts::pair_kernel<64, true, M> : (PairFn)ts::pair_kernel<64, false, M>; break;
    TS_PAIR(ts::kPlain)
    TS_PAIR(ts::kStatic)
    TS_PAIR(ts::kF32Out)
    TS_PAIR(ts::kStatic | ts::kF32Out)
#undef TS_PAIR
  }
  hipLaunchKernelGGL(fn, dim3(L.nseg, bh), dim3(256), (size_t)SL.bytes, stream, pp);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan pair: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

static int scan_fwd_impl(const ts_scan_desc* d, const ts_scan_io* io, void* workspace, size_t ws_bytes,
                         hipStream_t stream) {
  Layout L;
  int rc = compute_layout(d, &L);
  if (rc) return rc;
  if (!io) return fail(TS_ERR_VALUE, "scan: null io");
  if (d->want_final && !io->final_state) return fail(TS_ERR_VALUE, "scan: missing final_state buffer");
  if (d->init_state && !io->init_state) return fail(TS_ERR_VALUE, "scan: missing init_state buffer");
  if (d->T == 0) {
    // An empty piece leaves the carried state unchanged: the final state is
    // the initial one (or zero).  The prefix kernel over zero segments
    // writes exactly that.
    if (!d->want_final) return TS_OK;
    ts::FinalP F{io->final_state, d->init_state ? io->init_state : nullptr, L.dkp, L.dvp, d->dk, d->dv,
                 L.kx ? 1 : 0, L.vx ? 1 : 0};
    hipLaunchKernelGGL(ts::scan_prefix_kernel, dim3((L.nelem / 4 + 255) / 256, d->B * d->H), dim3(256), 0, stream,
                       (float*)nullptr, (const float*)nullptr, F, 0, 0, L.nelem);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: prefix launch failed: %s", hipGetErrorString(e));
    return TS_OK;
  }
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
  if (d->init_state && !io->init_state) return fail(TS_ERR_VALUE, "scan: missing init_state buffer");
  if (L.ws_bytes > 0 && (!workspace || ws_bytes < L.ws_bytes))
    return fail(TS_ERR_VALUE, "scan: workspace too small (%lld < %lld bytes)", (long long)ws_bytes,
                (long long)L.ws_bytes);
  if (L.ws_bytes > 0 && !aligned16(workspace)) return fail(TS_ERR_VALUE, "scan: workspace is not 16-byte aligned");

  ts::ScanP p;
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.dk = d->dk; p.dv = d->dv; p.dvp = L.dvp; p.vs = L.vs;
  p.nchunks = L.nchunks; p.seg_chunks = L.seg_chunks; p.nseg = L.nseg; p.nsum = L.nsum; p.nelem = L.nelem;
  p.ret = d->retention; p.reverse = d->reverse;
  p.q_ext = L.kx ? d->q_ext : TS_EXT_NONE;
  p.k_ext = L.kx ? d->k_ext : TS_EXT_NONE;
  p.v_ext = d->v_ext;
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
    p.segdec = p.seg + (size_t)d->B * d->H * L.nseg * (size_t)L.nelem;
  }

  const int bh = d->B * d->H;
  // a short continuation of a carried state: one token-by-token launch
  if (d->T <= ts::kStepMaxT && (d->init_state || d->want_final) && !d->reverse && !L.kx &&
      (d->v_ext == TS_EXT_NONE || d->v_ext == TS_EXT_ONES) &&
      (d->out_mode == TS_OUT_STORE || d->out_mode == TS_OUT_STORE_F32) && d->value_split == 0 &&
      d->states_in == 0 && L.dkp <= 128 && d->dv <= 128) {
    ts::StepP sp;
    memset(&sp, 0, sizeof(sp));
    sp.H = d->H; sp.T = d->T; sp.dk = d->dk; sp.dv = d->dv; sp.vx = L.vx ? 1 : 0; sp.ret = d->retention;
    sp.out_f32 = d->out_mode == TS_OUT_STORE ? 0 : 1; sp.has_init = d->init_state ? 1 : 0;
    sp.out_scale = d->out_scale;
    sp.q = io->q; sp.k = io->k; sp.v = io->v; sp.decay = io->decay; sp.out = io->out; sp.oe = io->out_ext;
    sp.log_alpha = io->log_alpha;
    sp.init = d->init_state ? io->init_state : nullptr;
    sp.fin = d->want_final ? io->final_state : nullptr;
    const bool bf = d->dtype == TS_BF16;
#define TS_STEP_CASE(DK)                                                                               \
  if (bf) hipLaunchKernelGGL((ts::scan_step_kernel<ts::bf16, DK>), dim3(bh), dim3(256), 0, stream, sp); \
  else hipLaunchKernelGGL((ts::scan_step_kernel<float, DK>), dim3(bh), dim3(256), 0, stream, sp);
    switch (L.dkp) {
      case 16: { TS_STEP_CASE(16) } break;
      case 32: { TS_STEP_CASE(32) } break;
      case 64: { TS_STEP_CASE(64) } break;
      default: { TS_STEP_CASE(128) } break;
    }
#undef TS_STEP_CASE
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: step launch failed: %s", hipGetErrorString(e));
    return TS_OK;
  }
  int mode = ts::kGeneral;
  if (d->retention != TS_RET_STREAM) {
    mode = (d->retention == TS_RET_STATIC ? ts::kStatic : 0) | (L.kx ? ts::kKeyExt : 0) | (L.vx ? ts::kValExt : 0) |
           (d->out_mode != TS_OUT_STORE ? ts::kF32Out : 0);
    // an fp32 output with a value-side ext column (its fp32 ext output) is general
    if ((mode & ts::kF32Out) && (mode & ts::kValExt)) mode = ts::kGeneral;
  }
  KernelFn fsum = pick_kernel(d->dtype == TS_BF16, L.dkp, L.nvw, false, mode);
  KernelFn fmain = pick_kernel(d->dtype == TS_BF16, L.dkp, L.nvw, true, mode);
  const size_t lds_sum = (size_t)ts::scan_layout(esize, L.dkp, L.vs, false).bytes;
  const size_t lds_main = (size_t)ts::scan_layout(esize, L.dkp, L.vs, true).bytes;
  if (lds_main > 160 * 1024)
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan: tile of %lld bytes exceeds LDS (dk_pad=%d slice=%d)",
                (long long)lds_main, L.dkp, L.vs);

  p.states_t = d->states_in == 2;
  p.has_init = d->init_state ? 1 : 0;
  if ((L.nsum > 0 || d->init_state) && (d->states_in == 0 || d->states_in == 3)) {
    // states_in 3: the workspace already holds the summaries (the prefix runs)
    if (d->states_in == 0 && L.nsum > 0 && (rc = launch(fsum, dim3(L.nsum, bh, L.nvs), lds_sum, stream, p)))
      return rc;
    ts::FinalP F{d->want_final ? io->final_state : nullptr, d->init_state ? io->init_state : nullptr, L.dkp, L.dvp,
                 d->dk, d->dv, L.kx ? 1 : 0, L.vx ? 1 : 0};
    hipLaunchKernelGGL(ts::scan_prefix_kernel, dim3((L.nelem / 4 + 255) / 256, bh), dim3(256), 0, stream, p.seg,
                       p.segdec, F, L.nseg, L.nsum, L.nelem);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: prefix launch failed: %s", hipGetErrorString(e));
  }
  return launch(fmain, dim3(L.nseg, bh, L.nvs), lds_main, stream, p);
}

int ts_scan_fwd(const ts_scan_desc* d, const ts_scan_io* io, void* workspace, size_t ws_bytes,
                hipStream_t stream) {
  return scan_fwd_impl(d, io, workspace, ws_bytes, stream);
}

int ts_scan_fwd_noalloc(const ts_scan_desc* d, const ts_scan_io* io, hipStream_t stream) {
  Layout L;
  int rc = compute_layout(d, &L);
  if (rc) return rc;
  if (d->states_in)
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan noalloc: kept segment states (states_in) need a workspace the "
                                        "caller owns across calls; use ts_scan_fwd");
  if (L.ws_bytes > (size_t)TS_SCAN_NOALLOC_MAX_WORKSPACE)
    return fail(TS_ERR_VALUE, "scan noalloc: this scan needs %zu bytes of workspace, above the %zu-byte scratch "
                              "buffer of ts_scan_fwd_noalloc; use ts_scan_fwd with a workspace",
                L.ws_bytes, (size_t)TS_SCAN_NOALLOC_MAX_WORKSPACE);
  void* ws = nullptr;
  if (L.ws_bytes > 0 && (rc = device_scratch(&ws))) return rc;
  return scan_fwd_impl(d, io, ws, L.ws_bytes, stream);
}

}  // extern "C"
