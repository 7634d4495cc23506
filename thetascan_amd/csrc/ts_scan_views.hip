// Several retentions of one q, k, v in one scan (gfx950).
//
// The multi-view call of the reference's chunk backend
// (src/thetascan/_core/ops/scan_chunk.py:246-339): a temporal bank scans the
// same streams under a plain sum and per-head static retentions, and the
// score tile S = Q K^T of every 64-token tile is the same for all of them.
// Here q, k and v are read once per pass and the score tile is formed once;
// each view applies its own decay mask to it and carries its own fp32 state.
//
// The passes are those of the one-view scan (ts_scan.hip): a summary kernel
// folds each segment's writes into a per-view summary, a prefix kernel scans
// the summaries over segments, and the main kernel re-walks each segment from
// the incoming states and writes every view's outputs (and key mass).  Inside
// a tile, wave w owns query block w and value block w: the scores of its
// queries stay in MFMA accumulators and feed the P.V contraction of every
// view; each view's state enters the outputs through a bf16 copy published in
// LDS (one per view, written between the tile's two barriers).  A view with
// no retention uses unit weights, which multiply exactly, so every view's
// result equals the one-view scan's with the same segments bit for bit.

#include "ts_common.h"
#include "ts_scan_impl.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct ViewsP {
  ScanP s;                     // shared streams, sizes, segmentation (ret/ext fields unused)
  int nv, mass;
  const float* log_alpha[TS_MAX_VIEWS];
  ts_strided out[TS_MAX_VIEWS], oe[TS_MAX_VIEWS];
  uint32_t out_rec[TS_MAX_VIEWS], oe_rec[TS_MAX_VIEWS];
  size_t seg_vstride, dec_vstride;  // floats between the views' summaries / segment decays
};

// LDS: K [C][kp], V [C][vp] (one stage), `nst` state copies [64][kp], then
// fp32: D [NV][DK], alpha^d [NV][68], and the masked powers [NV][4][kPwx]:
// copy s of view r holds f(j + s - 64) at j, f(d) = alpha_r^d for 0 <= d <= 64
// and 0 for d < 0, so the four powers f(d0 .. d0+3) of any window are one
// aligned 16-byte read (copy (d0 + 64) & 3 at j = d0 + 64 - that copy) and
// the causal / tile-length masks are in the table.
// The tables are kept where they leave the two workgroups per CU that the
// registers allow (at most 80 KB each); 128-wide keys with three views keep
// the per-element reads of alpha^d instead.
constexpr int kPwx = 128;
constexpr int kViewsLdsPerWg = 80 * 1024;
struct ViewsLayout {
  int kp, vp, st, nst, fbase, bytes;
  bool pwx;
};
__host__ __device__ constexpr ViewsLayout views_layout(int DK, int NV, bool main_kernel) {
  ViewsLayout L{};
  L.kp = DK + 8;
  L.vp = 64 + 8;
  L.st = 64 * L.kp;
  L.nst = main_kernel ? NV : 0;
  const int e_bytes = ((C * L.kp + C * L.vp + L.nst * L.st) * 2 + 15) / 16 * 16;
  L.fbase = e_bytes / 4;
  const int base = e_bytes + (NV * DK + NV * 68) * 4;
  L.pwx = base + NV * 4 * kPwx * 4 <= kViewsLdsPerWg;
  L.bytes = base + (L.pwx ? NV * 4 * kPwx * 4 : 0);
  return L;
}

// f(d0 .. d0 + 3) of one view's masked-power copies (-64 <= d0, d0 + 3 <= 67)
__device__ __forceinline__ floatx4 pow_window(const float* pwx, int d0) {
  const int j = d0 + 64;
  const int sft = j & 3;
  return *(const floatx4*)(pwx + sft * kPwx + (j - sft));
}

// One [64 x 8*PER_ROW] bf16 tile section (K or V rows), fetched into
// registers (16-byte vectors, thread tid owns vectors tid + 256 i) and stored
// to LDS later.  Offsets are recomputed per use rather than kept in registers.
template <int PER_ROW>
struct RowLoader {
  static constexpr int SLOTS = C * PER_ROW / 256;
  static_assert(SLOTS * 256 == C * PER_ROW, "the tile section must be whole 256-vector slots");
  uint4 r[SLOTS];
  __device__ __forceinline__ void fetch(rsrc_t data, int t0, int st_b, int width, int tid) {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / PER_ROW;
      const int c0 = (idx % PER_ROW) * 8;
      r[i] = bld16(data, c0 < width ? (uint32_t)((t0 + row) * st_b + c0 * 2) : kOOB);
    }
  }
  __device__ __forceinline__ void store(bf16* dst, int pitch, int tid) const {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int idx = tid + i * 256;
      *(uint4*)(dst + (idx / PER_ROW) * pitch + (idx % PER_ROW) * 8) = r[i];
    }
  }
};

template <int DK, int NV, bool MAIN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void views_kernel(ViewsP vp) {
  typedef bf16 E;
  typedef bf16x8 F8;
  typedef LdsIO<E> IO;
  typedef Tok<E> TK;
  constexpr int VEC = 8;
  constexpr int NK32 = DK / 32;
  constexpr int NKB = DK / 16;
  constexpr int NKO = NKB / 4;  // key blocks of D owned per wave
  const ScanP& p = vp.s;
  const bool mass = vp.mass != 0;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int g = lane >> 4;
  const int l16 = lane & 15;
  const int seg = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int wave_first = __builtin_amdgcn_readfirstlane(tid & ~63);

  constexpr ViewsLayout L = views_layout(DK, NV, MAIN);
  constexpr bool PWX = L.pwx;
  extern __shared__ __align__(16) unsigned char smem[];
  E* Ks = (E*)smem;
  E* Vs = Ks + C * L.kp;
  E* st_base = Vs + C * L.vp;
  float* s_d = (float*)smem + L.fbase;  // [NV][DK]
  float* s_pw = s_d + NV * DK;           // [NV][68]: alpha_r^d, d = 0..64
  float* s_pwx = s_pw + NV * 68;         // [NV][4][kPwx]: masked powers, shifted copies

  const int64_t bh_q = (int64_t)b * p.q.sb + (int64_t)h * p.q.sh;
  const int64_t bh_k = (int64_t)b * p.k.sb + (int64_t)h * p.k.sh;
  const int64_t bh_v = (int64_t)b * p.v.sb + (int64_t)h * p.v.sh;
  const int q_st_b = (int)p.q.st * 2;
  const int k_st_b = (int)p.k.st * 2;
  const int v_st_b = (int)p.v.st * 2;
  auto k_rsrc = [&]() { return make_rsrc((const E*)p.k.ptr + bh_k, p.k_rec); };
  auto v_rsrc = [&]() { return make_rsrc((const E*)p.v.ptr + bh_v, p.v_rec); };
  auto q_rsrc = [&]() { return make_rsrc((const E*)p.q.ptr + bh_q, p.q_rec); };

  float la[NV];
#pragma unroll
  for (int r = 0; r < NV; ++r) la[r] = vp.log_alpha[r] ? vp.log_alpha[r][h] : 0.0f;
  if (w == 0) {
#pragma unroll
    for (int r = 0; r < NV; ++r) {
      s_pw[r * 68 + lane] = expf(la[r] * (float)lane);
      if (lane == 0) s_pw[r * 68 + 64] = expf(la[r] * 64.0f);
    }
  }
  // masked powers: the same expf values (d = 0..64), zero below d = 0 and
  // above 64 (indices past 64 are never read by a window that matters)
  if constexpr (PWX) {
    for (int e = tid; e < NV * 4 * kPwx; e += 256) {
      const int r = e / (4 * kPwx), rem = e - r * 4 * kPwx;
      const int sft = rem / kPwx, j = rem - sft * kPwx;
      const int d = j + sft - 64;
      s_pwx[e] = d >= 0 && d <= 64 ? expf(la[r] * (float)d) : 0.0f;
    }
  }

  // ---- per-view states: S [key][value block w]; D of key blocks w + 4 j
  // for every view at once: row r of the accumulator is view r (lanes of
  // group 0 hold rows 0..3 as elements 0..3; every other row stays zero)
  floatx4 S[NV][NKB];
  floatx4 Dall[NKO];
#pragma unroll
  for (int r = 0; r < NV; ++r)
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) S[r][kb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < NKO; ++j) Dall[j] = floatx4{0.f, 0.f, 0.f, 0.f};
  float seg_log[NV];
#pragma unroll
  for (int r = 0; r < NV; ++r) seg_log[r] = 0.0f;

  const int c_begin = seg * p.seg_chunks;
  const int c_end = min(c_begin + p.seg_chunks, p.nchunks);
  bool state_zero = true;

  if (MAIN && seg > 0) {
    state_zero = false;
#pragma unroll
    for (int r = 0; r < NV; ++r) {
      const float* src = p.seg + r * vp.seg_vstride + ((size_t)bh * p.nseg + seg) * (size_t)p.nelem;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[r][kb][i] = src[(kb * 16 + 4 * g + i) * p.dvp + w * 16 + l16];
      if (g == 0) {
#pragma unroll
        for (int j = 0; j < NKO; ++j) Dall[j][r] = src[DK * p.dvp + p.dvp + (w + 4 * j) * 16 + l16];
      }
    }
  }

  // publish every view's state entering the tile (bf16 copies, D)
  auto publish = [&]() {
#pragma unroll
    for (int r = 0; r < NV; ++r) {
      E* st = st_base + r * L.st;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        IO::st4(st + (w * 16 + l16) * L.kp + kb * 16 + 4 * g, S[r][kb][0], S[r][kb][1], S[r][kb][2], S[r][kb][3]);
      if (mass && g == 0) {
#pragma unroll
        for (int j = 0; j < NKO; ++j) s_d[r * DK + (w + 4 * j) * 16 + l16] = Dall[j][r];
      }
    }
  };

  // ---- tile loading (registers one tile ahead, then LDS)
  RowLoader<DK / VEC> ldk;
  RowLoader<64 / VEC> ldv;
  auto fetch = [&](int t0) {
    ldk.fetch(k_rsrc(), t0, k_st_b, p.dk, tid);
    ldv.fetch(v_rsrc(), t0, v_st_b, p.dv, tid);
  };

  // ---- queries of this wave's block
  F8 qr[NK32];
  auto qload = [&](int t0) {
    const uint32_t ro = row_off(p, t0, w * 16 + l16, q_st_b);
    auto part = [&](int c) -> bf16x4 {
      const uint32_t off = c < p.dk ? ro + (uint32_t)(c * 2) : kOOB;
      return __builtin_bit_cast(bf16x4, bld8(q_rsrc(), off));
    };
#pragma unroll
    for (int j = 0; j < NK32; ++j) qr[j] = IO::cat(part(32 * j + 4 * g), part(32 * j + 16 + 4 * g));
  };

  F8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (E)1.0f;

  fetch(c_begin * C);
  if (MAIN) qload(c_begin * C);

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * C;
    const int len = min(C, p.T - t0);
    __syncthreads();  // the previous tile's K, V, state copies and D are no longer read
    ldk.store(Ks, L.kp, tid);
    ldv.store(Vs, L.vp, tid);
    if (c + 1 < c_end) fetch(t0 + C);  // next tile's K and V, in flight during this one
    if (MAIN && !state_zero) publish();
    __syncthreads();

#pragma unroll
    for (int r = 0; r < NV; ++r) seg_log[r] += la[r] * (float)len;

    if constexpr (MAIN) {
      const int query = w * 16 + l16;
      // raw causal scores of this query block (shared by every view)
      floatx4 sc[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        sc[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (kb > w) continue;
        const int krow = kb * 16 + l16;
#pragma unroll
        for (int j = 0; j < NK32; ++j) sc[kb] = mma32(frow8<E>(Ks, L.kp, krow, j, g), qr[j], sc[kb]);
      }
      // one view at a time (a rolled loop: the views share no registers here)
#pragma unroll 1
      for (int r = 0; r < NV; ++r) {
        const float* pw = s_pw + r * 68;
        const float* pwx = s_pwx + r * 4 * kPwx;
        floatx4 pr[4];
        if constexpr (PWX) {
          // key kb*16+4g+i sits query - key = c - i before the query: the
          // window f(c-3 .. c) holds its weight at element 3 - i (zero for a
          // key after the query, which also covers the blocks kb > w)
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            const floatx4 wv = pow_window(pwx, query - kb * 16 - 4 * g - 3);
#pragma unroll
            for (int i = 0; i < 4; ++i) pr[kb][i] = sc[kb][i] * wv[3 - i];
          }
        } else {
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int key = kb * 16 + 4 * g + i;
              pr[kb][i] = (kb < w || (kb == w && key <= query)) ? sc[kb][i] * pw[max(query - key, 0)] : 0.0f;
            }
        }
        const F8 p0 = IO::from_acc(pr[0], pr[1]);
        const F8 p1 = IO::from_acc(pr[2], pr[3]);
        const float cw = pw[query + 1];
        const E* st = st_base + r * L.st;
        const uint32_t ro = row_off(p, t0, query, (int)vp.out[r].st * 2);
        const rsrc_t out_rs = make_rsrc(bh_base(vp.out[r], b, h, 2), vp.out_rec[r]);
#pragma unroll
        for (int vb = 0; vb < 4; ++vb) {
          floatx4 acc = {0.f, 0.f, 0.f, 0.f};
          if (!state_zero) {
#pragma unroll
            for (int j = 0; j < NK32; ++j) acc = mma32(frow8<E>(st, L.kp, vb * 16 + l16, j, g), qr[j], acc);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] *= cw;
          }
          acc = mma32(TK::col8(Vs, L.vp, vb * 16, 0, lane), p0, acc);
          if (w >= 2) acc = mma32(TK::col8(Vs, L.vp, vb * 16, 1, lane), p1, acc);
          const int ocol = vb * 16 + 4 * g;
          bf16x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = (bf16)acc[i];
          bst8(out_rs, ocol < p.dv ? ro + (uint32_t)(ocol * 2) : kOOB, __builtin_bit_cast(uint2, o));
        }
        if (mass) {
          // key mass: cw <q, D> + sum over keys of P (unit ext column)
          floatx4 oacc = {0.f, 0.f, 0.f, 0.f};
          if (!state_zero) {
#pragma unroll
            for (int j = 0; j < NK32; ++j) oacc = mma32(bcast8<E>(s_d + r * DK, 32 * j, g), qr[j], oacc);
#pragma unroll
            for (int i = 0; i < 4; ++i) oacc[i] *= cw;
          }
          oacc = mma32(ones, p0, oacc);
          if (w >= 2) oacc = mma32(ones, p1, oacc);
          if (g == 0) {
            const rsrc_t oe_rs = make_rsrc(bh_base(vp.oe[r], b, h, 4), vp.oe_rec[r]);
            bstf(oe_rs, row_off(p, t0, query, (int)vp.oe[r].st * 4), oacc[0]);
          }
        }
      }
    }
    if (MAIN && c + 1 < c_end) qload(t0 + C);  // next tile's queries
    // ---- state updates: S_r = alpha_r^len S_r + K^T diag(w_r) V (value block w)
    F8 av[2];
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) av[kp] = TK::col8(Vs, L.vp, w * 16, kp, lane);
    // weights of this lane's keys of contraction block kp in view r: keys
    // 32kp+4g+e (e < 4) and 32kp+16+4g+(e-4) sit len-1-key before the tile's
    // end; the window f(c-3 .. c) holds key e's weight at element 3 - (e & 3)
    // (zero for a key past the tile's length)
    auto key_weights = [&](int r, int kp, float* wk) {
      if constexpr (PWX) {
        const float* pwx = s_pwx + r * 4 * kPwx;
        const int c0 = len - 1 - 32 * kp - 4 * g;
        const floatx4 lo = pow_window(pwx, c0 - 3), hi = pow_window(pwx, c0 - 16 - 3);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          wk[e] = lo[3 - e];
          wk[4 + e] = hi[3 - e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = 32 * kp + (e < 4 ? 4 * g + e : 12 + 4 * g + e);
          const float wv = s_pw[r * 68 + max(len - 1 - key, 0)];  // loaded unconditionally: no branch
          wk[e] = key < len ? wv : 0.0f;
        }
      }
    };
    // one view at a time (K fragments re-read from LDS per view: fewer live
    // registers than sharing them across the views' states)
#pragma unroll
    for (int r = 0; r < NV; ++r) {
      __builtin_amdgcn_sched_barrier(0);  // keep each view's loads with its MFMAs (register pressure)
      const float cdec = s_pw[r * 68 + len];
      F8 avw[2];
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        float wk[8];
        key_weights(r, kp, wk);
#pragma unroll
        for (int e = 0; e < 8; ++e) avw[kp][e] = (E)(tof(av[kp][e]) * wk[e]);
      }
      if (!(MAIN && state_zero)) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) S[r][kb][i] *= cdec;
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) S[r][kb] = mma32(TK::col8(Ks, L.kp, kb * 16, kp, lane), avw[kp], S[r][kb]);
    }
    if (mass) {
      // D_r = alpha_r^len D_r + K^T (unit ext column times view r's key
      // weights): A row r carries view r's weights, so one MFMA per key block
      // and contraction block updates every view
      floatx4 ddec = {1.f, 1.f, 1.f, 1.f};
      if (g == 0) {
#pragma unroll
        for (int i = 0; i < NV; ++i) ddec[i] = s_pw[i * 68 + len];
      }
#pragma unroll
      for (int j = 0; j < NKO; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) Dall[j][i] *= ddec[i];
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        F8 a;
        float wk[8];
        key_weights(min(l16, NV - 1), kp, wk);
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = (E)(l16 < NV ? wk[e] : 0.0f);
#pragma unroll
        for (int j = 0; j < NKO; ++j) Dall[j] = mma32(a, TK::col8(Ks, L.kp, (w + 4 * j) * 16, kp, lane), Dall[j]);
      }
    }
    state_zero = false;
  }

  if constexpr (!MAIN) {
#pragma unroll
    for (int r = 0; r < NV; ++r) {
      float* dst = p.seg + r * vp.seg_vstride + ((size_t)bh * p.nseg + seg) * (size_t)p.nelem;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[(kb * 16 + 4 * g + i) * p.dvp + w * 16 + l16] = S[r][kb][i];
      if (g == 0) {
        dst[DK * p.dvp + w * 16 + l16] = 0.0f;  // no key-side ext row
#pragma unroll
        for (int j = 0; j < NKO; ++j) dst[DK * p.dvp + p.dvp + (w + 4 * j) * 16 + l16] = Dall[j][r];
      }
      if (tid == 0) p.segdec[r * vp.dec_vstride + (size_t)bh * p.nseg + seg] = seg_log[r];
    }
  }
}

// Exclusive scan of every view's segment summaries (blockIdx.z = view).
__global__ void views_prefix_kernel(float* seg, const float* segdec, int nseg, int nsum, int nelem,
                                    size_t seg_vstride, size_t dec_vstride) {
  const int bh = blockIdx.y;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nelem) return;
  const int r = blockIdx.z;
  segment_prefix(seg + r * seg_vstride + (size_t)bh * nseg * nelem + e, segdec + r * dec_vstride + (size_t)bh * nseg,
                 nseg, nsum, nelem);
}

}  // namespace ts

namespace {

using ts::fail;

struct ViewsPlan {
  int DK, nchunks, seg_chunks, nseg, nsum, nelem;
  size_t seg_vstride, dec_vstride, ws_bytes;
};

int plan_views(const ts_scan_views_desc* d, ViewsPlan* P) {
  if (!d) return fail(TS_ERR_VALUE, "scan views: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0) return fail(TS_ERR_VALUE, "scan views: bad shape");
  if (d->n_views < 2 || d->n_views > TS_MAX_VIEWS)
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan views: %d views (2 .. %d per call)", d->n_views, TS_MAX_VIEWS);
  if (d->dtype != TS_BF16) return fail(TS_ERR_NOT_IMPLEMENTED, "scan views: bf16 streams only");
  if (d->dk < 8 || d->dk > 128 || d->dk % 8 || d->dv < 8 || d->dv > 64 || d->dv % 8)
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan views: widths dk %d (8..128) and dv %d (8..64), multiples of 8",
                d->dk, d->dv);
  if (d->seg_chunks < 0) return fail(TS_ERR_VALUE, "scan views: seg_chunks must be >= 0");
  P->DK = d->dk <= 64 ? 64 : 128;
  P->nchunks = (d->T + ts::C - 1) / ts::C;
  const int bh = d->B * d->H;
  if (d->seg_chunks > 0) {
    P->seg_chunks = d->seg_chunks;
  } else {
    // the one-view scan's rule (about two workgroups per CU), so the views
    // share its segments
    int want = 512 / bh;
    if (want < 1) want = 1;
    P->seg_chunks = (P->nchunks + want - 1) / want;
    if (P->seg_chunks < 1) P->seg_chunks = 1;
  }
  P->nseg = P->nchunks > 0 ? (P->nchunks + P->seg_chunks - 1) / P->seg_chunks : 0;
  P->nsum = P->nseg > 0 ? P->nseg - 1 : 0;
  P->nelem = P->DK * 64 + 64 + P->DK;
  P->seg_vstride = (size_t)bh * P->nseg * P->nelem;
  P->dec_vstride = (size_t)bh * P->nseg;
  P->ws_bytes = P->nsum > 0 ? (size_t)d->n_views * (P->seg_vstride + P->dec_vstride) * sizeof(float) + 256 : 0;
  return TS_OK;
}

typedef void (*ViewsFn)(ts::ViewsP);

template <int DK>
ViewsFn pick_views_dk(int nv, bool main_kernel) {
  if (nv == 2) return main_kernel ? ts::views_kernel<DK, 2, true> : ts::views_kernel<DK, 2, false>;
  return main_kernel ? ts::views_kernel<DK, 3, true> : ts::views_kernel<DK, 3, false>;
}

int views_launch(ViewsFn fn, dim3 grid, size_t lds, hipStream_t stream, const ts::ViewsP& p) {
  if (lds > 65536) {
    hipError_t e = ts::ensure_lds_limit((const void*)fn, (int)lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan views: LDS request failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(fn, grid, dim3(256), lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan views: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

bool aligned(const void* ptr, uintptr_t to) { return ((uintptr_t)ptr & (to - 1)) == 0; }

// Bytes spanned by one (batch, head) slice of a [.., T, width] stream.
int span_bytes(const char* name, const ts_strided& s, int T, int width, int esize, uint32_t* out) {
  *out = 0;
  if (s.st < 0) return fail(TS_ERR_VALUE, "scan views: negative time stride of %s", name);
  const int64_t last = ((int64_t)(T > 0 ? T - 1 : 0) * s.st + width) * esize;
  const int64_t reach = ((int64_t)T + 2 * ts::C) * s.st * esize + (int64_t)width * esize;
  if (reach >= ((int64_t)1 << 31))
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan views: one (batch, head) slice of %s spans more than 2 GiB", name);
  *out = (uint32_t)last;
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_scan_views_workspace_bytes(const ts_scan_views_desc* d, size_t* bytes) {
  ViewsPlan P;
  int rc = plan_views(d, &P);
  if (rc) return rc;
  if (bytes) *bytes = P.ws_bytes;
  return TS_OK;
}

int ts_scan_views_fwd(const ts_scan_views_desc* d, const ts_scan_views_io* io, void* workspace, size_t ws_bytes,
                      hipStream_t stream) {
  ViewsPlan P;
  int rc = plan_views(d, &P);
  if (rc) return rc;
  if (!io) return fail(TS_ERR_VALUE, "scan views: null io");
  if (d->T == 0) return TS_OK;
  const ts_strided* ins[3] = {&io->q, &io->k, &io->v};
  const char* names[3] = {"q", "k", "v"};
  for (int i = 0; i < 3; ++i) {
    const ts_strided& s = *ins[i];
    if (!s.ptr) return fail(TS_ERR_VALUE, "scan views: missing tensor %s", names[i]);
    if (!aligned(s.ptr, 16) || s.st % 8 || s.sh % 8 || s.sb % 8)
      return fail(TS_ERR_VALUE, "scan views: rows of %s must be 16-byte aligned", names[i]);
  }
  for (int r = 0; r < d->n_views; ++r) {
    const ts_strided& o = io->out[r];
    if (!o.ptr || !aligned(o.ptr, 8) || o.st % 4 || o.sh % 4 || o.sb % 4)
      return fail(TS_ERR_VALUE, "scan views: output %d missing or not 8-byte aligned", r);
    if (d->mass && !io->out_ext[r].ptr) return fail(TS_ERR_VALUE, "scan views: missing key mass output %d", r);
  }
  if (P.ws_bytes > 0 && (!workspace || ws_bytes < P.ws_bytes))
    return fail(TS_ERR_VALUE, "scan views: workspace too small (%zu < %zu bytes)", ws_bytes, P.ws_bytes);

  ts::ViewsP vp;
  memset(&vp, 0, sizeof(vp));
  ts::ScanP& p = vp.s;
  p.B = d->B; p.H = d->H; p.T = d->T; p.dk = d->dk; p.dv = d->dv; p.dvp = 64; p.vs = 64;
  p.nchunks = P.nchunks; p.seg_chunks = P.seg_chunks; p.nseg = P.nseg; p.nsum = P.nsum; p.nelem = P.nelem;
  p.q = io->q; p.k = io->k; p.v = io->v;
  if ((rc = span_bytes("q", p.q, d->T, d->dk, 2, &p.q_rec))) return rc;
  if ((rc = span_bytes("k", p.k, d->T, d->dk, 2, &p.k_rec))) return rc;
  if ((rc = span_bytes("v", p.v, d->T, d->dv, 2, &p.v_rec))) return rc;
  vp.nv = d->n_views;
  vp.mass = d->mass ? 1 : 0;
  for (int r = 0; r < d->n_views; ++r) {
    vp.log_alpha[r] = io->log_alpha[r];
    vp.out[r] = io->out[r];
    if ((rc = span_bytes("out", vp.out[r], d->T, d->dv, 2, &vp.out_rec[r]))) return rc;
    if (d->mass) {
      vp.oe[r] = io->out_ext[r];
      if ((rc = span_bytes("out_ext", vp.oe[r], d->T, 1, 4, &vp.oe_rec[r]))) return rc;
    }
  }
  vp.seg_vstride = P.seg_vstride;
  vp.dec_vstride = P.dec_vstride;
  if (P.ws_bytes > 0) {
    p.seg = (float*)workspace;
    p.segdec = p.seg + (size_t)d->n_views * P.seg_vstride;
  }

  const int bh = d->B * d->H;
  const bool dk128 = P.DK == 128;
  ViewsFn fsum = dk128 ? pick_views_dk<128>(d->n_views, false) : pick_views_dk<64>(d->n_views, false);
  ViewsFn fmain = dk128 ? pick_views_dk<128>(d->n_views, true) : pick_views_dk<64>(d->n_views, true);
  const size_t lds_sum = (size_t)ts::views_layout(P.DK, d->n_views, false).bytes;
  const size_t lds_main = (size_t)ts::views_layout(P.DK, d->n_views, true).bytes;
  if (P.nsum > 0) {
    if ((rc = views_launch(fsum, dim3(P.nsum, bh), lds_sum, stream, vp))) return rc;
    hipLaunchKernelGGL(ts::views_prefix_kernel, dim3((P.nelem + 255) / 256, bh, d->n_views), dim3(256), 0, stream,
                       p.seg, p.segdec, P.nseg, P.nsum, P.nelem, P.seg_vstride, P.dec_vstride);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan views: prefix launch failed: %s", hipGetErrorString(e));
  }
  return views_launch(fmain, dim3(P.nseg, bh), lds_main, stream, vp);
}

}  // extern "C"
