// Fused write-side feature map for gfx950 (forward and backward).
//
// A workgroup (4 waves) walks `groups` consecutive 64-token groups of one
// (batch, head).  Each group's input rows are fetched with coalesced 16-byte
// loads into registers one group ahead of their use, stored to LDS, and
// consumed from there; outputs are assembled as LDS rows and written back
// with 16-byte stores.  Wave w computes tokens 16w..16w+15 of a group.
//
// The tile is computed transposed, a^T = W1 xn^T, so the MFMA accumulator
// holds, per lane, one token and four consecutive features of every
// 16-feature block.  Per-token reductions (RMSNorm, feature mass, softmax
// max/sum, L2-norm dot products) are then lane-local sums plus two cross-lane
// steps, feature-RoPE pairs are lane-local, and the accumulator feeds the next
// MFMA (W2 h^T, W1^T da^T) directly as an operand with the contraction index
// permuted consistently in both operands.
//
// The backward also contracts each group's da^T xn and dresid^T h over its
// 64 tokens (MFMA on token-major LDS rows read transposed) into per-workgroup
// partial weight gradients, so dW1 and dW2 never need per-token tiles in HBM.
//
// Reference chain replaced: block.py:595-618 (input RoPE, L2 norm),
// engine.py:117-158 (_block_forward: W1, RMSNorm, threshold, feature map,
// W2), kernel_features.py:73-135 (softmax partition / ReLU^2 ridge),
// engine.py:74-86 (feature RoPE) and the base term of engine.py:522-528.

#include "ts_common.h"
#include "ts_tokens.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct FeatP {
  int B, H, T, m, in_rot, feat_rot, has_tau, kind, groups;
  float gain, s, eps, inv_m;
  Str x, phi, resid, dphi, dresid, dx, da, xn, h, dtau;
  const void* w1;
  const void* w2;
  const void* w1t;
  const void* w2t;
  const float* tau;
  const float* in_cos;
  const float* in_sin;
  const float* f_cos;
  const float* f_sin;
  float* dw1_part;   // [parts, H, m, D] (fused weight gradients)
  float* dw2_part;   // [parts, H, D, m]
  float* dtau_part;  // [parts, H]
  // segment summaries of the plain-sum scan whose keys are this call's
  // features and whose values are v (summary mode of the forward): the
  // workspace layout of that scan, one workgroup per segment
  Str v;
  float* seg;        // [B*H][nseg][nelem]: S [m][dvp], u [dvp], D [m]
  float* segdec;     // [B*H][nseg]
  int nseg, nsum, nelem, dvp, v_ones;
};

// One token row of x from LDS in the accumulator layout (dims 16db+4g+i):
// input RoPE (rotate_in(v, db) rotates block db), L2 norm.  Keeps the
// rotated x in xr, writes xn over the row, returns 1 / max(||x_rot||, eps)
// and sets `big` when ||x_rot|| > eps.
template <typename E, int D, typename RotIn>
__device__ __forceinline__ float load_xn(const FeatP& p, const RotIn& rotate_in, int g, E* xrow, float (*xr)[4],
                                         bool& big) {
#pragma unroll
  for (int db = 0; db < D / 16; ++db) ld4f<E>(xrow + db * 16 + 4 * g, xr[db]);
  float ss = 0.f;
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    if (db * 16 < p.in_rot) rotate_in(xr[db], db);  // uniform per block
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += xr[db][i] * xr[db][i];
  }
  const float nrm = sqrtf(sum_g(ss));
  big = nrm > p.eps;
  const float inv = rcp(fmaxf(nrm, p.eps));
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    float o[4] = {xr[db][0] * inv, xr[db][1] * inv, xr[db][2] * inv, xr[db][3] * inv};
    st4f<E>(xrow + db * 16 + 4 * g, o);
  }
  return inv;
}

// RoPE factors of one token for a kernel that applies both rotations: the
// first four 16-wide blocks of one rotation are preloaded (the input rotation
// when there is one, else the feature rotation: one register set, not two);
// any other block reads its tables where it is applied.
struct TokRope {
  RopeRegs<4> pre;
  bool in_pre;  // uniform: the preloaded factors serve the input rotation

  __device__ __forceinline__ void fetch(const FeatP& p, int t, bool valid, int g) {
    in_pre = p.in_rot > 0;
    pre.fetch(in_pre ? p.in_rot : p.feat_rot, in_pre ? p.in_cos : p.f_cos, in_pre ? p.in_sin : p.f_sin, t, valid,
              g);
  }
  __device__ __forceinline__ void apply_in(const FeatP& p, float* v, int db, int t, bool valid, int g,
                                           bool inverse) const {
    if (db < 4 && in_pre)
      pre.apply(v, db, p.in_rot, g, inverse);
    else
      rope4(v, db * 16 + 4 * g, p.in_rot, p.in_cos, p.in_sin, t, valid && db * 16 + 4 * g < p.in_rot, inverse);
  }
  __device__ __forceinline__ void apply_feat(const FeatP& p, float* v, int fb, int t, bool valid, int g,
                                             bool inverse) const {
    if (fb < 4 && !in_pre)
      pre.apply(v, fb, p.feat_rot, g, inverse);
    else
      rope4(v, fb * 16 + 4 * g, p.feat_rot, p.f_cos, p.f_sin, t, valid && fb * 16 + 4 * g < p.feat_rot, inverse);
  }
};

// In-register feature map of a^T (lane = token).  Leaves h in `hv`; returns
// the statistics the backward needs.  KIND is the ts_feature_kind (a
// compile-time constant, so neither map carries the other's code).
template <int KIND, int MB>
__device__ __forceinline__ void feature_map(const FeatP& p, float tau, const floatx4* a, int nfb, floatx4* hv,
                                            float& rinv, float& mass) {
  float ss = 0.f;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb)
    if (fb < nfb)
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += a[fb][i] * a[fb][i];
  rinv = rsqrtf(sum_g(ss) * p.inv_m + p.eps);
  if constexpr (KIND == TS_FEAT_RELU2) {
    float sf = 0.f;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float r = __builtin_amdgcn_fmed3f(fmaf(a[fb][i], rinv, -tau), 0.f, __FLT_MAX__);  // relu
        const float f = fb < nfb ? r * r : 0.f;
        hv[fb][i] = f;
        sf += f;
      }
    mass = sum_g(sf);
    const bool ok = mass > p.eps;
    const float inv = ok ? rcp(mass) : 0.f;
    const float uni = ok ? 0.f : p.inv_m;  // the uniform fallback below eps
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) hv[fb][i] = fmaf(hv[fb][i], inv, uni);
  } else {
    float m_ = -INFINITY;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
      if (fb < nfb)
#pragma unroll
        for (int i = 0; i < 4; ++i) m_ = fmaxf(m_, p.gain * (a[fb][i] * rinv - tau));
    const float mx = max_g(m_);
    float se = 0.f;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = fb < nfb ? __expf(p.gain * (a[fb][i] * rinv - tau) - mx) : 0.f;
        hv[fb][i] = e;
        se += e;
      }
    mass = sum_g(se);
    const float inv = rcp(mass);
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) hv[fb][i] *= inv;
  }
}

// LDS carve-up shared by the kernels and the host (element offsets of each
// tile; pitches are the tile width plus one 16-byte vector).
struct FeatLayout {
  int xp, mp;                    // row pitches of d-wide and m-wide tiles
  int xs, ps, rs, hs;            // tiles: x/xn(/resid), phi | dphi then da, dresid, h
  int w1, w1t, w2;               // weights: W1 [m][xp], W1^T [d][mp], W2 [d][mp] or W2^T [m][xp]
  int end;                       // total elements
};

__host__ __device__ constexpr FeatLayout feat_layout(int esize, int d, int m, bool fwd, bool resid, bool wgrad,
                                                     bool w_lds) {
  const int vec = 16 / esize;
  FeatLayout L{};
  L.xp = d + vec;
  L.mp = m + vec;
  int off = 0;
  L.xs = off; off += TT * L.xp;
  L.ps = off; off += TT * L.mp;
  L.rs = L.hs = -1;
  if (!fwd && resid) { L.rs = off; off += TT * L.xp; }
  if (!fwd && resid && wgrad) { L.hs = off; off += TT * L.mp; }
  L.w1 = L.w1t = L.w2 = -1;
  if (w_lds) {
    L.w1 = off; off += m * L.xp;
    if (fwd) {
      if (resid) { L.w2 = off; off += d * L.mp; }
    } else {
      // W1^T: transposing reads of the staged W1 where the feature blocks
      // pair up into 32-wide MFMA steps (m a multiple of 32), else a copy
      if ((m / 16) % 2) { L.w1t = off; off += d * L.mp; }
      if (resid) { L.w2 = off; off += m * L.xp; }
    }
  }
  L.end = off;
  return L;
}

constexpr int kLdsMax = 160 * 1024;

// Weights are staged in LDS exactly when the largest layout a kernel
// instantiation serves (full width MB*16, with W2) fits.
template <typename E, int D, int MB, bool FWD, bool WG>
constexpr bool weights_in_lds() {
  return feat_layout((int)sizeof(E), D, MB * 16, FWD, true, WG, true).end * (int)sizeof(E) + 64 <= kLdsMax;
}

// SUMM (bf16, D = 64, m = 64, no resid): the workgroup's groups are one
// segment of the scan that reads these features as keys and v as values; the
// workgroup also folds the segment's writes into the scan's summary
// S = sum_t phi_t v_t^T (and D = sum_t phi_t with the scan's ones column)
// with the scan summary pass's own MFMA sequence (same operands, same
// order), so the scan can skip that pass and read no features twice.
template <typename E, int D, int MB, int KIND, bool SUMM = false>
__global__ __launch_bounds__(256) void feature_fwd_kernel(FeatP p) {
  constexpr bool WL = weights_in_lds<E, D, MB, true, false>();
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  constexpr int nfb = MB;
  const int m = MB * 16;
  const bool want_resid = p.resid.ptr != nullptr;
  const FeatLayout L = feat_layout((int)sizeof(E), D, m, true, want_resid, false, WL);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  E* ps = base + L.ps;
  const E* w1 = (const E*)p.w1 + h * m * D;
  const E* w2 = (const E*)p.w2 + h * D * m;
  int wp1 = D, wp2 = m;
  if constexpr (WL) {
    stage_matrix<E>(w1, m, D, base + L.w1, L.xp, tid);
    if (want_resid) stage_matrix<E>(w2, D, m, base + L.w2, L.mp, tid);
    w1 = base + L.w1;
    w2 = base + L.w2;
    wp1 = L.xp;
    wp2 = L.mp;
  }
  const float tau = p.has_tau ? p.tau[h] : 0.f;
  const Rows<E> xsrc = rows_of<E>(p.x, b, h);

  // Each wave loads, computes and writes back its own 16 rows of every
  // group, so the group loop needs no workgroup barrier (only the weights'
  // staging does, once; the summary mode adds two per group).  The rows of
  // the next group are in flight while a group is computed.
  const int g0 = blockIdx.x * p.groups;
  // groups this workgroup owns (>= 1: the grid covers the tiles exactly)
  const int ng = min(p.groups, (p.T + TT - 1) / TT - g0);
  // rows of group g0 + gi, or (gi past the last group) the last group's own
  // rows again: cached, never stored
  auto fetch_group = [&](auto& rows, const Rows<E>& src, int gi) {
    const int gl = min(gi, ng - 1);
    rows.fetch_all(src, (g0 + gi) * TT, gi < ng ? p.T : min(p.T, (g0 + gl) * TT + TT));
  };
  WaveRows<E, D> ldx;
  ldx.init(D, w, lane);
  fetch_group(ldx, xsrc, 0);
  // summary mode: the value rows, this wave's value block of S and D
  constexpr int VP = 64 + 16 / (int)sizeof(E);  // pitch of the value tile
  E* vs = base + L.end;
  const bool summ = SUMM && (int)blockIdx.x < p.nsum;  // uniform
  WaveRows<E, 64> ldv;
  floatx4 S[MB], Dv = {0.f, 0.f, 0.f, 0.f};
  Rows<E> vsrc{};
  if constexpr (SUMM) {
#pragma unroll
    for (int kb = 0; kb < MB; ++kb) S[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
    vsrc = rows_of<E>(p.v, b, h);
    ldv.init(64, w, lane);
    if (summ) fetch_group(ldv, vsrc, 0);
  }
  __syncthreads();  // weights staged
  for (int grp = 0; grp < ng; ++grp) {
    const int t0 = (g0 + grp) * TT;
    wave_lds_sync();  // the previous group's rows written out
    ldx.store_valid(xs, L.xp, t0, p.T);
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    // input-RoPE factors ahead of the prefetch (needed first); the feature
    // rotation, applied after the map, reads its tables there (registers for
    // both would cost this kernel a resident wave per SIMD)
    RopeRegs<D / 16> ir;
    ir.fetch(p.in_rot, p.in_cos, p.in_sin, t, valid, g);
    fetch_group(ldx, xsrc, grp + 1);
    wave_lds_sync();

    E* xrow = xs + row * L.xp;
    float xr[D / 16][4];
    bool big;
    const float inv =
        load_xn<E, D>(p, [&](float* v, int db) { ir.apply(v, db, p.in_rot, g, false); }, g, xrow, xr, big);
    wave_lds_sync();  // this wave's xn rows complete before they feed its MFMAs

    floatx4 a[MB], hv[MB];
    gemm_a<E, D, MB>(w1, wp1, xs + w * 16 * L.xp, L.xp, l16, g, nfb, a);
    float rinv, mass;
    feature_map<KIND, MB>(p, tau, a, nfb, hv, rinv, mass);
    {
      E* prow = ps + row * L.mp;
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        if (fb < nfb) {
          float v[4] = {hv[fb][0], hv[fb][1], hv[fb][2], hv[fb][3]};
          if (fb * 16 < p.feat_rot)
            rope4(v, fb * 16 + 4 * g, p.feat_rot, p.f_cos, p.f_sin, t, valid && fb * 16 + 4 * g < p.feat_rot,
                  false);
          st4f<E>(prow + fb * 16 + 4 * g, v);
        }
      }
    }
    if (want_resid) {
      floatx4 base_[D / 16];
      gemm_back<E, D, MB>(w2, wp2, hv, l16, g, nfb, base_);
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = xr[db][i] * inv + p.s * base_[db][i];
        st4f<E>(xrow + db * 16 + 4 * g, v);  // resid over this lane's own xn entries
      }
    }
    wave_lds_sync();
    write_rows_wave<E>(ps, L.mp, rows_of<E>(p.phi, b, h), t0, p.T, m, w, lane);
    if (want_resid) write_rows_wave<E>(xs, L.xp, rows_of<E>(p.resid, b, h), t0, p.T, D, w, lane);
    if constexpr (SUMM) {
      if (summ) {
        ldv.store_valid(vs, VP, t0, p.T);  // rows past T are zero
        if (grp + 1 < ng) fetch_group(ldv, vsrc, grp + 1);
        __syncthreads();  // every wave's feature and value rows
        // S[key block kb][value block w] += phi^T v over the tile's 64 tokens
        typedef TokFrag<E> TK;
        const auto av0 = TK::get(vs, VP, w * 16, 0, lane);
        const auto av1 = TK::get(vs, VP, w * 16, 1, lane);
#pragma unroll
        for (int kb = 0; kb < MB; ++kb) {
          S[kb] = mma32(TK::get(ps, L.mp, kb * 16, 0, lane), av0, S[kb]);
          S[kb] = mma32(TK::get(ps, L.mp, kb * 16, 1, lane), av1, S[kb]);
        }
        if (p.v_ones) {
          // D over key block w: a broadcast row of the ones column (zero past T)
#pragma unroll
          for (int kp = 0; kp < 2; ++kp) {
            bf16x8 one;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int key = 32 * kp + (e < 4 ? 4 * g + e : 12 + 4 * g + e);
              one[e] = cvt<E>(t0 + key < p.T ? 1.0f : 0.0f);
            }
            Dv = mma32(one, TK::get(ps, L.mp, w * 16, kp, lane), Dv);
          }
        }
        __syncthreads();  // the tiles are read before the next group's rows replace them
      }
    }
  }
  if constexpr (SUMM) {
    if (summ) {
      // the scan summary pass's store: S [key][value] (pitch dvp), u = 0, D, and
      // the segment's log-decay 0 (plain sum)
      const int bh = b * p.H + h;
      float* dst = p.seg + ((size_t)bh * p.nseg + blockIdx.x) * (size_t)p.nelem;
#pragma unroll
      for (int kb = 0; kb < MB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[(kb * 16 + 4 * g + i) * p.dvp + w * 16 + l16] = S[kb][i];
      if (g == 0) {
        dst[m * p.dvp + w * 16 + l16] = 0.0f;
        dst[m * p.dvp + p.dvp + w * 16 + l16] = Dv[0];
      }
      if (tid == 0) p.segdec[(size_t)bh * p.nseg + blockIdx.x] = 0.0f;
    }
  }
}

// Weight-gradient blocks per wave of the fused backward: wave w owns the
// feature blocks fb = w, w + 4, ... of dW1 (and of dW2), each across all D/16
// head-dim blocks.
template <int D, int MB>
constexpr int wgrad_blocks() { return ((MB + 3) / 4) * (D / 16); }

// Resident waves per SIMD for the common bf16 widths: three for the ReLU^2
// key side (168 registers; its tiles take 46 KB of LDS), two with the
// residual stream or the softmax map.
template <typename E, int D, int MB, bool WG, bool RESID, int KIND>
__global__ __launch_bounds__(256, (sizeof(E) == 2 && D <= 64 && MB <= 4 ? (RESID || KIND != TS_FEAT_RELU2 ? 2 : 3) : 1))
    void feature_bwd_kernel(FeatP p) {
  typedef LdsIO<E> IO;
  typedef TokFrag<E> TF;
  constexpr bool WL = weights_in_lds<E, D, MB, false, WG>();
  constexpr int NB = WG ? wgrad_blocks<D, MB>() : 1;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  constexpr int nfb = MB;
  const int m = MB * 16;
  constexpr bool has_resid = RESID;
  const FeatLayout L = feat_layout((int)sizeof(E), D, m, false, has_resid, WG, WL);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;  // x, then xn
  E* ps = base + L.ps;  // dphi, then da
  E* rs = base + L.rs;  // dresid
  E* hs = base + L.hs;  // h
  float* red = (float*)(base + L.end);  // [4] wave partial sums
  // W1^T operands: transposing reads of the staged W1 (pairs of feature blocks)
  constexpr bool W1T_READ = WL && MB % 2 == 0;

  const E* w1 = (const E*)p.w1 + h * m * D;
  const E* w1t = (const E*)p.w1t + h * D * m;
  const E* w2t = (const E*)p.w2t + h * m * D;
  int wpa = D, wpt = m;
  if constexpr (WL) {
    stage_matrix<E>(w1, m, D, base + L.w1, L.xp, tid);
    if constexpr (!W1T_READ) {
      if (p.w1t) stage_matrix<E>(w1t, D, m, base + L.w1t, L.mp, tid);
      else stage_transposed<E>(w1, m, D, base + L.w1t, L.mp, tid);
    }
    if (has_resid) {
      if (p.w2t) stage_matrix<E>(w2t, m, D, base + L.w2, L.xp, tid);
      else stage_transposed<E>((const E*)p.w2 + h * D * m, D, m, base + L.w2, L.xp, tid);
    }
    w1 = base + L.w1;
    w1t = base + L.w1t;
    w2t = base + L.w2;
    wpa = L.xp;
    wpt = L.mp;
  }
  const float tau = p.has_tau ? p.tau[h] : 0.f;
  const Rows<E> xsrc = rows_of<E>(p.x, b, h);
  const Rows<E> psrc = rows_of<E>(p.dphi, b, h);
  const Rows<E> rsrc = rows_of<E>(p.dresid, b, h);

  floatx4 acc1[NB], acc2[NB];
#pragma unroll
  for (int k = 0; k < NB; ++k) acc1[k] = acc2[k] = floatx4{0.f, 0.f, 0.f, 0.f};
  float dtau_acc = 0.f;

  // Each wave loads its own 16 rows of every group (no barrier between the
  // rows' store and their first use); the weight-gradient contraction reads
  // all 64 rows, so the group still starts and ends on a workgroup barrier.
  WaveRows<E, D> ldx, ldr;
  WaveRows<E, MB * 16> ldp;
  ldx.init(D, w, lane);
  ldr.init(has_resid ? D : 0, w, lane);
  ldp.init(m, w, lane);
  const int g0 = blockIdx.x * p.groups;
  ldx.fetch_all(xsrc, g0 * TT, p.T);
  ldp.fetch_all(psrc, g0 * TT, p.T);
  if (has_resid) ldr.fetch_all(rsrc, g0 * TT, p.T);

  const int ng = min(p.groups, (p.T + TT - 1) / TT - g0);
  for (int grp = 0; grp < ng; ++grp) {
    const int t0 = (g0 + grp) * TT;
    __syncthreads();       // weights staged; previous group fully consumed
    ldx.store_valid(xs, L.xp, t0, p.T);
    ldp.store_valid(ps, L.mp, t0, p.T);
    if (has_resid) ldr.store_valid(rs, L.xp, t0, p.T);
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    TokRope rope;
    rope.fetch(p, t, valid, g);
    // next group's rows (after the last group, this group's own rows again:
    // cached, never stored)
    const int tmax = grp + 1 < ng ? p.T : min(p.T, t0 + TT);
    ldx.fetch_all(xsrc, t0 + TT, tmax);
    ldp.fetch_all(psrc, t0 + TT, tmax);
    if (has_resid) ldr.fetch_all(rsrc, t0 + TT, tmax);
    wave_lds_sync();

    E* xrow = xs + row * L.xp;
    float xr[D / 16][4];
    bool big;
    const float inv = load_xn<E, D>(
        p, [&](float* v, int db) { rope.apply_in(p, v, db, t, valid, g, false); }, g, xrow, xr, big);
    wave_lds_sync();  // this wave's xn rows complete before they feed its MFMAs

    floatx4 a[MB];
    gemm_a<E, D, MB>(w1, wpa, xs + w * 16 * L.xp, L.xp, l16, g, nfb, a);
    float ssa = 0.f;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) ssa += a[fb][i] * a[fb][i];
    const float rinv = rsqrtf(sum_g(ssa) * p.inv_m + p.eps);

    // dh = rotate^T(dphi) (+ s W2^T dresid); rows past T are zero in LDS
    floatx4 dh[MB];
    const E* rrow = rs + row * L.xp;
    if constexpr (has_resid) {
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        dh[fb] = floatx4{0.f, 0.f, 0.f, 0.f};
        const E* wrow = w2t + (fb * 16 + l16) * wpa;
#pragma unroll
        for (int kk = 0; kk < D / 32; ++kk)
          dh[fb] = mma32(IO::ld8(wrow + kk * 32 + 8 * g), IO::ld8(rrow + kk * 32 + 8 * g), dh[fb]);
        if (D % 32)
          dh[fb] = mma16(IO::ld4(wrow + (D / 32) * 32 + 4 * g), IO::ld4(rrow + (D / 32) * 32 + 4 * g), dh[fb]);
      }
    }
    {
      const E* prow = ps + row * L.mp;
      float v[MB][4];
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) ld4f<E>(prow + fb * 16 + 4 * g, v[fb]);
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        if (fb * 16 < p.feat_rot) rope.apply_feat(p, v[fb], fb, t, valid, g, true);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (has_resid) dh[fb][i] = fmaf(p.s, dh[fb][i], v[fb][i]);
          else dh[fb][i] = v[fb][i];
        }
      }
    }

    // The pre-activation gradient is dscale * dp (dp left in dh), with
    // sdp = sum_i dp_i and sda = sum_i dp_i a_i; hv holds h where it is written.
    // relu2: h = f / sum f, f = r^2, r = relu(pre) (the uniform 1/m below eps
    //   has no gradient): dpre_i = (2/mass) r_i (dh_i - sum_j dh_j h_j), so
    //   with u = dh r, dp = u - (sum_j u_j r_j / mass) r and dscale = 2/mass.
    // softmax: h = softmax(gain pre): dp = h (dh - sum_j dh_j h_j), dscale = gain.
    constexpr bool need_h = !WG || has_resid;
    floatx4 hv[MB];
    float dscale, sdp = 0.f, sda = 0.f;
    if constexpr (KIND == TS_FEAT_RELU2) {
      floatx4 r[MB];
      float sf = 0.f;
#pragma unroll
      for (int fb = 0; fb < MB; ++fb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          r[fb][i] = __builtin_amdgcn_fmed3f(fmaf(a[fb][i], rinv, -tau), 0.f, __FLT_MAX__);
          sf = fmaf(r[fb][i], r[fb][i], sf);
        }
      const float mass = sum_g(sf);
      const bool ok = mass > p.eps;
      const float inv_mass = ok ? rcp(mass) : 0.f;
      float su = 0.f;
#pragma unroll
      for (int fb = 0; fb < MB; ++fb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dh[fb][i] *= r[fb][i];
          su = fmaf(dh[fb][i], r[fb][i], su);
        }
      const float sdh = sum_g(su) * inv_mass;
#pragma unroll
      for (int fb = 0; fb < MB; ++fb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dh[fb][i] = fmaf(-sdh, r[fb][i], dh[fb][i]);
          sdp += dh[fb][i];
          sda = fmaf(dh[fb][i], a[fb][i], sda);
        }
      dscale = 2.f * inv_mass;
      if constexpr (need_h) {
        const float uni = ok ? 0.f : p.inv_m;
#pragma unroll
        for (int fb = 0; fb < MB; ++fb)
#pragma unroll
          for (int i = 0; i < 4; ++i) hv[fb][i] = fmaf(r[fb][i] * r[fb][i], inv_mass, uni);
      }
    } else {
      float rinv_, mass;
      feature_map<KIND, MB>(p, tau, a, nfb, hv, rinv_, mass);
      float sdh = 0.f;
#pragma unroll
      for (int fb = 0; fb < MB; ++fb)
#pragma unroll
        for (int i = 0; i < 4; ++i) sdh = fmaf(dh[fb][i], hv[fb][i], sdh);
      sdh = sum_g(sdh);
#pragma unroll
      for (int fb = 0; fb < MB; ++fb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dh[fb][i] = hv[fb][i] * (dh[fb][i] - sdh);
          sdp += dh[fb][i];
          sda = fmaf(dh[fb][i], a[fb][i], sda);
        }
      dscale = p.gain;
    }
    sdp = sum_g(sdp) * dscale;
    sda = sum_g(sda) * dscale;
    if (g == 0 && valid) {
      if (WG) dtau_acc -= sdp;
      else if (p.dtau.ptr) *rows_of<float>(p.dtau, b, h).at(t) = -sdp;
    }
    // RMSNorm backward: da = rinv dpre - rinv^3 (sum_j dpre_j a_j / m) a
    const float c1 = rinv * dscale, c3 = rinv * rinv * rinv * sda * p.inv_m;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) dh[fb][i] = c1 * dh[fb][i] - c3 * a[fb][i];


    if constexpr (WG) {
      // da over this lane's dphi entries; h for the dW2 contraction
      E* prow = ps + row * L.mp;
      E* hrow = hs + row * L.mp;
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        float v[4] = {dh[fb][0], dh[fb][1], dh[fb][2], dh[fb][3]};
        st4f<E>(prow + fb * 16 + 4 * g, v);
        if constexpr (has_resid) {
          float u[4] = {hv[fb][0], hv[fb][1], hv[fb][2], hv[fb][3]};
          st4f<E>(hrow + fb * 16 + 4 * g, u);
        }
      }
    } else if (valid) {
      E* da_out = p.da.ptr ? rows_of<E>(p.da, b, h).at(t) : nullptr;
      E* h_out = p.h.ptr ? rows_of<E>(p.h, b, h).at(t) : nullptr;
      E* xn_out = p.xn.ptr ? rows_of<E>(p.xn, b, h).at(t) : nullptr;
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        float v[4] = {dh[fb][0], dh[fb][1], dh[fb][2], dh[fb][3]};
        if (da_out) st4f<E>(da_out + fb * 16 + 4 * g, v);
        float u[4] = {hv[fb][0], hv[fb][1], hv[fb][2], hv[fb][3]};
        if (h_out) st4f<E>(h_out + fb * 16 + 4 * g, u);
      }
      if (xn_out) {
#pragma unroll
        for (int db = 0; db < D / 16; ++db) {
          float v[4];
          ld4f<E>(xrow + db * 16 + 4 * g, v);
          st4f<E>(xn_out + db * 16 + 4 * g, v);
        }
      }
    }

    // dxn^T = W1^T da^T  (W1^T as transposing reads of the staged W1, or given as [D x m])
    floatx4 dxn[D / 16];
    if constexpr (W1T_READ) {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        dxn[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < MB / 2; ++j)
          dxn[db] = mma32(TF::get(w1, wpa, db * 16, j, lane), IO::from_acc(dh[2 * j], dh[2 * j + 1]), dxn[db]);
      }
    } else {
      gemm_back<E, D, MB>(w1t, wpt, dh, l16, g, nfb, dxn);
    }
    // residual path, L2-norm backward (x / max(||x||, eps): the projection
    // term only where ||x|| > eps), input-RoPE backward at dims 16db+4g+i
    float dot = 0.f;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      if (has_resid) {
        float r[4];
        ld4f<E>(rrow + db * 16 + 4 * g, r);
#pragma unroll
        for (int i = 0; i < 4; ++i) dxn[db][i] += r[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) dot += dxn[db][i] * xr[db][i];
    }
    dot = sum_g(dot);  // every lane takes part in the cross-lane sum
    dot = big ? dot * inv * inv : 0.f;
    {
      // dx straight from registers: four consecutive dims per lane
      E* dxrow = valid ? rows_of<E>(p.dx, b, h).at(t) : nullptr;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (dxn[db][i] - xr[db][i] * dot) * inv;
        if (db * 16 < p.in_rot) rope.apply_in(p, v, db, t, valid, g, true);
        if (valid) st4f<E>(dxrow + db * 16 + 4 * g, v);
      }
    }
    __syncthreads();  // da, h, xn rows of all four waves complete (the contraction reads them all)

    if constexpr (WG) {
      // dW1[f][e] += sum_t da[t][f] xn[t][e];  dW2[e][f] += sum_t dresid[t][e] h[t][f]
#pragma unroll
      for (int j = 0; j < (MB + 3) / 4; ++j) {
        const int fb = w + 4 * j;
        if (fb < nfb) {
#pragma unroll
          for (int kp = 0; kp < 2; ++kp) {
            const auto fa = TF::get(ps, L.mp, fb * 16, kp, lane);
            const auto fh = has_resid ? TF::get(hs, L.mp, fb * 16, kp, lane) : fa;
#pragma unroll
            for (int db = 0; db < D / 16; ++db) {
              const int k = j * (D / 16) + db;
              acc1[k] = mma32(fa, TF::get(xs, L.xp, db * 16, kp, lane), acc1[k]);
              if (has_resid) acc2[k] = mma32(TF::get(rs, L.xp, db * 16, kp, lane), fh, acc2[k]);
            }
          }
        }
      }
    }
  }  // token groups

  if constexpr (WG) {
    const int part = b * gridDim.x + blockIdx.x;
    float* d1 = p.dw1_part + ((size_t)part * p.H + h) * (size_t)m * D;
    float* d2 = p.dw2_part + ((size_t)part * p.H + h) * (size_t)D * m;
#pragma unroll
    for (int k = 0; k < NB; ++k) {
      const int fb = w + 4 * (k / (D / 16)), db = k % (D / 16);
      if (fb < nfb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          d1[(fb * 16 + 4 * g + i) * D + db * 16 + l16] = acc1[k][i];
          if (has_resid) d2[(db * 16 + 4 * g + i) * m + fb * 16 + l16] = p.s * acc2[k][i];
        }
      }
    }
    if (p.dtau_part) {
      float v = dtau_acc;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
      if (lane == 0) red[w] = v;
      __syncthreads();
      if (tid == 0) p.dtau_part[(size_t)part * p.H + h] = red[0] + red[1] + red[2] + red[3];
    }
  }
}


// ------------------------------------------------------------------ wide maps
//
// Feature widths of 192 and 384 (bf16, head widths 32 and 64): the per-lane
// feature arrays of the kernels above would not fit in registers, so these
// walk the feature axis 64 features at a time, re-forming the chunk's
// a^T = W1 xn^T on MFMA in every pass that needs it (RMSNorm sum, mass or
// softmax max/sum, then h; in the backward dh . h, sum dp and dp . a, then
// da).  W1 (and W2) are staged in LDS once per workgroup; W1^T and W2^T
// operands are transposing LDS reads of the staged rows.  The backward
// writes da, xn, h and dtau per token for the weight-gradient GEMMs (no
// fused weight-gradient partials at these widths).

struct WideLayout {
  int xp, cp, mp;
  int xs, cs, rs, os, w1, w2;  // element offsets
  int end;
};

__host__ __device__ constexpr WideLayout wide_layout(int d, int m, bool fwd, bool resid) {
  WideLayout L{};
  L.xp = d + 8;
  L.cp = 64 + 8;
  L.mp = m + 8;
  int off = 0;
  L.xs = off; off += TT * L.xp;
  L.cs = L.rs = L.os = -1;
  if (fwd) {
    L.cs = off; off += TT * L.cp;
  } else {
    if (resid) { L.rs = off; off += TT * L.xp; }
    L.os = off; off += TT * L.xp;
  }
  L.w1 = off; off += m * L.xp;
  L.w2 = -1;
  if (resid) { L.w2 = off; off += d * L.mp; }
  L.end = off;
  return L;
}

// a^T of feature chunk c (blocks 4c..4c+3) for this wave's 16 tokens.
template <int D>
__device__ __forceinline__ void wide_a(const bf16* w1s, int xp, const bf16* xs_w, int c, int l16, int g, floatx4* a) {
  gemm_a<bf16, D, 4>(w1s + c * 64 * xp, xp, xs_w, xp, l16, g, 4, a);
}

// Per-token statistics over the whole width: rinv (RMSNorm) and the
// normalizer (ReLU^2 mass, or the softmax max mx and sum).
template <int D, int KIND, int NC>
__device__ __forceinline__ void wide_stats(const FeatP& p, float tau, const bf16* w1s, int xp, const bf16* xs_w,
                                           int l16, int g, float& rinv, float& mass, float& mx) {
  float ss = 0.f;
#pragma unroll 1
  for (int c = 0; c < NC; ++c) {
    floatx4 a[4];
    wide_a<D>(w1s, xp, xs_w, c, l16, g, a);
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += a[f][i] * a[f][i];
  }
  rinv = rsqrtf(sum_g(ss) * p.inv_m + p.eps);
  mx = 0.f;
  if constexpr (KIND == TS_FEAT_RELU2) {
    float sf = 0.f;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4];
      wide_a<D>(w1s, xp, xs_w, c, l16, g, a);
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pre = fmaxf(a[f][i] * rinv - tau, 0.f);
          sf += pre * pre;
        }
    }
    mass = sum_g(sf);
  } else {
    float m_ = -INFINITY;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4];
      wide_a<D>(w1s, xp, xs_w, c, l16, g, a);
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) m_ = fmaxf(m_, p.gain * (a[f][i] * rinv - tau));
    }
    mx = max_g(m_);
    float se = 0.f;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4];
      wide_a<D>(w1s, xp, xs_w, c, l16, g, a);
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) se += __expf(p.gain * (a[f][i] * rinv - tau) - mx);
    }
    mass = sum_g(se);
  }
}

// h of one chunk from its a and the statistics.
template <int KIND>
__device__ __forceinline__ void wide_h(const FeatP& p, float tau, const floatx4* a, float rinv, float mass, float mx,
                                       floatx4* hc) {
  if constexpr (KIND == TS_FEAT_RELU2) {
    const bool ok = mass > p.eps;
    const float inv = ok ? rcp(mass) : 0.f;
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pre = fmaxf(a[f][i] * rinv - tau, 0.f);
        hc[f][i] = ok ? pre * pre * inv : p.inv_m;
      }
  } else {
    const float inv = rcp(mass);
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) hc[f][i] = __expf(p.gain * (a[f][i] * rinv - tau) - mx) * inv;
  }
}

template <int D, int MB, int KIND>
__global__ __launch_bounds__(256) void feature_fwd_wide_kernel(FeatP p) {
  typedef bf16 E;
  typedef LdsIO<E> IO;
  constexpr int NC = MB / 4;
  constexpr int m = MB * 16;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const bool want_resid = p.resid.ptr != nullptr;
  const WideLayout L = wide_layout(D, m, true, want_resid);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  E* cs = base + L.cs;
  E* w1s = base + L.w1;
  E* w2s = base + L.w2;
  stage_matrix<E>((const E*)p.w1 + (size_t)h * m * D, m, D, w1s, L.xp, tid);
  if (want_resid) stage_matrix<E>((const E*)p.w2 + (size_t)h * D * m, D, m, w2s, L.mp, tid);
  const float tau = p.has_tau ? p.tau[h] : 0.f;
  const Rows<E> xsrc = rows_of<E>(p.x, b, h);
  const Rows<E> phi = rows_of<E>(p.phi, b, h);

  RowTile<E, D> ldx;
  ldx.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldx.fetch(xsrc, g0 * TT, p.T);
  const int ng = min(p.groups, (p.T + TT - 1) / TT - g0);
  for (int grp = 0; grp < ng; ++grp) {
    const int t0 = (g0 + grp) * TT;
    __syncthreads();  // weights staged; previous group's rows written out
    ldx.store(xs, L.xp);
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    RopeRegs<D / 16> ir;
    ir.fetch(p.in_rot, p.in_cos, p.in_sin, t, valid, g);
    ldx.fetch(xsrc, t0 + TT, grp + 1 < ng ? p.T : 0);
    __syncthreads();

    E* xrow = xs + row * L.xp;
    const E* xs_w = xs + w * 16 * L.xp;
    float xr[D / 16][4];
    bool big;
    const float inv =
        load_xn<E, D>(p, [&](float* v, int db) { ir.apply(v, db, p.in_rot, g, false); }, g, xrow, xr, big);
    wave_lds_sync();  // this wave's xn rows complete before they feed its MFMAs

    float rinv, mass, mx;
    wide_stats<D, KIND, NC>(p, tau, w1s, L.xp, xs_w, l16, g, rinv, mass, mx);
    floatx4 rb[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) rb[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], hc[4];
      wide_a<D>(w1s, L.xp, xs_w, c, l16, g, a);
      wide_h<KIND>(p, tau, a, rinv, mass, mx, hc);
      if (want_resid) {
#pragma unroll
        for (int db = 0; db < D / 16; ++db) {
          const E* wrow = w2s + (db * 16 + l16) * L.mp + c * 64;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
            rb[db] = mma32(IO::cat(IO::ld4(wrow + 32 * jj + 4 * g), IO::ld4(wrow + 32 * jj + 16 + 4 * g)),
                           IO::from_acc(hc[2 * jj], hc[2 * jj + 1]), rb[db]);
        }
      }
      E* crow = cs + row * L.cp;
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float v[4] = {hc[f][0], hc[f][1], hc[f][2], hc[f][3]};
        const int col = c * 64 + f * 16 + 4 * g;
        if (c * 64 + f * 16 < p.feat_rot)
          rope4(v, col, p.feat_rot, p.f_cos, p.f_sin, t, valid && col < p.feat_rot, false);
        st4f<E>(crow + f * 16 + 4 * g, v);
      }
      __syncthreads();
      write_rows<E>(cs, L.cp, Rows<E>{phi.base + c * 64, phi.st}, t0, p.T, 64, tid);
      __syncthreads();
    }
    if (want_resid) {
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = xr[db][i] * inv + p.s * rb[db][i];
        st4f<E>(xrow + db * 16 + 4 * g, v);
      }
      __syncthreads();
      write_rows<E>(xs, L.xp, rows_of<E>(p.resid, b, h), t0, p.T, D, tid);
    }
  }
}

template <int D, int MB, bool RESID, int KIND>
__global__ __launch_bounds__(256) void feature_bwd_wide_kernel(FeatP p) {
  typedef bf16 E;
  typedef LdsIO<E> IO;
  typedef TokFrag<E> TF;
  constexpr int NC = MB / 4;
  constexpr int m = MB * 16;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const WideLayout L = wide_layout(D, m, false, RESID);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  E* rs = base + L.rs;
  E* os = base + L.os;
  E* w1s = base + L.w1;
  E* w2s = base + L.w2;
  stage_matrix<E>((const E*)p.w1 + (size_t)h * m * D, m, D, w1s, L.xp, tid);
  if (RESID) stage_matrix<E>((const E*)p.w2 + (size_t)h * D * m, D, m, w2s, L.mp, tid);
  const float tau = p.has_tau ? p.tau[h] : 0.f;
  const Rows<E> xsrc = rows_of<E>(p.x, b, h);
  const Rows<E> rsrc = rows_of<E>(p.dresid, b, h);
  const Rows<E> psrc = rows_of<E>(p.dphi, b, h);

  RowTile<E, D> ldx, ldr;
  ldx.init(D, tid);
  ldr.init(RESID ? D : 0, tid);
  const int g0 = blockIdx.x * p.groups;
  ldx.fetch(xsrc, g0 * TT, p.T);
  if (RESID) ldr.fetch(rsrc, g0 * TT, p.T);
  const int ng = min(p.groups, (p.T + TT - 1) / TT - g0);
  for (int grp = 0; grp < ng; ++grp) {
    const int t0 = (g0 + grp) * TT;
    __syncthreads();  // weights staged; previous group fully consumed
    ldx.store(xs, L.xp);
    if (RESID) ldr.store(rs, L.xp);
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    RopeRegs<D / 16> ir;
    ir.fetch(p.in_rot, p.in_cos, p.in_sin, t, valid, g);
    const int next_T = grp + 1 < ng ? p.T : 0;
    ldx.fetch(xsrc, t0 + TT, next_T);
    if (RESID) ldr.fetch(rsrc, t0 + TT, next_T);
    __syncthreads();

    const E* prow = psrc.at(valid ? t : 0);
    E* xrow = xs + row * L.xp;
    const E* xs_w = xs + w * 16 * L.xp;
    float xr[D / 16][4];
    bool big;
    const float inv =
        load_xn<E, D>(p, [&](float* v, int db) { ir.apply(v, db, p.in_rot, g, false); }, g, xrow, xr, big);
    wave_lds_sync();  // this wave's xn rows complete before they feed its MFMAs

    float rinv, mass, mx;
    wide_stats<D, KIND, NC>(p, tau, w1s, L.xp, xs_w, l16, g, rinv, mass, mx);
    const E* rrow = rs + row * L.xp;
    // a, h and dh = rotate^T(dphi) + s W2^T dresid of chunk c
    auto chunk = [&](int c, floatx4* a, floatx4* hc, floatx4* dh) {
      uint2 dpr[4];
#pragma unroll
      for (int f = 0; f < 4; ++f)
        dpr[f] = valid ? *(const uint2*)(prow + c * 64 + f * 16 + 4 * g) : make_uint2(0u, 0u);
      wide_a<D>(w1s, L.xp, xs_w, c, l16, g, a);
      wide_h<KIND>(p, tau, a, rinv, mass, mx, hc);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        dh[f] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (RESID) {
#pragma unroll
          for (int kk = 0; kk < D / 32; ++kk)
            dh[f] = mma32(TF::get(w2s, L.mp, c * 64 + f * 16, kk, lane),
                          IO::cat(IO::ld4(rrow + 32 * kk + 4 * g), IO::ld4(rrow + 32 * kk + 16 + 4 * g)), dh[f]);
#pragma unroll
          for (int i = 0; i < 4; ++i) dh[f][i] *= p.s;
        }
        float v[4] = {__uint_as_float(dpr[f].x << 16), __uint_as_float(dpr[f].x & 0xffff0000u),
                      __uint_as_float(dpr[f].y << 16), __uint_as_float(dpr[f].y & 0xffff0000u)};
        const int col = c * 64 + f * 16 + 4 * g;
        if (c * 64 + f * 16 < p.feat_rot)
          rope4(v, col, p.feat_rot, p.f_cos, p.f_sin, t, valid && col < p.feat_rot, true);
#pragma unroll
        for (int i = 0; i < 4; ++i) dh[f][i] += v[i];
      }
    };
    // pass 1: sdh = dh . h
    float sdh = 0.f;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], hc[4], dh[4];
      chunk(c, a, hc, dh);
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) sdh += dh[f][i] * hc[f][i];
    }
    sdh = sum_g(sdh);
    const float scale = KIND == TS_FEAT_RELU2 ? (mass > p.eps ? 2.0f * rcp(mass) : 0.f) : p.gain;
    // dp of a chunk (left in dh)
    auto dp_of = [&](const floatx4* a, const floatx4* hc, floatx4* dh) {
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (KIND == TS_FEAT_RELU2)
            dh[f][i] = (dh[f][i] - sdh) * scale * fmaxf(a[f][i] * rinv - tau, 0.f);
          else
            dh[f][i] = scale * hc[f][i] * (dh[f][i] - sdh);
        }
    };
    // pass 2: sum dp, dp . a
    float sdp = 0.f, sda = 0.f;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], hc[4], dh[4];
      chunk(c, a, hc, dh);
      dp_of(a, hc, dh);
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sdp += dh[f][i];
          sda += dh[f][i] * a[f][i];
        }
    }
    sdp = sum_g(sdp);
    sda = sum_g(sda);
    if (g == 0 && valid && p.dtau.ptr) *rows_of<float>(p.dtau, b, h).at(t) = -sdp;
    const float c3 = rinv * rinv * rinv * sda * p.inv_m;
    // pass 3: da = rinv dp - c3 a per chunk -> dxn^T += W1^T da^T; da and h out
    floatx4 dxn[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) dxn[db] = floatx4{0.f, 0.f, 0.f, 0.f};
    E* da_out = valid && p.da.ptr ? rows_of<E>(p.da, b, h).at(t) : nullptr;
    E* h_out = valid && p.h.ptr ? rows_of<E>(p.h, b, h).at(t) : nullptr;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], hc[4], da[4];
      chunk(c, a, hc, da);
      dp_of(a, hc, da);
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int i = 0; i < 4; ++i) da[f][i] = rinv * da[f][i] - c3 * a[f][i];
#pragma unroll
      for (int db = 0; db < D / 16; ++db)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
          dxn[db] = mma32(TF::get(w1s + c * 64 * L.xp, L.xp, db * 16, jj, lane),
                          IO::from_acc(da[2 * jj], da[2 * jj + 1]), dxn[db]);
      if (da_out) {
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          float v[4] = {da[f][0], da[f][1], da[f][2], da[f][3]};
          st4f<E>(da_out + c * 64 + f * 16 + 4 * g, v);
        }
      }
      if (h_out) {
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          float u[4] = {hc[f][0], hc[f][1], hc[f][2], hc[f][3]};
          st4f<E>(h_out + c * 64 + f * 16 + 4 * g, u);
        }
      }
    }
    if (valid && p.xn.ptr) {
      E* xn_out = rows_of<E>(p.xn, b, h).at(t);
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        float v[4];
        ld4f<E>(xrow + db * 16 + 4 * g, v);
        st4f<E>(xn_out + db * 16 + 4 * g, v);
      }
    }
    // residual path, L2-norm backward (x / max(||x||, eps): the projection
    // term only where ||x|| > eps), input-RoPE backward at dims 16db+4g+i
    float dot = 0.f;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      if (RESID) {
        float r[4];
        ld4f<E>(rrow + db * 16 + 4 * g, r);
#pragma unroll
        for (int i = 0; i < 4; ++i) dxn[db][i] += r[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) dot += dxn[db][i] * xr[db][i];
    }
    dot = sum_g(dot);  // every lane takes part in the cross-lane sum
    dot = big ? dot * inv * inv : 0.f;
    {
      E* orow = os + row * L.xp;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (dxn[db][i] - xr[db][i] * dot) * inv;
        if (db * 16 < p.in_rot) ir.apply(v, db, p.in_rot, g, true);
        st4f<E>(orow + db * 16 + 4 * g, v);
      }
    }
    __syncthreads();  // dx rows of all four waves complete
    write_rows<E>(os, L.xp, rows_of<E>(p.dx, b, h), t0, p.T, D, tid);
  }
}

}  // namespace ts

// ============================================================== host side
namespace {

using ts::fail;

typedef void (*FeatFn)(ts::FeatP);

template <typename E, int D, int MB, int KIND>
FeatFn pick4(bool fwd, bool wgrad, bool resid) {
  if (fwd) return (FeatFn)ts::feature_fwd_kernel<E, D, MB, KIND>;
  if (wgrad) {
    if constexpr (ts::wgrad_blocks<D, MB>() <= 8)
      return resid ? (FeatFn)ts::feature_bwd_kernel<E, D, MB, true, true, KIND>
                   : (FeatFn)ts::feature_bwd_kernel<E, D, MB, true, false, KIND>;
    return nullptr;
  }
  return resid ? (FeatFn)ts::feature_bwd_kernel<E, D, MB, false, true, KIND>
               : (FeatFn)ts::feature_bwd_kernel<E, D, MB, false, false, KIND>;
}

template <typename E, int D, int MB>
FeatFn pick3(int kind, bool fwd, bool wgrad, bool resid) {
  return kind == TS_FEAT_RELU2 ? pick4<E, D, MB, TS_FEAT_RELU2>(fwd, wgrad, resid)
                               : pick4<E, D, MB, TS_FEAT_SOFTMAX>(fwd, wgrad, resid);
}

// Kernels exist for head widths d in {16, 32, 64, 128} and feature widths
// m in {16, 32, 64, 128, 256} (the feature-block count is a compile-time
// constant, so no per-block predicates remain in the kernels).
template <typename E, int D>
FeatFn pick_mb(int m, int kind, bool fwd, bool wgrad, bool resid) {
  switch (m) {
    case 16: return pick3<E, D, 1>(kind, fwd, wgrad, resid);
    case 32: return pick3<E, D, 2>(kind, fwd, wgrad, resid);
    case 64: return pick3<E, D, 4>(kind, fwd, wgrad, resid);
    case 128: return pick3<E, D, 8>(kind, fwd, wgrad, resid);
    case 256: return pick3<E, D, 16>(kind, fwd, wgrad, resid);
  }
  return nullptr;
}

template <typename E>
FeatFn pick_feature(int d, int m, int kind, bool fwd, bool wgrad, bool resid) {
  switch (d) {
    case 16: return pick_mb<E, 16>(m, kind, fwd, wgrad, resid);
    case 32: return pick_mb<E, 32>(m, kind, fwd, wgrad, resid);
    case 64: return pick_mb<E, 64>(m, kind, fwd, wgrad, resid);
    case 128: return pick_mb<E, 128>(m, kind, fwd, wgrad, resid);
  }
  return nullptr;
}

// Feature widths the wide kernels take (bf16, head widths 32 and 64).
bool is_wide(const ts_feature_desc* d) { return d->m == 192 || d->m == 384; }

template <int D, int MB, int KIND>
FeatFn pick_wide4(bool fwd, bool resid) {
  if (fwd) return (FeatFn)ts::feature_fwd_wide_kernel<D, MB, KIND>;
  return resid ? (FeatFn)ts::feature_bwd_wide_kernel<D, MB, true, KIND>
               : (FeatFn)ts::feature_bwd_wide_kernel<D, MB, false, KIND>;
}

template <int D, int MB>
FeatFn pick_wide3(int kind, bool fwd, bool resid) {
  return kind == TS_FEAT_RELU2 ? pick_wide4<D, MB, TS_FEAT_RELU2>(fwd, resid)
                               : pick_wide4<D, MB, TS_FEAT_SOFTMAX>(fwd, resid);
}

template <int D>
FeatFn pick_wide2(int m, int kind, bool fwd, bool resid) {
  switch (m) {
    case 192: return pick_wide3<D, 12>(kind, fwd, resid);
    case 384: return pick_wide3<D, 24>(kind, fwd, resid);
  }
  return nullptr;
}

FeatFn pick(const ts_feature_desc* d, bool fwd, bool wgrad, bool resid = false) {
  if (is_wide(d)) {
    if (d->dtype != TS_BF16 || wgrad) return nullptr;
    switch (d->d) {
      case 32: return pick_wide2<32>(d->m, d->kind, fwd, resid);
      case 64: return pick_wide2<64>(d->m, d->kind, fwd, resid);
    }
    return nullptr;
  }
  return d->dtype == TS_BF16 ? pick_feature<ts::bf16>(d->d, d->m, d->kind, fwd, wgrad, resid)
                             : pick_feature<float>(d->d, d->m, d->kind, fwd, wgrad, resid);
}

int check_feature_desc(const ts_feature_desc* d) {
  if (!d) return fail(TS_ERR_VALUE, "feature: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0) return fail(TS_ERR_VALUE, "feature: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "feature: unknown dtype");
  if (d->kind != TS_FEAT_RELU2 && d->kind != TS_FEAT_SOFTMAX)
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature: kind %d has no fused kernel", d->kind);
  if (d->m != 16 && d->m != 32 && d->m != 64 && d->m != 128 && d->m != 256 && !is_wide(d))
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature: no fused kernel for feature width m=%d", d->m);
  if (is_wide(d) && (d->dtype != TS_BF16 || (d->d != 32 && d->d != 64)))
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature: width m=%d runs in bf16 with head width 32 or 64", d->m);
  if (d->in_rot < 0 || d->in_rot > d->d || d->in_rot % 4)
    return fail(TS_ERR_VALUE, "feature: input rotation must be a multiple of 4 within d");
  if (d->feat_rot < 0 || d->feat_rot > d->m || d->feat_rot % 4)
    return fail(TS_ERR_VALUE, "feature: feature rotation must be a multiple of 4 within m");
  if (!pick(d, true, false)) return fail(TS_ERR_NOT_IMPLEMENTED, "feature: no fused kernel for head width d=%d", d->d);
  return TS_OK;
}

// Stream descriptor for the kernels: 16-byte aligned rows and a time stride
// whose offsets up to T + 64 rows fit in 32 bits.
int to_str(const char* name, const ts_strided& s, int esize, int T, ts::Str* out) {
  *out = ts::Str{const_cast<void*>(s.ptr), s.sb, s.sh, 0};
  if (!s.ptr) return TS_OK;
  const int vec = 16 / esize;
  if (((uintptr_t)s.ptr & 15u) || s.sb % vec || s.sh % vec || s.st % vec || s.st < 0)
    return fail(TS_ERR_VALUE, "feature: rows of %s must be 16-byte aligned", name);
  if ((int64_t)(T + ts::TT) * s.st >= ((int64_t)1 << 31))
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature: time stride of %s too large", name);
  out->st = (int)s.st;
  return TS_OK;
}

// Per-token fp32 scalar stream (dtau): no alignment requirement.
int to_str_scalar(const ts_strided& s, int T, ts::Str* out) {
  *out = ts::Str{const_cast<void*>(s.ptr), s.sb, s.sh, (int)s.st};
  if (s.ptr && (int64_t)(T + ts::TT) * s.st >= ((int64_t)1 << 31))
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature: time stride of dtau too large");
  return TS_OK;
}

constexpr size_t kLdsTwoPerCu = 80 * 1024;

struct Plan {
  bool wgrad;
  size_t lds;
  int groups;
  dim3 grid;
};

// Weights in LDS: the same compile-time rule as weights_in_lds().
bool kernel_wl(int es, int d, int m, bool fwd, bool wgrad) {
  return (size_t)ts::feat_layout(es, d, m, fwd, true, wgrad, true).end * es + 64 <= (size_t)ts::kLdsMax;
}

size_t lds_bytes(int es, int d, int m, bool fwd, bool resid, bool wgrad) {
  const bool wl = kernel_wl(es, d, m, fwd, wgrad);
  return (size_t)ts::feat_layout(es, d, m, fwd, resid, wgrad, wl).end * es + 4 * sizeof(float);
}

// Launch plan of one call: fused weight gradients when a kernel exists for
// the shape and its tiles fit in LDS.  Forward: enough 64-token groups per
// workgroup to leave about four resident workgroups per CU.  Backward: the
// groups of each (batch, head) split over as many workgroups as the device
// holds at once (the occupancy calculator's count for the kernel), so that
// one wave of workgroups covers the call.
int plan_feature(const ts_feature_desc* d, bool fwd, bool resid, bool want_wgrad, Plan* P) {
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  P->wgrad = !fwd && want_wgrad && pick(d, false, true) != nullptr &&
             lds_bytes(es, d->d, d->m, fwd, resid, true) <= (size_t)ts::kLdsMax;
  P->lds = is_wide(d) ? (size_t)ts::wide_layout(d->d, d->m, fwd, resid).end * es
                      : lds_bytes(es, d->d, d->m, fwd, resid, P->wgrad);
  if (P->lds > (size_t)ts::kLdsMax) return fail(TS_ERR_NOT_IMPLEMENTED, "feature: tiles need %zu bytes of LDS", P->lds);
  const int tiles = (d->T + ts::TT - 1) / ts::TT;
  int groups = 1;
  if (fwd) {
    while (groups < 16 && (long)((tiles + 2 * groups - 1) / (2 * groups)) * d->H * d->B >= 1024) groups *= 2;
  } else {
    long slots = ts::resident_workgroups((const void*)pick(d, false, P->wgrad, resid), (int)P->lds);
    if (slots <= 0) slots = 512;  // two per CU on 256 CUs
    const long per_bh = slots / ((long)d->H * d->B) > 1 ? slots / ((long)d->H * d->B) : 1;
    const long g = (tiles + per_bh - 1) / per_bh;
    groups = (int)(g < 1 ? 1 : g > 16 ? 16 : g);
  }
  P->groups = groups;
  P->grid = dim3((tiles + groups - 1) / groups, d->H, d->B);
  return TS_OK;
}

int launch_feature(FeatFn fn, const Plan& P, hipStream_t stream, ts::FeatP& p) {
  p.groups = P.groups;
  if (P.lds > 65536) {
    hipError_t e = ts::ensure_lds_limit((const void*)fn, (int)P.lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "feature: LDS request failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(fn, P.grid, dim3(256), P.lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "feature: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

void fill_common(const ts_feature_desc* d, ts::FeatP& p) {
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.m = d->m;
  p.in_rot = d->in_rot; p.feat_rot = d->feat_rot; p.has_tau = d->has_tau; p.kind = d->kind;
  p.gain = d->gain; p.s = d->resid_scale; p.eps = d->eps; p.inv_m = 1.0f / (float)d->m;
}

}  // namespace

extern "C" {

int ts_feature_fwd(const ts_feature_desc* d, const ts_feature_io* io, hipStream_t stream) {
  int rc = check_feature_desc(d);
  if (rc) return rc;
  if (!io || !io->x.ptr || !io->w1 || !io->phi.ptr) return fail(TS_ERR_VALUE, "feature: missing tensors");
  if (io->resid.ptr && !io->w2) return fail(TS_ERR_VALUE, "feature: resid needs w2");
  if (d->has_tau && !io->tau) return fail(TS_ERR_VALUE, "feature: missing tau");
  if ((d->in_rot && (!io->in_cos || !io->in_sin)) || (d->feat_rot && (!io->f_cos || !io->f_sin)))
    return fail(TS_ERR_VALUE, "feature: missing rope tables");
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  ts::FeatP p;
  fill_common(d, p);
  if ((rc = to_str("x", io->x, es, d->T, &p.x)) || (rc = to_str("phi", io->phi, es, d->T, &p.phi)) ||
      (rc = to_str("resid", io->resid, es, d->T, &p.resid)))
    return rc;
  if (d->T == 0) return TS_OK;
  p.w1 = io->w1; p.w2 = io->w2; p.tau = io->tau;
  p.in_cos = io->in_cos; p.in_sin = io->in_sin; p.f_cos = io->f_cos; p.f_sin = io->f_sin;
  Plan P;
  if ((rc = plan_feature(d, true, io->resid.ptr != nullptr, false, &P))) return rc;
  return launch_feature(pick(d, true, false), P, stream, p);
}

int ts_feature_fwd_summary(const ts_feature_desc* d, const ts_feature_io* io, ts_strided v,
                           const ts_scan_desc* scan, void* workspace, size_t ws_bytes, hipStream_t stream) {
  int rc = check_feature_desc(d);
  if (rc) return rc;
  if (!io || !io->x.ptr || !io->w1 || !io->phi.ptr || !v.ptr || !scan)
    return fail(TS_ERR_VALUE, "feature summary: missing tensors");
  if (io->resid.ptr) return fail(TS_ERR_VALUE, "feature summary: keys carry no residual");
  if (d->has_tau && !io->tau) return fail(TS_ERR_VALUE, "feature: missing tau");
  if ((d->in_rot && (!io->in_cos || !io->in_sin)) || (d->feat_rot && (!io->f_cos || !io->f_sin)))
    return fail(TS_ERR_VALUE, "feature: missing rope tables");
  if (d->dtype != TS_BF16 || d->d != 64 || d->m != 64)
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature summary: bf16 with d = m = 64 only");
  if (scan->B != d->B || scan->H != d->H || scan->T != d->T || scan->dk != d->m || scan->dv != 64 ||
      scan->dtype != TS_BF16 || scan->retention != TS_RET_NONE || scan->reverse || scan->q_ext != TS_EXT_NONE ||
      scan->k_ext != TS_EXT_NONE || (scan->v_ext != TS_EXT_NONE && scan->v_ext != TS_EXT_ONES) ||
      scan->want_final || scan->init_state || scan->value_split)
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature summary: the scan must be a plain 64 x 64 bf16 sum over these "
                                        "features (optionally with its ones column)");
  ts::ScanSegments sg;
  if ((rc = ts::scan_segments(scan, &sg))) return rc;
  if (sg.dvp != 64 || sg.dkp != 64) return fail(TS_ERR_NOT_IMPLEMENTED, "feature summary: padded widths");
  if (sg.ws_bytes > 0 && (!workspace || ws_bytes < sg.ws_bytes || ((uintptr_t)workspace & 15)))
    return fail(TS_ERR_VALUE, "feature summary: workspace needs %zu bytes, 16-byte aligned", sg.ws_bytes);
  const int es = 2;
  ts::FeatP p;
  fill_common(d, p);
  if ((rc = to_str("x", io->x, es, d->T, &p.x)) || (rc = to_str("phi", io->phi, es, d->T, &p.phi)) ||
      (rc = to_str("v", v, es, d->T, &p.v)))
    return rc;
  if (d->T == 0) return TS_OK;
  p.w1 = io->w1; p.tau = io->tau;
  p.in_cos = io->in_cos; p.in_sin = io->in_sin; p.f_cos = io->f_cos; p.f_sin = io->f_sin;
  p.seg = (float*)workspace;
  p.segdec = p.seg ? p.seg + (size_t)d->B * d->H * sg.nseg * (size_t)sg.nelem : nullptr;
  p.nseg = sg.nseg; p.nsum = sg.ws_bytes > 0 ? sg.nsum : 0; p.nelem = sg.nelem; p.dvp = sg.dvp;
  p.v_ones = scan->v_ext == TS_EXT_ONES ? 1 : 0;
  Plan P;
  if ((rc = plan_feature(d, true, false, false, &P))) return rc;
  // one workgroup per segment of the scan
  P.groups = sg.seg_chunks;
  P.grid = dim3((unsigned)sg.nseg, d->H, d->B);
  P.lds += (size_t)ts::TT * (64 + 8) * es;
  FeatFn fn = d->kind == TS_FEAT_RELU2 ? (FeatFn)ts::feature_fwd_kernel<ts::bf16, 64, 4, TS_FEAT_RELU2, true>
                                       : (FeatFn)ts::feature_fwd_kernel<ts::bf16, 64, 4, TS_FEAT_SOFTMAX, true>;
  return launch_feature(fn, P, stream, p);
}

int ts_feature_bwd_parts(const ts_feature_desc* d, int32_t has_dresid, int32_t* parts) {
  int rc = check_feature_desc(d);
  if (rc) return rc;
  Plan P;
  if ((rc = plan_feature(d, false, has_dresid != 0, true, &P))) return rc;
  if (parts) *parts = P.wgrad ? (int32_t)(P.grid.x * P.grid.z) : 0;
  return TS_OK;
}

int ts_feature_bwd_transposed(const ts_feature_desc* d, int32_t has_dresid, int32_t fused_wgrad, int32_t* needed) {
  int rc = check_feature_desc(d);
  if (rc) return rc;
  Plan P;
  if ((rc = plan_feature(d, false, has_dresid != 0, fused_wgrad != 0, &P))) return rc;
  if (needed) *needed = is_wide(d) || kernel_wl(d->dtype == TS_BF16 ? 2 : 4, d->d, d->m, false, P.wgrad) ? 0 : 1;
  return TS_OK;
}

int ts_feature_bwd(const ts_feature_desc* d, const ts_feature_bwd_io* io, hipStream_t stream) {
  int rc = check_feature_desc(d);
  if (rc) return rc;
  if (!io || !io->x.ptr || !io->w1 || !io->dphi.ptr || !io->dx.ptr)
    return fail(TS_ERR_VALUE, "feature bwd: missing tensors");
  if (io->dresid.ptr && !io->w2t && !io->w2) return fail(TS_ERR_VALUE, "feature bwd: dresid needs w2 or w2t");
  if (d->has_tau && !io->tau) return fail(TS_ERR_VALUE, "feature bwd: missing tau");
  if ((d->in_rot && (!io->in_cos || !io->in_sin)) || (d->feat_rot && (!io->f_cos || !io->f_sin)))
    return fail(TS_ERR_VALUE, "feature bwd: missing rope tables");
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  ts::FeatP p;
  fill_common(d, p);
  if ((rc = to_str("x", io->x, es, d->T, &p.x)) || (rc = to_str("dphi", io->dphi, es, d->T, &p.dphi)) ||
      (rc = to_str("dx", io->dx, es, d->T, &p.dx)) || (rc = to_str("dresid", io->dresid, es, d->T, &p.dresid)))
    return rc;
  const bool want_wgrad = io->dw1_part != nullptr;
  if (!want_wgrad) {
    if ((rc = to_str("da", io->da, es, d->T, &p.da)) || (rc = to_str("xn", io->xn, es, d->T, &p.xn)) ||
        (rc = to_str("h", io->h, es, d->T, &p.h)) || (rc = to_str_scalar(io->dtau, d->T, &p.dtau)))
      return rc;
  }
  Plan P;
  if ((rc = plan_feature(d, false, io->dresid.ptr != nullptr, want_wgrad, &P))) return rc;
  if (want_wgrad && !P.wgrad)
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature bwd: no fused weight-gradient kernel for d=%d m=%d", d->d, d->m);
  if (want_wgrad && io->dresid.ptr && !io->dw2_part)
    return fail(TS_ERR_VALUE, "feature bwd: fused weight gradients with dresid need dw2_part");
  if (want_wgrad && d->has_tau && !io->dtau_part)
    return fail(TS_ERR_VALUE, "feature bwd: fused weight gradients with tau need dtau_part");
  if (is_wide(d)) {
    if (io->dresid.ptr && !io->w2) return fail(TS_ERR_VALUE, "feature bwd: width m=%d with dresid needs w2", d->m);
  } else if (!kernel_wl(es, d->d, d->m, false, P.wgrad) && (!io->w1t || (io->dresid.ptr && !io->w2t))) {
    return fail(TS_ERR_VALUE, "feature bwd: weights too large for LDS need w1t (and w2t)");
  }
  if (d->T == 0) return TS_OK;
  p.w1 = io->w1; p.w1t = io->w1t; p.w2t = io->w2t; p.w2 = io->w2; p.tau = io->tau;
  p.in_cos = io->in_cos; p.in_sin = io->in_sin; p.f_cos = io->f_cos; p.f_sin = io->f_sin;
  if (want_wgrad) {
    p.dw1_part = io->dw1_part; p.dw2_part = io->dw2_part; p.dtau_part = io->dtau_part;
  }
  return launch_feature(pick(d, false, P.wgrad, io->dresid.ptr != nullptr), P, stream, p);
}

}  // extern "C"
