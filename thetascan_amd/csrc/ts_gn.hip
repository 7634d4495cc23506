// GN-family write payloads for gfx950: the damped Gauss-Newton fast-weight
// update of a one-hidden-layer memory with a ReLU^2 or tanh hidden layer
// (forward and backward).
//
// Per token x (key, [d]) and v (value, [d]), with per-head W1 [m, d],
// W2 [d, m] and an optional per-feature threshold tau [m]
// (engine.py:117-158, 180-195, 215-255; depth L, s = 1/sqrt(L)):
//
//   a = W1 x,   rinv = (mean(a^2) + eps)^-1/2,   pre = a rinv - tau
//   h = sigma(pre),   sp = sigma'(pre)    (relu2: relu(pre)^2, 2 relu(pre);
//                                          tanh: tanh(pre), 1 - h^2)
//   u = W2 h,   r = v - (x + s u)                       (residual of theta0)
//   den = (|h|^2 + |x|^2 (W2 o W2)(sp rinv)^2) / L + damping  (Jacobi diagonal;
//         the reference's damping is eps)
//   lam = r / den,   g = s sp (W2^T lam) rinv
//
// Outputs: h (the LA2 keys), s lam (LA2 values) and g (LA1 values).  The
// backward recomputes the forward from x and v, writes dx and dv, and emits
// head-major weight-gradient tiles ([slot, H, B*T, w]) that batched GEMMs
// contract over tokens: dW1 = da^T x, dW2 = lam^T dz + du^T h + 2 W2 o
// (drq^T s2), dtau = -sum dpre.
//
// Layout and MFMA usage follow the feature kernels (ts_tokens.h): lane =
// token, the contraction over d or m runs on 16x16x32 MFMAs whose operands
// are LDS weight rows and accumulator fragments of the previous product.

#include "ts_common.h"
#include "ts_gn_act.h"
#include "ts_tokens.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct GnP {
  int B, H, T, groups, has_tau, act;
  float s, inv_L, eps, inv_m, damp;
  Str x, v, h, lam, g;             // forward inputs / outputs
  Str dh, dlam, dg, dxin, dx, dv;  // backward
  const void* w1;                  // [H, m, d]
  const void* w2;                  // [H, d, m]
  const void* w1t;                 // [H, d, m]
  const void* w2t;                 // [H, m, d]
  const float* tau;                // [H, m]
  void* tm;                        // [4 (+1), H, B*T, m]: dz, h, da, s2 (, dpre with tau)
  void* td;                        // [4, H, B*T, d]: lam, du, x, drq
};

// LDS carve-up (elements of E): x tile, then the weights when they fit.
struct GnLayout {
  int xp, mp;
  int xs, w1, w2, w1t, w2t;
  int end;
};
__host__ __device__ constexpr GnLayout gn_layout(int esize, int d, int m, bool fwd, bool w_lds) {
  const int vec = 16 / esize;
  GnLayout L{};
  L.xp = d + vec;
  L.mp = m + vec;
  int off = 0;
  L.xs = off; off += TT * L.xp;
  L.w1 = L.w2 = L.w1t = L.w2t = -1;
  if (w_lds) {
    L.w1 = off; off += m * L.xp;
    L.w2 = off; off += d * L.mp;
    L.w2t = off; off += m * L.xp;
    if (!fwd) { L.w1t = off; off += d * L.mp; }
  }
  L.end = off;
  return L;
}
// The read stage's own carve-up: the forward stages W1 and W2, the backward
// W1, W1^T and W2^T (the write layout's other matrices would only cost
// resident workgroups).
__host__ __device__ constexpr GnLayout gn_read_layout(int esize, int d, int m, bool fwd, bool w_lds) {
  const int vec = 16 / esize;
  GnLayout L{};
  L.xp = d + vec;
  L.mp = m + vec;
  int off = 0;
  L.xs = off; off += TT * L.xp;
  L.w1 = L.w2 = L.w1t = L.w2t = -1;
  if (w_lds) {
    L.w1 = off; off += m * L.xp;
    if (fwd) {
      L.w2 = off; off += d * L.mp;
    } else {
      L.w1t = off; off += d * L.mp;
      L.w2t = off; off += m * L.xp;
    }
  }
  L.end = off;
  return L;
}
constexpr int kGnLdsMax = 160 * 1024;
template <typename E, int D, int MB, bool FWD>
constexpr bool gn_weights_in_lds() {
  return gn_layout((int)sizeof(E), D, MB * 16, FWD, true).end * (int)sizeof(E) <= kGnLdsMax;
}
template <typename E, int D, int MB, bool FWD>
constexpr bool gn_read_weights_in_lds() {
  return gn_read_layout((int)sizeof(E), D, MB * 16, FWD, true).end * (int)sizeof(E) <= kGnLdsMax;
}

// The four thresholds of features fb*16 + 4g .. +3 (zeros without tau).
__device__ __forceinline__ void tau4(const float* tau, bool has_tau, int fb, int g, float* tv) {
  if (has_tau) {
    const floatx4 t4 = *(const floatx4*)(tau + fb * 16 + 4 * g);
    tv[0] = t4[0]; tv[1] = t4[1]; tv[2] = t4[2]; tv[3] = t4[3];
  } else {
    tv[0] = tv[1] = tv[2] = tv[3] = 0.f;
  }
}

// Four consecutive elements of row t (zero past T).
template <typename E>
__device__ __forceinline__ void ld4_row(const Str& s, int b, int h, int t, int c, bool valid, float* o) {
  if (valid && s.ptr) {
    ld4f<E>(rows_of<E>(s, b, h).at(t) + c, o);
  } else {
    o[0] = o[1] = o[2] = o[3] = 0.f;
  }
}
template <typename E>
__device__ __forceinline__ void st4_row(const Str& s, int b, int h, int t, int c, bool valid, const float* v) {
  if (valid) st4f<E>(rows_of<E>(s, b, h).at(t) + c, v);
}
// Row n of a head-major tile [.., N, w].
template <typename E>
__device__ __forceinline__ void st4_tile(void* base, int64_t row, int w, int c, bool valid, const float* v) {
  if (valid) st4f<E>((E*)base + row * w + c, v);
}

// out[db] = (Wt o Wt) reg: gemm_back with every weight squared on its way
// into the MFMA (the reference squares W2 elementwise, engine.py:244).
template <typename E, int D, int MB>
__device__ __forceinline__ void gemm_back_sq(const E* wt, int wp, const floatx4* reg, int l16, int g, floatx4* out) {
  typedef LdsIO<E> IO;
  auto sq4 = [](typename Frag<E>::f4 v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = tof(v[i]);
      v[i] = cvt<E>(f * f);
    }
    return v;
  };
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    out[db] = floatx4{0.f, 0.f, 0.f, 0.f};
    const E* wrow = wt + (db * 16 + l16) * wp;
#pragma unroll
    for (int j = 0; j < MB / 2; ++j)
      out[db] = mma32(IO::cat(sq4(IO::ld4(wrow + 32 * j + 4 * g)), sq4(IO::ld4(wrow + 32 * j + 16 + 4 * g))),
                      IO::from_acc(reg[2 * j], reg[2 * j + 1]), out[db]);
    if (MB & 1)
      out[db] = mma16(sq4(IO::ld4(wrow + 16 * (MB - 1) + 4 * g)), IO::from_acc4(reg[MB - 1]), out[db]);
  }
}

// The forward chain of one token (lane = token, four features per block).
template <typename E, int D, int MB>
struct GnToken {
  float xr[D / 16][4];  // x (dims 16db+4g+i)
  float vr[D / 16][4];  // v
  floatx4 a[MB];        // W1 x
  floatx4 rq[D / 16];   // (W2 o W2) (sp rinv)^2
  floatx4 lam[D / 16];  // lambda
  floatx4 den[D / 16];
  float rinv, xx, hh;
};

template <typename E, int D, int MB>
__device__ __forceinline__ void gn_forward_token(const GnP& p, int b, int h, int t, bool valid, int l16, int g,
                                                 const E* xrow, const E* xs_w, int xp, const E* w1, int wp1,
                                                 const E* w2, int wp2, const float* tau, GnToken<E, D, MB>& k,
                                                 floatx4* hv, floatx4* s2v) {
  float xx = 0.f;
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    ld4f<E>(xrow + db * 16 + 4 * g, k.xr[db]);
    ld4_row<E>(p.v, b, h, t, db * 16 + 4 * g, valid, k.vr[db]);
#pragma unroll
    for (int i = 0; i < 4; ++i) xx += k.xr[db][i] * k.xr[db][i];
  }
  k.xx = sum_g(xx);
  gemm_a<E, D, MB>(w1, wp1, xs_w, xp, l16, g, MB, k.a);
  float ss = 0.f;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb)
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += k.a[fb][i] * k.a[fb][i];
  k.rinv = rsqrtf(sum_g(ss) * p.inv_m + p.eps);
  float hh = 0.f;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb) {
    float tv[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.has_tau) {
      const floatx4 t4 = *(const floatx4*)(tau + fb * 16 + 4 * g);
      tv[0] = t4[0]; tv[1] = t4[1]; tv[2] = t4[2]; tv[3] = t4[3];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pre = k.a[fb][i] * k.rinv - tv[i];
      const float hval = gn_act(p.act, pre);
      hv[fb][i] = hval;
      const float sv = gn_slope(p.act, pre, hval) * k.rinv;
      s2v[fb][i] = sv * sv;
      hh += hval * hval;
    }
  }
  k.hh = sum_g(hh);
  floatx4 u[D / 16];
  gemm_back<E, D, MB>(w2, wp2, hv, l16, g, MB, u);
  gemm_back_sq<E, D, MB>(w2, wp2, s2v, l16, g, k.rq);
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float r = k.vr[db][i] - k.xr[db][i] - p.s * u[db][i];
      const float dn = (k.hh + k.xx * k.rq[db][i]) * p.inv_L + p.damp;
      k.den[db][i] = dn;
      k.lam[db][i] = r / dn;
    }
}

// Two waves per SIMD for the bf16 forward up to 64-wide tokens and 128 hidden
// features: at 128 hidden features that spills 44 registers and still runs
// 25 % faster than one wave without spills (B8 T2048 H8: 135 -> 101 us).
// (The backward at that width would spill 229 and measured 33 % slower.)
template <typename E, int D, int MB>
__global__ __launch_bounds__(256, (sizeof(E) == 2 && D <= 64 && MB <= 8 ? 2 : 1)) void gn_write_fwd_kernel(GnP p) {
  constexpr int M = MB * 16;
  constexpr bool WL = gn_weights_in_lds<E, D, MB, true>();
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const GnLayout L = gn_layout((int)sizeof(E), D, M, true, WL);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  const E* w1 = (const E*)p.w1 + h * M * D;
  const E* w2 = (const E*)p.w2 + h * D * M;
  const E* w2t = (const E*)p.w2t + h * M * D;
  int wp1 = D, wp2 = M;
  if constexpr (WL) {
    stage_matrix<E>(w1, M, D, base + L.w1, L.xp, tid);
    stage_matrix<E>(w2, D, M, base + L.w2, L.mp, tid);
    stage_matrix<E>(w2t, M, D, base + L.w2t, L.xp, tid);
    w1 = base + L.w1;
    w2 = base + L.w2;
    w2t = base + L.w2t;
    wp1 = L.xp;
    wp2 = L.mp;
  }
  const float* tau = p.has_tau ? p.tau + h * M : nullptr;
  const Rows<E> xsrc = rows_of<E>(p.x, b, h);
  RowTile<E, D> ldx;
  ldx.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldx.fetch(xsrc, g0 * TT, p.T);
  for (int grp = 0; grp < p.groups; ++grp) {
    const int t0 = (g0 + grp) * TT;
    if (t0 >= p.T) break;  // uniform over the workgroup
    __syncthreads();       // weights staged; previous group consumed
    ldx.store(xs, L.xp);
    if (grp + 1 < p.groups) ldx.fetch(xsrc, t0 + TT, p.T);
    __syncthreads();
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    GnToken<E, D, MB> k;
    floatx4 hv[MB], s2v[MB];
    gn_forward_token<E, D, MB>(p, b, h, t, valid, l16, g, xs + row * L.xp, xs + w * 16 * L.xp, L.xp, w1, wp1, w2,
                               wp2, tau, k, hv, s2v);
    floatx4 z[MB];
    gemm_back<E, M, D / 16>(w2t, wp1, k.lam, l16, g, D / 16, z);
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      float hvv[4], gv[4], tv[4];
      tau4(tau, p.has_tau, fb, g, tv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hvv[i] = hv[fb][i];
        const float sp = gn_slope(p.act, k.a[fb][i] * k.rinv - tv[i], hv[fb][i]);
        gv[i] = p.s * sp * z[fb][i] * k.rinv;
      }
      st4_row<E>(p.h, b, h, t, fb * 16 + 4 * g, valid, hvv);
      st4_row<E>(p.g, b, h, t, fb * 16 + 4 * g, valid, gv);
    }
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float lv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) lv[i] = p.s * k.lam[db][i];
      st4_row<E>(p.lam, b, h, t, db * 16 + 4 * g, valid, lv);
    }
  }
}

template <typename E, int D, int MB>
__global__ __launch_bounds__(256) void gn_write_bwd_kernel(GnP p) {
  constexpr int M = MB * 16;
  constexpr bool WL = gn_weights_in_lds<E, D, MB, false>();
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const GnLayout L = gn_layout((int)sizeof(E), D, M, false, WL);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  const E* w1 = (const E*)p.w1 + h * M * D;
  const E* w2 = (const E*)p.w2 + h * D * M;
  const E* w2t = (const E*)p.w2t + h * M * D;
  const E* w1t = (const E*)p.w1t + h * D * M;
  int wpd = D, wpm = M;  // pitches of [.][D] and [.][M] weight rows
  if constexpr (WL) {
    stage_matrix<E>(w1, M, D, base + L.w1, L.xp, tid);
    stage_matrix<E>(w2, D, M, base + L.w2, L.mp, tid);
    stage_matrix<E>(w2t, M, D, base + L.w2t, L.xp, tid);
    stage_matrix<E>(w1t, D, M, base + L.w1t, L.mp, tid);
    w1 = base + L.w1;
    w2 = base + L.w2;
    w2t = base + L.w2t;
    w1t = base + L.w1t;
    wpd = L.xp;
    wpm = L.mp;
  }
  const float* tau = p.has_tau ? p.tau + h * M : nullptr;
  const int64_t N = (int64_t)p.B * p.T;
  // slot-major tiles: slot k of head h starts at k * H * N * w + h * N * w
  E* tm = (E*)p.tm + (int64_t)h * N * M;  // dz, h, da, s2 (, dpre)
  E* td = (E*)p.td + (int64_t)h * N * D;  // lam, du, x, drq
  const int64_t HNM = (int64_t)p.H * N * M, HND = (int64_t)p.H * N * D;
  const Rows<E> xsrc = rows_of<E>(p.x, b, h);
  RowTile<E, D> ldx;
  ldx.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldx.fetch(xsrc, g0 * TT, p.T);
  for (int grp = 0; grp < p.groups; ++grp) {
    const int t0 = (g0 + grp) * TT;
    if (t0 >= p.T) break;  // uniform over the workgroup
    __syncthreads();
    ldx.store(xs, L.xp);
    if (grp + 1 < p.groups) ldx.fetch(xsrc, t0 + TT, p.T);
    __syncthreads();
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    const int64_t n = (int64_t)b * p.T + t;
    GnToken<E, D, MB> k;
    floatx4 hv[MB], s2v[MB];
    gn_forward_token<E, D, MB>(p, b, h, t, valid, l16, g, xs + row * L.xp, xs + w * 16 * L.xp, L.xp, w1, wpd, w2,
                               wpm, tau, k, hv, s2v);
    // tiles known after the forward: h, s2, lam, x
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      float o[4] = {hv[fb][0], hv[fb][1], hv[fb][2], hv[fb][3]};
      st4_tile<E>(tm + 1 * HNM, n, M, fb * 16 + 4 * g, valid, o);
      float o2[4] = {s2v[fb][0], s2v[fb][1], s2v[fb][2], s2v[fb][3]};
      st4_tile<E>(tm + 3 * HNM, n, M, fb * 16 + 4 * g, valid, o2);
    }
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float o[4] = {k.lam[db][0], k.lam[db][1], k.lam[db][2], k.lam[db][3]};
      st4_tile<E>(td + 0 * HND, n, D, db * 16 + 4 * g, valid, o);
      st4_tile<E>(td + 2 * HND, n, D, db * 16 + 4 * g, valid, k.xr[db]);
    }
    // ---- g = s sp z rinv, z = W2^T lam
    floatx4 dz[MB], dsp[MB];
    float drinv = 0.f;
    {
      floatx4 z[MB];
      gemm_back<E, M, D / 16>(w2t, wpd, k.lam, l16, g, D / 16, z);
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        float dgv[4], tv[4];
        ld4_row<E>(p.dg, b, h, t, fb * 16 + 4 * g, valid, dgv);
        tau4(tau, p.has_tau, fb, g, tv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float sp = gn_slope(p.act, k.a[fb][i] * k.rinv - tv[i], hv[fb][i]);
          const float sdg = p.s * dgv[i];
          dz[fb][i] = sdg * sp * k.rinv;
          dsp[fb][i] = sdg * z[fb][i] * k.rinv;
          drinv += sdg * sp * z[fb][i];
        }
        float o[4] = {dz[fb][0], dz[fb][1], dz[fb][2], dz[fb][3]};
        st4_tile<E>(tm + 0 * HNM, n, M, fb * 16 + 4 * g, valid, o);
      }
    }
    // ---- lam -> r, den -> (hh, xx, rq)
    floatx4 dr[D / 16], drq[D / 16];
    float dhh = 0.f, dxx = 0.f;
    {
      floatx4 wdz[D / 16];
      gemm_back<E, D, MB>(w2, wpm, dz, l16, g, MB, wdz);
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        float dlv[4];
        ld4_row<E>(p.dlam, b, h, t, db * 16 + 4 * g, valid, dlv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float dl = p.s * dlv[i] + wdz[db][i];
          dr[db][i] = dl / k.den[db][i];
          const float dD = -dl * k.lam[db][i] / k.den[db][i] * p.inv_L;
          dhh += dD;
          dxx += dD * k.rq[db][i];
          drq[db][i] = dD;  // times xx below (after the group sum)
        }
      }
      dhh = sum_g(dhh);
      dxx = sum_g(dxx);
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
#pragma unroll
        for (int i = 0; i < 4; ++i) drq[db][i] *= k.xx;
        float o[4] = {drq[db][0], drq[db][1], drq[db][2], drq[db][3]};
        st4_tile<E>(td + 3 * HND, n, D, db * 16 + 4 * g, valid, o);
      }
    }
    // ---- rq = (W2 o W2) s2, s2 = (sp rinv)^2
    {
      floatx4 ds2[MB];
      gemm_back_sq<E, M, D / 16>(w2t, wpd, drq, l16, g, ds2);
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        float tv[4];
        tau4(tau, p.has_tau, fb, g, tv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float sp = gn_slope(p.act, k.a[fb][i] * k.rinv - tv[i], hv[fb][i]);
          const float dsv = 2.f * sp * k.rinv * ds2[fb][i];
          dsp[fb][i] += dsv * k.rinv;
          drinv += dsv * sp;
        }
      }
    }
    // ---- r = v - x - s W2 h
    floatx4 du[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float dvv[4], duv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dvv[i] = dr[db][i];
        du[db][i] = -p.s * dr[db][i];
        duv[i] = du[db][i];
      }
      st4_row<E>(p.dv, b, h, t, db * 16 + 4 * g, valid, dvv);
      st4_tile<E>(td + 1 * HND, n, D, db * 16 + 4 * g, valid, duv);
    }
    floatx4 da[MB];
    {
      floatx4 dhu[MB];
      gemm_back<E, M, D / 16>(w2t, wpd, du, l16, g, D / 16, dhu);
      float ra = 0.f;
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        float dhv[4];
        ld4_row<E>(p.dh, b, h, t, fb * 16 + 4 * g, valid, dhv);
        float tv[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.has_tau) {
          const floatx4 t4 = *(const floatx4*)(tau + fb * 16 + 4 * g);
          tv[0] = t4[0]; tv[1] = t4[1]; tv[2] = t4[2]; tv[3] = t4[3];
        }
        float dpv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pre = k.a[fb][i] * k.rinv - tv[i];
          const float dht = dhv[i] + dhu[fb][i] + 2.f * hv[fb][i] * dhh;
          const float dpre = valid ? gn_dpre(p.act, pre, hv[fb][i], dht, dsp[fb][i]) : 0.f;
          dpv[i] = dpre;
          da[fb][i] = dpre;  // completed below once drinv is known
          ra += dpre * k.a[fb][i];
        }
        if (p.has_tau) st4_tile<E>(tm + 4 * HNM, n, M, fb * 16 + 4 * g, valid, dpv);
      }
      drinv = sum_g(drinv + ra);
    }
    const float c3 = drinv * k.rinv * k.rinv * k.rinv * p.inv_m;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) da[fb][i] = da[fb][i] * k.rinv - c3 * k.a[fb][i];
      float o[4] = {da[fb][0], da[fb][1], da[fb][2], da[fb][3]};
      st4_tile<E>(tm + 2 * HNM, n, M, fb * 16 + 4 * g, valid, o);
    }
    floatx4 wda[D / 16];
    gemm_back<E, D, MB>(w1t, wpm, da, l16, g, MB, wda);
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float dxi[4], o[4];
      ld4_row<E>(p.dxin, b, h, t, db * 16 + 4 * g, valid, dxi);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = dxi[i] - dr[db][i] + 2.f * k.xr[db][i] * dxx + wda[db][i];
      st4_row<E>(p.dx, b, h, t, db * 16 + 4 * g, valid, o);
    }
  }
}

// ------------------------------------------------------------ GN read stage
//
// One stage of the GN read (engine.py:467-506): per query q,
//   a = W1 q + c,  c = 0 | num | num / (mass + eps)   (corr = 0 | 1 | 2)
//   pre = a rsqrt(mean a^2 + eps) - tau,  h = sigma(pre) (relu2 or tanh)
//   resid = q + s W2 h                                  (want_resid)
// Stage 1 of the normalized two-stage read is corr = 0 without resid (its h
// are the queries of the feature-mass scan); stage 2 adds the normalized
// stage-1 read (corr = 2) and produces the queries of the memory scan and the
// residual the read epilogue adds the memory to.  The backward emits dq, the
// gradients of num and mass, and head-major tiles for dW1 = da^T q,
// dW2 = (s dresid)^T h and dtau = -sum dpre.
struct GnReadP {
  int B, H, T, groups, has_tau, corr, want_resid, act;
  float s, eps, inv_m;
  Str q, num, h, resid, dh, dresid, dq, dnum;
  const float* mass;  // fp32 [B,H,T] with element strides msb, msh, mst
  float* dmass;
  int64_t msb, msh, mst;
  const void* w1;   // [H, m, d]
  const void* w2;   // [H, d, m]
  const void* w1t;  // [H, d, m]
  const void* w2t;  // [H, m, d]
  const float* tau;
  void* tm;  // [2 (+1), H, B*T, m]: da, h (, dpre with tau)
  void* td;  // [2, H, B*T, d]: q, s dresid
};

template <typename E, int D, int MB>
__device__ __forceinline__ float gn_read_preact(const GnReadP& p, int b, int h, int t, bool valid, int l16, int g,
                                                const E* xs_w, int xp, const E* w1, int wp1, floatx4* a,
                                                float& cinv) {
  gemm_a<E, D, MB>(w1, wp1, xs_w, xp, l16, g, MB, a);
  cinv = 1.f;
  if (p.corr) {
    if (p.corr == 2) cinv = valid ? 1.f / (p.mass[b * p.msb + h * p.msh + (int64_t)t * p.mst] + p.eps) : 0.f;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      float c[4];
      ld4_row<E>(p.num, b, h, t, fb * 16 + 4 * g, valid, c);
#pragma unroll
      for (int i = 0; i < 4; ++i) a[fb][i] += c[i] * cinv;
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb)
#pragma unroll
    for (int i = 0; i < 4; ++i) ss += a[fb][i] * a[fb][i];
  return rsqrtf(sum_g(ss) * p.inv_m + p.eps);
}

template <int MB>
__device__ __forceinline__ void tau_of(const float* tau, int fb, int g, bool on, float* tv) {
  tv[0] = tv[1] = tv[2] = tv[3] = 0.f;
  if (on) {
    const floatx4 t4 = *(const floatx4*)(tau + fb * 16 + 4 * g);
    tv[0] = t4[0]; tv[1] = t4[1]; tv[2] = t4[2]; tv[3] = t4[3];
  }
}

template <typename E, int D, int MB>
__global__ __launch_bounds__(256) void gn_read_fwd_kernel(GnReadP p) {
  constexpr int M = MB * 16;
  constexpr bool WL = gn_read_weights_in_lds<E, D, MB, true>();
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const GnLayout L = gn_read_layout((int)sizeof(E), D, M, true, WL);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  const E* w1 = (const E*)p.w1 + h * M * D;
  const E* w2 = p.want_resid ? (const E*)p.w2 + h * D * M : nullptr;
  int wp1 = D, wp2 = M;
  if constexpr (WL) {
    stage_matrix<E>(w1, M, D, base + L.w1, L.xp, tid);
    if (p.want_resid) stage_matrix<E>(w2, D, M, base + L.w2, L.mp, tid);
    w1 = base + L.w1;
    w2 = base + L.w2;
    wp1 = L.xp;
    wp2 = L.mp;
  }
  const float* tau = p.has_tau ? p.tau + h * M : nullptr;
  const Rows<E> qsrc = rows_of<E>(p.q, b, h);
  RowTile<E, D> ldq;
  ldq.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldq.fetch(qsrc, g0 * TT, p.T);
  for (int grp = 0; grp < p.groups; ++grp) {
    const int t0 = (g0 + grp) * TT;
    if (t0 >= p.T) break;  // uniform over the workgroup
    __syncthreads();
    ldq.store(xs, L.xp);
    if (grp + 1 < p.groups) ldq.fetch(qsrc, t0 + TT, p.T);
    __syncthreads();
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    floatx4 a[MB], hv[MB];
    float cinv;
    const float rinv = gn_read_preact<E, D, MB>(p, b, h, t, valid, l16, g, xs + w * 16 * L.xp, L.xp, w1, wp1, a,
                                                cinv);
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      float tv[4], o[4];
      tau_of<MB>(tau, fb, g, p.has_tau, tv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hv[fb][i] = gn_act(p.act, a[fb][i] * rinv - tv[i]);
        o[i] = hv[fb][i];
      }
      st4_row<E>(p.h, b, h, t, fb * 16 + 4 * g, valid, o);
    }
    if (p.want_resid) {
      floatx4 u[D / 16];
      gemm_back<E, D, MB>(w2, wp2, hv, l16, g, MB, u);
      const E* qrow = xs + row * L.xp;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        float qv[4];
        ld4f<E>(qrow + db * 16 + 4 * g, qv);
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] += p.s * u[db][i];
        st4_row<E>(p.resid, b, h, t, db * 16 + 4 * g, valid, qv);
      }
    }
  }
}

template <typename E, int D, int MB>
__global__ __launch_bounds__(256) void gn_read_bwd_kernel(GnReadP p) {
  constexpr int M = MB * 16;
  constexpr bool WL = gn_read_weights_in_lds<E, D, MB, false>();
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const GnLayout L = gn_read_layout((int)sizeof(E), D, M, false, WL);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  const E* w1 = (const E*)p.w1 + h * M * D;
  const E* w1t = (const E*)p.w1t + h * D * M;
  const E* w2t = p.want_resid ? (const E*)p.w2t + h * M * D : nullptr;
  int wpd = D, wpm = M;
  if constexpr (WL) {
    stage_matrix<E>(w1, M, D, base + L.w1, L.xp, tid);
    stage_matrix<E>(w1t, D, M, base + L.w1t, L.mp, tid);
    if (p.want_resid) stage_matrix<E>(w2t, M, D, base + L.w2t, L.xp, tid);
    w1 = base + L.w1;
    w1t = base + L.w1t;
    w2t = base + L.w2t;
    wpd = L.xp;
    wpm = L.mp;
  }
  const float* tau = p.has_tau ? p.tau + h * M : nullptr;
  const int64_t N = (int64_t)p.B * p.T;
  // slot-major tiles: slot k of head h starts at k * H * N * w + h * N * w
  E* tm = (E*)p.tm + (int64_t)h * N * M;  // da, h (, dpre)
  E* td = (E*)p.td + (int64_t)h * N * D;  // q, s dresid
  const int64_t HNM = (int64_t)p.H * N * M, HND = (int64_t)p.H * N * D;
  const Rows<E> qsrc = rows_of<E>(p.q, b, h);
  RowTile<E, D> ldq;
  ldq.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldq.fetch(qsrc, g0 * TT, p.T);
  for (int grp = 0; grp < p.groups; ++grp) {
    const int t0 = (g0 + grp) * TT;
    if (t0 >= p.T) break;  // uniform over the workgroup
    __syncthreads();
    ldq.store(xs, L.xp);
    if (grp + 1 < p.groups) ldq.fetch(qsrc, t0 + TT, p.T);
    __syncthreads();
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    const int64_t n = (int64_t)b * p.T + t;
    floatx4 a[MB];
    float cinv;
    const float rinv = gn_read_preact<E, D, MB>(p, b, h, t, valid, l16, g, xs + w * 16 * L.xp, L.xp, w1, wpd, a,
                                                cinv);
    float dres[D / 16][4], qv[D / 16][4];
    floatx4 dres4[D / 16];
    const E* qrow = xs + row * L.xp;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      ld4f<E>(qrow + db * 16 + 4 * g, qv[db]);
      ld4_row<E>(p.dresid, b, h, t, db * 16 + 4 * g, valid && p.want_resid, dres[db]);
      float sd[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dres4[db][i] = dres[db][i];
        sd[i] = p.s * dres[db][i];
      }
      st4_tile<E>(td + 0 * HND, n, D, db * 16 + 4 * g, valid, qv[db]);
      st4_tile<E>(td + 1 * HND, n, D, db * 16 + 4 * g, valid, sd);
    }
    floatx4 dhr[MB];
    if (p.want_resid) {
      gemm_back<E, M, D / 16>(w2t, wpd, dres4, l16, g, D / 16, dhr);
    } else {
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) dhr[fb] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    floatx4 da[MB];
    float ra = 0.f;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      float tv[4], dhv[4], hvv[4], dpv[4];
      tau_of<MB>(tau, fb, g, p.has_tau, tv);
      ld4_row<E>(p.dh, b, h, t, fb * 16 + 4 * g, valid, dhv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pre = a[fb][i] * rinv - tv[i];
        hvv[i] = gn_act(p.act, pre);
        const float dpre = valid ? gn_dpre(p.act, pre, hvv[i], dhv[i] + p.s * dhr[fb][i], 0.f) : 0.f;
        dpv[i] = dpre;
        da[fb][i] = dpre;
        ra += dpre * a[fb][i];
      }
      st4_tile<E>(tm + 1 * HNM, n, M, fb * 16 + 4 * g, valid, hvv);
      if (p.has_tau) st4_tile<E>(tm + 2 * HNM, n, M, fb * 16 + 4 * g, valid, dpv);
    }
    ra = sum_g(ra);
    const float c3 = ra * rinv * rinv * rinv * p.inv_m;
    float dm = 0.f;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      float o[4], dn[4];
      float c[4] = {0.f, 0.f, 0.f, 0.f};
      if (p.corr == 2) ld4_row<E>(p.num, b, h, t, fb * 16 + 4 * g, valid, c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        da[fb][i] = da[fb][i] * rinv - c3 * a[fb][i];
        o[i] = da[fb][i];
        dn[i] = da[fb][i] * cinv;
        dm += da[fb][i] * c[i];
      }
      st4_tile<E>(tm + 0 * HNM, n, M, fb * 16 + 4 * g, valid, o);
      if (p.corr) st4_row<E>(p.dnum, b, h, t, fb * 16 + 4 * g, valid, dn);
    }
    if (p.corr == 2) {
      dm = sum_g(dm);
      if (g == 0 && valid) p.dmass[b * p.msb + h * p.msh + (int64_t)t * p.mst] = -dm * cinv * cinv;
    }
    floatx4 wda[D / 16];
    gemm_back<E, D, MB>(w1t, wpm, da, l16, g, MB, wda);
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = dres[db][i] + wda[db][i];
      st4_row<E>(p.dq, b, h, t, db * 16 + 4 * g, valid, o);
    }
  }
}

// ------------------------------------------------------------ wide widths
//
// Hidden widths of 192 and 384 (bf16, head widths 32 and 64): the per-lane
// m-vectors of the kernels above would not fit in registers (they spill to
// scratch), so these walk the hidden axis 64 features at a time.  Each pass
// over the chunks re-forms what it needs of a = W1 x (RMSNorm sum, then h,
// s^2 and the W2 products; in the backward the products that feed drinv and
// the per-chunk dpre) on MFMA, keeping only d-vectors and per-token scalars
// across chunks.  W1 and W2 (or W2^T for the read backward) are staged in
// LDS once per workgroup; W1^T and W2^T operands of the write kernels are
// transposing LDS reads of the staged rows.

struct GnWideLayout {
  int xp, mp;
  int xs, w1, w2;  // element offsets; w2 holds W2 [d][mp] or W2^T [m][xp]
  int end;
};
// w2_rows: 0 (no W2), 1 (W2 as [d][m + 8]), 2 (W2^T as [m][d + 8])
__host__ __device__ constexpr GnWideLayout gn_wide_layout(int d, int m, int w2_rows) {
  GnWideLayout L{};
  L.xp = d + 8;
  L.mp = m + 8;
  int off = 0;
  L.xs = off; off += TT * L.xp;
  L.w1 = off; off += m * L.xp;
  L.w2 = -1;
  if (w2_rows == 1) { L.w2 = off; off += d * L.mp; }
  if (w2_rows == 2) { L.w2 = off; off += m * L.xp; }
  L.end = off;
  return L;
}

__device__ __forceinline__ bf16x8 sq8(bf16x8 v) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float f = tof(v[i]);
    v[i] = (bf16)(f * f);
  }
  return v;
}

// a of chunk c (feature blocks 4c..4c+3) for this wave's 16 tokens
template <int D>
__device__ __forceinline__ void gnw_a(const bf16* w1s, int xp, const bf16* xs_w, int c, int l16, int g, floatx4* a) {
  gemm_a<bf16, D, 4>(w1s + c * 64 * xp, xp, xs_w, xp, l16, g, 4, a);
}
// out[db] += (W2 or W2 o W2)[:, chunk c] reg  (W2 staged as [D][mp])
template <int D, bool SQ>
__device__ __forceinline__ void gnw_w2(const bf16* w2s, int mp, int c, const floatx4* reg, int l16, int g,
                                       floatx4* out) {
  typedef LdsIO<bf16> IO;
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    const bf16* wrow = w2s + (db * 16 + l16) * mp + c * 64;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      bf16x8 wa = IO::cat(IO::ld4(wrow + 32 * jj + 4 * g), IO::ld4(wrow + 32 * jj + 16 + 4 * g));
      if (SQ) wa = sq8(wa);
      out[db] = mma32(wa, IO::from_acc(reg[2 * jj], reg[2 * jj + 1]), out[db]);
    }
  }
}
// out[f] = (W2 or W2 o W2)[:, chunk c]^T dvec  (transposing reads of W2 [D][mp])
template <int D, bool SQ>
__device__ __forceinline__ void gnw_w2t(const bf16* w2s, int mp, int c, const floatx4* dvec, int lane,
                                        floatx4* out) {
  typedef LdsIO<bf16> IO;
  typedef TokFrag<bf16> TF;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    out[f] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk) {
      bf16x8 wa = TF::get(w2s, mp, c * 64 + f * 16, kk, lane);
      if (SQ) wa = sq8(wa);
      out[f] = mma32(wa, IO::from_acc(dvec[2 * kk], dvec[2 * kk + 1]), out[f]);
    }
  }
}
// out[db] += W1[chunk c]^T reg  (transposing reads of W1 [m][xp])
template <int D>
__device__ __forceinline__ void gnw_w1t(const bf16* w1s, int xp, int c, const floatx4* reg, int lane,
                                        floatx4* out) {
  typedef LdsIO<bf16> IO;
  typedef TokFrag<bf16> TF;
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      out[db] = mma32(TF::get(w1s + c * 64 * xp, xp, db * 16, jj, lane), IO::from_acc(reg[2 * jj], reg[2 * jj + 1]),
                      out[db]);
}

// The forward chain of one token over the chunks: rinv, hh, u = W2 h,
// rq = (W2 o W2) s^2, then lam and den.  Per chunk it hands h and s^2 to
// `sink` (the tiles of the backward, the h output of the forward).
template <int D, int MB, typename Sink>
__device__ __forceinline__ void gnw_forward(const GnP& p, const float* tau, const bf16* w1s, int xp, const bf16* w2s,
                                            int mp, const bf16* xs_w, int l16, int g, const float (*xr)[4],
                                            const float (*vr)[4], float xx, float& rinv, float& hh, floatx4* lam,
                                            floatx4* den, floatx4* rq, Sink sink) {
  constexpr int NC = MB / 4;
  float ss = 0.f;
#pragma unroll 1
  for (int c = 0; c < NC; ++c) {
    floatx4 a[4];
    gnw_a<D>(w1s, xp, xs_w, c, l16, g, a);
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += a[f][i] * a[f][i];
  }
  rinv = rsqrtf(sum_g(ss) * p.inv_m + p.eps);
  floatx4 u[D / 16];
#pragma unroll
  for (int db = 0; db < D / 16; ++db) u[db] = rq[db] = floatx4{0.f, 0.f, 0.f, 0.f};
  float hsum = 0.f;
#pragma unroll 1
  for (int c = 0; c < NC; ++c) {
    floatx4 a[4], hv[4], s2v[4];
    gnw_a<D>(w1s, xp, xs_w, c, l16, g, a);
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      float tv[4];
      tau_of<MB>(tau, 4 * c + f, g, p.has_tau, tv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pre = a[f][i] * rinv - tv[i];
        const float hval = gn_act(p.act, pre);
        hv[f][i] = hval;
        const float sv = gn_slope(p.act, pre, hval) * rinv;
        s2v[f][i] = sv * sv;
        hsum += hval * hval;
      }
    }
    gnw_w2<D, false>(w2s, mp, c, hv, l16, g, u);
    gnw_w2<D, true>(w2s, mp, c, s2v, l16, g, rq);
    sink(c, hv, s2v);
  }
  hh = sum_g(hsum);
#pragma unroll
  for (int db = 0; db < D / 16; ++db)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float r = vr[db][i] - xr[db][i] - p.s * u[db][i];
      const float dn = (hh + xx * rq[db][i]) * p.inv_L + p.damp;
      den[db][i] = dn;
      lam[db][i] = r / dn;
    }
}

template <int D, int MB>
__global__ __launch_bounds__(256) void gn_write_fwd_wide_kernel(GnP p) {
  typedef bf16 E;
  constexpr int M = MB * 16;
  constexpr int NC = MB / 4;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const GnWideLayout L = gn_wide_layout(D, M, 1);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  E* w1s = base + L.w1;
  E* w2s = base + L.w2;
  stage_matrix<E>((const E*)p.w1 + (size_t)h * M * D, M, D, w1s, L.xp, tid);
  stage_matrix<E>((const E*)p.w2 + (size_t)h * D * M, D, M, w2s, L.mp, tid);
  const float* tau = p.has_tau ? p.tau + h * M : nullptr;
  const Rows<E> xsrc = rows_of<E>(p.x, b, h);
  RowTile<E, D> ldx;
  ldx.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldx.fetch(xsrc, g0 * TT, p.T);
  for (int grp = 0; grp < p.groups; ++grp) {
    const int t0 = (g0 + grp) * TT;
    if (t0 >= p.T) break;  // uniform over the workgroup
    __syncthreads();       // weights staged; previous group consumed
    ldx.store(xs, L.xp);
    if (grp + 1 < p.groups) ldx.fetch(xsrc, t0 + TT, p.T);
    __syncthreads();
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    const E* xs_w = xs + w * 16 * L.xp;
    float xr[D / 16][4], vr[D / 16][4];
    float xx = 0.f;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      ld4f<E>(xs + row * L.xp + db * 16 + 4 * g, xr[db]);
      ld4_row<E>(p.v, b, h, t, db * 16 + 4 * g, valid, vr[db]);
#pragma unroll
      for (int i = 0; i < 4; ++i) xx += xr[db][i] * xr[db][i];
    }
    xx = sum_g(xx);
    float rinv, hh;
    floatx4 lam[D / 16], den[D / 16], rq[D / 16];
    gnw_forward<D, MB>(p, tau, w1s, L.xp, w2s, L.mp, xs_w, l16, g, xr, vr, xx, rinv, hh, lam, den, rq,
                       [&](int c, const floatx4* hv, const floatx4*) {
#pragma unroll
                         for (int f = 0; f < 4; ++f) {
                           float o[4] = {hv[f][0], hv[f][1], hv[f][2], hv[f][3]};
                           st4_row<E>(p.h, b, h, t, c * 64 + f * 16 + 4 * g, valid, o);
                         }
                       });
    // g = s sp (W2^T lam) rinv per chunk
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], z[4];
      gnw_a<D>(w1s, L.xp, xs_w, c, l16, g, a);
      gnw_w2t<D, false>(w2s, L.mp, c, lam, lane, z);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float tv[4], gv[4];
        tau_of<MB>(tau, 4 * c + f, g, p.has_tau, tv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pre = a[f][i] * rinv - tv[i];
          gv[i] = p.s * gn_slope(p.act, pre, gn_act(p.act, pre)) * z[f][i] * rinv;
        }
        st4_row<E>(p.g, b, h, t, c * 64 + f * 16 + 4 * g, valid, gv);
      }
    }
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float lv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) lv[i] = p.s * lam[db][i];
      st4_row<E>(p.lam, b, h, t, db * 16 + 4 * g, valid, lv);
    }
  }
}

template <int D, int MB>
__global__ __launch_bounds__(256) void gn_write_bwd_wide_kernel(GnP p) {
  typedef bf16 E;
  constexpr int M = MB * 16;
  constexpr int NC = MB / 4;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const GnWideLayout L = gn_wide_layout(D, M, 1);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  E* w1s = base + L.w1;
  E* w2s = base + L.w2;
  stage_matrix<E>((const E*)p.w1 + (size_t)h * M * D, M, D, w1s, L.xp, tid);
  stage_matrix<E>((const E*)p.w2 + (size_t)h * D * M, D, M, w2s, L.mp, tid);
  const float* tau = p.has_tau ? p.tau + h * M : nullptr;
  const int64_t N = (int64_t)p.B * p.T;
  // slot-major tiles: slot k of head h starts at k * H * N * w + h * N * w
  E* tm = (E*)p.tm + (int64_t)h * N * M;  // dz, h, da, s2 (, dpre)
  E* td = (E*)p.td + (int64_t)h * N * D;  // lam, du, x, drq
  const int64_t HNM = (int64_t)p.H * N * M, HND = (int64_t)p.H * N * D;
  const Rows<E> xsrc = rows_of<E>(p.x, b, h);
  RowTile<E, D> ldx;
  ldx.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldx.fetch(xsrc, g0 * TT, p.T);
  for (int grp = 0; grp < p.groups; ++grp) {
    const int t0 = (g0 + grp) * TT;
    if (t0 >= p.T) break;  // uniform over the workgroup
    __syncthreads();
    ldx.store(xs, L.xp);
    if (grp + 1 < p.groups) ldx.fetch(xsrc, t0 + TT, p.T);
    __syncthreads();
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    const int64_t n = (int64_t)b * p.T + t;
    const E* xs_w = xs + w * 16 * L.xp;
    float xr[D / 16][4], vr[D / 16][4];
    float xx = 0.f;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      ld4f<E>(xs + row * L.xp + db * 16 + 4 * g, xr[db]);
      ld4_row<E>(p.v, b, h, t, db * 16 + 4 * g, valid, vr[db]);
#pragma unroll
      for (int i = 0; i < 4; ++i) xx += xr[db][i] * xr[db][i];
    }
    xx = sum_g(xx);
    float rinv, hh;
    floatx4 lam[D / 16], den[D / 16], rq[D / 16];
    gnw_forward<D, MB>(p, tau, w1s, L.xp, w2s, L.mp, xs_w, l16, g, xr, vr, xx, rinv, hh, lam, den, rq,
                       [&](int c, const floatx4* hv, const floatx4* s2v) {
#pragma unroll
                         for (int f = 0; f < 4; ++f) {
                           float o[4] = {hv[f][0], hv[f][1], hv[f][2], hv[f][3]};
                           st4_tile<E>(tm + 1 * HNM, n, M, c * 64 + f * 16 + 4 * g, valid, o);
                           float o2[4] = {s2v[f][0], s2v[f][1], s2v[f][2], s2v[f][3]};
                           st4_tile<E>(tm + 3 * HNM, n, M, c * 64 + f * 16 + 4 * g, valid, o2);
                         }
                       });
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float o[4] = {lam[db][0], lam[db][1], lam[db][2], lam[db][3]};
      st4_tile<E>(td + 0 * HND, n, D, db * 16 + 4 * g, valid, o);
      st4_tile<E>(td + 2 * HND, n, D, db * 16 + 4 * g, valid, xr[db]);
    }
    // ---- pass 1: g = s sp z rinv (z = W2^T lam) -> dz, and its share of drinv
    float drinv = 0.f;
    floatx4 wdz[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) wdz[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], z[4], dz[4];
      gnw_a<D>(w1s, L.xp, xs_w, c, l16, g, a);
      gnw_w2t<D, false>(w2s, L.mp, c, lam, lane, z);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float tv[4], dgv[4];
        tau_of<MB>(tau, 4 * c + f, g, p.has_tau, tv);
        ld4_row<E>(p.dg, b, h, t, c * 64 + f * 16 + 4 * g, valid, dgv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pre = a[f][i] * rinv - tv[i];
          const float sp = gn_slope(p.act, pre, gn_act(p.act, pre));
          const float sdg = p.s * dgv[i];
          dz[f][i] = sdg * sp * rinv;
          drinv += sdg * sp * z[f][i];
        }
        float o[4] = {dz[f][0], dz[f][1], dz[f][2], dz[f][3]};
        st4_tile<E>(tm + 0 * HNM, n, M, c * 64 + f * 16 + 4 * g, valid, o);
      }
      gnw_w2<D, false>(w2s, L.mp, c, dz, l16, g, wdz);
    }
    // ---- lam -> r, den -> (hh, xx, rq)
    floatx4 dr[D / 16], drq[D / 16], du[D / 16];
    float dhh = 0.f, dxx = 0.f;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float dlv[4];
      ld4_row<E>(p.dlam, b, h, t, db * 16 + 4 * g, valid, dlv);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float dl = p.s * dlv[i] + wdz[db][i];
        dr[db][i] = dl / den[db][i];
        const float dD = -dl * lam[db][i] / den[db][i] * p.inv_L;
        dhh += dD;
        dxx += dD * rq[db][i];
        drq[db][i] = dD;
      }
    }
    dhh = sum_g(dhh);
    dxx = sum_g(dxx);
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float dvv[4], duv[4], o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        drq[db][i] *= xx;
        o[i] = drq[db][i];
        dvv[i] = dr[db][i];
        du[db][i] = -p.s * dr[db][i];
        duv[i] = du[db][i];
      }
      st4_tile<E>(td + 3 * HND, n, D, db * 16 + 4 * g, valid, o);
      st4_row<E>(p.dv, b, h, t, db * 16 + 4 * g, valid, dvv);
      st4_tile<E>(td + 1 * HND, n, D, db * 16 + 4 * g, valid, duv);
    }
    // dpre of chunk c (with its a): sigma' dht + sigma'' dsp, dht = dh + W2^T du + 2 h dhh,
    // dsp = s dg z rinv + 2 sp rinv ((W2 o W2)^T drq) rinv; adds the chunk's share to drinv
    auto dpre_chunk = [&](int c, floatx4* a, floatx4* dpre, float& drv) {
      floatx4 z[4], ds2[4], dhu[4];
      gnw_a<D>(w1s, L.xp, xs_w, c, l16, g, a);
      gnw_w2t<D, false>(w2s, L.mp, c, lam, lane, z);
      gnw_w2t<D, true>(w2s, L.mp, c, drq, lane, ds2);
      gnw_w2t<D, false>(w2s, L.mp, c, du, lane, dhu);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float tv[4], dgv[4], dhv[4];
        tau_of<MB>(tau, 4 * c + f, g, p.has_tau, tv);
        ld4_row<E>(p.dg, b, h, t, c * 64 + f * 16 + 4 * g, valid, dgv);
        ld4_row<E>(p.dh, b, h, t, c * 64 + f * 16 + 4 * g, valid, dhv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pre = a[f][i] * rinv - tv[i];
          const float hval = gn_act(p.act, pre);
          const float sp = gn_slope(p.act, pre, hval);
          const float dsv = 2.f * sp * rinv * ds2[f][i];
          const float dsp = p.s * dgv[i] * z[f][i] * rinv + dsv * rinv;
          drv += dsv * sp;
          const float dht = dhv[i] + dhu[f][i] + 2.f * hval * dhh;
          dpre[f][i] = valid ? gn_dpre(p.act, pre, hval, dht, dsp) : 0.f;
        }
      }
    };
    // ---- pass 2: drinv from the s^2 path and from dpre . a
    float ra = 0.f;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], dpre[4];
      dpre_chunk(c, a, dpre, drinv);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ra += dpre[f][i] * a[f][i];
        if (p.has_tau) {
          float o[4] = {dpre[f][0], dpre[f][1], dpre[f][2], dpre[f][3]};
          st4_tile<E>(tm + 4 * HNM, n, M, c * 64 + f * 16 + 4 * g, valid, o);
        }
      }
    }
    drinv = sum_g(drinv + ra);
    const float c3 = drinv * rinv * rinv * rinv * p.inv_m;
    // ---- pass 3: da = dpre rinv - c3 a -> W1^T da
    floatx4 wda[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) wda[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], da[4];
      float unused = 0.f;
      dpre_chunk(c, a, da, unused);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
#pragma unroll
        for (int i = 0; i < 4; ++i) da[f][i] = da[f][i] * rinv - c3 * a[f][i];
        float o[4] = {da[f][0], da[f][1], da[f][2], da[f][3]};
        st4_tile<E>(tm + 2 * HNM, n, M, c * 64 + f * 16 + 4 * g, valid, o);
      }
      gnw_w1t<D>(w1s, L.xp, c, da, lane, wda);
    }
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float dxi[4], o[4];
      ld4_row<E>(p.dxin, b, h, t, db * 16 + 4 * g, valid, dxi);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = dxi[i] - dr[db][i] + 2.f * xr[db][i] * dxx + wda[db][i];
      st4_row<E>(p.dx, b, h, t, db * 16 + 4 * g, valid, o);
    }
  }
}

// a + correction of chunk c for the read stage (c = num or num / (mass + eps))
template <int D>
__device__ __forceinline__ void gnw_read_a(const GnReadP& p, int b, int h, int t, bool valid, const bf16* w1s, int xp,
                                           const bf16* xs_w, int c, int l16, int g, float cinv, floatx4* a) {
  gnw_a<D>(w1s, xp, xs_w, c, l16, g, a);
  if (p.corr) {
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      float cv[4];
      ld4_row<bf16>(p.num, b, h, t, c * 64 + f * 16 + 4 * g, valid, cv);
#pragma unroll
      for (int i = 0; i < 4; ++i) a[f][i] += cv[i] * cinv;
    }
  }
}

template <int D, int MB>
__device__ __forceinline__ float gnw_read_rinv(const GnReadP& p, int b, int h, int t, bool valid, const bf16* w1s,
                                               int xp, const bf16* xs_w, int l16, int g, float& cinv) {
  cinv = 1.f;
  if (p.corr == 2) cinv = valid ? 1.f / (p.mass[b * p.msb + h * p.msh + (int64_t)t * p.mst] + p.eps) : 0.f;
  float ss = 0.f;
#pragma unroll 1
  for (int c = 0; c < MB / 4; ++c) {
    floatx4 a[4];
    gnw_read_a<D>(p, b, h, t, valid, w1s, xp, xs_w, c, l16, g, cinv, a);
#pragma unroll
    for (int f = 0; f < 4; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += a[f][i] * a[f][i];
  }
  return rsqrtf(sum_g(ss) * p.inv_m + p.eps);
}

template <int D, int MB>
__global__ __launch_bounds__(256) void gn_read_fwd_wide_kernel(GnReadP p) {
  typedef bf16 E;
  constexpr int M = MB * 16;
  constexpr int NC = MB / 4;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const GnWideLayout L = gn_wide_layout(D, M, p.want_resid ? 1 : 0);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  E* w1s = base + L.w1;
  E* w2s = base + L.w2;
  stage_matrix<E>((const E*)p.w1 + (size_t)h * M * D, M, D, w1s, L.xp, tid);
  if (p.want_resid) stage_matrix<E>((const E*)p.w2 + (size_t)h * D * M, D, M, w2s, L.mp, tid);
  const float* tau = p.has_tau ? p.tau + h * M : nullptr;
  const Rows<E> qsrc = rows_of<E>(p.q, b, h);
  RowTile<E, D> ldq;
  ldq.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldq.fetch(qsrc, g0 * TT, p.T);
  for (int grp = 0; grp < p.groups; ++grp) {
    const int t0 = (g0 + grp) * TT;
    if (t0 >= p.T) break;  // uniform over the workgroup
    __syncthreads();
    ldq.store(xs, L.xp);
    if (grp + 1 < p.groups) ldq.fetch(qsrc, t0 + TT, p.T);
    __syncthreads();
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    const E* xs_w = xs + w * 16 * L.xp;
    float cinv;
    const float rinv = gnw_read_rinv<D, MB>(p, b, h, t, valid, w1s, L.xp, xs_w, l16, g, cinv);
    floatx4 u[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) u[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], hv[4];
      gnw_read_a<D>(p, b, h, t, valid, w1s, L.xp, xs_w, c, l16, g, cinv, a);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float tv[4], o[4];
        tau_of<MB>(tau, 4 * c + f, g, p.has_tau, tv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hv[f][i] = gn_act(p.act, a[f][i] * rinv - tv[i]);
          o[i] = hv[f][i];
        }
        st4_row<E>(p.h, b, h, t, c * 64 + f * 16 + 4 * g, valid, o);
      }
      if (p.want_resid) gnw_w2<D, false>(w2s, L.mp, c, hv, l16, g, u);
    }
    if (p.want_resid) {
      const E* qrow = xs + row * L.xp;
#pragma unroll
      for (int db = 0; db < D / 16; ++db) {
        float qv[4];
        ld4f<E>(qrow + db * 16 + 4 * g, qv);
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] += p.s * u[db][i];
        st4_row<E>(p.resid, b, h, t, db * 16 + 4 * g, valid, qv);
      }
    }
  }
}

template <int D, int MB>
__global__ __launch_bounds__(256) void gn_read_bwd_wide_kernel(GnReadP p) {
  typedef bf16 E;
  typedef LdsIO<E> IO;
  constexpr int M = MB * 16;
  constexpr int NC = MB / 4;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const GnWideLayout L = gn_wide_layout(D, M, p.want_resid ? 2 : 0);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* xs = base + L.xs;
  E* w1s = base + L.w1;
  E* w2ts = base + L.w2;  // W2^T [m][xp]
  stage_matrix<E>((const E*)p.w1 + (size_t)h * M * D, M, D, w1s, L.xp, tid);
  if (p.want_resid) stage_matrix<E>((const E*)p.w2t + (size_t)h * M * D, M, D, w2ts, L.xp, tid);
  const float* tau = p.has_tau ? p.tau + h * M : nullptr;
  const int64_t N = (int64_t)p.B * p.T;
  E* tm = (E*)p.tm + (int64_t)h * N * M;  // da, h (, dpre)
  E* td = (E*)p.td + (int64_t)h * N * D;  // q, s dresid
  const int64_t HNM = (int64_t)p.H * N * M, HND = (int64_t)p.H * N * D;
  const Rows<E> qsrc = rows_of<E>(p.q, b, h);
  RowTile<E, D> ldq;
  ldq.init(D, tid);
  const int g0 = blockIdx.x * p.groups;
  ldq.fetch(qsrc, g0 * TT, p.T);
  for (int grp = 0; grp < p.groups; ++grp) {
    const int t0 = (g0 + grp) * TT;
    if (t0 >= p.T) break;  // uniform over the workgroup
    __syncthreads();
    ldq.store(xs, L.xp);
    if (grp + 1 < p.groups) ldq.fetch(qsrc, t0 + TT, p.T);
    __syncthreads();
    const int row = w * 16 + l16;
    const int t = t0 + row;
    const bool valid = t < p.T;
    const int64_t n = (int64_t)b * p.T + t;
    const E* xs_w = xs + w * 16 * L.xp;
    float cinv;
    const float rinv = gnw_read_rinv<D, MB>(p, b, h, t, valid, w1s, L.xp, xs_w, l16, g, cinv);
    float dres[D / 16][4];
    floatx4 dres4[D / 16];
    const E* qrow = xs + row * L.xp;
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float qv[4], sd[4];
      ld4f<E>(qrow + db * 16 + 4 * g, qv);
      ld4_row<E>(p.dresid, b, h, t, db * 16 + 4 * g, valid && p.want_resid, dres[db]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dres4[db][i] = dres[db][i];
        sd[i] = p.s * dres[db][i];
      }
      st4_tile<E>(td + 0 * HND, n, D, db * 16 + 4 * g, valid, qv);
      st4_tile<E>(td + 1 * HND, n, D, db * 16 + 4 * g, valid, sd);
    }
    // dpre of chunk c: sigma'(pre) (dh + s W2^T dresid)
    auto dpre_chunk = [&](int c, floatx4* a, floatx4* dpre) {
      floatx4 dhr[4];
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        dhr[f] = floatx4{0.f, 0.f, 0.f, 0.f};
        if (p.want_resid) {
          const E* wrow = w2ts + (c * 64 + f * 16 + l16) * L.xp;
#pragma unroll
          for (int kk = 0; kk < D / 32; ++kk)
            dhr[f] = mma32(IO::cat(IO::ld4(wrow + 32 * kk + 4 * g), IO::ld4(wrow + 32 * kk + 16 + 4 * g)),
                           IO::from_acc(dres4[2 * kk], dres4[2 * kk + 1]), dhr[f]);
        }
      }
      gnw_read_a<D>(p, b, h, t, valid, w1s, L.xp, xs_w, c, l16, g, cinv, a);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float tv[4], dhv[4];
        tau_of<MB>(tau, 4 * c + f, g, p.has_tau, tv);
        ld4_row<E>(p.dh, b, h, t, c * 64 + f * 16 + 4 * g, valid, dhv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pre = a[f][i] * rinv - tv[i];
          const float hval = gn_act(p.act, pre);
          dpre[f][i] = valid ? gn_dpre(p.act, pre, hval, dhv[i] + p.s * dhr[f][i], 0.f) : 0.f;
        }
      }
    };
    float ra = 0.f;
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], dpre[4];
      dpre_chunk(c, a, dpre);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float tv[4], hvv[4], dpv[4];
        tau_of<MB>(tau, 4 * c + f, g, p.has_tau, tv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          hvv[i] = gn_act(p.act, a[f][i] * rinv - tv[i]);
          dpv[i] = dpre[f][i];
          ra += dpre[f][i] * a[f][i];
        }
        st4_tile<E>(tm + 1 * HNM, n, M, c * 64 + f * 16 + 4 * g, valid, hvv);
        if (p.has_tau) st4_tile<E>(tm + 2 * HNM, n, M, c * 64 + f * 16 + 4 * g, valid, dpv);
      }
    }
    ra = sum_g(ra);
    const float c3 = ra * rinv * rinv * rinv * p.inv_m;
    float dm = 0.f;
    floatx4 wda[D / 16];
#pragma unroll
    for (int db = 0; db < D / 16; ++db) wda[db] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      floatx4 a[4], da[4];
      dpre_chunk(c, a, da);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        float o[4], dn[4];
        float cv[4] = {0.f, 0.f, 0.f, 0.f};
        if (p.corr == 2) ld4_row<E>(p.num, b, h, t, c * 64 + f * 16 + 4 * g, valid, cv);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          da[f][i] = da[f][i] * rinv - c3 * a[f][i];
          o[i] = da[f][i];
          dn[i] = da[f][i] * cinv;
          dm += da[f][i] * cv[i];
        }
        st4_tile<E>(tm + 0 * HNM, n, M, c * 64 + f * 16 + 4 * g, valid, o);
        if (p.corr) st4_row<E>(p.dnum, b, h, t, c * 64 + f * 16 + 4 * g, valid, dn);
      }
      gnw_w1t<D>(w1s, L.xp, c, da, lane, wda);
    }
    if (p.corr == 2) {
      dm = sum_g(dm);
      if (g == 0 && valid) p.dmass[b * p.msb + h * p.msh + (int64_t)t * p.mst] = -dm * cinv * cinv;
    }
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = dres[db][i] + wda[db][i];
      st4_row<E>(p.dq, b, h, t, db * 16 + 4 * g, valid, o);
    }
  }
}

}  // namespace ts

namespace {

using ts::fail;

bool gn_is_wide(const ts_gn_desc* d);

int check_gn(const ts_gn_desc* d) {
  if (!d) return fail(TS_ERR_VALUE, "gn: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0) return fail(TS_ERR_VALUE, "gn: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "gn: unknown dtype");
  if (d->d != 16 && d->d != 32 && d->d != 64 && d->d != 128)
    return fail(TS_ERR_NOT_IMPLEMENTED, "gn: head width %d (16, 32, 64 or 128)", d->d);
  if (d->m < 16 || d->m % 16 || (d->m > 128 && d->m != 192 && d->m != 256 && !gn_is_wide(d)))
    return fail(TS_ERR_NOT_IMPLEMENTED,
                "gn: hidden width %d (a multiple of 16 up to 128, 192 or 256; 384 in bf16 at head widths 32, 64)", d->m);
  if (d->H > 65535 || d->B > 65535) return fail(TS_ERR_NOT_IMPLEMENTED, "gn: grid too large");
  if (d->act != TS_GN_RELU2 && d->act != TS_GN_TANH && d->act != TS_GN_SILU)
    return fail(TS_ERR_VALUE, "gn: unknown nonlinearity %d", d->act);
  if (!(d->damping > 0.f)) return fail(TS_ERR_VALUE, "gn: damping must be > 0");
  return TS_OK;
}

bool gn_stream_ok(const ts_strided& s, int vec) {
  return s.ptr == nullptr || (((uintptr_t)s.ptr & 15u) == 0 && s.sb % vec == 0 && s.sh % vec == 0 && s.st % vec == 0 &&
                              s.st <= 0x7fffffff);
}

ts::Str gn_str(const ts_strided& s) { return ts::Str{const_cast<void*>(s.ptr), s.sb, s.sh, (int)s.st}; }

typedef void (*GnKernel)(ts::GnP);

template <typename E, bool FWD, int D>
GnKernel gn_pick_m(int m) {
#define TS_GN(MB) \
  return FWD ? (GnKernel)ts::gn_write_fwd_kernel<E, D, MB> : (GnKernel)ts::gn_write_bwd_kernel<E, D, MB>;
  switch (m) {
    case 16: TS_GN(1)
    case 32: TS_GN(2)
    case 48: TS_GN(3)
    case 64: TS_GN(4)
    case 80: TS_GN(5)
    case 96: TS_GN(6)
    case 112: TS_GN(7)
    case 128: TS_GN(8)
    case 192: TS_GN(12)
    case 256: TS_GN(16)
  }
#undef TS_GN
  return nullptr;
}

template <typename E, bool FWD>
GnKernel gn_pick(int d, int m) {
  switch (d) {
    case 16: return gn_pick_m<E, FWD, 16>(m);
    case 32: return gn_pick_m<E, FWD, 32>(m);
    case 64: return gn_pick_m<E, FWD, 64>(m);
    case 128: return gn_pick_m<E, FWD, 128>(m);
  }
  return nullptr;
}

// Hidden widths the chunked kernels take (bf16, head widths 32 and 64).
bool gn_is_wide(const ts_gn_desc* d) {
  return d->dtype == TS_BF16 && (d->d == 32 || d->d == 64) && (d->m == 192 || d->m == 384);
}

template <int D>
GnKernel gn_wide_pick_d(int m, bool fwd) {
  switch (m) {
    case 192: return fwd ? (GnKernel)ts::gn_write_fwd_wide_kernel<D, 12> : (GnKernel)ts::gn_write_bwd_wide_kernel<D, 12>;
    case 384: return fwd ? (GnKernel)ts::gn_write_fwd_wide_kernel<D, 24> : (GnKernel)ts::gn_write_bwd_wide_kernel<D, 24>;
  }
  return nullptr;
}
GnKernel gn_wide_pick(const ts_gn_desc* d, bool fwd) {
  return d->d == 32 ? gn_wide_pick_d<32>(d->m, fwd) : gn_wide_pick_d<64>(d->m, fwd);
}

int gn_lds_bytes(const ts_gn_desc* d, bool fwd) {
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  const ts::GnLayout full = ts::gn_layout(es, d->d, d->m, fwd, true);
  const bool wl = full.end * es <= ts::kGnLdsMax;
  return ts::gn_layout(es, d->d, d->m, fwd, wl).end * es;
}

int gn_read_lds_bytes(const ts_gn_desc* d, bool fwd) {
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  const ts::GnLayout full = ts::gn_read_layout(es, d->d, d->m, fwd, true);
  const bool wl = full.end * es <= ts::kGnLdsMax;
  return ts::gn_read_layout(es, d->d, d->m, fwd, wl).end * es;
}

// Groups of 64 tokens per workgroup: enough workgroups to fill 256 CUs.
int gn_groups(const ts_gn_desc* d) {
  const int ngroups = (d->T + ts::TT - 1) / ts::TT;
  const int64_t slices = (int64_t)d->B * d->H;
  int per = 1;
  while (per < ngroups && slices * ((ngroups + 2 * per - 1) / (2 * per)) >= 512) per *= 2;
  return per;
}

void gn_fill(const ts_gn_desc* d, ts::GnP& p) {
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T;
  p.groups = gn_groups(d);
  p.has_tau = d->has_tau;
  p.s = d->s; p.inv_L = d->inv_depth; p.eps = d->eps; p.act = d->act; p.damp = d->damping;
  p.inv_m = 1.0f / (float)d->m;
}

int gn_launch(const ts_gn_desc* d, const ts::GnP& p, bool fwd, hipStream_t stream) {
  const bool wide = gn_is_wide(d);
  GnKernel k = wide ? gn_wide_pick(d, fwd)
               : d->dtype == TS_BF16 ? (fwd ? gn_pick<ts::bf16, true>(d->d, d->m) : gn_pick<ts::bf16, false>(d->d, d->m))
                                     : (fwd ? gn_pick<float, true>(d->d, d->m) : gn_pick<float, false>(d->d, d->m));
  if (!k) return fail(TS_ERR_NOT_IMPLEMENTED, "gn: no kernel for d=%d m=%d", d->d, d->m);
  const int lds = wide ? ts::gn_wide_layout(d->d, d->m, 1).end * 2 : gn_lds_bytes(d, fwd);
  if (lds > ts::kGnLdsMax) return fail(TS_ERR_NOT_IMPLEMENTED, "gn: tile of %d bytes exceeds LDS", lds);
  if (lds > 65536) {
    hipError_t e = ts::ensure_lds_limit((const void*)k, lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "gn: LDS request failed: %s", hipGetErrorString(e));
  }
  const int ngroups = (d->T + ts::TT - 1) / ts::TT;
  const dim3 grid((unsigned)((ngroups + p.groups - 1) / p.groups), (unsigned)d->H, (unsigned)d->B);
  hipLaunchKernelGGL(k, grid, dim3(256), lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "gn: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

typedef void (*GnReadKernel)(ts::GnReadP);

template <typename E, bool FWD, int D>
GnReadKernel gn_read_pick_m(int m) {
#define TS_GNR(MB) \
  return FWD ? (GnReadKernel)ts::gn_read_fwd_kernel<E, D, MB> : (GnReadKernel)ts::gn_read_bwd_kernel<E, D, MB>;
  switch (m) {
    case 16: TS_GNR(1)
    case 32: TS_GNR(2)
    case 48: TS_GNR(3)
    case 64: TS_GNR(4)
    case 80: TS_GNR(5)
    case 96: TS_GNR(6)
    case 112: TS_GNR(7)
    case 128: TS_GNR(8)
    case 192: TS_GNR(12)
    case 256: TS_GNR(16)
  }
#undef TS_GNR
  return nullptr;
}

template <typename E, bool FWD>
GnReadKernel gn_read_pick(int d, int m) {
  switch (d) {
    case 16: return gn_read_pick_m<E, FWD, 16>(m);
    case 32: return gn_read_pick_m<E, FWD, 32>(m);
    case 64: return gn_read_pick_m<E, FWD, 64>(m);
    case 128: return gn_read_pick_m<E, FWD, 128>(m);
  }
  return nullptr;
}

int check_gn_read(const ts_gn_read_desc* r, ts_gn_desc* d) {
  if (!r) return fail(TS_ERR_VALUE, "gn read: null descriptor");
  if (r->corr < 0 || r->corr > 2) return fail(TS_ERR_VALUE, "gn read: corr must be 0, 1 or 2");
  memset(d, 0, sizeof(*d));
  d->B = r->B; d->H = r->H; d->T = r->T; d->d = r->d; d->m = r->m; d->dtype = r->dtype; d->has_tau = r->has_tau;
  d->s = r->s; d->inv_depth = 1.f; d->eps = r->eps; d->act = r->act;
  d->damping = 1.f;  // the read stage has no Jacobi diagonal
  return check_gn(d);
}

void gn_read_fill(const ts_gn_read_desc* r, const ts_gn_desc* d, ts::GnReadP& p, const ts_strided& mass) {
  memset(&p, 0, sizeof(p));
  p.B = r->B; p.H = r->H; p.T = r->T;
  p.groups = gn_groups(d);
  p.has_tau = r->has_tau; p.corr = r->corr; p.want_resid = r->want_resid;
  p.s = r->s; p.eps = r->eps; p.inv_m = 1.0f / (float)r->m; p.act = r->act;
  p.mass = (const float*)mass.ptr;
  p.msb = mass.sb; p.msh = mass.sh; p.mst = mass.st;
}

template <int D>
GnReadKernel gn_read_wide_pick_d(int m, bool fwd) {
  switch (m) {
    case 192: return fwd ? (GnReadKernel)ts::gn_read_fwd_wide_kernel<D, 12> : (GnReadKernel)ts::gn_read_bwd_wide_kernel<D, 12>;
    case 384: return fwd ? (GnReadKernel)ts::gn_read_fwd_wide_kernel<D, 24> : (GnReadKernel)ts::gn_read_bwd_wide_kernel<D, 24>;
  }
  return nullptr;
}

int gn_read_launch(const ts_gn_desc* d, const ts::GnReadP& p, bool fwd, hipStream_t stream) {
  const bool wide = gn_is_wide(d);
  GnReadKernel k =
      wide ? (d->d == 32 ? gn_read_wide_pick_d<32>(d->m, fwd) : gn_read_wide_pick_d<64>(d->m, fwd))
      : d->dtype == TS_BF16 ? (fwd ? gn_read_pick<ts::bf16, true>(d->d, d->m) : gn_read_pick<ts::bf16, false>(d->d, d->m))
                            : (fwd ? gn_read_pick<float, true>(d->d, d->m) : gn_read_pick<float, false>(d->d, d->m));
  if (!k) return fail(TS_ERR_NOT_IMPLEMENTED, "gn read: no kernel for d=%d m=%d", d->d, d->m);
  const int lds = wide ? ts::gn_wide_layout(d->d, d->m, p.want_resid ? (fwd ? 1 : 2) : 0).end * 2
                       : gn_read_lds_bytes(d, fwd);
  if (lds > ts::kGnLdsMax) return fail(TS_ERR_NOT_IMPLEMENTED, "gn read: tile of %d bytes exceeds LDS", lds);
  if (lds > 65536) {
    hipError_t e = ts::ensure_lds_limit((const void*)k, lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "gn read: LDS request failed: %s", hipGetErrorString(e));
  }
  const int ngroups = (d->T + ts::TT - 1) / ts::TT;
  const dim3 grid((unsigned)((ngroups + p.groups - 1) / p.groups), (unsigned)d->H, (unsigned)d->B);
  hipLaunchKernelGGL(k, grid, dim3(256), lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "gn read: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_gn_write_fwd(const ts_gn_desc* d, const ts_gn_io* io, hipStream_t stream) {
  int rc = check_gn(d);
  if (rc) return rc;
  if (!io || !io->x.ptr || !io->v.ptr || !io->w1 || !io->w2 || !io->w2t || !io->h.ptr || !io->lam.ptr || !io->g.ptr)
    return fail(TS_ERR_VALUE, "gn: missing tensors");
  if (d->has_tau && !io->tau) return fail(TS_ERR_VALUE, "gn: missing tau");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  for (const ts_strided* s : {&io->x, &io->v, &io->h, &io->lam, &io->g})
    if (!gn_stream_ok(*s, vec)) return fail(TS_ERR_VALUE, "gn: streams need 16-byte aligned rows");
  if (d->T == 0) return TS_OK;
  ts::GnP p;
  gn_fill(d, p);
  p.x = gn_str(io->x); p.v = gn_str(io->v);
  p.h = gn_str(io->h); p.lam = gn_str(io->lam); p.g = gn_str(io->g);
  p.w1 = io->w1; p.w2 = io->w2; p.w2t = io->w2t; p.tau = io->tau;
  return gn_launch(d, p, true, stream);
}

int ts_gn_write_bwd(const ts_gn_desc* d, const ts_gn_bwd_io* io, hipStream_t stream) {
  int rc = check_gn(d);
  if (rc) return rc;
  if (!io || !io->x.ptr || !io->v.ptr || !io->w1 || !io->w2 || !io->w1t || !io->w2t || !io->dx.ptr || !io->dv.ptr ||
      !io->tiles_m || !io->tiles_d)
    return fail(TS_ERR_VALUE, "gn bwd: missing tensors");
  if (d->has_tau && !io->tau) return fail(TS_ERR_VALUE, "gn bwd: missing tau");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  for (const ts_strided* s : {&io->x, &io->v, &io->dh, &io->dlam, &io->dg, &io->dx_in, &io->dx, &io->dv})
    if (!gn_stream_ok(*s, vec)) return fail(TS_ERR_VALUE, "gn bwd: streams need 16-byte aligned rows");
  if (d->T == 0) return TS_OK;
  ts::GnP p;
  gn_fill(d, p);
  p.x = gn_str(io->x); p.v = gn_str(io->v);
  p.dh = gn_str(io->dh); p.dlam = gn_str(io->dlam); p.dg = gn_str(io->dg); p.dxin = gn_str(io->dx_in);
  p.dx = gn_str(io->dx); p.dv = gn_str(io->dv);
  p.w1 = io->w1; p.w2 = io->w2; p.w1t = io->w1t; p.w2t = io->w2t; p.tau = io->tau;
  p.tm = io->tiles_m; p.td = io->tiles_d;
  return gn_launch(d, p, false, stream);
}


int ts_gn_read_fwd(const ts_gn_read_desc* r, const ts_gn_read_io* io, hipStream_t stream) {
  ts_gn_desc d;
  int rc = check_gn_read(r, &d);
  if (rc) return rc;
  if (!io || !io->q.ptr || !io->w1 || !io->h.ptr) return fail(TS_ERR_VALUE, "gn read: missing tensors");
  if (r->want_resid && (!io->w2 || !io->resid.ptr)) return fail(TS_ERR_VALUE, "gn read: missing W2 or resid");
  if (r->corr && !io->num.ptr) return fail(TS_ERR_VALUE, "gn read: missing num");
  if (r->corr == 2 && !io->mass.ptr) return fail(TS_ERR_VALUE, "gn read: missing mass");
  if (r->has_tau && !io->tau) return fail(TS_ERR_VALUE, "gn read: missing tau");
  const int vec = r->dtype == TS_BF16 ? 8 : 4;
  for (const ts_strided* s : {&io->q, &io->num, &io->h, &io->resid})
    if (!gn_stream_ok(*s, vec)) return fail(TS_ERR_VALUE, "gn read: streams need 16-byte aligned rows");
  if (r->T == 0) return TS_OK;
  ts::GnReadP p;
  gn_read_fill(r, &d, p, io->mass);
  p.q = gn_str(io->q); p.num = gn_str(io->num); p.h = gn_str(io->h); p.resid = gn_str(io->resid);
  p.w1 = io->w1; p.w2 = io->w2; p.tau = io->tau;
  return gn_read_launch(&d, p, true, stream);
}

int ts_gn_read_bwd(const ts_gn_read_desc* r, const ts_gn_read_bwd_io* io, hipStream_t stream) {
  ts_gn_desc d;
  int rc = check_gn_read(r, &d);
  if (rc) return rc;
  if (!io || !io->q.ptr || !io->w1 || !io->w1t || !io->dq.ptr || !io->tiles_m || !io->tiles_d)
    return fail(TS_ERR_VALUE, "gn read bwd: missing tensors");
  if (r->want_resid && !io->w2t) return fail(TS_ERR_VALUE, "gn read bwd: missing W2^T");
  if (r->corr && (!io->num.ptr || !io->dnum.ptr)) return fail(TS_ERR_VALUE, "gn read bwd: missing num");
  if (r->corr == 2 && (!io->mass.ptr || !io->dmass)) return fail(TS_ERR_VALUE, "gn read bwd: missing mass");
  if (r->has_tau && !io->tau) return fail(TS_ERR_VALUE, "gn read bwd: missing tau");
  const int vec = r->dtype == TS_BF16 ? 8 : 4;
  for (const ts_strided* s : {&io->q, &io->num, &io->dh, &io->dresid, &io->dq, &io->dnum})
    if (!gn_stream_ok(*s, vec)) return fail(TS_ERR_VALUE, "gn read bwd: streams need 16-byte aligned rows");
  if (r->T == 0) return TS_OK;
  ts::GnReadP p;
  gn_read_fill(r, &d, p, io->mass);
  p.q = gn_str(io->q); p.num = gn_str(io->num);
  p.dh = gn_str(io->dh); p.dresid = gn_str(io->dresid); p.dq = gn_str(io->dq); p.dnum = gn_str(io->dnum);
  p.dmass = io->dmass;
  p.w1 = io->w1; p.w1t = io->w1t; p.w2t = io->w2t; p.tau = io->tau;
  p.tm = io->tiles_m; p.td = io->tiles_d;
  return gn_read_launch(&d, p, false, stream);
}

}  // extern "C"
