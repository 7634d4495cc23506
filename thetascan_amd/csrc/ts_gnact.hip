// Per-row GN hidden activation with its Jacobian scales (gfx950), forward
// and backward: the nonlinear core of one block of a GN fast network.
//
//   elementwise act (relu2, silu, tanh):
//     ra = (mean a^2 + eps)^-1/2,  z = a ra - tau,  h = sigma(z),
//     sa = sigma'(z) ra
//   SwiGLU (engine.py:117-158 with cfg.nonlin == "swiglu"):
//     za = a ra,  zb = b rb,  h = silu(zb) za,
//     sa = silu(zb) ra,  sb = za silu'(zb) rb
//
// sa (and sb) are the per-feature scales by which the reference multiplies
// W2 in the Jacobian-transpose payload and the Gauss-Newton diagonal
// (engine.py:180-255: _g_from_lambda, _w2s, _lambda_solve), so a caller forms
// g = s sa (W2^T lam) and rowsq = (W2 o W2)(sa^2 [+ sb^2]) with plain GEMMs.
//
// Backward (dh, dsa, dsb given; a missing one reads as zeros):
//   dz  = sigma'(z) dh + sigma''(z) ra dsa
//   dra = sum_j sigma'(z_j) dsa_j + sum_j dz_j a_j
//   da  = ra dz - dra ra^3 a / m                   (dtau = -sum_tokens dz)
// and for SwiGLU
//   dza = silu(zb) dh + silu'(zb) rb dsb
//   dzb = silu'(zb) za dh + silu'(zb) ra dsa + za silu''(zb) rb dsb
//   dra = sum silu(zb) dsa + sum dza a,  drb = sum za silu'(zb) dsb + sum dzb b
//   da  = ra dza - dra ra^3 a / m,  db = rb dzb - drb rb^3 b / m.
//
// One thread owns one token row and walks it in 16-byte vectors (three
// passes in the backward: the RMS, the row sums, the outputs), so any width
// that is a multiple of the vector runs without holding the row in
// registers.

#include "ts_common.h"
#include "ts_gn_act.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct GnActP {
  int T, m, act, has_tau;
  float eps, inv_m;
  ts_strided a, b, h, sa, sb, dh, dsa, dsb, da, db, dz;
  const float* tau;  // [H, m]
};

template <typename E>
__device__ __forceinline__ const E* gnact_row(const ts_strided& s, int b, int h, int t) {
  return (const E*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st;
}

template <typename E>
__device__ __forceinline__ void gnact_ld(const ts_strided& s, int b, int h, int t, int j, float* o) {
  constexpr int VEC = 16 / (int)sizeof(E);
  if (!s.ptr) {
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[e] = 0.f;
    return;
  }
  Vec16<E> u;
  u.raw = *(const uint4*)(gnact_row<E>(s, b, h, t) + j);
#pragma unroll
  for (int e = 0; e < VEC; ++e) o[e] = tof(u.e[e]);
}

template <typename E>
__device__ __forceinline__ void gnact_st(const ts_strided& s, int b, int h, int t, int j, const float* v) {
  constexpr int VEC = 16 / (int)sizeof(E);
  if (!s.ptr) return;
  Vec16<E> u;
#pragma unroll
  for (int e = 0; e < VEC; ++e) u.e[e] = cvt<E>(v[e]);
  *(uint4*)(const_cast<E*>(gnact_row<E>(s, b, h, t)) + j) = u.raw;
}

// Inverse RMS of a row.
template <typename E>
__device__ __forceinline__ float gnact_rinv(const GnActP& p, const ts_strided& s, int b, int h, int t) {
  constexpr int VEC = 16 / (int)sizeof(E);
  float ss = 0.f;
  for (int j = 0; j < p.m; j += VEC) {
    float x[VEC];
    gnact_ld<E>(s, b, h, t, j, x);
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss += x[e] * x[e];
  }
  return rsqrtf(ss * p.inv_m + p.eps);
}

__device__ __forceinline__ float silu_d2(float pre) { return gn_dpre(TS_GN_SILU, pre, 0.f, 0.f, 1.f); }

template <typename E>
__global__ __launch_bounds__(256) void gnact_fwd_kernel(GnActP p) {
  constexpr int VEC = 16 / (int)sizeof(E);
  const int h = blockIdx.y, b = blockIdx.z;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= p.T) return;
  const bool glu = p.act == TS_GN_SWIGLU;
  const float ra = gnact_rinv<E>(p, p.a, b, h, t);
  const float rb = glu ? gnact_rinv<E>(p, p.b, b, h, t) : 0.f;
  for (int j = 0; j < p.m; j += VEC) {
    float x[VEC], y[VEC], hv[VEC], s1[VEC], s2[VEC];
    gnact_ld<E>(p.a, b, h, t, j, x);
    if (glu) {
      gnact_ld<E>(p.b, b, h, t, j, y);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float za = x[e] * ra, zb = y[e] * rb;
        const float sg = gn_act(TS_GN_SILU, zb);
        hv[e] = sg * za;
        s1[e] = sg * ra;
        s2[e] = za * gn_slope(TS_GN_SILU, zb, sg) * rb;
      }
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float z = x[e] * ra - (p.has_tau ? p.tau[h * p.m + j + e] : 0.f);
        hv[e] = gn_act(p.act, z);
        s1[e] = gn_slope(p.act, z, hv[e]) * ra;
      }
    }
    gnact_st<E>(p.h, b, h, t, j, hv);
    gnact_st<E>(p.sa, b, h, t, j, s1);
    if (glu) gnact_st<E>(p.sb, b, h, t, j, s2);
  }
}

// One vector of the backward chain: dz (dza, dzb) of features j .. j+VEC-1,
// and their shares of the row sums dra, drb.
template <typename E>
__device__ __forceinline__ void gnact_dz(const GnActP& p, int b, int h, int t, int j, float ra, float rb,
                                         float* x, float* y, float* dza, float* dzb, float& dra, float& drb) {
  constexpr int VEC = 16 / (int)sizeof(E);
  float dh[VEC], ds1[VEC], ds2[VEC];
  gnact_ld<E>(p.a, b, h, t, j, x);
  gnact_ld<E>(p.dh, b, h, t, j, dh);
  gnact_ld<E>(p.dsa, b, h, t, j, ds1);
  if (p.act == TS_GN_SWIGLU) {
    gnact_ld<E>(p.b, b, h, t, j, y);
    gnact_ld<E>(p.dsb, b, h, t, j, ds2);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float za = x[e] * ra, zb = y[e] * rb;
      const float sg = gn_act(TS_GN_SILU, zb);
      const float d1 = gn_slope(TS_GN_SILU, zb, sg);
      const float d2 = silu_d2(zb);
      dza[e] = sg * dh[e] + d1 * rb * ds2[e];
      dzb[e] = d1 * za * dh[e] + d1 * ra * ds1[e] + za * d2 * rb * ds2[e];
      dra += sg * ds1[e] + dza[e] * x[e];
      drb += za * d1 * ds2[e] + dzb[e] * y[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float z = x[e] * ra - (p.has_tau ? p.tau[h * p.m + j + e] : 0.f);
      const float hv = gn_act(p.act, z);
      dza[e] = gn_dpre(p.act, z, hv, dh[e], ra * ds1[e]);
      dra += gn_slope(p.act, z, hv) * ds1[e] + dza[e] * x[e];
    }
  }
}

template <typename E>
__global__ __launch_bounds__(256) void gnact_bwd_kernel(GnActP p) {
  constexpr int VEC = 16 / (int)sizeof(E);
  const int h = blockIdx.y, b = blockIdx.z;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= p.T) return;
  const bool glu = p.act == TS_GN_SWIGLU;
  const float ra = gnact_rinv<E>(p, p.a, b, h, t);
  const float rb = glu ? gnact_rinv<E>(p, p.b, b, h, t) : 0.f;
  float dra = 0.f, drb = 0.f;
  for (int j = 0; j < p.m; j += VEC) {
    float x[VEC], y[VEC], dza[VEC], dzb[VEC];
    gnact_dz<E>(p, b, h, t, j, ra, rb, x, y, dza, dzb, dra, drb);
  }
  const float ca = dra * ra * ra * ra * p.inv_m, cb = drb * rb * rb * rb * p.inv_m;
  for (int j = 0; j < p.m; j += VEC) {
    float x[VEC], y[VEC], dza[VEC], dzb[VEC], o[VEC];
    float unused_a = 0.f, unused_b = 0.f;
    gnact_dz<E>(p, b, h, t, j, ra, rb, x, y, dza, dzb, unused_a, unused_b);
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[e] = ra * dza[e] - ca * x[e];
    gnact_st<E>(p.da, b, h, t, j, o);
    if (glu) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = rb * dzb[e] - cb * y[e];
      gnact_st<E>(p.db, b, h, t, j, o);
    } else {
      gnact_st<E>(p.dz, b, h, t, j, dza);
    }
  }
}

}  // namespace ts

namespace {

using ts::fail;

bool gnact_rows(const ts_strided& s, int es, bool required) {
  if (!s.ptr) return !required;
  return ((uintptr_t)s.ptr & 15) == 0 && (s.sb * es) % 16 == 0 && (s.sh * es) % 16 == 0 && (s.st * es) % 16 == 0;
}

int check_gnact(const ts_gn_act_desc* d) {
  if (!d) return fail(TS_ERR_VALUE, "gn act: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0 || d->m < 1) return fail(TS_ERR_VALUE, "gn act: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "gn act: unknown dtype");
  if (d->act != TS_GN_RELU2 && d->act != TS_GN_TANH && d->act != TS_GN_SILU && d->act != TS_GN_SWIGLU)
    return fail(TS_ERR_VALUE, "gn act: unknown nonlinearity %d", d->act);
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  if (d->m % vec) return fail(TS_ERR_NOT_IMPLEMENTED, "gn act: width %d is not a multiple of %d", d->m, vec);
  if (d->act == TS_GN_SWIGLU && d->has_tau) return fail(TS_ERR_VALUE, "gn act: SwiGLU takes no threshold");
  if (d->H > 65535 || d->B > 65535) return fail(TS_ERR_NOT_IMPLEMENTED, "gn act: too many heads or batches");
  return TS_OK;
}

void fill_gnact(const ts_gn_act_desc* d, const float* tau, ts::GnActP& p) {
  memset(&p, 0, sizeof(p));
  p.T = d->T; p.m = d->m; p.act = d->act; p.has_tau = d->has_tau ? 1 : 0;
  p.eps = d->eps; p.inv_m = 1.0f / (float)d->m;
  p.tau = tau;
}

int gnact_run(const ts_gn_act_desc* d, const ts::GnActP& p, bool bwd, hipStream_t stream) {
  if ((int64_t)d->B * d->T == 0) return TS_OK;
  const dim3 grid((unsigned)((d->T + 255) / 256), (unsigned)d->H, (unsigned)d->B);
  if (d->dtype == TS_BF16) {
    if (bwd) hipLaunchKernelGGL(ts::gnact_bwd_kernel<ts::bf16>, grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(ts::gnact_fwd_kernel<ts::bf16>, grid, dim3(256), 0, stream, p);
  } else {
    if (bwd) hipLaunchKernelGGL(ts::gnact_bwd_kernel<float>, grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(ts::gnact_fwd_kernel<float>, grid, dim3(256), 0, stream, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "gn act: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_gn_act_fwd(const ts_gn_act_desc* d, ts_strided a, ts_strided b, const float* tau, ts_strided h,
                  ts_strided sa, ts_strided sb, hipStream_t stream) {
  int rc = check_gnact(d);
  if (rc) return rc;
  const bool glu = d->act == TS_GN_SWIGLU;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!gnact_rows(a, es, true) || !gnact_rows(b, es, glu) || !gnact_rows(h, es, true) || !gnact_rows(sa, es, false) ||
      !gnact_rows(sb, es, false))
    return fail(TS_ERR_VALUE, "gn act: rows must be present and 16-byte aligned");
  if (d->has_tau && !tau) return fail(TS_ERR_VALUE, "gn act: missing tau");
  if (!glu && sb.ptr) return fail(TS_ERR_VALUE, "gn act: sb belongs to SwiGLU");
  ts::GnActP p;
  fill_gnact(d, tau, p);
  p.a = a; p.b = glu ? b : ts_strided{nullptr, 0, 0, 0}; p.h = h; p.sa = sa; p.sb = sb;
  return gnact_run(d, p, false, stream);
}

int ts_gn_act_bwd(const ts_gn_act_desc* d, ts_strided a, ts_strided b, const float* tau, ts_strided dh,
                  ts_strided dsa, ts_strided dsb, ts_strided da, ts_strided db, ts_strided dz, hipStream_t stream) {
  int rc = check_gnact(d);
  if (rc) return rc;
  const bool glu = d->act == TS_GN_SWIGLU;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!gnact_rows(a, es, true) || !gnact_rows(b, es, glu) || !gnact_rows(dh, es, false) ||
      !gnact_rows(dsa, es, false) || !gnact_rows(dsb, es, false) || !gnact_rows(da, es, true) ||
      !gnact_rows(db, es, glu) || !gnact_rows(dz, es, false))
    return fail(TS_ERR_VALUE, "gn act bwd: rows must be present and 16-byte aligned");
  if (d->has_tau && !tau) return fail(TS_ERR_VALUE, "gn act: missing tau");
  if (!glu && (dsb.ptr || db.ptr)) return fail(TS_ERR_VALUE, "gn act bwd: dsb and db belong to SwiGLU");
  if (glu && dz.ptr) return fail(TS_ERR_VALUE, "gn act bwd: SwiGLU has no threshold gradient");
  ts::GnActP p;
  fill_gnact(d, tau, p);
  p.a = a; p.dh = dh; p.dsa = dsa; p.da = da; p.dz = dz;
  if (glu) {
    p.b = b; p.dsb = dsb; p.db = db;
  }
  return gnact_run(d, p, true, stream);
}

}  // extern "C"
