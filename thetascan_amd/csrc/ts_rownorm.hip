// Row RMSNorm with an optional half-split rotary turn and per-head gain, for
// the hybrid language model around the ThetaScan layers (gfx950).
//
// Per row x [W] (a token of one head, or a token of the residual stream):
//
//   r = (mean(x^2) + eps)^-1/2,   n = x r
//   y = g_h R_t(n)    R_t: (n1, n2) -> (n1 c + n2 s, n2 c - n1 s) on the
//                     halves n1 = n[:W/2], n2 = n[W/2:] with the position's
//                     phases c = cos[t], s = sin[t] (when rotating)
//
// in fp32 with one rounding at the store; r per row is kept for the
// backward:
//
//   dn = g_h R_t^T(dy),  R^T: (d1, d2) -> (d1 c - d2 s, d1 s + d2 c)
//   dx = r dn - x r^3 sum(dn x) / W,   dg_h = sum over the head's rows of
//   <dy, R_t(n)> (one fp32 sum per row; the caller adds the rows)
//
// Lane layout: eight consecutive features per lane (one 16-byte load of
// bf16, two of fp32), W / 8 lanes per row (a power of two up to 64), so a
// row's sums are xor butterflies inside the row's lanes and a lane's rotary
// partner (the other half) is the lane W / 16 away.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct RowNormP {
  int B, H, T, W, rope, lanes;  // lanes per row = W / 8
  float eps;
  ts_strided x, dy;             // [B,H,T,W] views (feature axis contiguous)
  void* y;                      // out: contiguous [B,H,T,W]
  void* dx;                     // out: contiguous [B,H,T,W]
  float* rstd;                  // [B*H*T]
  float* dg_row;                // [B*H*T] or null
  const float* cos;             // [T, W/2]
  const float* sin;
  const float* gain;            // [H] or null
};

template <typename E>
__device__ __forceinline__ void rn_ld8(const E* p, float* v) {
  if constexpr (sizeof(E) == 2) {
    const uint4 r = *(const uint4*)p;
    const bf16x8 b = __builtin_bit_cast(bf16x8, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)b[e];
  } else {
    const floatx4 a = *(const floatx4*)p, b = *(const floatx4*)(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[e];
      v[4 + e] = b[e];
    }
  }
}

template <typename E>
__device__ __forceinline__ void rn_st8(E* p, const float* v) {
  if constexpr (sizeof(E) == 2) {
    bf16x8 b;
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = (bf16)v[e];
    *(uint4*)p = __builtin_bit_cast(uint4, b);
  } else {
    *(floatx4*)p = floatx4{v[0], v[1], v[2], v[3]};
    *(floatx4*)(p + 4) = floatx4{v[4], v[5], v[6], v[7]};
  }
}

// Sum over the `lanes` lanes of a row (adjacent, aligned lanes of one wave).
__device__ __forceinline__ float rn_row_sum(float s, int lanes) {
  for (int o = 1; o < lanes; o <<= 1) s += __shfl_xor(s, o, 64);
  return s;
}

struct RnRow {
  int64_t r;  // row index b*H*T + h*T + t
  int b, h, t, c0;
  bool valid;
};

__device__ __forceinline__ RnRow rn_row(const RowNormP& p) {
  RnRow w;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows = (int64_t)p.B * p.H * p.T;
  w.r = idx / p.lanes;
  w.c0 = (int)(idx - w.r * p.lanes) * 8;
  w.valid = w.r < rows;
  const int64_t rr = w.valid ? w.r : 0;
  w.t = (int)(rr % p.T);
  const int64_t bh = rr / p.T;
  w.h = (int)(bh % p.H);
  w.b = (int)(bh / p.H);
  return w;
}

// The rotary turn of this lane's eight features given the partner lane's
// (the other half of the row); `inverse` applies R^T.
__device__ __forceinline__ void rn_rotate(const RowNormP& p, const RnRow& w, const float* own, const float* other,
                                          bool inverse, float* out) {
  const int half = p.W / 2;
  const bool first = w.c0 < half;
  const int j0 = first ? w.c0 : w.c0 - half;
  const float* cr = p.cos + (int64_t)w.t * half + j0;
  const float* sr = p.sin + (int64_t)w.t * half + j0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c = cr[e], s = sr[e];
    // forward: first half n1 c + n2 s, second half n2 c - n1 s;
    // inverse: first half d1 c - d2 s, second half d1 s + d2 c
    const float sgn = first != inverse ? 1.f : -1.f;
    out[e] = own[e] * c + sgn * other[e] * s;
  }
}

template <typename E>
__global__ __launch_bounds__(256) void rownorm_fwd_kernel(RowNormP p) {
  const RnRow w = rn_row(p);
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (w.valid) rn_ld8<E>((const E*)p.x.ptr + w.b * p.x.sb + w.h * p.x.sh + (int64_t)w.t * p.x.st + w.c0, v);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  ss = rn_row_sum(ss, p.lanes);
  const float r = rsqrtf(ss / (float)p.W + p.eps);
  float n[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = v[e] * r;
  float o[8];
  if (p.rope) {
    float other[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) other[e] = __shfl_xor(n[e], p.lanes / 2, 64);
    rn_rotate(p, w, n, other, false, o);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = n[e];
  }
  const float g = p.gain ? p.gain[w.h] : 1.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] *= g;
  if (w.valid) {
    rn_st8<E>((E*)p.y + w.r * p.W + w.c0, o);
    if (w.c0 == 0) p.rstd[w.r] = r;
  }
}

template <typename E>
__global__ __launch_bounds__(256) void rownorm_bwd_kernel(RowNormP p) {
  const RnRow w = rn_row(p);
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, d[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float r = 0.f;
  if (w.valid) {
    rn_ld8<E>((const E*)p.x.ptr + w.b * p.x.sb + w.h * p.x.sh + (int64_t)w.t * p.x.st + w.c0, v);
    rn_ld8<E>((const E*)p.dy.ptr + w.b * p.dy.sb + w.h * p.dy.sh + (int64_t)w.t * p.dy.st + w.c0, d);
    r = p.rstd[w.r];
  }
  const float g = p.gain ? p.gain[w.h] : 1.f;
  float n[8], dn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) n[e] = v[e] * r;
  float dg = 0.f;
  if (p.rope) {
    float other[8], rn[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) other[e] = __shfl_xor(n[e], p.lanes / 2, 64);
    rn_rotate(p, w, n, other, false, rn);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dg += d[e] * rn[e];
      other[e] = __shfl_xor(d[e], p.lanes / 2, 64);
    }
    rn_rotate(p, w, d, other, true, dn);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dg += d[e] * n[e];
      dn[e] = d[e];
    }
  }
  float dot = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    dn[e] *= g;
    dot += dn[e] * v[e];
  }
  dot = rn_row_sum(dot, p.lanes);
  dg = rn_row_sum(dg, p.lanes);
  const float c3 = r * r * r * dot / (float)p.W;
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = r * dn[e] - c3 * v[e];
  if (w.valid) {
    rn_st8<E>((E*)p.dx + w.r * p.W + w.c0, o);
    if (p.dg_row && w.c0 == 0) p.dg_row[w.r] = dg;
  }
}

}  // namespace ts

namespace {

using ts::fail;

int rn_prepare(const ts_rownorm_desc* d, ts_strided x, const float* cos, const float* sin, ts::RowNormP* p) {
  if (!d || d->B < 1 || d->H < 1 || d->T < 0) return fail(TS_ERR_VALUE, "row norm: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "row norm: unknown dtype");
  const int lanes = d->W / 8;
  if (d->W % 8 || lanes < 1 || lanes > 64 || (lanes & (lanes - 1)))
    return fail(TS_ERR_NOT_IMPLEMENTED, "row norm: width %d (8, 16, 32, ... 512)", d->W);
  if (d->rope && (lanes < 2 || !cos || !sin))
    return fail(TS_ERR_VALUE, "row norm: the rotary turn needs a width of at least 16 and its phase tables");
  if (!(d->eps >= 0.f)) return fail(TS_ERR_VALUE, "row norm: eps must be >= 0");
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!x.ptr || ((uintptr_t)x.ptr % 16) || (x.sb * es) % 16 || (x.sh * es) % 16 || (x.st * es) % 16)
    return fail(TS_ERR_VALUE, "row norm: rows must be 16-byte aligned");
  memset(p, 0, sizeof(*p));
  p->B = d->B; p->H = d->H; p->T = d->T; p->W = d->W; p->rope = d->rope ? 1 : 0; p->lanes = lanes;
  p->eps = d->eps;
  p->x = x;
  p->cos = cos;
  p->sin = sin;
  return TS_OK;
}

template <typename E, bool FWD>
int rn_launch(const ts::RowNormP& p, hipStream_t stream) {
  const int64_t threads = (int64_t)p.B * p.H * p.T * p.lanes;
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (FWD) hipLaunchKernelGGL((ts::rownorm_fwd_kernel<E>), grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL((ts::rownorm_bwd_kernel<E>), grid, dim3(256), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "row norm: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace

extern "C" {

int ts_rownorm_fwd(const ts_rownorm_desc* d, ts_strided x, const float* cos, const float* sin, const float* gain,
                   void* y, float* rstd, hipStream_t stream) {
  ts::RowNormP p;
  int rc = rn_prepare(d, x, cos, sin, &p);
  if (rc) return rc;
  if (!y || !aligned16(y) || !rstd) return fail(TS_ERR_VALUE, "row norm: missing or unaligned output");
  if (d->T == 0) return TS_OK;
  p.y = y;
  p.rstd = rstd;
  p.gain = gain;
  return d->dtype == TS_BF16 ? rn_launch<ts::bf16, true>(p, stream) : rn_launch<float, true>(p, stream);
}

int ts_rownorm_bwd(const ts_rownorm_desc* d, ts_strided x, ts_strided dy, const float* cos, const float* sin,
                   const float* gain, const float* rstd, void* dx, float* dg_row, hipStream_t stream) {
  ts::RowNormP p;
  int rc = rn_prepare(d, x, cos, sin, &p);
  if (rc) return rc;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!dy.ptr || !aligned16(dy.ptr) || (dy.sb * es) % 16 || (dy.sh * es) % 16 || (dy.st * es) % 16)
    return fail(TS_ERR_VALUE, "row norm: dy rows must be 16-byte aligned");
  if (!dx || !aligned16(dx) || !rstd) return fail(TS_ERR_VALUE, "row norm: missing or unaligned dx / rstd");
  if (d->T == 0) return TS_OK;
  p.dy = dy;
  p.dx = dx;
  p.rstd = const_cast<float*>(rstd);
  p.gain = gain;
  p.dg_row = dg_row;
  return d->dtype == TS_BF16 ? rn_launch<ts::bf16, false>(p, stream) : rn_launch<float, false>(p, stream);
}

}  // extern "C"
