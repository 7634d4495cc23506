// Fused write-side feature map for gfx950 (forward and backward).
//
// One workgroup (4 waves) owns 64 tokens of one (batch, head).  Row passes
// use four threads per token; the two small GEMMs of the tile (a = xn W1^T
// and base = h W2^T, or their transposes in the backward) run on MFMA from
// LDS-staged operands.  Reference chain replaced: block.py:595-618 (input
// RoPE, L2 norm), engine.py:117-158 (_block_forward: W1, RMSNorm, threshold,
// feature map, W2), kernel_features.py:73-135 (softmax partition / ReLU^2
// ridge), engine.py:74-86 (feature RoPE) and the base term of
// engine.py:522-528.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct FeatP {
  int B, H, T, m, in_rot, feat_rot, has_tau, kind;
  float gain, s, eps;
  ts_strided x, phi, resid;
  const void* w1;
  const void* w2;
  const void* w1t;
  const void* w2t;
  const float* tau;
  const float* in_cos;
  const float* in_sin;
  const float* f_cos;
  const float* f_sin;
  ts_strided dphi, dresid, dx, da, xn, h, dtau;
};

constexpr int TT = 64;  // tokens per workgroup

__device__ __forceinline__ float red4_sum(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  return v;
}
__device__ __forceinline__ float red4_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 1, 64));
  v = fmaxf(v, __shfl_xor(v, 2, 64));
  return v;
}

template <typename E>
__device__ __forceinline__ void load_row(const E* src, float* dst, int n, bool valid) {
  for (int i = 0; i < n; ++i) dst[i] = valid ? tof(src[i]) : 0.0f;
}

// Four-element store (8 bytes for bf16, 16 for fp32).
template <typename E>
__device__ __forceinline__ void store4(E* dst, float a, float b, float c, float d) {
  LdsIO<E>::st4(dst, a, b, c, d);
}

// out[rows 64][cols 16*nb] = A[64 x K] * B^T where B is [ncols x K] row-major
// (global), A row-major in LDS.  Blocks are distributed over the 4 waves.
template <typename E, int K>
__device__ __forceinline__ void tile_gemm_nt(const E* A, int apitch, const E* Bg, int ncols,
                                             float* out, int opitch, int w, int l16, int g) {
  typedef LdsIO<E> IO;
  const int nblk = 4 * (ncols / 16);
  for (int blk = w; blk < nblk; blk += 4) {
    const int rb = blk & 3, cb = blk >> 2;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const E* arow = A + (rb * 16 + l16) * apitch;
    const E* brow = Bg + (size_t)(cb * 16 + l16) * K;
#pragma unroll
    for (int kk = 0; kk < K / 32; ++kk)
      acc = mma32(IO::ld8(arow + kk * 32 + 8 * g), IO::ld8(brow + kk * 32 + 8 * g), acc);
    if (K % 32)
      acc = mma16(IO::ld4(arow + (K / 32) * 32 + 4 * g), IO::ld4(brow + (K / 32) * 32 + 4 * g), acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(rb * 16 + 4 * g + i) * opitch + cb * 16 + l16] = acc[i];
  }
}

// Same with a runtime contraction length k (multiple of 16).
template <typename E>
__device__ __forceinline__ void tile_gemm_nt_rt(const E* A, int apitch, const E* Bg, int k, int ncols,
                                                float* out, int opitch, int w, int l16, int g) {
  typedef LdsIO<E> IO;
  const int nblk = 4 * (ncols / 16);
  const int k32 = k / 32;
  for (int blk = w; blk < nblk; blk += 4) {
    const int rb = blk & 3, cb = blk >> 2;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const E* arow = A + (rb * 16 + l16) * apitch;
    const E* brow = Bg + (size_t)(cb * 16 + l16) * k;
    for (int kk = 0; kk < k32; ++kk)
      acc = mma32(IO::ld8(arow + kk * 32 + 8 * g), IO::ld8(brow + kk * 32 + 8 * g), acc);
    if (k % 32) acc = mma16(IO::ld4(arow + k32 * 32 + 4 * g), IO::ld4(brow + k32 * 32 + 4 * g), acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(rb * 16 + 4 * g + i) * opitch + cb * 16 + l16] = acc[i];
  }
}

// Row pass 1: rotate (input RoPE) and L2-normalise this thread's D/4 slice of x.
template <typename E, int D>
__device__ __forceinline__ void xn_row(const FeatP& p, int b, int h, int t, int part, float* xv,
                                       float& nrm) {
  constexpr int CH = D / 4;
  const bool valid = t < p.T;
  const E* src = (const E*)p.x.ptr + (int64_t)b * p.x.sb + (int64_t)h * p.x.sh +
                 (int64_t)(valid ? t : 0) * p.x.st + part * CH;
  load_row<E>(src, xv, CH, valid);
  if (p.in_rot > 0 && valid) {
    const int half = p.in_rot / 2;
#pragma unroll
    for (int i = 0; i < CH; i += 2) {
      const int c = part * CH + i;
      if (c < p.in_rot) {
        const float cs = p.in_cos[(int64_t)t * half + c / 2];
        const float sn = p.in_sin[(int64_t)t * half + c / 2];
        const float x1 = xv[i], x2 = xv[i + 1];
        xv[i] = x1 * cs - x2 * sn;
        xv[i + 1] = x1 * sn + x2 * cs;
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) ss += xv[i] * xv[i];
  nrm = sqrtf(red4_sum(ss));
}

// Feature map of one row slice held in LDS (fp32 `a`), in place -> h.
// Returns the statistics the backward needs through references.
__device__ __forceinline__ void feature_row(const FeatP& p, int h, float* arow, int mc, float& rinv,
                                            float& mass) {
  float ss = 0.f;
  for (int j = 0; j < mc; ++j) ss += arow[j] * arow[j];
  ss = red4_sum(ss);
  rinv = rsqrtf(ss / (float)p.m + p.eps);
  const float tau = p.has_tau ? p.tau[h] : 0.0f;
  if (p.kind == TS_FEAT_RELU2) {
    float sf = 0.f;
    for (int j = 0; j < mc; ++j) {
      const float pre = arow[j] * rinv - tau;
      const float f = pre > 0.f ? pre * pre : 0.f;
      arow[j] = f;
      sf += f;
    }
    mass = red4_sum(sf);
    const bool ok = mass > p.eps;
    const float inv = ok ? 1.0f / mass : 0.0f;
    const float uni = 1.0f / (float)p.m;
    for (int j = 0; j < mc; ++j) arow[j] = ok ? arow[j] * inv : uni;
  } else {
    float mx = -INFINITY;
    for (int j = 0; j < mc; ++j) {
      const float l = p.gain * (arow[j] * rinv - tau);
      arow[j] = l;
      mx = fmaxf(mx, l);
    }
    mx = red4_max(mx);
    float se = 0.f;
    for (int j = 0; j < mc; ++j) {
      const float e = expf(arow[j] - mx);
      arow[j] = e;
      se += e;
    }
    mass = red4_sum(se);
    const float inv = 1.0f / mass;
    for (int j = 0; j < mc; ++j) arow[j] *= inv;
  }
}

template <typename E, int D>
__global__ __launch_bounds__(256) void feature_fwd_kernel(FeatP p) {
  constexpr int VEC = 16 / (int)sizeof(E);
  constexpr int XP = D + VEC;
  constexpr int CH = D / 4;
  const int m = p.m, mc = m / 4;
  const int AP = m + 4;
  const int HP = m + VEC;
  const int BP = D + 4;
  const int b = blockIdx.z, h = blockIdx.y, t0 = blockIdx.x * TT;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const int row = tid >> 2, part = tid & 3;
  const int t = t0 + row;
  const bool valid = t < p.T;
  const bool want_resid = p.resid.ptr != nullptr;

  extern __shared__ __align__(16) unsigned char smem[];
  E* Xn = (E*)smem;
  float* As = (float*)(Xn + TT * XP);
  E* Hs = (E*)(As + TT * (AP > BP ? AP : BP));
  float* Bs = As;  // base tile reuses the pre-activation tile

  float xv[CH];
  float nrm;
  xn_row<E, D>(p, b, h, t, part, xv, nrm);
  const float inv = 1.0f / fmaxf(nrm, p.eps);
#pragma unroll
  for (int i = 0; i < CH; ++i) Xn[row * XP + part * CH + i] = cvt<E>(xv[i] * inv);
  __syncthreads();

  tile_gemm_nt<E, D>(Xn, XP, (const E*)p.w1 + (size_t)h * m * D, m, As, AP, w, l16, g);
  __syncthreads();

  float* arow = As + row * AP + part * mc;
  float rinv, mass;
  feature_row(p, h, arow, mc, rinv, mass);
  if (want_resid)
    for (int j = 0; j < mc; ++j) Hs[row * HP + part * mc + j] = cvt<E>(arow[j]);
  if (valid) {
    E* dst = (E*)p.phi.ptr + (int64_t)b * p.phi.sb + (int64_t)h * p.phi.sh + (int64_t)t * p.phi.st;
    const int fhalf = p.feat_rot / 2;
    for (int j0 = 0; j0 < mc; j0 += 4) {
      const int c = part * mc + j0;
      float o[4] = {arow[j0], arow[j0 + 1], arow[j0 + 2], arow[j0 + 3]};
#pragma unroll
      for (int e = 0; e < 4; e += 2) {
        if (c + e < p.feat_rot) {
          const float cs = p.f_cos[(int64_t)t * fhalf + (c + e) / 2];
          const float sn = p.f_sin[(int64_t)t * fhalf + (c + e) / 2];
          const float h1 = o[e], h2 = o[e + 1];
          o[e] = h1 * cs - h2 * sn;
          o[e + 1] = h1 * sn + h2 * cs;
        }
      }
      store4<E>(dst + c, o[0], o[1], o[2], o[3]);
    }
  }
  if (!want_resid) return;
  __syncthreads();

  tile_gemm_nt_rt<E>(Hs, HP, (const E*)p.w2 + (size_t)h * D * m, m, D, Bs, BP, w, l16, g);
  __syncthreads();
  if (valid) {
    E* dst = (E*)p.resid.ptr + (int64_t)b * p.resid.sb + (int64_t)h * p.resid.sh +
             (int64_t)t * p.resid.st + part * CH;
#pragma unroll
    for (int i = 0; i < CH; i += 4) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = tof(Xn[row * XP + part * CH + i + e]) + p.s * Bs[row * BP + part * CH + i + e];
      store4<E>(dst + i, o[0], o[1], o[2], o[3]);
    }
  }
}

template <typename E, int D>
__global__ __launch_bounds__(256) void feature_bwd_kernel(FeatP p) {
  constexpr int VEC = 16 / (int)sizeof(E);
  constexpr int XP = D + VEC;
  constexpr int CH = D / 4;
  const int m = p.m, mc = m / 4;
  const int AP = m + 4;
  const int HP = m + VEC;
  const int b = blockIdx.z, h = blockIdx.y, t0 = blockIdx.x * TT;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const int row = tid >> 2, part = tid & 3;
  const int t = t0 + row;
  const bool valid = t < p.T;
  const bool has_resid = p.dresid.ptr != nullptr;

  extern __shared__ __align__(16) unsigned char smem[];
  E* Xn = (E*)smem;
  E* Rs = Xn + TT * XP;                  // s * dresid (MFMA operand)
  float* As = (float*)(Rs + TT * XP);    // a = W1 xn
  float* Gs = As + TT * AP;              // W2^T (s dresid), later dxn
  E* Ds = (E*)(Gs + TT * (AP > D + 4 ? AP : D + 4));  // da (MFMA operand)

  float xv[CH];
  float nrm;
  xn_row<E, D>(p, b, h, t, part, xv, nrm);
  const float inv = 1.0f / fmaxf(nrm, p.eps);
#pragma unroll
  for (int i = 0; i < CH; ++i) Xn[row * XP + part * CH + i] = cvt<E>(xv[i] * inv);
  float drv[CH];
  if (has_resid) {
    const float* src = (const float*)p.dresid.ptr + (int64_t)b * p.dresid.sb + (int64_t)h * p.dresid.sh +
                       (int64_t)(valid ? t : 0) * p.dresid.st + part * CH;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      drv[i] = valid ? src[i] : 0.f;
      Rs[row * XP + part * CH + i] = cvt<E>(p.s * drv[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < CH; ++i) drv[i] = 0.f;
  }
  __syncthreads();

  tile_gemm_nt<E, D>(Xn, XP, (const E*)p.w1 + (size_t)h * m * D, m, As, AP, w, l16, g);
  if (has_resid) tile_gemm_nt<E, D>(Rs, XP, (const E*)p.w2t + (size_t)h * m * D, m, Gs, AP, w, l16, g);
  __syncthreads();

  // ---- row pass over features: h, dh, dpre, da
  float* arow = As + row * AP + part * mc;
  float* grow = Gs + row * AP + part * mc;
  float ss = 0.f;
  for (int j = 0; j < mc; ++j) ss += arow[j] * arow[j];
  ss = red4_sum(ss);
  const float rinv = rsqrtf(ss / (float)m + p.eps);
  const float tau = p.has_tau ? p.tau[h] : 0.0f;
  // forward statistics
  float mass = 0.f, mx = -INFINITY;
  if (p.kind == TS_FEAT_RELU2) {
    for (int j = 0; j < mc; ++j) {
      const float pre = arow[j] * rinv - tau;
      mass += pre > 0.f ? pre * pre : 0.f;
    }
    mass = red4_sum(mass);
  } else {
    for (int j = 0; j < mc; ++j) mx = fmaxf(mx, p.gain * (arow[j] * rinv - tau));
    mx = red4_max(mx);
    for (int j = 0; j < mc; ++j) mass += expf(p.gain * (arow[j] * rinv - tau) - mx);
    mass = red4_sum(mass);
  }
  const bool ok = p.kind != TS_FEAT_RELU2 || mass > p.eps;
  const float minv = 1.0f / mass;
  auto hval = [&](float a) -> float {
    const float pre = a * rinv - tau;
    if (p.kind == TS_FEAT_RELU2) return ok ? (pre > 0.f ? pre * pre : 0.f) * minv : 1.0f / (float)m;
    return expf(p.gain * pre - mx) * minv;
  };
  // dh = unrotated dphi (+ W2^T s dresid), kept in grow
  const float* dsrc = (const float*)p.dphi.ptr + (int64_t)b * p.dphi.sb + (int64_t)h * p.dphi.sh +
                      (int64_t)(valid ? t : 0) * p.dphi.st + part * mc;
  const int fhalf = p.feat_rot / 2;
  float sdh = 0.f;
  for (int j = 0; j < mc; j += 2) {
    const int c = part * mc + j;
    float d1 = valid ? dsrc[j] : 0.f, d2 = valid ? dsrc[j + 1] : 0.f;
    if (c < p.feat_rot && valid) {
      const float cs = p.f_cos[(int64_t)t * fhalf + c / 2];
      const float sn = p.f_sin[(int64_t)t * fhalf + c / 2];
      const float e1 = d1 * cs + d2 * sn;
      const float e2 = -d1 * sn + d2 * cs;
      d1 = e1;
      d2 = e2;
    }
    if (has_resid) {
      d1 += grow[j];
      d2 += grow[j + 1];
    }
    grow[j] = d1;
    grow[j + 1] = d2;
    sdh += d1 * hval(arow[j]) + d2 * hval(arow[j + 1]);
  }
  sdh = red4_sum(sdh);
  // dpre (stored in grow), sum(dpre), sum(dpre * a)
  float sdp = 0.f, sda = 0.f;
  for (int j = 0; j < mc; ++j) {
    const float a = arow[j];
    const float pre = a * rinv - tau;
    float dp;
    if (p.kind == TS_FEAT_RELU2) {
      dp = ok ? (grow[j] - sdh) * minv * 2.0f * fmaxf(pre, 0.f) : 0.f;
    } else {
      dp = p.gain * hval(a) * (grow[j] - sdh);
    }
    grow[j] = dp;
    sdp += dp;
    sda += dp * a;
  }
  sdp = red4_sum(sdp);
  sda = red4_sum(sda);
  if (p.dtau.ptr && part == 0 && valid)
    ((float*)p.dtau.ptr)[(int64_t)b * p.dtau.sb + (int64_t)h * p.dtau.sh + (int64_t)t * p.dtau.st] = -sdp;
  const float c3 = rinv * rinv * rinv * sda / (float)m;
  E* da_out = p.da.ptr ? (E*)p.da.ptr + (int64_t)b * p.da.sb + (int64_t)h * p.da.sh + (int64_t)t * p.da.st +
                             part * mc
                       : nullptr;
  E* h_out = p.h.ptr ? (E*)p.h.ptr + (int64_t)b * p.h.sb + (int64_t)h * p.h.sh + (int64_t)t * p.h.st + part * mc
                     : nullptr;
  for (int j = 0; j < mc; j += 4) {
    float dv[4], hv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dv[e] = rinv * grow[j + e] - c3 * arow[j + e];
      Ds[row * HP + part * mc + j + e] = cvt<E>(dv[e]);
      hv[e] = hval(arow[j + e]);
    }
    if (valid && da_out) store4<E>(da_out + j, dv[0], dv[1], dv[2], dv[3]);
    if (valid && h_out) store4<E>(h_out + j, hv[0], hv[1], hv[2], hv[3]);
  }
  __syncthreads();

  // ---- dxn = da W1  (W1^T given row-major as [D x m])
  float* Xg = Gs;
  tile_gemm_nt_rt<E>(Ds, HP, (const E*)p.w1t + (size_t)h * D * m, m, D, Xg, D + 4, w, l16, g);
  __syncthreads();

  // ---- row pass: residual path, L2-norm and input-RoPE backward
  float dxn[CH];
  float dot = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    dxn[i] = Xg[row * (D + 4) + part * CH + i] + drv[i];
    dot += dxn[i] * xv[i] * inv;
  }
  dot = red4_sum(dot);
  float dxr[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i)
    dxr[i] = nrm > p.eps ? (dxn[i] - xv[i] * inv * dot) / nrm : dxn[i] / p.eps;
  if (p.in_rot > 0 && valid) {
    const int half = p.in_rot / 2;
#pragma unroll
    for (int i = 0; i < CH; i += 2) {
      const int c = part * CH + i;
      if (c < p.in_rot) {
        const float cs = p.in_cos[(int64_t)t * half + c / 2];
        const float sn = p.in_sin[(int64_t)t * half + c / 2];
        const float g1 = dxr[i], g2 = dxr[i + 1];
        dxr[i] = g1 * cs + g2 * sn;
        dxr[i + 1] = -g1 * sn + g2 * cs;
      }
    }
  }
  if (valid) {
    E* dst = (E*)p.dx.ptr + (int64_t)b * p.dx.sb + (int64_t)h * p.dx.sh + (int64_t)t * p.dx.st + part * CH;
#pragma unroll
    for (int i = 0; i < CH; i += 4) store4<E>(dst + i, dxr[i], dxr[i + 1], dxr[i + 2], dxr[i + 3]);
    if (p.xn.ptr) {
      E* xo = (E*)p.xn.ptr + (int64_t)b * p.xn.sb + (int64_t)h * p.xn.sh + (int64_t)t * p.xn.st + part * CH;
#pragma unroll
      for (int i = 0; i < CH; i += 4)
        store4<E>(xo + i, xv[i] * inv, xv[i + 1] * inv, xv[i + 2] * inv, xv[i + 3] * inv);
    }
  }
}

}  // namespace ts

// ============================================================== host side
namespace {

using ts::fail;

typedef void (*FeatFn)(ts::FeatP);

template <typename E>
FeatFn pick_feature(int d, bool fwd) {
  switch (d) {
#define TS_CASE(D) \
  case D:          \
    return fwd ? (FeatFn)ts::feature_fwd_kernel<E, D> : (FeatFn)ts::feature_bwd_kernel<E, D>;
    TS_CASE(16)
    TS_CASE(32)
    TS_CASE(48)
    TS_CASE(64)
    TS_CASE(96)
    TS_CASE(128)
#undef TS_CASE
  }
  return nullptr;
}

int check_feature_desc(const ts_feature_desc* d) {
  if (!d) return fail(TS_ERR_VALUE, "feature: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0) return fail(TS_ERR_VALUE, "feature: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "feature: unknown dtype");
  if (d->kind != TS_FEAT_RELU2 && d->kind != TS_FEAT_SOFTMAX)
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature: kind %d has no fused kernel", d->kind);
  if (d->m < 16 || d->m > 256 || d->m % 16)
    return fail(TS_ERR_NOT_IMPLEMENTED, "feature: width m=%d outside 16..256 (multiple of 16)", d->m);
  if (d->in_rot < 0 || d->in_rot > d->d || d->in_rot % 2) return fail(TS_ERR_VALUE, "feature: bad input rotation");
  if (d->feat_rot < 0 || d->feat_rot > d->m || d->feat_rot % 2)
    return fail(TS_ERR_VALUE, "feature: bad feature rotation");
  return TS_OK;
}

size_t fwd_lds(int esize, int d, int m) {
  const int vec = 16 / esize;
  const size_t a = (size_t)ts::TT * ((m > d ? m : d) + 4) * 4;
  return (size_t)ts::TT * (d + vec) * esize + a + (size_t)ts::TT * (m + vec) * esize;
}

size_t bwd_lds(int esize, int d, int m) {
  const int vec = 16 / esize;
  const size_t g = (size_t)ts::TT * ((m > d ? m : d) + 4) * 4;
  return 2 * (size_t)ts::TT * (d + vec) * esize + (size_t)ts::TT * (m + 4) * 4 + g + (size_t)ts::TT * (m + vec) * esize;
}

int launch_feature(FeatFn fn, const ts_feature_desc* d, size_t lds, hipStream_t stream, const ts::FeatP& p) {
  if (!fn) return fail(TS_ERR_NOT_IMPLEMENTED, "feature: head width d=%d has no fused kernel", d->d);
  if (lds > 160 * 1024) return fail(TS_ERR_NOT_IMPLEMENTED, "feature: tile needs %zu bytes of LDS", lds);
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "feature: LDS request failed: %s", hipGetErrorString(e));
  }
  dim3 grid((d->T + ts::TT - 1) / ts::TT, d->H, d->B);
  hipLaunchKernelGGL(fn, grid, dim3(256), lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "feature: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

void fill_common(const ts_feature_desc* d, ts::FeatP& p) {
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.m = d->m;
  p.in_rot = d->in_rot; p.feat_rot = d->feat_rot; p.has_tau = d->has_tau; p.kind = d->kind;
  p.gain = d->gain; p.s = d->resid_scale; p.eps = d->eps;
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
  if (d->T == 0) return TS_OK;
  ts::FeatP p;
  fill_common(d, p);
  p.x = io->x; p.phi = io->phi; p.resid = io->resid;
  p.w1 = io->w1; p.w2 = io->w2; p.tau = io->tau;
  p.in_cos = io->in_cos; p.in_sin = io->in_sin; p.f_cos = io->f_cos; p.f_sin = io->f_sin;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  FeatFn fn = d->dtype == TS_BF16 ? pick_feature<ts::bf16>(d->d, true) : pick_feature<float>(d->d, true);
  return launch_feature(fn, d, fwd_lds(es, d->d, d->m), stream, p);
}

int ts_feature_bwd(const ts_feature_desc* d, const ts_feature_bwd_io* io, hipStream_t stream) {
  int rc = check_feature_desc(d);
  if (rc) return rc;
  if (!io || !io->x.ptr || !io->w1 || !io->w1t || !io->dphi.ptr || !io->dx.ptr)
    return fail(TS_ERR_VALUE, "feature bwd: missing tensors");
  if (io->dresid.ptr && !io->w2t) return fail(TS_ERR_VALUE, "feature bwd: dresid needs w2t");
  if (d->has_tau && !io->tau) return fail(TS_ERR_VALUE, "feature bwd: missing tau");
  if (d->T == 0) return TS_OK;
  ts::FeatP p;
  fill_common(d, p);
  p.x = io->x; p.w1 = io->w1; p.w1t = io->w1t; p.w2t = io->w2t; p.tau = io->tau;
  p.in_cos = io->in_cos; p.in_sin = io->in_sin; p.f_cos = io->f_cos; p.f_sin = io->f_sin;
  p.dphi = io->dphi; p.dresid = io->dresid; p.dx = io->dx; p.da = io->da; p.xn = io->xn; p.h = io->h;
  p.dtau = io->dtau;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  FeatFn fn = d->dtype == TS_BF16 ? pick_feature<ts::bf16>(d->d, false) : pick_feature<float>(d->d, false);
  return launch_feature(fn, d, bwd_lds(es, d->d, d->m), stream, p);
}

}  // extern "C"
