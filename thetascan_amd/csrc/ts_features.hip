// Fused write-side feature map for gfx950 (forward and backward).
//
// One workgroup = 4 waves = 64 tokens of one (batch, head); each wave owns 16
// tokens end to end.  The tile is computed transposed, a^T = W1 xn^T, so the
// MFMA accumulator already holds, per lane, one token and four consecutive
// features of every 16-feature block.  Every per-token reduction (RMSNorm,
// feature mass, softmax max/sum, L2-norm dot products) is then a lane-local
// sum plus two cross-lane steps, feature-RoPE pairs are lane-local, and the
// accumulator feeds the next MFMA (W2 h^T, W1^T da^T) directly as an operand
// with the contraction index permuted consistently in both operands.  Only
// the L2-normalised inputs are staged in LDS (as the B operand of a^T).
//
// Reference chain replaced: block.py:595-618 (input RoPE, L2 norm),
// engine.py:117-158 (_block_forward: W1, RMSNorm, threshold, feature map,
// W2), kernel_features.py:73-135 (softmax partition / ReLU^2 ridge),
// engine.py:74-86 (feature RoPE) and the base term of engine.py:522-528.

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
  int groups;  // 64-token groups per workgroup
  int w_lds;   // weights staged in LDS
};

constexpr int TT = 64;  // tokens per workgroup (16 per wave)

__device__ __forceinline__ float sum_g(float v) {  // over the 4 lane groups of a token
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}
__device__ __forceinline__ float max_g(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  return v;
}

template <typename E>
__device__ __forceinline__ E* at(const ts_strided& s, int b, int h, int t) {
  return (E*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st;
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

// Rotate pairs (c, c+1), (c+2, c+3) of a four-feature group starting at even c.
__device__ __forceinline__ void rot4(float* v, int c, int rot, const float* cs_tab, const float* sn_tab,
                                     int64_t row, bool inverse) {
#pragma unroll
  for (int e = 0; e < 4; e += 2) {
    if (c + e < rot) {
      const float cs = cs_tab[row + (c + e) / 2];
      const float sn = inverse ? -sn_tab[row + (c + e) / 2] : sn_tab[row + (c + e) / 2];
      const float a = v[e], b = v[e + 1];
      v[e] = a * cs - b * sn;
      v[e + 1] = a * sn + b * cs;
    }
  }
}

// Row pass over x (four lanes per token, d/4 contiguous dims each): input
// RoPE, L2 norm; writes xn to the wave's LDS rows and returns ||x_rot||.
template <typename E, int D>
__device__ __forceinline__ float stage_xn(const FeatP& p, int b, int h, int t, int g, E* xs_row) {
  constexpr int CH = D / 4;
  const bool valid = t < p.T;
  float xv[CH];
  const E* src = at<E>(p.x, b, h, valid ? t : 0) + g * CH;
#pragma unroll
  for (int i = 0; i < CH; i += 4) {
    if (valid) {
      ld4f<E>(src + i, xv + i);
    } else {
      xv[i] = xv[i + 1] = xv[i + 2] = xv[i + 3] = 0.f;
    }
  }
  if (p.in_rot > 0 && valid) {
    const int64_t row = (int64_t)t * (p.in_rot / 2);
#pragma unroll
    for (int i = 0; i < CH; i += 4) rot4(xv + i, g * CH + i, p.in_rot, p.in_cos, p.in_sin, row, false);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) ss += xv[i] * xv[i];
  const float nrm = sqrtf(sum_g(ss));
  const float inv = 1.0f / fmaxf(nrm, p.eps);
#pragma unroll
  for (int i = 0; i < CH; i += 4) {
    float o[4] = {xv[i] * inv, xv[i + 1] * inv, xv[i + 2] * inv, xv[i + 3] * inv};
    st4f<E>(xs_row + g * CH + i, o);
  }
  return nrm;
}

// acc[fb] = (W1 xn^T) block fb: lane holds token l16, features 16fb+4g+i.
// W1 rows (length D) start every `wp` elements (LDS or global).
template <typename E, int D, int MB>
__device__ __forceinline__ void gemm_a(const E* w1, int wp, const E* xs, int l16, int g, int nfb, floatx4* acc) {
  typedef LdsIO<E> IO;
  constexpr int XP = D + 16 / (int)sizeof(E);
  const E* xrow = xs + l16 * XP;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb) {
    acc[fb] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (fb < nfb) {
      const E* wrow = w1 + (size_t)(fb * 16 + l16) * wp;
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
    const E* wrow = wt + (size_t)(db * 16 + l16) * wp;
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

// Copy a [rows x cols] row-major global matrix into LDS rows of pitch `pitch`.
template <typename E>
__device__ __forceinline__ void stage_matrix(const E* src, int rows, int cols, E* dst, int pitch, int tid) {
  constexpr int VEC = 16 / (int)sizeof(E);
  const int per_row = cols / VEC;
  for (int idx = tid; idx < rows * per_row; idx += 256) {
    const int r = idx / per_row, c = (idx - r * per_row) * VEC;
    *(uint4*)(dst + r * pitch + c) = *(const uint4*)(src + (size_t)r * cols + c);
  }
}

// In-register feature map of a^T (lane = token).  Leaves h in `hv`; returns
// the statistics the backward needs.
template <int MB>
__device__ __forceinline__ void feature_map(const FeatP& p, float tau, const floatx4* a, int nfb, floatx4* hv,
                                            float& rinv, float& mass, float& mx) {
  float ss = 0.f;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb)
    if (fb < nfb)
#pragma unroll
      for (int i = 0; i < 4; ++i) ss += a[fb][i] * a[fb][i];
  rinv = rsqrtf(sum_g(ss) / (float)p.m + p.eps);
  mx = 0.f;
  if (p.kind == TS_FEAT_RELU2) {
    float sf = 0.f;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pre = a[fb][i] * rinv - tau;
        const float f = (fb < nfb && pre > 0.f) ? pre * pre : 0.f;
        hv[fb][i] = f;
        sf += f;
      }
    mass = sum_g(sf);
    const bool ok = mass > p.eps;
    const float inv = ok ? 1.0f / mass : 0.f;
    const float uni = 1.0f / (float)p.m;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) hv[fb][i] = ok ? hv[fb][i] * inv : uni;
  } else {
    float m_ = -INFINITY;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
      if (fb < nfb)
#pragma unroll
        for (int i = 0; i < 4; ++i) m_ = fmaxf(m_, p.gain * (a[fb][i] * rinv - tau));
    mx = max_g(m_);
    float se = 0.f;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = fb < nfb ? expf(p.gain * (a[fb][i] * rinv - tau) - mx) : 0.f;
        hv[fb][i] = e;
        se += e;
      }
    mass = sum_g(se);
    const float inv = 1.0f / mass;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb)
#pragma unroll
      for (int i = 0; i < 4; ++i) hv[fb][i] *= inv;
  }
}

// Weights live in LDS when p.w_lds (staged once per workgroup, shared by its
// 4 waves x NG token groups); otherwise they are read from global memory.
template <typename E, int D, int MB>
__global__ __launch_bounds__(256) void feature_fwd_kernel(FeatP p) {
  constexpr int VEC = 16 / (int)sizeof(E);
  constexpr int XP = D + VEC;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const int m = p.m, nfb = m / 16;
  const bool want_resid = p.resid.ptr != nullptr;
  extern __shared__ __align__(16) unsigned char smem[];
  E* xs = (E*)smem + w * 16 * XP;
  const E* w1 = (const E*)p.w1 + (size_t)h * m * D;
  const E* w2 = want_resid ? (const E*)p.w2 + (size_t)h * D * m : nullptr;
  int wp1 = D, wp2 = m;
  if (p.w_lds) {
    E* ws1 = (E*)smem + TT * XP;
    E* ws2 = ws1 + m * (D + VEC);
    stage_matrix<E>(w1, m, D, ws1, D + VEC, tid);
    if (want_resid) stage_matrix<E>(w2, D, m, ws2, m + VEC, tid);
    w1 = ws1;
    w2 = ws2;
    wp1 = D + VEC;
    wp2 = m + VEC;
  }
  const float tau = p.has_tau ? p.tau[h] : 0.f;

  for (int grp = 0; grp < p.groups; ++grp) {
    const int t = (blockIdx.x * p.groups + grp) * TT + w * 16 + l16;
    const bool valid = t < p.T;
    __syncthreads();  // weights staged / previous group done with xs
    stage_xn<E, D>(p, b, h, t, g, xs + l16 * XP);
    __syncthreads();

    floatx4 a[MB], hv[MB];
    gemm_a<E, D, MB>(w1, wp1, xs, l16, g, nfb, a);
    float rinv, mass, mx;
    feature_map<MB>(p, tau, a, nfb, hv, rinv, mass, mx);
    if (valid) {
      E* dst = at<E>(p.phi, b, h, t);
      const int64_t frow = (int64_t)t * (p.feat_rot / 2);
#pragma unroll
      for (int fb = 0; fb < MB; ++fb) {
        if (fb < nfb) {
          float v[4] = {hv[fb][0], hv[fb][1], hv[fb][2], hv[fb][3]};
          if (p.feat_rot > 0) rot4(v, fb * 16 + 4 * g, p.feat_rot, p.f_cos, p.f_sin, frow, false);
          st4f<E>(dst + fb * 16 + 4 * g, v);
        }
      }
    }
    if (want_resid) {
      floatx4 base[D / 16];
      gemm_back<E, D, MB>(w2, wp2, hv, l16, g, nfb, base);
      if (valid) {
        E* dst = at<E>(p.resid, b, h, t);
#pragma unroll
        for (int db = 0; db < D / 16; ++db) {
          float xn[4];
          ld4f<E>(xs + l16 * XP + db * 16 + 4 * g, xn);
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = xn[i] + p.s * base[db][i];
          st4f<E>(dst + db * 16 + 4 * g, v);
        }
      }
    }
  }
}

template <typename E, int D, int MB>
__global__ __launch_bounds__(256) void feature_bwd_kernel(FeatP p) {
  typedef LdsIO<E> IO;
  constexpr int VEC = 16 / (int)sizeof(E);
  constexpr int XP = D + VEC;
  const int b = blockIdx.z, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g = lane >> 4;
  const int m = p.m, nfb = m / 16;
  const bool has_resid = p.dresid.ptr != nullptr;
  extern __shared__ __align__(16) unsigned char smem[];
  E* xs = (E*)smem + w * 16 * XP;
  const E* w1 = (const E*)p.w1 + (size_t)h * m * D;
  const E* w1t = (const E*)p.w1t + (size_t)h * D * m;
  const E* w2t = has_resid ? (const E*)p.w2t + (size_t)h * m * D : nullptr;
  int wpa = D, wpt = m;
  if (p.w_lds) {
    E* ws1 = (E*)smem + TT * XP;
    E* ws1t = ws1 + m * (D + VEC);
    E* ws2t = ws1t + D * (m + VEC);
    stage_matrix<E>(w1, m, D, ws1, D + VEC, tid);
    stage_matrix<E>(w1t, D, m, ws1t, m + VEC, tid);
    if (has_resid) stage_matrix<E>(w2t, m, D, ws2t, D + VEC, tid);
    w1 = ws1;
    w1t = ws1t;
    w2t = ws2t;
    wpa = D + VEC;
    wpt = m + VEC;
  }
  const float tau = p.has_tau ? p.tau[h] : 0.f;

  for (int grp = 0; grp < p.groups; ++grp) {
  const int t = (blockIdx.x * p.groups + grp) * TT + w * 16 + l16;
  const bool valid = t < p.T;
  const int tc = valid ? t : 0;
  __syncthreads();  // weights staged / previous group done with xs
  const float nrm = stage_xn<E, D>(p, b, h, t, g, xs + l16 * XP);
  __syncthreads();
  if (valid && p.xn.ptr) {
    constexpr int CH = D / 4;
    E* dst = at<E>(p.xn, b, h, t) + g * CH;
#pragma unroll
    for (int i = 0; i < CH; i += 4) {
      float v[4];
      ld4f<E>(xs + l16 * XP + g * CH + i, v);
      st4f<E>(dst + i, v);
    }
  }

  floatx4 a[MB], hv[MB];
  gemm_a<E, D, MB>(w1, wpa, xs, l16, g, nfb, a);
  float rinv, mass, mx;
  feature_map<MB>(p, tau, a, nfb, hv, rinv, mass, mx);

  // dh = rotate^T(dphi) (+ s W2^T dresid)
  floatx4 dh[MB];
  if (has_resid) {
    const E* drow = at<E>(p.dresid, b, h, tc);
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      dh[fb] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (fb < nfb) {
        const E* wrow = w2t + (size_t)(fb * 16 + l16) * wpa;
#pragma unroll
        for (int kk = 0; kk < D / 32; ++kk)
          dh[fb] = mma32(IO::ld8(wrow + kk * 32 + 8 * g), IO::ld8(drow + kk * 32 + 8 * g), dh[fb]);
        if (D % 32)
          dh[fb] = mma16(IO::ld4(wrow + (D / 32) * 32 + 4 * g), IO::ld4(drow + (D / 32) * 32 + 4 * g), dh[fb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) dh[fb][i] = valid ? dh[fb][i] * p.s : 0.f;
      }
    }
  } else {
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) dh[fb] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  float sdh = 0.f;
  if (valid) {
    const E* src = at<E>(p.dphi, b, h, t);
    const int64_t frow = (int64_t)t * (p.feat_rot / 2);
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      if (fb < nfb) {
        float v[4];
        ld4f<E>(src + fb * 16 + 4 * g, v);
        if (p.feat_rot > 0) rot4(v, fb * 16 + 4 * g, p.feat_rot, p.f_cos, p.f_sin, frow, true);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dh[fb][i] += v[i];
          sdh += dh[fb][i] * hv[fb][i];
        }
      }
    }
  }
  sdh = sum_g(sdh);
  // dpre -> da (RMSNorm backward); reuse dh as da
  const bool ok = p.kind != TS_FEAT_RELU2 || mass > p.eps;
  const float minv = 1.0f / mass;
  float sdp = 0.f, sda = 0.f;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float dp = 0.f;
      if (fb < nfb) {
        if (p.kind == TS_FEAT_RELU2) {
          const float pre = a[fb][i] * rinv - tau;
          dp = ok ? (dh[fb][i] - sdh) * minv * 2.0f * fmaxf(pre, 0.f) : 0.f;
        } else {
          dp = p.gain * hv[fb][i] * (dh[fb][i] - sdh);
        }
      }
      dh[fb][i] = dp;
      sdp += dp;
      sda += dp * a[fb][i];
    }
  }
  sdp = sum_g(sdp);
  sda = sum_g(sda);
  if (p.dtau.ptr && g == 0 && valid) *at<float>(p.dtau, b, h, t) = -sdp;
  const float c3 = rinv * rinv * rinv * sda / (float)p.m;
#pragma unroll
  for (int fb = 0; fb < MB; ++fb)
#pragma unroll
    for (int i = 0; i < 4; ++i) dh[fb][i] = rinv * dh[fb][i] - c3 * a[fb][i];
  if (valid) {
    E* da_out = p.da.ptr ? at<E>(p.da, b, h, t) : nullptr;
    E* h_out = p.h.ptr ? at<E>(p.h, b, h, t) : nullptr;
#pragma unroll
    for (int fb = 0; fb < MB; ++fb) {
      if (fb < nfb) {
        float v[4] = {dh[fb][0], dh[fb][1], dh[fb][2], dh[fb][3]};
        if (da_out) st4f<E>(da_out + fb * 16 + 4 * g, v);
        float u[4] = {hv[fb][0], hv[fb][1], hv[fb][2], hv[fb][3]};
        if (h_out) st4f<E>(h_out + fb * 16 + 4 * g, u);
      }
    }
  }

  // dxn^T = W1^T da^T  (W1^T given as [D x m])
  floatx4 dxn[D / 16];
  gemm_back<E, D, MB>(w1t, wpt, dh, l16, g, nfb, dxn);
  // residual path, L2-norm backward, input-RoPE backward at dims 16db+4g+i
  const E* xsrc = at<E>(p.x, b, h, tc);
  const E* drow = has_resid ? at<E>(p.dresid, b, h, tc) : nullptr;
  const float inv = 1.0f / fmaxf(nrm, p.eps);
  const int64_t irow = (int64_t)tc * (p.in_rot / 2);
  float xr[D / 16][4];
  float dot = 0.f;
#pragma unroll
  for (int db = 0; db < D / 16; ++db) {
    ld4f<E>(xsrc + db * 16 + 4 * g, xr[db]);
    if (p.in_rot > 0) rot4(xr[db], db * 16 + 4 * g, p.in_rot, p.in_cos, p.in_sin, irow, false);
    if (drow) {
      float r[4];
      ld4f<E>(drow + db * 16 + 4 * g, r);
#pragma unroll
      for (int i = 0; i < 4; ++i) dxn[db][i] += r[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) dot += dxn[db][i] * xr[db][i] * inv;
  }
  dot = sum_g(dot);
  if (valid) {
    E* dst = at<E>(p.dx, b, h, t);
#pragma unroll
    for (int db = 0; db < D / 16; ++db) {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        v[i] = nrm > p.eps ? (dxn[db][i] - xr[db][i] * inv * dot) / nrm : dxn[db][i] / p.eps;
      if (p.in_rot > 0) rot4(v, db * 16 + 4 * g, p.in_rot, p.in_cos, p.in_sin, irow, true);
      st4f<E>(dst + db * 16 + 4 * g, v);
    }
  }
  }  // token groups
}

}  // namespace ts

// ============================================================== host side
namespace {

using ts::fail;

typedef void (*FeatFn)(ts::FeatP);

template <typename E, int D>
FeatFn pick_mb(int m, bool fwd) {
  if (m <= 64) return fwd ? (FeatFn)ts::feature_fwd_kernel<E, D, 4> : (FeatFn)ts::feature_bwd_kernel<E, D, 4>;
  if (m <= 128) return fwd ? (FeatFn)ts::feature_fwd_kernel<E, D, 8> : (FeatFn)ts::feature_bwd_kernel<E, D, 8>;
  return fwd ? (FeatFn)ts::feature_fwd_kernel<E, D, 16> : (FeatFn)ts::feature_bwd_kernel<E, D, 16>;
}

template <typename E>
FeatFn pick_feature(int d, int m, bool fwd) {
  switch (d) {
    case 16: return pick_mb<E, 16>(m, fwd);
    case 32: return pick_mb<E, 32>(m, fwd);
    case 48: return pick_mb<E, 48>(m, fwd);
    case 64: return pick_mb<E, 64>(m, fwd);
    case 96: return pick_mb<E, 96>(m, fwd);
    case 128: return pick_mb<E, 128>(m, fwd);
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
  if (d->in_rot < 0 || d->in_rot > d->d || d->in_rot % 4)
    return fail(TS_ERR_VALUE, "feature: input rotation must be a multiple of 4 within d");
  if (d->feat_rot < 0 || d->feat_rot > d->m || d->feat_rot % 4)
    return fail(TS_ERR_VALUE, "feature: feature rotation must be a multiple of 4 within m");
  return TS_OK;
}

int launch_feature(FeatFn fn, const ts_feature_desc* d, bool fwd, bool resid, hipStream_t stream, ts::FeatP& p) {
  if (!fn) return fail(TS_ERR_NOT_IMPLEMENTED, "feature: head width d=%d has no fused kernel", d->d);
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  const int vec = 16 / es;
  const size_t xs_bytes = (size_t)ts::TT * (d->d + vec) * es;
  size_t w_bytes = (size_t)d->m * (d->d + vec) * es;              // W1 rows
  if (fwd) {
    if (resid) w_bytes += (size_t)d->d * (d->m + vec) * es;       // W2 rows
  } else {
    w_bytes += (size_t)d->d * (d->m + vec) * es;                  // W1^T rows
    if (resid) w_bytes += (size_t)d->m * (d->d + vec) * es;       // W2^T rows
  }
  p.w_lds = xs_bytes + w_bytes <= 64 * 1024;
  const size_t lds = xs_bytes + (p.w_lds ? w_bytes : 0);
  // Enough token groups per workgroup to amortise the weight staging while
  // keeping >= 4 workgroups per CU at long sequences.
  const int tiles = (d->T + ts::TT - 1) / ts::TT;
  int groups = 1;
  while (groups < 4 && (long)((tiles + 2 * groups - 1) / (2 * groups)) * d->H * d->B >= 1024) groups *= 2;
  p.groups = groups;
  dim3 grid((tiles + groups - 1) / groups, d->H, d->B);
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
  FeatFn fn = d->dtype == TS_BF16 ? pick_feature<ts::bf16>(d->d, d->m, true) : pick_feature<float>(d->d, d->m, true);
  return launch_feature(fn, d, true, io->resid.ptr != nullptr, stream, p);
}

int ts_feature_bwd(const ts_feature_desc* d, const ts_feature_bwd_io* io, hipStream_t stream) {
  int rc = check_feature_desc(d);
  if (rc) return rc;
  if (!io || !io->x.ptr || !io->w1 || !io->w1t || !io->dphi.ptr || !io->dx.ptr)
    return fail(TS_ERR_VALUE, "feature bwd: missing tensors");
  if (io->dresid.ptr && !io->w2t) return fail(TS_ERR_VALUE, "feature bwd: dresid needs w2t");
  if (d->has_tau && !io->tau) return fail(TS_ERR_VALUE, "feature bwd: missing tau");
  if ((d->in_rot && (!io->in_cos || !io->in_sin)) || (d->feat_rot && (!io->f_cos || !io->f_sin)))
    return fail(TS_ERR_VALUE, "feature bwd: missing rope tables");
  if (d->T == 0) return TS_OK;
  ts::FeatP p;
  fill_common(d, p);
  p.x = io->x; p.w1 = io->w1; p.w1t = io->w1t; p.w2t = io->w2t; p.tau = io->tau;
  p.in_cos = io->in_cos; p.in_sin = io->in_sin; p.f_cos = io->f_cos; p.f_sin = io->f_sin;
  p.dphi = io->dphi; p.dresid = io->dresid; p.dx = io->dx; p.da = io->da; p.xn = io->xn; p.h = io->h;
  p.dtau = io->dtau;
  FeatFn fn = d->dtype == TS_BF16 ? pick_feature<ts::bf16>(d->d, d->m, false) : pick_feature<float>(d->d, d->m, false);
  return launch_feature(fn, d, false, io->dresid.ptr != nullptr, stream, p);
}

}  // extern "C"
