// Mass of absolute features (gfx950): the normalizer of a read whose features
// can be negative (a tanh GN fast network), and its backward.
//
//   mass_t = sum_j |q_tj| C_tj,   C_u = a_u C_{u-1} + |k_u|
//
// C is the decayed prefix of |keys| along the scan order (plain, static
// per-head or per-token retention, the view's own), so |num_t| / mass_t <=
// max |value| for the normalized read num / (mass + eps).  Backward:
//
//   dq_tj = dmass_t sign(q_tj) C_tj
//   dk_ij = sign(k_ij) R_ij,   R_u = a'_u R_{u-1} + dmass_u |q_u|  (anti-causal)
//
// with the anti-causal step decay a'_u of the token the state steps out of,
// exactly the adjoint of the causal prefix.  Each pass has ts_wcumsum's
// time-parallel form: a summary pass (every (b, h, segment, four features)
// folds its segment from zero: last value and decay product) and a main pass
// (fold the earlier segments, walk the segment once).  The [B,H,T,F] prefix is
// never stored: the forward reduces |q| C over the features of a row in
// registers (the row's F/4 threads are adjacent lanes of one wave), the
// backward forms dq and dk where the prefixes are made.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

enum { AM_MASS = 0, AM_DQ = 1, AM_DK = 2 };

struct AbsMassP {
  int B, H, T, F, S, L, ret;
  ts_strided q, k, mass, dmass, out, decay;  // mass / dmass: fp32 [B,H,T] (feature stride unused)
  const float* log_alpha;
  float* tot;   // [B*H, S, F]
  float* prod;  // [B*H, S]
};

template <typename E>
__device__ __forceinline__ floatx4 am_ld4(const E* p) {
  if constexpr (sizeof(E) == 2) {
    const uint2 r = *(const uint2*)p;
    const bf16x4 v = __builtin_bit_cast(bf16x4, r);
    return floatx4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  } else {
    return *(const floatx4*)p;
  }
}

template <typename E>
__device__ __forceinline__ void am_st4(E* p, floatx4 v) {
  if constexpr (sizeof(E) == 2) {
    bf16x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (bf16)v[i];
    *(uint2*)p = __builtin_bit_cast(uint2, o);
  } else {
    *(floatx4*)p = v;
  }
}

__device__ __forceinline__ floatx4 am_abs(floatx4 v) {
  return floatx4{fabsf(v[0]), fabsf(v[1]), fabsf(v[2]), fabsf(v[3])};
}
__device__ __forceinline__ float am_sign(float x) { return x > 0.f ? 1.f : (x < 0.f ? -1.f : 0.f); }

struct AmThread {
  int f, seg, b, h;
  int64_t r;
  float a_static;
  const float* db;
};

// Thread (b, h, segment, features f .. f+3); false past the end.
__device__ __forceinline__ bool am_thread(const AbsMassP& p, AmThread& w) {
  const int FV = p.F / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)p.B * p.H * p.S * FV) return false;
  w.f = (int)(idx % FV) * 4;
  w.r = idx / FV;
  w.seg = (int)(w.r % p.S);
  const int bh = (int)(w.r / p.S);
  w.b = bh / p.H;
  w.h = bh % p.H;
  w.a_static = p.ret == TS_RET_STATIC ? expf(p.log_alpha[w.h]) : 1.0f;
  w.db = p.ret == TS_RET_STREAM
             ? (const float*)p.decay.ptr + (int64_t)w.b * p.decay.sb + (int64_t)w.h * p.decay.sh
             : nullptr;
  return true;
}

// Step decay of scan step u (causal: the token's own decay; anti-causal: the
// decay of the token the state steps out of, 1 past the end).
template <int MODE>
__device__ __forceinline__ float am_step(const AbsMassP& p, const AmThread& w, int u) {
  if (p.ret == TS_RET_STATIC) return w.a_static;
  if (p.ret != TS_RET_STREAM) return 1.0f;
  const int tp = MODE == AM_DK ? p.T - 1 - u : u;
  const int src = MODE == AM_DK ? tp + 1 : tp;
  return src < p.T ? expf(w.db[(int64_t)src * p.decay.st]) : 1.0f;
}

template <typename E>
__device__ __forceinline__ const E* am_row(const ts_strided& s, int b, int h, int t) {
  return (const E*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st;
}
__device__ __forceinline__ float am_scalar(const ts_strided& s, int b, int h, int t) {
  return *((const float*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st);
}

// The prefix's input at scan step u (token tp): |k| causally, dmass |q|
// anti-causally.
template <typename E, int MODE>
__device__ __forceinline__ floatx4 am_input(const AbsMassP& p, const AmThread& w, int tp) {
  if constexpr (MODE == AM_DK) {
    const float dm = am_scalar(p.dmass, w.b, w.h, tp);
    const floatx4 aq = am_abs(am_ld4<E>(am_row<E>(p.q, w.b, w.h, tp) + w.f));
    return floatx4{dm * aq[0], dm * aq[1], dm * aq[2], dm * aq[3]};
  } else {
    return am_abs(am_ld4<E>(am_row<E>(p.k, w.b, w.h, tp) + w.f));
  }
}

// Steps are taken eight at a time: the loads of all eight are issued before
// the first is folded (the step chain itself is sequential, its loads are
// not), with the tail's surplus loads clamped to the segment's last step.
constexpr int kAmUnroll = 8;

template <typename E, int MODE>
__global__ __launch_bounds__(256) void absmass_summary_kernel(AbsMassP p) {
  AmThread w;
  if (!am_thread(p, w)) return;
  const int u0 = w.seg * p.L;
  const int u1 = min(u0 + p.L, p.T);
  floatx4 z = {0.f, 0.f, 0.f, 0.f};
  float P = 1.0f;
  for (int u = u0; u < u1; u += kAmUnroll) {
    floatx4 x[kAmUnroll];
    float a[kAmUnroll];
#pragma unroll
    for (int i = 0; i < kAmUnroll; ++i) {
      const int uu = min(u + i, u1 - 1);
      const int tp = MODE == AM_DK ? p.T - 1 - uu : uu;
      a[i] = am_step<MODE>(p, w, uu);
      x[i] = am_input<E, MODE>(p, w, tp);
    }
#pragma unroll
    for (int i = 0; i < kAmUnroll; ++i) {
      if (u + i < u1) {
        const float c = u + i == u0 ? 0.f : a[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) z[e] = c * z[e] + x[i][e];
        P *= a[i];
      }
    }
  }
  *(floatx4*)(p.tot + w.r * p.F + w.f) = z;
  if (w.f == 0) p.prod[w.r] = P;
}

template <typename E, int MODE>
__global__ __launch_bounds__(256) void absmass_main_kernel(AbsMassP p) {
  AmThread w;
  if (!am_thread(p, w)) return;
  const int FV = p.F / 4;  // a power of two <= 64: the row's threads are adjacent, aligned lanes
  const int64_t row0 = (w.r / p.S) * p.S;
  floatx4 z = {0.f, 0.f, 0.f, 0.f};  // the state entering this segment
  for (int j0 = 0; j0 < w.seg; j0 += kAmUnroll) {
    float P[kAmUnroll];
    floatx4 t4[kAmUnroll];
#pragma unroll
    for (int i = 0; i < kAmUnroll; ++i) {
      const int j = min(j0 + i, w.seg - 1);
      P[i] = p.prod[row0 + j];
      t4[i] = *(const floatx4*)(p.tot + (row0 + j) * p.F + w.f);
    }
#pragma unroll
    for (int i = 0; i < kAmUnroll; ++i) {
      if (j0 + i < w.seg) {
#pragma unroll
        for (int e = 0; e < 4; ++e) z[e] = P[i] * z[e] + t4[i][e];
      }
    }
  }
  const int u0 = w.seg * p.L;
  const int u1 = min(u0 + p.L, p.T);
  for (int u = u0; u < u1; u += kAmUnroll) {
    floatx4 x[kAmUnroll], y[kAmUnroll];
    float a[kAmUnroll], dm[kAmUnroll];
#pragma unroll
    for (int i = 0; i < kAmUnroll; ++i) {
      const int uu = min(u + i, u1 - 1);
      const int tp = MODE == AM_DK ? p.T - 1 - uu : uu;
      a[i] = am_step<MODE>(p, w, uu);
      x[i] = am_input<E, MODE>(p, w, tp);
      // the row the step's output reads besides the prefix: q (mass, dq) or k (dk)
      y[i] = am_ld4<E>(am_row<E>(MODE == AM_DK ? p.k : p.q, w.b, w.h, tp) + w.f);
      dm[i] = MODE == AM_DQ ? am_scalar(p.dmass, w.b, w.h, tp) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kAmUnroll; ++i) {
      // uniform over a row's lanes (one segment), so the row's shuffles below
      // run with every partner lane active
      if (u + i < u1) {
        const int tp = MODE == AM_DK ? p.T - 1 - (u + i) : u + i;
        const float c = u + i == 0 ? 0.f : a[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) z[e] = c * z[e] + x[i][e];
        if constexpr (MODE == AM_MASS) {
          const floatx4 aq = am_abs(y[i]);
          float s = aq[0] * z[0] + aq[1] * z[1] + aq[2] * z[2] + aq[3] * z[3];
          for (int o = 1; o < FV; o <<= 1) s += __shfl_xor(s, o, 64);
          if (w.f == 0)
            *((float*)p.mass.ptr + (int64_t)w.b * p.mass.sb + (int64_t)w.h * p.mass.sh + (int64_t)tp * p.mass.st) = s;
        } else if constexpr (MODE == AM_DQ) {
          floatx4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = dm[i] * am_sign(y[i][e]) * z[e];
          am_st4<E>(const_cast<E*>(am_row<E>(p.out, w.b, w.h, tp)) + w.f, o);
        } else {
          floatx4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = am_sign(y[i][e]) * z[e];
          am_st4<E>(const_cast<E*>(am_row<E>(p.out, w.b, w.h, tp)) + w.f, o);
        }
      }
    }
  }
}

}  // namespace ts

namespace {

using ts::fail;

// Segments of the scan order: about 2^TS_AM_INFLIGHT_LOG2 features in
// flight, at least 16 steps per segment.
#ifndef TS_AM_INFLIGHT_LOG2
#define TS_AM_INFLIGHT_LOG2 19
#endif
void am_segments(const ts_abs_mass_desc* d, int* S, int* L) {
  const int64_t lanes = (int64_t)d->B * d->H * d->F;
  int64_t want = ((int64_t)1 << TS_AM_INFLIGHT_LOG2) / (lanes > 0 ? lanes : 1);
  const int64_t most = (d->T + 15) / 16;
  if (want > most) want = most;
  if (want < 1) want = 1;
  *L = (int)((d->T + want - 1) / want);
  if (*L < 1) *L = 1;
  *S = (d->T + *L - 1) / *L;
}

int check_am(const ts_abs_mass_desc* d) {
  if (!d || d->B < 1 || d->H < 1 || d->T < 0 || d->F < 4) return fail(TS_ERR_VALUE, "abs mass: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "abs mass: unknown dtype");
  if (d->retention < TS_RET_NONE || d->retention > TS_RET_STREAM) return fail(TS_ERR_VALUE, "abs mass: bad retention");
  const int fv = d->F / 4;
  if (d->F % 4 || fv > 64 || (fv & (fv - 1)))
    return fail(TS_ERR_NOT_IMPLEMENTED, "abs mass: width %d (4, 8, 16, ... 256)", d->F);
  return TS_OK;
}

bool am_rows(const ts_strided& s, int es) {
  const int64_t a = 4;  // four features per access
  return s.ptr && ((uintptr_t)s.ptr % (4 * es)) == 0 && s.sb % a == 0 && s.sh % a == 0 && s.st % a == 0;
}

template <typename E, int MODE>
int am_launch(const ts::AbsMassP& p, hipStream_t stream) {
  const int64_t n = (int64_t)p.B * p.H * p.S * (p.F / 4);
  const dim3 grid((unsigned)((n + 255) / 256));
  if (p.S > 1) hipLaunchKernelGGL((ts::absmass_summary_kernel<E, MODE>), grid, dim3(256), 0, stream, p);
  hipLaunchKernelGGL((ts::absmass_main_kernel<E, MODE>), grid, dim3(256), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "abs mass: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

template <int MODE>
int am_run(const ts_abs_mass_desc* d, const ts::AbsMassP& p, hipStream_t stream) {
  return d->dtype == TS_BF16 ? am_launch<ts::bf16, MODE>(p, stream) : am_launch<float, MODE>(p, stream);
}

int am_prepare(const ts_abs_mass_desc* d, ts_strided q, ts_strided k, const float* log_alpha, ts_strided decay,
               void* workspace, size_t ws_bytes, ts::AbsMassP* p) {
  int rc = check_am(d);
  if (rc) return rc;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!am_rows(q, es) || !am_rows(k, es)) return fail(TS_ERR_VALUE, "abs mass: q and k rows must be aligned to 4 features");
  if (d->retention == TS_RET_STATIC && !log_alpha) return fail(TS_ERR_VALUE, "abs mass: missing log_alpha");
  if (d->retention == TS_RET_STREAM && !decay.ptr) return fail(TS_ERR_VALUE, "abs mass: missing decay");
  size_t need = 0;
  if ((rc = ts_abs_mass_workspace_bytes(d, &need))) return rc;
  if (need && (!workspace || ws_bytes < need || ((uintptr_t)workspace & 15u)))
    return fail(TS_ERR_VALUE, "abs mass: workspace needs %zu bytes, 16-byte aligned", need);
  memset(p, 0, sizeof(*p));
  p->B = d->B; p->H = d->H; p->T = d->T; p->F = d->F; p->ret = d->retention;
  am_segments(d, &p->S, &p->L);
  p->q = q; p->k = k; p->decay = decay; p->log_alpha = log_alpha;
  p->tot = (float*)workspace;
  p->prod = p->tot ? p->tot + (size_t)d->B * d->H * p->S * d->F : nullptr;
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_abs_mass_workspace_bytes(const ts_abs_mass_desc* d, size_t* bytes) {
  int rc = check_am(d);
  if (rc) return rc;
  int S = 0, L = 0;
  am_segments(d, &S, &L);
  if (bytes) *bytes = d->T == 0 ? 0 : (size_t)d->B * d->H * S * ((size_t)d->F + 1) * sizeof(float) + 256;
  return TS_OK;
}

int ts_abs_mass_fwd(const ts_abs_mass_desc* d, ts_strided q, ts_strided k, const float* log_alpha, ts_strided decay,
                    ts_strided mass, void* workspace, size_t ws_bytes, hipStream_t stream) {
  ts::AbsMassP p;
  int rc = am_prepare(d, q, k, log_alpha, decay, workspace, ws_bytes, &p);
  if (rc) return rc;
  if (!mass.ptr) return fail(TS_ERR_VALUE, "abs mass: missing mass");
  if (d->T == 0) return TS_OK;
  p.mass = mass;
  return am_run<ts::AM_MASS>(d, p, stream);
}

int ts_abs_mass_bwd(const ts_abs_mass_desc* d, ts_strided q, ts_strided k, ts_strided dmass, const float* log_alpha,
                    ts_strided decay, ts_strided dq, ts_strided dk, void* workspace, size_t ws_bytes,
                    hipStream_t stream) {
  ts::AbsMassP p;
  int rc = am_prepare(d, q, k, log_alpha, decay, workspace, ws_bytes, &p);
  if (rc) return rc;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!dmass.ptr || (dq.ptr && !am_rows(dq, es)) || (dk.ptr && !am_rows(dk, es)))
    return fail(TS_ERR_VALUE, "abs mass bwd: missing dmass or unaligned dq / dk rows");
  if (d->T == 0) return TS_OK;
  p.dmass = dmass;
  if (dq.ptr) {
    p.out = dq;
    if ((rc = am_run<ts::AM_DQ>(d, p, stream))) return rc;
  }
  if (dk.ptr) {
    p.out = dk;
    if ((rc = am_run<ts::AM_DK>(d, p, stream))) return rc;
  }
  return TS_OK;
}

}  // extern "C"
