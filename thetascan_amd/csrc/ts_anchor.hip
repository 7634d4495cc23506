// Value-anchor deposit of the kernel memory (gfx950), forward and backward.
//
//   vn = v / max(||v||, eps);   r = softmax(gain * C vn)      (C [V, d] per head)
//
// The deposit a value-anchor memory writes instead of the raw value
// (src/thetascan/_core/ops/engine.py:284-296): the value's softmax code over
// a codebook of V anchors.  One thread owns one token of one head: it keeps
// the token's d values and V logits in registers and reads the codebook,
// staged in LDS per workgroup, as broadcast rows.  The backward writes dv and
// dl / max(||v||, eps) per token (head-major [H, B*T, VP], zero past V), the
// left operand of the codebook gradient dC = sum_t (dl_t / n_t) v_t^T that
// the caller contracts over tokens.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct AnchorP {
  int B, H, T, V, c_heads;
  float gain, eps;
  ts_strided v, r, dr, dv;
  const float* c;   // [c_heads, V, d]
  void* dls;        // [H, B*T, VP] (backward)
};

template <typename E>
__device__ __forceinline__ void load_row(const E* src, float* out, int n) {
  constexpr int VEC = 16 / (int)sizeof(E);
  for (int j = 0; j < n; j += VEC) {
    Vec16<E> u;
    u.raw = *(const uint4*)(src + j);
#pragma unroll
    for (int e = 0; e < VEC; ++e) out[j + e] = tof(u.e[e]);
  }
}

// Logits gain * C vn of one token, their softmax, and 1 / max(||v||, eps).
template <int D, int VP>
__device__ __forceinline__ float anchor_code(const AnchorP& p, const float* cs, const float* vr, float* vn, float* r,
                                             float& n) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < D; ++j) ss += vr[j] * vr[j];
  n = sqrtf(ss);
  const float inv = 1.0f / fmaxf(n, p.eps);
#pragma unroll
  for (int j = 0; j < D; ++j) vn[j] = vr[j] * inv;
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < VP; ++c) {
    float l = 0.f;
    if (c < p.V) {
#pragma unroll
      for (int j = 0; j < D; ++j) l += cs[c * D + j] * vn[j];
      l *= p.gain;
      mx = fmaxf(mx, l);
    }
    r[c] = l;
  }
  float se = 0.f;
#pragma unroll
  for (int c = 0; c < VP; ++c) {
    const float e = c < p.V ? expf(r[c] - mx) : 0.f;
    r[c] = e;
    se += e;
  }
  const float is = 1.0f / se;
#pragma unroll
  for (int c = 0; c < VP; ++c) r[c] *= is;
  return inv;
}

template <int D, int VP>
__device__ __forceinline__ void stage_codebook(const AnchorP& p, float* cs, int h) {
  const float* src = p.c + (size_t)(p.c_heads == 1 ? 0 : h) * p.V * D;
  for (int i = threadIdx.x; i < p.V * D; i += blockDim.x) cs[i] = src[i];
  __syncthreads();
}

template <typename E, int D, int VP>
__global__ __launch_bounds__(256) void anchor_fwd_kernel(AnchorP p) {
  __shared__ float cs[VP * D];
  const int h = blockIdx.y, b = blockIdx.z;
  stage_codebook<D, VP>(p, cs, h);
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= p.T) return;
  const E* vrow = (const E*)p.v.ptr + (int64_t)b * p.v.sb + (int64_t)h * p.v.sh + (int64_t)t * p.v.st;
  float vr[D], vn[D], r[VP], n;
  load_row<E>(vrow, vr, D);
  anchor_code<D, VP>(p, cs, vr, vn, r, n);
  E* rrow = (E*)p.r.ptr + (int64_t)b * p.r.sb + (int64_t)h * p.r.sh + (int64_t)t * p.r.st;
#pragma unroll
  for (int c = 0; c < VP; ++c)
    if (c < p.V) rrow[c] = cvt<E>(r[c]);
}

template <typename E, int D, int VP>
__global__ __launch_bounds__(256) void anchor_bwd_kernel(AnchorP p) {
  __shared__ float cs[VP * D];
  const int h = blockIdx.y, b = blockIdx.z;
  stage_codebook<D, VP>(p, cs, h);
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= p.T) return;
  const E* vrow = (const E*)p.v.ptr + (int64_t)b * p.v.sb + (int64_t)h * p.v.sh + (int64_t)t * p.v.st;
  const E* drow = (const E*)p.dr.ptr + (int64_t)b * p.dr.sb + (int64_t)h * p.dr.sh + (int64_t)t * p.dr.st;
  float vr[D], vn[D], r[VP], n;
  load_row<E>(vrow, vr, D);
  const float inv = anchor_code<D, VP>(p, cs, vr, vn, r, n);
  // softmax backward: dl_c = gain r_c (dr_c - sum_k dr_k r_k)
  float dl[VP], sdr = 0.f;
#pragma unroll
  for (int c = 0; c < VP; ++c) {
    dl[c] = c < p.V ? tof(drow[c]) : 0.f;
    sdr += dl[c] * r[c];
  }
#pragma unroll
  for (int c = 0; c < VP; ++c) dl[c] = p.gain * r[c] * (dl[c] - sdr);
  // dvn = C^T dl, then through vn = v / max(||v||, eps) (the projection
  // term only where ||v|| > eps, as the clamp's gradient)
  float dvn[D], dot = 0.f;
#pragma unroll
  for (int j = 0; j < D; ++j) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < VP; ++c)
      if (c < p.V) s += dl[c] * cs[c * D + j];
    dvn[j] = s;
    dot += s * vn[j];
  }
  if (!(n > p.eps)) dot = 0.f;
  E* dvrow = (E*)p.dv.ptr + (int64_t)b * p.dv.sb + (int64_t)h * p.dv.sh + (int64_t)t * p.dv.st;
  constexpr int VEC = 16 / (int)sizeof(E);
#pragma unroll
  for (int j = 0; j < D; j += VEC) {
    Vec16<E> u;
#pragma unroll
    for (int e = 0; e < VEC; ++e) u.e[e] = cvt<E>((dvn[j + e] - vn[j + e] * dot) * inv);
    *(uint4*)(dvrow + j) = u.raw;
  }
  E* lrow = (E*)p.dls + ((int64_t)h * p.B * p.T + (int64_t)b * p.T + t) * VP;
#pragma unroll
  for (int c = 0; c < VP; c += VEC) {
    Vec16<E> u;
#pragma unroll
    for (int e = 0; e < VEC; ++e) u.e[e] = cvt<E>(dl[c + e] * inv);
    *(uint4*)(lrow + c) = u.raw;
  }
}

}  // namespace ts

namespace {

using ts::fail;

int anchor_vp(int V) { return V <= 16 ? 16 : V <= 32 ? 32 : V <= 64 ? 64 : 0; }

int check_anchor(const ts_anchor_desc* d) {
  if (!d) return fail(TS_ERR_VALUE, "anchor: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0 || d->V < 2) return fail(TS_ERR_VALUE, "anchor: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "anchor: unknown dtype");
  if (d->c_heads != 1 && d->c_heads != d->H) return fail(TS_ERR_VALUE, "anchor: codebook heads must be 1 or H");
  if (d->d != 16 && d->d != 32 && d->d != 64 && d->d != 128)
    return fail(TS_ERR_NOT_IMPLEMENTED, "anchor: value width %d (16, 32, 64 or 128)", d->d);
  if (!anchor_vp(d->V)) return fail(TS_ERR_NOT_IMPLEMENTED, "anchor: %d anchors (at most 64)", d->V);
  if (d->H > 65535 || d->B > 65535) return fail(TS_ERR_NOT_IMPLEMENTED, "anchor: too many heads or batches");
  return TS_OK;
}

void fill_anchor(const ts_anchor_desc* d, ts::AnchorP& p) {
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.V = d->V; p.c_heads = d->c_heads;
  p.gain = d->gain; p.eps = d->eps;
}

template <typename E, int D>
void launch_anchor(int vp, bool bwd, dim3 grid, hipStream_t s, const ts::AnchorP& p) {
#define TS_ANCHOR_CASE(VP)                                                                              \
  if (bwd) hipLaunchKernelGGL((ts::anchor_bwd_kernel<E, D, VP>), grid, dim3(256), 0, s, p);            \
  else hipLaunchKernelGGL((ts::anchor_fwd_kernel<E, D, VP>), grid, dim3(256), 0, s, p);
  if (vp == 16) { TS_ANCHOR_CASE(16) }
  else if (vp == 32) { TS_ANCHOR_CASE(32) }
  else { TS_ANCHOR_CASE(64) }
#undef TS_ANCHOR_CASE
}

template <typename E>
void dispatch_anchor(int d, int vp, bool bwd, dim3 grid, hipStream_t s, const ts::AnchorP& p) {
  switch (d) {
    case 16: launch_anchor<E, 16>(vp, bwd, grid, s, p); break;
    case 32: launch_anchor<E, 32>(vp, bwd, grid, s, p); break;
    case 64: launch_anchor<E, 64>(vp, bwd, grid, s, p); break;
    default: launch_anchor<E, 128>(vp, bwd, grid, s, p); break;
  }
}

int anchor_run(const ts_anchor_desc* d, const ts::AnchorP& p, bool bwd, hipStream_t stream, const char* what) {
  if ((int64_t)d->B * d->T == 0) return TS_OK;
  const dim3 grid((unsigned)((d->T + 255) / 256), (unsigned)d->H, (unsigned)d->B);
  const int vp = anchor_vp(d->V);
  if (d->dtype == TS_BF16) dispatch_anchor<ts::bf16>(d->d, vp, bwd, grid, stream, p);
  else dispatch_anchor<float>(d->d, vp, bwd, grid, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TS_OK;
}

bool row_ok(const ts_strided& s, int es) {
  return s.ptr && ((uintptr_t)s.ptr & 15) == 0 && (s.sb * es) % 16 == 0 && (s.sh * es) % 16 == 0 &&
         (s.st * es) % 16 == 0;
}

}  // namespace

extern "C" {

int ts_anchor_width(const ts_anchor_desc* d, int32_t* vp) {
  int rc = check_anchor(d);
  if (rc) return rc;
  if (vp) *vp = anchor_vp(d->V);
  return TS_OK;
}

int ts_anchor_fwd(const ts_anchor_desc* d, ts_strided v, const float* codebook, ts_strided r, hipStream_t stream) {
  int rc = check_anchor(d);
  if (rc) return rc;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!codebook || !r.ptr) return fail(TS_ERR_VALUE, "anchor: missing tensors");
  if (!row_ok(v, es)) return fail(TS_ERR_VALUE, "anchor: value rows must be 16-byte aligned");
  ts::AnchorP p;
  fill_anchor(d, p);
  p.v = v; p.r = r; p.c = codebook;
  return anchor_run(d, p, false, stream, "anchor");
}

int ts_anchor_bwd(const ts_anchor_desc* d, ts_strided v, const float* codebook, ts_strided dr, ts_strided dv,
                  void* dls, hipStream_t stream) {
  int rc = check_anchor(d);
  if (rc) return rc;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!codebook || !dr.ptr || !dls) return fail(TS_ERR_VALUE, "anchor bwd: missing tensors");
  if (!row_ok(v, es) || !row_ok(dv, es) || ((uintptr_t)dls & 15))
    return fail(TS_ERR_VALUE, "anchor bwd: rows must be 16-byte aligned");
  ts::AnchorP p;
  fill_anchor(d, p);
  p.v = v; p.dr = dr; p.dv = dv; p.c = codebook; p.dls = dls;
  return anchor_run(d, p, true, stream, "anchor bwd");
}

}  // extern "C"
