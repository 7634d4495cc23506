// Kernel-family feature maps with their learned controls (gfx950), forward
// and backward: the softmax partition with a scalar, per-head or
// per-feature gain, an additive per-feature shift (score bias and/or the
// learned threshold) and the relative-to-max sparsity variants, and the ReLU^2
// ridge with a shift -- optionally after the RMSNorm of the raw W1 products.
//
//   z   = rmsnorm(a) (rms) or a;   u = z + shift
//   softmax: l = gain * u; dense = softmax(l); e = exp(l - max l)
//            margin = (l - max l) - log(clamp(rho, eps, 1 - eps))
//            gate   = sigmoid(margin / temp)  (relative_soft)
//                   | [margin >= 0]           (relative_st*: forward value; the
//                                              gradient is the sigmoid's)
//            sparse = e gate / max(sum e gate, eps)
//            phi = dense | sparse | dense + alpha (sparse - dense)
//   relu2:   f = relu(u)^2;  phi = f / sum f  (uniform 1/m when sum f <= eps)
//
// Reference: src/thetascan/_core/ops/kernel_features.py:43-135
// (relative_threshold_features, softmax_partition_features,
// relu2_ridge_features) after the RMSNorm of engine.py:117-158.
//
// One thread owns one token of one head and keeps its row in registers
// (m <= 64).  The backward recomputes the forward, writes da (or dz) and
// per-workgroup partial sums of the control gradients, reduced across the
// workgroup's rows in lane order (reproducible bit for bit).

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct KmapP {
  int B, H, T, m, kind, rms, gain_mode, sparsity;
  float gain, temp, eps;
  ts_strided a, phi, dphi, da;
  const float* shift;  // [H, m] or null
  const float* gainv;  // [H] or [H, m]
  const float* rho;    // [H]
  const float* alpha;  // [H]
  float* dshift_part;  // [parts, H, m]
  float* dgain_part;   // [parts, H] or [parts, H, m]
  float* drho_part;    // [parts, H]
  float* dalpha_part;  // [parts, H]
};

template <typename E, int M>
__device__ __forceinline__ void kmap_load(const E* row, float* z) {
  constexpr int VEC = 16 / (int)sizeof(E);
#pragma unroll
  for (int j = 0; j < M; j += VEC) {
    Vec16<E> u;
    u.raw = *(const uint4*)(row + j);
#pragma unroll
    for (int e = 0; e < VEC; ++e) z[j + e] = tof(u.e[e]);
  }
}

template <typename E, int M>
__device__ __forceinline__ void kmap_store(E* row, const float* v) {
  constexpr int VEC = 16 / (int)sizeof(E);
#pragma unroll
  for (int j = 0; j < M; j += VEC) {
    Vec16<E> u;
#pragma unroll
    for (int e = 0; e < VEC; ++e) u.e[e] = cvt<E>(v[j + e]);
    *(uint4*)(row + j) = u.raw;
  }
}

__device__ __forceinline__ float kmap_gain(const KmapP& p, int h, int j) {
  return p.gain_mode == 0 ? p.gain : p.gain_mode == 1 ? p.gainv[h] : p.gainv[h * p.m + j];
}

// The row after the RMSNorm and shift (u, in place) and 1 / rms.
template <int M>
__device__ __forceinline__ float kmap_pre(const KmapP& p, int h, float* u) {
  float rinv = 1.0f;
  if (p.rms) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) ss += u[j] * u[j];
    rinv = rsqrtf(ss / (float)p.m + p.eps);
  }
#pragma unroll
  for (int j = 0; j < M; ++j) u[j] = u[j] * rinv + (p.shift ? p.shift[h * p.m + j] : 0.f);
  return rinv;
}

// Softmax statistics of a row: max logit, sum of exp, sum of the gated exp,
// and log(clamped rho).
struct SoftStats {
  float mx, se, sw, lr;
};

template <int M>
__device__ __forceinline__ SoftStats kmap_soft_stats(const KmapP& p, int h, const float* u) {
  SoftStats s;
  s.mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < M; ++j) s.mx = fmaxf(s.mx, kmap_gain(p, h, j) * u[j]);
  s.lr = 0.f;
  if (p.sparsity) s.lr = logf(fminf(fmaxf(p.rho[h], p.eps), 1.0f - p.eps));
  s.se = 0.f;
  s.sw = 0.f;
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const float sh = kmap_gain(p, h, j) * u[j] - s.mx;
    const float e = expf(sh);
    s.se += e;
    if (p.sparsity) {
      const float margin = sh - s.lr;
      const float gate = p.sparsity == TS_SPARSE_SOFT ? 1.0f / (1.0f + expf(-margin / p.temp))
                                                      : (margin >= 0.f ? 1.0f : 0.0f);
      s.sw += e * gate;
    }
  }
  return s;
}

template <typename E, int M>
__global__ __launch_bounds__(256) void kmap_fwd_kernel(KmapP p) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= p.T) return;
  float u[M];
  kmap_load<E, M>((const E*)p.a.ptr + (int64_t)b * p.a.sb + (int64_t)h * p.a.sh + (int64_t)t * p.a.st, u);
  kmap_pre<M>(p, h, u);
  float out[M];
  if (p.kind == TS_KMAP_RELU2) {
    float mass = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const float r = fmaxf(u[j], 0.f);
      out[j] = r * r;
      mass += out[j];
    }
    const bool ok = mass > p.eps;
    const float inv = ok ? 1.0f / mass : 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) out[j] = ok ? out[j] * inv : 1.0f / (float)p.m;
  } else {
    const SoftStats s = kmap_soft_stats<M>(p, h, u);
    const float ise = 1.0f / s.se, isw = 1.0f / fmaxf(s.sw, p.eps);
    const float al = p.sparsity == TS_SPARSE_ST_BLEND ? p.alpha[h] : 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const float sh = kmap_gain(p, h, j) * u[j] - s.mx;
      const float e = expf(sh);
      const float dense = e * ise;
      float v = dense;
      if (p.sparsity) {
        const float margin = sh - s.lr;
        const float gate = p.sparsity == TS_SPARSE_SOFT ? 1.0f / (1.0f + expf(-margin / p.temp))
                                                        : (margin >= 0.f ? 1.0f : 0.0f);
        const float sp = e * gate * isw;
        v = p.sparsity == TS_SPARSE_ST_BLEND ? dense + al * (sp - dense) : sp;
      }
      out[j] = v;
    }
  }
  kmap_store<E, M>((E*)p.phi.ptr + (int64_t)b * p.phi.sb + (int64_t)h * p.phi.sh + (int64_t)t * p.phi.st, out);
}

// Sum of v over the 256 threads of the workgroup, in lane then wave order;
// the result is valid in thread 0.
__device__ __forceinline__ float kmap_block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

template <typename E, int M>
__global__ __launch_bounds__(256) void kmap_bwd_kernel(KmapP p) {
  __shared__ float red[4];
  const int h = blockIdx.y, b = blockIdx.z;
  const int t = blockIdx.x * 256 + threadIdx.x;
  const bool live = t < p.T;
  const int tc = live ? t : 0;
  float u[M], gr[M];
  kmap_load<E, M>((const E*)p.a.ptr + (int64_t)b * p.a.sb + (int64_t)h * p.a.sh + (int64_t)tc * p.a.st, u);
  kmap_load<E, M>((const E*)p.dphi.ptr + (int64_t)b * p.dphi.sb + (int64_t)h * p.dphi.sh + (int64_t)tc * p.dphi.st,
                  gr);
  if (!live) {
#pragma unroll
    for (int j = 0; j < M; ++j) gr[j] = 0.f;
  }
  const float rinv = kmap_pre<M>(p, h, u);
  float drho = 0.f, dalpha = 0.f;
  // gr becomes dl (the gradient of the logits, or of u for relu2)
  if (p.kind == TS_KMAP_RELU2) {
    float mass = 0.f, sgh = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const float r = fmaxf(u[j], 0.f);
      mass += r * r;
      sgh += gr[j] * r * r;
    }
    const bool ok = mass > p.eps;
    const float inv = ok ? 1.0f / mass : 0.f;
    sgh *= inv;
#pragma unroll
    for (int j = 0; j < M; ++j) gr[j] = ok ? 2.0f * fmaxf(u[j], 0.f) * (gr[j] - sgh) * inv : 0.f;
  } else {
    const SoftStats s = kmap_soft_stats<M>(p, h, u);
    const float ise = 1.0f / s.se;
    const bool wok = s.sw > p.eps;
    const float isw = 1.0f / fmaxf(s.sw, p.eps);
    const float al = p.sparsity == TS_SPARSE_ST_BLEND ? p.alpha[h] : 0.f;
    const float cd = p.sparsity == TS_SPARSE_NONE ? 1.f : p.sparsity == TS_SPARSE_ST_BLEND ? 1.f - al : 0.f;
    const float cs = p.sparsity == TS_SPARSE_NONE ? 0.f : p.sparsity == TS_SPARSE_ST_BLEND ? al : 1.f;
    // row sums: sum gd dense, sum gs sparse, and the blend's dalpha
    float sdd = 0.f, sss = 0.f;
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const float sh = kmap_gain(p, h, j) * u[j] - s.mx;
      const float e = expf(sh);
      const float dense = e * ise;
      sdd += cd * gr[j] * dense;
      if (p.sparsity) {
        const float margin = sh - s.lr;
        const float soft = 1.0f / (1.0f + expf(-margin / p.temp));
        const float gate = p.sparsity == TS_SPARSE_SOFT ? soft : (margin >= 0.f ? 1.0f : 0.0f);
        const float sp = e * gate * isw;
        sss += cs * gr[j] * sp;
        if (p.sparsity == TS_SPARSE_ST_BLEND) dalpha += gr[j] * (sp - dense);
      }
    }
    float dmax = 0.f;
    int nmax = 0;
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const float l = kmap_gain(p, h, j) * u[j];
      const float sh = l - s.mx;
      const float e = expf(sh);
      const float dense = e * ise;
      float dl = dense * (cd * gr[j] - sdd);
      if (p.sparsity) {
        const float margin = sh - s.lr;
        const float soft = 1.0f / (1.0f + expf(-margin / p.temp));
        const float gate = p.sparsity == TS_SPARSE_SOFT ? soft : (margin >= 0.f ? 1.0f : 0.0f);
        // sparse = w / max(sum w, eps), w = e gate (the clamp passes no gradient to sum w)
        const float dw = wok ? (cs * gr[j] - sss) * isw : cs * gr[j] * isw;
        const float dmargin = dw * e * soft * (1.0f - soft) / p.temp;
        const float dsh = dw * gate * e + dmargin;
        drho += dmargin;
        dl += dsh;
        dmax -= dsh;
      }
      nmax += l == s.mx ? 1 : 0;
      gr[j] = dl;
    }
    // the max's gradient goes to the maximal logits in equal shares
    if (p.sparsity) {
      const float share = dmax / (float)nmax;
#pragma unroll
      for (int j = 0; j < M; ++j)
        if (kmap_gain(p, h, j) * u[j] == s.mx) gr[j] += share;
    }
    const float rc = p.sparsity ? p.rho[h] : 0.f;
    drho = (p.sparsity && rc >= p.eps && rc <= 1.0f - p.eps) ? -drho / rc : 0.f;
  }
  // du = gain dl (softmax) or dl (relu2); the per-feature control gradients
  // are du (shift) and dl u (gain)
  float sdu_a = 0.f, dgain_h = 0.f;
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const float du = p.kind == TS_KMAP_RELU2 ? gr[j] : kmap_gain(p, h, j) * gr[j];
    if (p.kind != TS_KMAP_RELU2 && p.gain_mode == 1) dgain_h += gr[j] * u[j];
    const float zn = u[j] - (p.shift ? p.shift[h * p.m + j] : 0.f);  // a * rinv
    sdu_a += du * zn;
    if (p.gain_mode == 2 && p.kind != TS_KMAP_RELU2) u[j] = gr[j] * u[j];  // per-feature dgain row
    gr[j] = du;
  }
  if (live) {
    // RMSNorm backward: da = rinv (du - (sum_i du_i zn_i / m) zn), zn = a rinv
    float da[M];
#pragma unroll
    for (int j = 0; j < M; ++j) da[j] = gr[j];
    if (p.rms) {
      // reload a (u may now hold the per-feature gain gradients)
      float a[M];
      kmap_load<E, M>((const E*)p.a.ptr + (int64_t)b * p.a.sb + (int64_t)h * p.a.sh + (int64_t)t * p.a.st, a);
      const float c = sdu_a / (float)p.m;
#pragma unroll
      for (int j = 0; j < M; ++j) da[j] = rinv * (gr[j] - c * a[j] * rinv);
    }
    kmap_store<E, M>((E*)p.da.ptr + (int64_t)b * p.da.sb + (int64_t)h * p.da.sh + (int64_t)t * p.da.st, da);
  }
  // per-workgroup partial sums of the control gradients
  const int part = b * gridDim.x + blockIdx.x;
  if (p.dshift_part) {
    for (int j = 0; j < M; ++j) {
      const float v = kmap_block_sum(live ? gr[j] : 0.f, red);
      if (threadIdx.x == 0) p.dshift_part[((size_t)part * p.H + h) * p.m + j] = v;
    }
  }
  if (p.dgain_part && p.gain_mode == 2 && p.kind != TS_KMAP_RELU2) {
    for (int j = 0; j < M; ++j) {
      const float v = kmap_block_sum(live ? u[j] : 0.f, red);
      if (threadIdx.x == 0) p.dgain_part[((size_t)part * p.H + h) * p.m + j] = v;
    }
  }
  if (p.dgain_part && p.gain_mode == 1 && p.kind != TS_KMAP_RELU2) {
    const float v = kmap_block_sum(live ? dgain_h : 0.f, red);
    if (threadIdx.x == 0) p.dgain_part[(size_t)part * p.H + h] = v;
  }
  if (p.drho_part) {
    const float v = kmap_block_sum(live ? drho : 0.f, red);
    if (threadIdx.x == 0) p.drho_part[(size_t)part * p.H + h] = v;
  }
  if (p.dalpha_part) {
    const float v = kmap_block_sum(live ? dalpha : 0.f, red);
    if (threadIdx.x == 0) p.dalpha_part[(size_t)part * p.H + h] = v;
  }
}

}  // namespace ts

namespace {

using ts::fail;

int kmap_width(int m) { return m == 16 ? 16 : m == 32 ? 32 : m == 48 ? 48 : m == 64 ? 64 : 0; }

int check_kmap(const ts_kmap_desc* d, const ts_kmap_params* prm) {
  if (!d || !prm) return fail(TS_ERR_VALUE, "kmap: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0 || d->m < 1) return fail(TS_ERR_VALUE, "kmap: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "kmap: unknown dtype");
  if (d->kind != TS_KMAP_SOFTMAX && d->kind != TS_KMAP_RELU2) return fail(TS_ERR_VALUE, "kmap: unknown map");
  if (!kmap_width(d->m)) return fail(TS_ERR_NOT_IMPLEMENTED, "kmap: feature width %d (16, 32, 48 or 64)", d->m);
  if (d->gain_mode < 0 || d->gain_mode > 2 || (d->gain_mode && !prm->gain))
    return fail(TS_ERR_VALUE, "kmap: gain mode %d without its gains", d->gain_mode);
  if (d->sparsity < TS_SPARSE_NONE || d->sparsity > TS_SPARSE_ST_BLEND) return fail(TS_ERR_VALUE, "kmap: unknown sparsity");
  if (d->kind == TS_KMAP_RELU2 && (d->sparsity || d->gain_mode))
    return fail(TS_ERR_VALUE, "kmap: the ReLU^2 ridge takes no gain or sparsity");
  if (d->sparsity && !prm->rho) return fail(TS_ERR_VALUE, "kmap: sparsity needs the relative threshold");
  if (d->sparsity == TS_SPARSE_ST_BLEND && !prm->alpha) return fail(TS_ERR_VALUE, "kmap: the blend needs alpha");
  if (d->sparsity && !(d->temperature > 0.f)) return fail(TS_ERR_VALUE, "relative threshold temperature must be positive");
  if (d->H > 65535 || d->B > 65535) return fail(TS_ERR_NOT_IMPLEMENTED, "kmap: too many heads or batches");
  return TS_OK;
}

bool rows16(const ts_strided& s, int es) {
  return s.ptr && ((uintptr_t)s.ptr & 15) == 0 && (s.sb * es) % 16 == 0 && (s.sh * es) % 16 == 0 &&
         (s.st * es) % 16 == 0;
}

void fill_kmap(const ts_kmap_desc* d, const ts_kmap_params* prm, ts::KmapP& p) {
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.m = d->m; p.kind = d->kind; p.rms = d->rms ? 1 : 0;
  p.gain_mode = d->gain_mode; p.sparsity = d->sparsity;
  p.gain = d->gain; p.temp = d->temperature; p.eps = d->eps;
  p.shift = prm->shift; p.gainv = prm->gain; p.rho = prm->rho; p.alpha = prm->alpha;
}

template <typename E>
void launch_kmap(int m, bool bwd, dim3 grid, hipStream_t s, const ts::KmapP& p) {
#define TS_KMAP_CASE(M)                                                                            \
  if (bwd) hipLaunchKernelGGL((ts::kmap_bwd_kernel<E, M>), grid, dim3(256), 0, s, p);             \
  else hipLaunchKernelGGL((ts::kmap_fwd_kernel<E, M>), grid, dim3(256), 0, s, p);
  switch (m) {
    case 16: { TS_KMAP_CASE(16) } break;
    case 32: { TS_KMAP_CASE(32) } break;
    case 48: { TS_KMAP_CASE(48) } break;
    default: { TS_KMAP_CASE(64) } break;
  }
#undef TS_KMAP_CASE
}

int kmap_run(const ts_kmap_desc* d, const ts::KmapP& p, bool bwd, hipStream_t stream, const char* what) {
  if ((int64_t)d->B * d->T == 0) return TS_OK;
  const dim3 grid((unsigned)((d->T + 255) / 256), (unsigned)d->H, (unsigned)d->B);
  if (d->dtype == TS_BF16) launch_kmap<ts::bf16>(d->m, bwd, grid, stream, p);
  else launch_kmap<float>(d->m, bwd, grid, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_kmap_parts(const ts_kmap_desc* d, const ts_kmap_params* prm, int32_t* parts) {
  int rc = check_kmap(d, prm);
  if (rc) return rc;
  if (parts) *parts = (int32_t)(d->B * ((d->T + 255) / 256));
  return TS_OK;
}

int ts_kmap_fwd(const ts_kmap_desc* d, const ts_kmap_params* prm, ts_strided a, ts_strided phi, hipStream_t stream) {
  int rc = check_kmap(d, prm);
  if (rc) return rc;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!rows16(a, es) || !rows16(phi, es)) return fail(TS_ERR_VALUE, "kmap: rows must be 16-byte aligned");
  ts::KmapP p;
  fill_kmap(d, prm, p);
  p.a = a; p.phi = phi;
  return kmap_run(d, p, false, stream, "kmap");
}

int ts_kmap_bwd(const ts_kmap_desc* d, const ts_kmap_params* prm, ts_strided a, ts_strided dphi,
                const ts_kmap_grads* g, hipStream_t stream) {
  int rc = check_kmap(d, prm);
  if (rc) return rc;
  if (!g) return fail(TS_ERR_VALUE, "kmap bwd: missing gradients");
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  if (!rows16(a, es) || !rows16(dphi, es) || !rows16(g->da, es))
    return fail(TS_ERR_VALUE, "kmap bwd: rows must be 16-byte aligned");
  if ((g->dgain_part && !d->gain_mode) || (g->drho_part && !d->sparsity) ||
      (g->dalpha_part && d->sparsity != TS_SPARSE_ST_BLEND) || (g->dshift_part && !prm->shift))
    return fail(TS_ERR_VALUE, "kmap bwd: gradient of an absent control");
  ts::KmapP p;
  fill_kmap(d, prm, p);
  p.a = a; p.dphi = dphi; p.da = g->da;
  p.dshift_part = g->dshift_part; p.dgain_part = g->dgain_part; p.drho_part = g->drho_part;
  p.dalpha_part = g->dalpha_part;
  return kmap_run(d, p, true, stream, "kmap bwd");
}

}  // extern "C"
