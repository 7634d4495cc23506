// Read epilogue (normalised read + residual + output gate) and decayed
// prefix sums for gfx950.  Both are HBM-bound streaming kernels.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct ReadP {
  int B, H, T, d, normalize, gate;
  float s, eps;
  ts_strided num, mass, resid, g, y, dy, dnum, dmass, dresid, dg;
  const float* gbias;  // [H, d] added to the gate pre-activation (or null)
};

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float dsilu(float x) {
  const float sg = 1.0f / (1.0f + expf(-x));
  return sg * (1.0f + x * (1.0f - sg));
}

template <typename E>
__device__ __forceinline__ const E* rowp(const ts_strided& s, int b, int h, int t) {
  return (const E*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st;
}
template <typename E>
__device__ __forceinline__ E* rowp_w(const ts_strided& s, int b, int h, int t) {
  return (E*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st;
}

template <typename E>
__device__ __forceinline__ void ld_vec(const E* p, float* out) {
  Vec16<E> v;
  v.raw = *(const uint4*)p;
#pragma unroll
  for (int e = 0; e < Vec16<E>::N; ++e) out[e] = tof(v.e[e]);
}
template <typename E>
__device__ __forceinline__ void st_vec(E* p, const float* in) {
  Vec16<E> v;
#pragma unroll
  for (int e = 0; e < Vec16<E>::N; ++e) v.e[e] = cvt<E>(in[e]);
  *(uint4*)p = v.raw;
}

// Work mapping of the read kernels: a row (one (b, h, t)) is split into
// 16-byte chunks; `p2` consecutive lanes (a power of two >= chunks per row)
// own one row, so every load and store instruction covers whole contiguous
// row segments, and a row reduction is a log2(p2)-step butterfly.
struct RowMap {
  int64_t row;
  int chunk;
  bool active;
};

__device__ __forceinline__ RowMap row_map(int64_t nrows, int nchunk, int p2) {
  const int64_t gtid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  RowMap r;
  r.row = gtid / p2;
  r.chunk = (int)(gtid % p2);
  r.active = r.row < nrows && r.chunk < nchunk;
  return r;
}

__device__ __forceinline__ float row_sum(float v, int p2) {
  for (int o = 1; o < p2; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// y = (resid + s * num / (mass + eps)) * silu(g)     (engine.py:440-442, 526-528; gates.py:34-40)
template <typename E>
__global__ __launch_bounds__(256) void read_fwd_kernel(ReadP p, int p2) {
  constexpr int N = Vec16<E>::N;
  const int64_t nrows = (int64_t)p.B * p.H * p.T;
  const RowMap rm = row_map(nrows, p.d / N, p2);
  if (!rm.active) return;
  const int t = (int)(rm.row % p.T);
  const int h = (int)((rm.row / p.T) % p.H);
  const int b = (int)(rm.row / ((int64_t)p.T * p.H));
  const int c = rm.chunk * N;
  float scale = p.s;
  if (p.normalize) scale = p.s / (rowp<float>(p.mass, b, h, t)[0] + p.eps);
  float nv[N], rv[N], gv[N], out[N];
  ld_vec<E>(rowp<E>(p.num, b, h, t) + c, nv);
  if (p.resid.ptr) ld_vec<E>(rowp<E>(p.resid, b, h, t) + c, rv);
  if (p.gate) {
    ld_vec<E>(rowp<E>(p.g, b, h, t) + c, gv);
    if (p.gbias)
#pragma unroll
      for (int e = 0; e < N; ++e) gv[e] += p.gbias[h * p.d + c + e];
  }
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float v = (p.resid.ptr ? rv[e] : 0.0f) + scale * nv[e];
    out[e] = p.gate ? v * silu(gv[e]) : v;
  }
  st_vec<E>(rowp_w<E>(p.y, b, h, t) + c, out);
}

template <typename E>
__global__ __launch_bounds__(256) void read_bwd_kernel(ReadP p, int p2) {
  constexpr int N = Vec16<E>::N;
  const int64_t nrows = (int64_t)p.B * p.H * p.T;
  const RowMap rm = row_map(nrows, p.d / N, p2);
  // inactive lanes still take part in the row butterfly with zeros
  const int64_t row = rm.row < nrows ? rm.row : nrows - 1;
  const int t = (int)(row % p.T);
  const int h = (int)((row / p.T) % p.H);
  const int b = (int)(row / ((int64_t)p.T * p.H));
  const int c = rm.chunk * N;
  float denom = 1.0f;
  if (p.normalize) denom = rowp<float>(p.mass, b, h, t)[0] + p.eps;
  const float scale = p.s / denom;
  float dot = 0.0f;
  if (rm.active) {
    float nv[N], rv[N], gv[N], dv[N], o_dnum[N], o_dg[N], o_dres[N];
    ld_vec<E>(rowp<E>(p.num, b, h, t) + c, nv);
    ld_vec<E>(rowp<E>(p.dy, b, h, t) + c, dv);
    if (p.resid.ptr) ld_vec<E>(rowp<E>(p.resid, b, h, t) + c, rv);
    if (p.gate) {
      ld_vec<E>(rowp<E>(p.g, b, h, t) + c, gv);
      if (p.gbias)
#pragma unroll
        for (int e = 0; e < N; ++e) gv[e] += p.gbias[h * p.d + c + e];
    }
#pragma unroll
    for (int e = 0; e < N; ++e) {
      float dpre = dv[e];
      if (p.gate) {
        const float ypre = (p.resid.ptr ? rv[e] : 0.0f) + scale * nv[e];
        o_dg[e] = dv[e] * ypre * dsilu(gv[e]);
        dpre = dv[e] * silu(gv[e]);
      }
      o_dnum[e] = scale * dpre;
      o_dres[e] = dpre;
      dot += dpre * nv[e];
    }
    st_vec<E>(rowp_w<E>(p.dnum, b, h, t) + c, o_dnum);
    if (p.dresid.ptr) st_vec<E>(rowp_w<E>(p.dresid, b, h, t) + c, o_dres);
    if (p.gate) st_vec<E>(rowp_w<E>(p.dg, b, h, t) + c, o_dg);
  }
  if (p.normalize) {
    dot = row_sum(dot, p2);
    if (rm.active && rm.chunk == 0) rowp_w<float>(p.dmass, b, h, t)[0] = -p.s * dot / (denom * denom);
  }
}

// z_t = a_t z_{t-1} + x_t  over T for every (b, h, feature).
__global__ __launch_bounds__(256) void wcumsum_kernel(int B, int H, int T, int F, int ret, int reverse,
                                                      ts_strided x, ts_strided out, const float* log_alpha,
                                                      ts_strided decay) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)B * H * F) return;
  const int f = (int)(idx % F);
  const int h = (int)((idx / F) % H);
  const int b = (int)(idx / ((int64_t)F * H));
  const float* xb = (const float*)x.ptr + (int64_t)b * x.sb + (int64_t)h * x.sh + f;
  float* ob = (float*)out.ptr + (int64_t)b * out.sb + (int64_t)h * out.sh + f;
  const float a_static = ret == TS_RET_STATIC ? expf(log_alpha[h]) : 1.0f;
  const float* db = ret == TS_RET_STREAM
                        ? (const float*)decay.ptr + (int64_t)b * decay.sb + (int64_t)h * decay.sh
                        : nullptr;
  float z = 0.0f;
  for (int s = 0; s < T; ++s) {
    const int tp = reverse ? T - 1 - s : s;
    float a = a_static;
    if (db) {
      // a_t multiplies the state when stepping into t; anti-causal scans
      // step from t+1 into t and use the decay of t+1.
      const int src = reverse ? tp + 1 : tp;
      a = src < T ? expf(db[(int64_t)src * decay.st]) : 1.0f;
    }
    z = (s == 0 ? 0.0f : a * z) + xb[(int64_t)tp * x.st];
    ob[(int64_t)tp * out.st] = z;
  }
}

// out[i] = scale * (sum_s a[s][i] + sum_s b[s][i]): the partial weight-gradient
// slots of one or two ts_feature_bwd calls.  A block covers `opb` consecutive
// outputs; its 256 / opb thread rows split the slots between them (four
// independent loads in flight per thread) and combine through LDS.
__global__ __launch_bounds__(256) void sum_slots_kernel(const float* a, int na, const float* b, int nb, int64_t n,
                                                        void* out, int out_bf16, float scale, int opb) {
  __shared__ float red[256];
  const int tid = threadIdx.x;
  const int c = tid % opb, j = tid / opb, sub = 256 / opb;
  const int64_t i = (int64_t)blockIdx.x * opb + c;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (i < n) {
    const int total = na + nb;
    int s = j;
    for (; s + 3 * sub < total; s += 4 * sub) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = s + u * sub;
        acc[u] += t < na ? a[(int64_t)t * n + i] : b[(int64_t)(t - na) * n + i];
      }
    }
    for (; s < total; s += sub) acc[0] += s < na ? a[(int64_t)s * n + i] : b[(int64_t)(s - na) * n + i];
  }
  red[tid] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  if (j == 0 && i < n) {
    float v = 0.f;
    for (int r = 0; r < sub; ++r) v += red[r * opb + c];
    v *= scale;
    if (out_bf16)
      ((bf16*)out)[i] = (bf16)v;
    else
      ((float*)out)[i] = v;
  }
}

// parts[blk][c] = sum of x[r * stride + c] over the `rows_per_block` rows of
// block blk.  A block is 256 / (cols / 8) row lanes x (cols / 8) column
// groups of eight (one 16-byte load of bf16, two of fp32); row lanes step by
// their count with four loads in flight and combine through LDS.
template <typename E>
__global__ __launch_bounds__(256) void col_sums_kernel(const E* x, int64_t rows, int cols, int64_t stride,
                                                       float* parts, int rows_per_block) {
  __shared__ float red[256 * 8];
  const int groups = cols / 8;
  const int tid = threadIdx.x;
  const int cg = tid % groups, rl = tid / groups, lanes = 256 / groups;
  const int c = cg * 8;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < rows ? r0 + rows_per_block : rows;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (rl < lanes) {
    int64_t r = r0 + rl;
    for (; r + 3 * lanes < r1; r += 4 * lanes) {
      Vec16<E> v[4][8 / Vec16<E>::N];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int h = 0; h < 8 / Vec16<E>::N; ++h)
          v[u][h].raw = *(const uint4*)(x + (r + u * lanes) * stride + c + h * Vec16<E>::N);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int h = 0; h < 8 / Vec16<E>::N; ++h)
#pragma unroll
          for (int e = 0; e < Vec16<E>::N; ++e) acc[h * Vec16<E>::N + e] += tof(v[u][h].e[e]);
    }
    for (; r < r1; r += lanes) {
#pragma unroll
      for (int h = 0; h < 8 / Vec16<E>::N; ++h) {
        Vec16<E> v;
        v.raw = *(const uint4*)(x + r * stride + c + h * Vec16<E>::N);
#pragma unroll
        for (int e = 0; e < Vec16<E>::N; ++e) acc[h * Vec16<E>::N + e] += tof(v.e[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[tid * 8 + e] = acc[e];
  __syncthreads();
  if (rl == 0) {
    float* out = parts + (int64_t)blockIdx.x * cols + c;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = 0.f;
      for (int l = 0; l < lanes; ++l) v += red[(l * groups + cg) * 8 + e];
      out[e] = v;
    }
  }
}

}  // namespace ts

namespace {

using ts::fail;

int check_read(const ts_read_desc* d) {
  if (!d) return fail(TS_ERR_VALUE, "read: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0 || d->d < 1) return fail(TS_ERR_VALUE, "read: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "read: unknown dtype");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  if (d->d % vec) return fail(TS_ERR_VALUE, "read: width %d is not a multiple of 16 bytes", d->d);
  if (d->d / vec > 64) return fail(TS_ERR_NOT_IMPLEMENTED, "read: width %d is too wide", d->d);
  return TS_OK;
}

// Lanes per row: chunks of 16 bytes rounded up to a power of two (<= 64).
int lanes_per_row(const ts_read_desc* d) {
  const int chunks = d->d / (d->dtype == TS_BF16 ? 8 : 4);
  int p2 = 1;
  while (p2 < chunks) p2 <<= 1;
  return p2;
}

void fill_read(const ts_read_desc* d, ts::ReadP& p) {
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.d = d->d;
  p.normalize = d->normalize; p.gate = d->gate; p.s = d->scale; p.eps = d->eps;
}

int finish(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_read_fwd(const ts_read_desc* d, const ts_read_io* io, hipStream_t stream) {
  int rc = check_read(d);
  if (rc) return rc;
  if (!io || !io->num.ptr || !io->y.ptr) return fail(TS_ERR_VALUE, "read: missing tensors");
  if (d->normalize && !io->mass.ptr) return fail(TS_ERR_VALUE, "read: missing mass");
  if (d->gate && !io->g.ptr) return fail(TS_ERR_VALUE, "read: missing gate");
  const int64_t rows = (int64_t)d->B * d->H * d->T;
  if (rows == 0) return TS_OK;
  ts::ReadP p;
  fill_read(d, p);
  p.num = io->num; p.mass = io->mass; p.resid = io->resid; p.g = io->g; p.y = io->y;
  p.gbias = io->g_bias;
  const int p2 = lanes_per_row(d);
  const dim3 grid((unsigned)((rows * p2 + 255) / 256));
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL(ts::read_fwd_kernel<ts::bf16>, grid, dim3(256), 0, stream, p, p2);
  else
    hipLaunchKernelGGL(ts::read_fwd_kernel<float>, grid, dim3(256), 0, stream, p, p2);
  return finish("read");
}

int ts_read_bwd(const ts_read_desc* d, const ts_read_bwd_io* io, hipStream_t stream) {
  int rc = check_read(d);
  if (rc) return rc;
  if (!io || !io->num.ptr || !io->dy.ptr || !io->dnum.ptr) return fail(TS_ERR_VALUE, "read bwd: missing tensors");
  if (d->normalize && (!io->mass.ptr || !io->dmass.ptr)) return fail(TS_ERR_VALUE, "read bwd: missing mass");
  if (d->gate && (!io->g.ptr || !io->dg.ptr)) return fail(TS_ERR_VALUE, "read bwd: missing gate");
  const int64_t rows = (int64_t)d->B * d->H * d->T;
  if (rows == 0) return TS_OK;
  ts::ReadP p;
  fill_read(d, p);
  p.num = io->num; p.mass = io->mass; p.resid = io->resid; p.g = io->g; p.dy = io->dy;
  p.dnum = io->dnum; p.dmass = io->dmass; p.dresid = io->dresid; p.dg = io->dg;
  p.gbias = io->g_bias;
  const int p2 = lanes_per_row(d);
  const dim3 grid((unsigned)((rows * p2 + 255) / 256));
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL(ts::read_bwd_kernel<ts::bf16>, grid, dim3(256), 0, stream, p, p2);
  else
    hipLaunchKernelGGL(ts::read_bwd_kernel<float>, grid, dim3(256), 0, stream, p, p2);
  return finish("read bwd");
}

int ts_sum_slots(const float* a, int32_t na, const float* b, int32_t nb, int64_t n, void* out, int32_t out_dtype,
                 float scale, hipStream_t stream) {
  if (n < 0 || na < 0 || nb < 0) return fail(TS_ERR_VALUE, "sum_slots: bad sizes");
  if ((na && !a) || (nb && !b) || !out) return fail(TS_ERR_VALUE, "sum_slots: missing buffers");
  if (out_dtype != TS_BF16 && out_dtype != TS_F32) return fail(TS_ERR_VALUE, "sum_slots: unknown dtype");
  if (n == 0) return TS_OK;
  // outputs per block: as many as keep >= 512 blocks, at least 4 slot rows per output
  int opb = 64;
  while (opb > 4 && (n + opb - 1) / opb < 512) opb >>= 1;
  hipLaunchKernelGGL(ts::sum_slots_kernel, dim3((unsigned)((n + opb - 1) / opb)), dim3(256), 0, stream, a, na, b, nb,
                     n, out, out_dtype == TS_BF16 ? 1 : 0, scale, opb);
  return finish("sum_slots");
}

int ts_col_sums(const void* x, int32_t dtype, int64_t rows, int32_t cols, int64_t row_stride, float* parts,
                int32_t slices, hipStream_t stream) {
  if (!x || !parts || rows < 0 || cols < 0 || slices < 1) return fail(TS_ERR_VALUE, "col_sums: bad arguments");
  if (dtype != TS_BF16 && dtype != TS_F32) return fail(TS_ERR_VALUE, "col_sums: unknown dtype");
  if (cols % 8 || row_stride % 8 || ((uintptr_t)x & 15u))
    return fail(TS_ERR_VALUE, "col_sums: columns and rows must be 8-element aligned");
  if (cols / 8 > 256) return fail(TS_ERR_NOT_IMPLEMENTED, "col_sums: more than 2048 columns");
  if (cols == 0) return TS_OK;
  const int rows_per_block = (int)((rows + slices - 1) / slices);
  if (dtype == TS_BF16)
    hipLaunchKernelGGL(ts::col_sums_kernel<ts::bf16>, dim3((unsigned)slices), dim3(256), 0, stream,
                       (const ts::bf16*)x, rows, cols, row_stride, parts, rows_per_block);
  else
    hipLaunchKernelGGL(ts::col_sums_kernel<float>, dim3((unsigned)slices), dim3(256), 0, stream, (const float*)x,
                       rows, cols, row_stride, parts, rows_per_block);
  return finish("col_sums");
}

int ts_wcumsum(const ts_wcumsum_desc* d, ts_strided x, ts_strided out, const float* log_alpha,
               ts_strided decay, hipStream_t stream) {
  if (!d || d->B < 1 || d->H < 1 || d->T < 0 || d->F < 1) return fail(TS_ERR_VALUE, "wcumsum: bad shape");
  if (!x.ptr || !out.ptr) return fail(TS_ERR_VALUE, "wcumsum: missing tensors");
  if (d->retention == TS_RET_STATIC && !log_alpha) return fail(TS_ERR_VALUE, "wcumsum: missing log_alpha");
  if (d->retention == TS_RET_STREAM && !decay.ptr) return fail(TS_ERR_VALUE, "wcumsum: missing decay");
  const int64_t n = (int64_t)d->B * d->H * d->F;
  if (d->T == 0) return TS_OK;
  hipLaunchKernelGGL(ts::wcumsum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, d->B, d->H, d->T,
                     d->F, d->retention, d->reverse, x, out, log_alpha, decay);
  return finish("wcumsum");
}

}  // extern "C"
