// Row-wise elementwise glue of the hybrid language model's blocks (gfx950):
// the residual mixes and scaled residual adds, and the ReLU^2 of the MLP.
//
//   scale-add:  y = a (.) x + b (.) u        a, b: per-column factors [W] of the
//                                            rows' dtype (NULL: 1), rows of width W
//     backward: dx = a (.) g,  du = b (.) g,
//               da = sum_rows g (.) x,  db = sum_rows g (.) u
//   ReLU^2:     h = relu(z)^2,  dz = 2 relu(z) g
//
// fp32 arithmetic, one rounding at each store.  Eight consecutive columns per
// thread (one 16-byte access of bf16, two of fp32).  The column sums of the
// backward are per-workgroup fp32 partials [P][W] (each workgroup owns a
// fixed run of rows and keeps its columns' sums in registers, then adds its
// row lanes through LDS), summed by ts_sum_slots in slot order, so results
// do not depend on timing.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

template <typename E>
__device__ __forceinline__ void rg_ld8(const E* p, float* v) {
  if constexpr (sizeof(E) == 2) {
    const bf16x8 b = __builtin_bit_cast(bf16x8, *(const uint4*)p);
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
__device__ __forceinline__ void rg_st8(E* p, const float* v) {
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

// Eight per-column factors (of the rows' dtype) from column c, or ones.
template <typename E>
__device__ __forceinline__ void rg_factors(const E* f, int c, float* v) {
  if (f) {
    rg_ld8<E>(f + c, v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 1.0f;
  }
}

struct GlueP {
  int64_t rows;
  int W;
  const void* x;
  const void* u;
  const void* g;
  const void* a;  // per-column factors [W] of the rows' dtype (NULL: 1)
  const void* b;
  void* y;   // forward output, or dx
  void* du;
  float* da_part;  // [P][W]
  float* db_part;
  int64_t rows_per_block;
};

template <typename E>
__global__ __launch_bounds__(256) void scale_add_fwd_kernel(GlueP p) {
  const int vw = p.W / 8;
  const int64_t n = p.rows * vw;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int c = (int)(i % vw) * 8;
    const int64_t off = i * 8;
    float x[8], u[8], a[8], b[8];
    rg_ld8<E>((const E*)p.x + off, x);
    rg_ld8<E>((const E*)p.u + off, u);
    rg_factors<E>((const E*)p.a, c, a);
    rg_factors<E>((const E*)p.b, c, b);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = fmaf(a[e], x[e], b[e] * u[e]);
    rg_st8<E>((E*)p.y + off, x);
  }
}

// A workgroup of 256 threads is (256 / vw) row lanes x vw column groups
// (vw = W / 8 <= 256) and walks rows [blk * rows_per_block, ...).
template <typename E>
__global__ __launch_bounds__(256) void scale_add_bwd_kernel(GlueP p) {
  __shared__ float red[2][256 * 8];
  const int vw = p.W / 8;
  const int tid = threadIdx.x;
  const int cg = tid % vw, rl = tid / vw, lanes = 256 / vw;
  const int c = cg * 8;
  const int64_t r0 = (int64_t)blockIdx.x * p.rows_per_block;
  const int64_t r1 = min(r0 + p.rows_per_block, p.rows);
  float a[8], b[8], sa[8], sb[8];
  rg_factors<E>((const E*)p.a, c, a);
  rg_factors<E>((const E*)p.b, c, b);
#pragma unroll
  for (int e = 0; e < 8; ++e) sa[e] = sb[e] = 0.f;
  if (rl < lanes) {
    for (int64_t r = r0 + rl; r < r1; r += lanes) {
      const int64_t off = r * p.W + c;
      float g[8];
      rg_ld8<E>((const E*)p.g + off, g);
      if (p.y) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = a[e] * g[e];
        rg_st8<E>((E*)p.y + off, o);
      }
      if (p.du) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = b[e] * g[e];
        rg_st8<E>((E*)p.du + off, o);
      }
      if (p.da_part) {
        float x[8];
        rg_ld8<E>((const E*)p.x + off, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) sa[e] = fmaf(g[e], x[e], sa[e]);
      }
      if (p.db_part) {
        float u[8];
        rg_ld8<E>((const E*)p.u + off, u);
#pragma unroll
        for (int e = 0; e < 8; ++e) sb[e] = fmaf(g[e], u[e], sb[e]);
      }
    }
  }
  if (!p.da_part && !p.db_part) return;  // uniform
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[0][tid * 8 + e] = sa[e];
    red[1][tid * 8 + e] = sb[e];
  }
  __syncthreads();
  if (rl == 0) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float* dst = k == 0 ? p.da_part : p.db_part;
      if (!dst) continue;
      dst += (int64_t)blockIdx.x * p.W + c;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = 0.f;
        for (int l = 0; l < lanes; ++l) v += red[k][(l * vw + cg) * 8 + e];
        dst[e] = v;
      }
    }
  }
}

template <typename E, bool BWD>
__global__ __launch_bounds__(256) void relu2_kernel(GlueP p) {
  const int64_t n = p.rows * (p.W / 8);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t off = i * 8;
    float z[8];
    rg_ld8<E>((const E*)p.x + off, z);
    if constexpr (BWD) {
      float g[8];
      rg_ld8<E>((const E*)p.g + off, g);
#pragma unroll
      for (int e = 0; e < 8; ++e) z[e] = (2.0f * fmaxf(z[e], 0.0f)) * g[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float r = fmaxf(z[e], 0.0f);
        z[e] = r * r;
      }
    }
    rg_st8<E>((E*)p.y + off, z);
  }
}

// Softcapped cross entropy: one wave per row of V logits (V / 64 per lane,
// in runs of eight), c = cap tanh(z / cap) in fp32, the row's max and
// exp-sum by xor butterflies.  The backward recomputes c from z and the
// forward's log-sum-exp, so no [rows, V] fp32 tensor is ever stored.
template <typename E, bool BWD>
__global__ __launch_bounds__(256) void softcap_xent_kernel(GlueP p, const int64_t* target, float cap, float* loss,
                                                           float* lse, const float* g, float g_scale) {
  constexpr int kMaxRun = 8;  // runs of eight logits per lane: V <= 4096
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;  // uniform per wave
  const int runs = p.W / 512 > 0 ? p.W / 512 : 1;  // eight-logit runs per lane (W a multiple of 512, or 8..504)
  const E* zr = (const E*)p.x + row * p.W;
  const float inv_cap = 1.0f / cap;
  float c[kMaxRun][8];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kMaxRun; ++k) {
    const int col = (k * 64 + lane) * 8;
    if (k < runs && col < p.W) {
      rg_ld8<E>(zr + col, c[k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        c[k][e] = cap * tanhf(c[k][e] * inv_cap);
        mx = fmaxf(mx, c[k][e]);
      }
    }
  }
  for (int o = 1; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  const int64_t y = target[row];
  float l;
  if constexpr (!BWD) {
    float se = 0.f, cy = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxRun; ++k) {
      const int col = (k * 64 + lane) * 8;
      if (k < runs && col < p.W) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          se += __expf(c[k][e] - mx);
          if (col + e == y) cy = c[k][e];
        }
      }
    }
    for (int o = 1; o < 64; o <<= 1) {
      se += __shfl_xor(se, o, 64);
      cy += __shfl_xor(cy, o, 64);
    }
    l = mx + __logf(se);
    if (lane == 0) {
      lse[row] = l;
      // a target outside [0, W) has no logit: NaN rather than a wrong loss
      loss[row] = (y >= 0 && y < p.W) ? l - cy : __builtin_nanf("");
    }
  } else {
    l = lse[row];
    const float gr = (y >= 0 && y < p.W) ? *g * g_scale : __builtin_nanf("");
    E* dz = (E*)p.y + row * p.W;
#pragma unroll
    for (int k = 0; k < kMaxRun; ++k) {
      const int col = (k * 64 + lane) * 8;
      if (k < runs && col < p.W) {
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float t = c[k][e] * inv_cap;  // tanh(z / cap)
          const float pr = __expf(c[k][e] - l) - (col + e == y ? 1.0f : 0.0f);
          o[e] = gr * pr * (1.0f - t * t);
        }
        rg_st8<E>(dz + col, o);
      }
    }
  }
}

}  // namespace ts

namespace {

using ts::fail;

constexpr int kGlueBlocks = 2048;  // grid of the elementwise walks (grid-stride)
constexpr int kGlueParts = 1024;   // row slices of the backward's column sums

int check_rows(const ts_rows_desc* d, const char* what) {
  if (!d || d->rows < 0 || d->W < 8) return fail(TS_ERR_VALUE, "%s: bad shape", what);
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "%s: unknown dtype", what);
  if (d->W % 8) return fail(TS_ERR_NOT_IMPLEMENTED, "%s: width %d (a multiple of 8)", what, d->W);
  return TS_OK;
}

bool aligned(const void* p) { return !p || ((uintptr_t)p & 15u) == 0; }

int glue_finish(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TS_OK;
}

unsigned walk_grid(const ts_rows_desc* d) {
  const int64_t n = d->rows * (d->W / 8);
  const int64_t blocks = (n + 255) / 256;
  return (unsigned)(blocks < kGlueBlocks ? (blocks > 0 ? blocks : 1) : kGlueBlocks);
}

}  // namespace

extern "C" {

int ts_scale_add_fwd(const ts_rows_desc* d, const void* x, const void* u, const void* a, const void* b, void* y,
                     hipStream_t stream) {
  int rc = check_rows(d, "scale_add");
  if (rc) return rc;
  if (!x || !u || !y) return fail(TS_ERR_VALUE, "scale_add: missing x, u or y");
  if (!aligned(x) || !aligned(u) || !aligned(y) || !aligned(a) || !aligned(b))
    return fail(TS_ERR_VALUE, "scale_add: tensors and factors must be 16-byte aligned");
  if (d->rows == 0) return TS_OK;
  ts::GlueP p;
  memset(&p, 0, sizeof(p));
  p.rows = d->rows; p.W = d->W; p.x = x; p.u = u; p.a = a; p.b = b; p.y = y;
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL(ts::scale_add_fwd_kernel<ts::bf16>, dim3(walk_grid(d)), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(ts::scale_add_fwd_kernel<float>, dim3(walk_grid(d)), dim3(256), 0, stream, p);
  return glue_finish("scale_add");
}

int ts_scale_add_parts(const ts_rows_desc* d, int32_t* parts) {
  int rc = check_rows(d, "scale_add");
  if (rc) return rc;
  if (d->W / 8 > 256) return fail(TS_ERR_NOT_IMPLEMENTED, "scale_add: more than 2048 columns");
  const int64_t p = d->rows < kGlueParts ? (d->rows > 0 ? d->rows : 1) : kGlueParts;
  if (parts) *parts = (int32_t)p;
  return TS_OK;
}

int ts_scale_add_bwd(const ts_rows_desc* d, const void* g, const void* x, const void* u, const void* a,
                     const void* b, void* dx, void* du, float* da_part, float* db_part, hipStream_t stream) {
  int32_t parts = 0;
  int rc = ts_scale_add_parts(d, &parts);
  if (rc) return rc;
  if (!g || (da_part && !x) || (db_part && !u)) return fail(TS_ERR_VALUE, "scale_add bwd: missing g, x or u");
  if (!aligned(g) || !aligned(x) || !aligned(u) || !aligned(dx) || !aligned(du) || !aligned(a) || !aligned(b) ||
      !aligned(da_part) || !aligned(db_part))
    return fail(TS_ERR_VALUE, "scale_add bwd: tensors, factors and partials must be 16-byte aligned");
  // no rows: the one workgroup writes zero partials (if any are wanted)
  if (d->rows == 0 && !da_part && !db_part) return TS_OK;
  ts::GlueP p;
  memset(&p, 0, sizeof(p));
  p.rows = d->rows; p.W = d->W; p.g = g; p.x = x; p.u = u; p.a = a; p.b = b;
  p.y = dx; p.du = du; p.da_part = da_part; p.db_part = db_part;
  p.rows_per_block = (d->rows + parts - 1) / parts;
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL(ts::scale_add_bwd_kernel<ts::bf16>, dim3((unsigned)parts), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(ts::scale_add_bwd_kernel<float>, dim3((unsigned)parts), dim3(256), 0, stream, p);
  return glue_finish("scale_add bwd");
}

int ts_relu2_fwd(const ts_rows_desc* d, const void* z, void* h, hipStream_t stream) {
  int rc = check_rows(d, "relu2");
  if (rc) return rc;
  if (!z || !h || !aligned(z) || !aligned(h)) return fail(TS_ERR_VALUE, "relu2: z and h must be 16-byte aligned");
  if (d->rows == 0) return TS_OK;
  ts::GlueP p;
  memset(&p, 0, sizeof(p));
  p.rows = d->rows; p.W = d->W; p.x = z; p.y = h;
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL((ts::relu2_kernel<ts::bf16, false>), dim3(walk_grid(d)), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((ts::relu2_kernel<float, false>), dim3(walk_grid(d)), dim3(256), 0, stream, p);
  return glue_finish("relu2");
}

int ts_relu2_bwd(const ts_rows_desc* d, const void* z, const void* g, void* dz, hipStream_t stream) {
  int rc = check_rows(d, "relu2 bwd");
  if (rc) return rc;
  if (!z || !g || !dz || !aligned(z) || !aligned(g) || !aligned(dz))
    return fail(TS_ERR_VALUE, "relu2 bwd: z, g and dz must be 16-byte aligned");
  if (d->rows == 0) return TS_OK;
  ts::GlueP p;
  memset(&p, 0, sizeof(p));
  p.rows = d->rows; p.W = d->W; p.x = z; p.g = g; p.y = dz;
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL((ts::relu2_kernel<ts::bf16, true>), dim3(walk_grid(d)), dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((ts::relu2_kernel<float, true>), dim3(walk_grid(d)), dim3(256), 0, stream, p);
  return glue_finish("relu2 bwd");
}

int ts_softcap_xent_fwd(const ts_rows_desc* d, const void* z, const int64_t* target, float cap, float* loss,
                        float* lse, hipStream_t stream) {
  int rc = check_rows(d, "softcap_xent");
  if (rc) return rc;
  if (d->W > 4096 || (d->W > 512 && d->W % 512)) return fail(TS_ERR_NOT_IMPLEMENTED, "softcap_xent: width %d", d->W);
  if (!z || !target || !loss || !lse || !aligned(z) || !(cap > 0.f))
    return fail(TS_ERR_VALUE, "softcap_xent: missing or unaligned arguments, or cap <= 0");
  if (d->rows == 0) return TS_OK;
  ts::GlueP p;
  memset(&p, 0, sizeof(p));
  p.rows = d->rows; p.W = d->W; p.x = z;
  const dim3 grid((unsigned)((d->rows + 3) / 4));
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL((ts::softcap_xent_kernel<ts::bf16, false>), grid, dim3(256), 0, stream, p, target, cap, loss, lse,
                       (const float*)nullptr, 0.f);
  else
    hipLaunchKernelGGL((ts::softcap_xent_kernel<float, false>), grid, dim3(256), 0, stream, p, target, cap, loss, lse,
                       (const float*)nullptr, 0.f);
  return glue_finish("softcap_xent");
}

int ts_softcap_xent_bwd(const ts_rows_desc* d, const void* z, const int64_t* target, float cap, const float* lse,
                        const float* g, float g_scale, void* dz, hipStream_t stream) {
  int rc = check_rows(d, "softcap_xent bwd");
  if (rc) return rc;
  if (d->W > 4096 || (d->W > 512 && d->W % 512))
    return fail(TS_ERR_NOT_IMPLEMENTED, "softcap_xent bwd: width %d", d->W);
  if (!z || !target || !lse || !g || !dz || !aligned(z) || !aligned(dz) || !(cap > 0.f))
    return fail(TS_ERR_VALUE, "softcap_xent bwd: missing or unaligned arguments, or cap <= 0");
  if (d->rows == 0) return TS_OK;
  ts::GlueP p;
  memset(&p, 0, sizeof(p));
  p.rows = d->rows; p.W = d->W; p.x = z; p.y = dz;
  const dim3 grid((unsigned)((d->rows + 3) / 4));
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL((ts::softcap_xent_kernel<ts::bf16, true>), grid, dim3(256), 0, stream, p, target, cap,
                       (float*)nullptr, (float*)lse, g, g_scale);
  else
    hipLaunchKernelGGL((ts::softcap_xent_kernel<float, true>), grid, dim3(256), 0, stream, p, target, cap,
                       (float*)nullptr, (float*)lse, g, g_scale);
  return glue_finish("softcap_xent bwd");
}

}  // extern "C"
