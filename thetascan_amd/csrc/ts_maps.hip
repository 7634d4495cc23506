// Projected B-spline feature map and temporal-bank blend for gfx950.
//
// Both are streaming kernels bound by HBM: the spline map reads one
// coordinate and writes n_basis features per coordinate; the blend reads
// n_in views and writes one.  Work is laid out as a 2-D grid of
// (tile of one (b, h) slice, b * H + h) so that every block works for a
// single head: per-head parameters are uniform (scalar registers) and the
// parameter-gradient partial sums need no atomics.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <float.h>
#include <math.h>
#include <string.h>

namespace ts {

// ------------------------------------------------------------- helpers

template <typename E>
__device__ __forceinline__ E* at(const ts_strided& s, int b, int h, int64_t t) {
  return (E*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + t * s.st;
}

// Sums v[0..N) over the 256 threads of the block; thread i < N gets sum i.
template <int N>
__device__ __forceinline__ float block_sums(float (&v)[N], float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v[i] += __shfl_xor(v[i], o, 64);
  if (lane == 0)
#pragma unroll
    for (int i = 0; i < N; ++i) red[wave * N + i] = v[i];
  __syncthreads();
  float s = 0.f;
  if (threadIdx.x < N) s = red[threadIdx.x] + red[N + threadIdx.x] + red[2 * N + threadIdx.x] + red[3 * N + threadIdx.x];
  return s;
}

// ------------------------------------------------------ B-spline map

constexpr int kSplineTile = 256;  // coordinates per block (one per thread: table reads are not hoisted)
constexpr int kSplineTab = 600;    // floats in the knot/reciprocal table (32 + 7 basis functions)

// Flat table of a (NI, DMAX) instantiation, NI = nb bucket + DMAX intervals:
//   [0, NI]                  knots t[0..NI] (past the last knot: +bound)
//   NI+1 + (r-1)*NI + i      1 / (t[i+r] - t[i])        (r = 1..DMAX)
//   NI+1 + (DMAX+r-1)*NI + i 1 / (t[i+r+1] - t[i+1])
// Reciprocals are 0 where the span is empty (the reference's
// where(den > 0, ..., 0)) and for every entry past an order's last basis
// function, so the recursion below runs over all NI entries without guards:
// the extra entries stay exactly zero.
__host__ __device__ constexpr int spline_tab_size(int ni, int dmax) { return ni + 1 + 2 * dmax * ni; }

struct SplineP {
  int B, H, T, P, nb, deg;
  int tiles, vec;
  float scale, bound, hi, inv_p;  // hi = nextafter(bound, -inf)
  const float* scale_h;
  ts_strided pre, out, dout, dpre;
  float* dscale_part;
  // RMS-normalized input (the norm variants): pre is the raw W1 product,
  // normalized over each token's P projections and shifted per projection
  float eps;
  const float* shift;   // [H, P] or null
  float* dshift_part;   // [H][B * tiles][P] or null
  float tab[kSplineTab];
};

// The coordinate a thread maps: the raw value, or (RMS) its token's
// RMS-normalized value plus the shift, with zn = a / rms and 1 / rms.  The
// P coordinates of a token sit in P consecutive lanes (P a power of two
// dividing 64; a block starts on a token), so the token's sum of squares is
// an xor butterfly over P lanes; every lane takes part.
template <typename E, bool RMS>
__device__ __forceinline__ float spline_input(const SplineP& p, int b, int h, int64_t t, int c, bool valid,
                                              float& zn, float& rinv) {
  const float a = valid ? tof(at<const E>(p.pre, b, h, t)[c]) : 0.f;
  zn = a;
  rinv = 1.f;
  if constexpr (RMS) {
    float ss = a * a;
    for (int o = 1; o < p.P; o <<= 1) ss += __shfl_xor(ss, o, 64);
    rinv = rsqrtf(ss / (float)p.P + p.eps);
    zn = a * rinv;
    return zn + (p.shift ? p.shift[h * p.P + c] : 0.f);
  }
  return a;
}

// Copies the table into LDS (block-wide; ends with a barrier).
template <int NI, int DMAX>
__device__ __forceinline__ void spline_table(const SplineP& p, float* tab) {
  constexpr int N = spline_tab_size(NI, DMAX);
  static_assert(N <= kSplineTab, "spline table");
  for (int i = threadIdx.x; i < N; i += 256) tab[i] = p.tab[i];
  __syncthreads();
}

// Cox-de Boor recursion over every knot interval (kernel_features.py:186-201),
// with the derivative d/dx carried alongside when GRAD.  Fully unrolled over
// the bucket sizes NI and DMAX so b[] stays in registers; the orders past the
// runtime degree are skipped by a uniform branch.
template <int NI, int DMAX, bool GRAD>
__device__ __forceinline__ void spline_basis(const float* tab, int deg, float x, float (&b)[NI], float (&db)[NI]) {
  const float* kn = tab;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    b[i] = (x >= kn[i] && x < kn[i + 1]) ? 1.f : 0.f;
    db[i] = 0.f;
  }
#pragma unroll
  for (int r = 1; r <= DMAX; ++r) {
    if (r > deg) break;
    const float* il = tab + NI + 1 + (r - 1) * NI;
    const float* ir = tab + NI + 1 + (DMAX + r - 1) * NI;
#pragma unroll
    for (int i = 0; i + r < NI; ++i) {
      const float L = (x - kn[i]) * il[i];
      const float R = (kn[i + r + 1] - x) * ir[i];
      if (GRAD) db[i] = il[i] * b[i] + L * db[i] - ir[i] * b[i + 1] + R * db[i + 1];
      b[i] = L * b[i] + R * b[i + 1];
    }
  }
}

template <typename E, int NB, int DMAX, bool RMS>
__global__ __launch_bounds__(256) void bspline_fwd_kernel(SplineP p) {
  constexpr int NI = NB + DMAX;
  __shared__ float tab[spline_tab_size(NI, DMAX)];
  spline_table<NI, DMAX>(p, tab);
  const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
  const float scale = p.scale_h ? p.scale_h[h] : p.scale;
  const int64_t n = (int64_t)p.T * p.P;
  const int64_t q0 = (int64_t)blockIdx.x * kSplineTile;
  const int64_t q = q0 + threadIdx.x;
  const int64_t t = q / p.P;
  const int c = (int)(q - t * p.P);
  float zn, rinv;
  const float pre = spline_input<E, RMS>(p, b, h, t, c, q < n, zn, rinv);
  if (q < n) {
    const float x0 = pre * scale;
    const float x = fminf(fminf(fmaxf(x0, -p.bound), p.bound), p.hi);
    float bs[NI], dbs[NI];
    spline_basis<NI, DMAX, false>(tab, p.deg, x, bs, dbs);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < NB; ++j) sum += fmaxf(bs[j], 0.f);
    const float inv = 1.0f / fmaxf(sum, FLT_MIN);
    E* dst = at<E>(p.out, b, h, t) + (int64_t)c * p.nb;
    if (p.vec) {
      constexpr int V = Vec16<E>::N;
#pragma unroll
      for (int j0 = 0; j0 < NB; j0 += V) {
        if (j0 < p.nb) {
          Vec16<E> v;
#pragma unroll
          for (int e = 0; e < V; ++e) v.e[e] = cvt<E>(fmaxf(bs[j0 + e], 0.f) * inv * p.inv_p);
          *(uint4*)(dst + j0) = v.raw;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j)
        if (j < p.nb) dst[j] = cvt<E>(fmaxf(bs[j], 0.f) * inv * p.inv_p);
    }
  }
}

template <typename E, int NB, int DMAX, bool RMS>
__global__ __launch_bounds__(256) void bspline_bwd_kernel(SplineP p) {
  constexpr int NI = NB + DMAX;
  __shared__ float tab[spline_tab_size(NI, DMAX)];
  __shared__ float red[4 * 64];
  spline_table<NI, DMAX>(p, tab);
  const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
  const float scale = p.scale_h ? p.scale_h[h] : p.scale;
  const int64_t n = (int64_t)p.T * p.P;
  const int64_t q0 = (int64_t)blockIdx.x * kSplineTile;
  const int64_t q = q0 + threadIdx.x;
  const int64_t t = q / p.P;
  const int c = (int)(q - t * p.P);
  float zn, rinv;
  const float pre = spline_input<E, RMS>(p, b, h, t, c, q < n, zn, rinv);
  float acc[1] = {0.f};
  float dz = 0.f;  // gradient of the map's input (before the scale)
  if (q < n) {
    const float x0 = pre * scale;
    const float x1 = fminf(fmaxf(x0, -p.bound), p.bound);
    const float x = fminf(x1, p.hi);
    float bs[NI], dbs[NI];
    spline_basis<NI, DMAX, true>(tab, p.deg, x, bs, dbs);
    float g[NB];
    const E* src = at<const E>(p.dout, b, h, t) + (int64_t)c * p.nb;
    if (p.vec) {
      constexpr int V = Vec16<E>::N;
#pragma unroll
      for (int j0 = 0; j0 < NB; j0 += V) {
        if (j0 < p.nb) {
          Vec16<E> v;
          v.raw = *(const uint4*)(src + j0);
#pragma unroll
          for (int e = 0; e < V; ++e) g[j0 + e] = tof(v.e[e]);
        } else {
#pragma unroll
          for (int e = 0; e < V; ++e) g[j0 + e] = 0.f;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j) g[j] = j < p.nb ? tof(src[j]) : 0.f;
    }
    // out_j = v_j / max(S, tiny) / P with v_j = max(b_j, 0), S = sum v_j
    // (entries past n_basis are exactly zero and add nothing)
    float S = 0.f, dS = 0.f, gv = 0.f, gdv = 0.f;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const bool pos = bs[j] >= 0.f;
      const float v = pos ? bs[j] : 0.f, dv = pos ? dbs[j] : 0.f;
      S += v;
      dS += dv;
      gv += g[j] * v;
      gdv += g[j] * dv;
    }
    const bool live = S >= FLT_MIN;
    const float Sc = live ? S : FLT_MIN;
    const float dSc = live ? dS : 0.f;
    float dx = (gdv * Sc - gv * dSc) / (Sc * Sc) * p.inv_p;
    // clamp(x0, -bound, bound) passes the gradient on [-bound, bound];
    // minimum(x1, hi) passes it below hi and half of it at equality.
    if (!(x0 >= -p.bound && x0 <= p.bound)) dx = 0.f;
    if (x1 > p.hi) dx = 0.f;
    else if (x1 == p.hi) dx *= 0.5f;
    dz = dx * scale;
    acc[0] += dx * pre;
  }
  if constexpr (RMS) {
    // RMSNorm backward over the token's P lanes: da = rinv (dz - (sum dz zn / P) zn)
    float s = dz * zn;
    for (int o = 1; o < p.P; o <<= 1) s += __shfl_xor(s, o, 64);
    if (q < n) at<E>(p.dpre, b, h, t)[c] = cvt<E>(rinv * (dz - s / (float)p.P * zn));
  } else {
    if (q < n) at<E>(p.dpre, b, h, t)[c] = cvt<E>(dz);
  }
  if (p.dscale_part) {
    const float s = block_sums<1>(acc, red);
    if (threadIdx.x == 0) p.dscale_part[(int64_t)h * p.B * p.tiles + (int64_t)b * p.tiles + blockIdx.x] = s;
  }
  if (RMS && p.dshift_part) {
    // per projection c: the lanes c, c + P, ... of each wave, then the waves
    float v = dz;
    for (int o = p.P; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane < p.P) red[wave * 64 + lane] = v;
    __syncthreads();
    if ((int)threadIdx.x < p.P) {
      const float tot = red[threadIdx.x] + red[64 + threadIdx.x] + red[128 + threadIdx.x] + red[192 + threadIdx.x];
      p.dshift_part[((int64_t)h * p.B * p.tiles + (int64_t)b * p.tiles + blockIdx.x) * p.P + threadIdx.x] = tot;
    }
  }
}

// ---------------------------------------------------------- bank blend

constexpr int kBlendMax = 8;
constexpr int kBlendElems = 8192;  // elements of one view per block (rows * d)

// Rows per block: a whole number of rows holding about kBlendElems elements.
// The tiling depends on the shape alone, so the backward's partial-sum layout
// is the same for the vector and the scalar kernel.
__host__ __device__ inline int blend_rows(int d) { return d >= kBlendElems ? 1 : kBlendElems / d; }

struct BlendP {
  int B, H, T, d, n, tiles, rows;
  const float* coef;
  ts_strided in[kBlendMax];
  ts_strided y, dy;
  ts_strided din[kBlendMax];
  float* dpart;
  ts_strided g;      // output-gate pre-activation (forward only; NULL: no gate)
  const float* gb;   // gate bias [H*d] (NULL: none)
};

// Chunk c of the (b, h) slice: row t = c / per_row, columns W*(c % per_row)..
// Block x covers rows [x * rows, (x + 1) * rows).
template <typename E, bool V>
__global__ __launch_bounds__(256) void blend_fwd_kernel(BlendP p) {
  constexpr int W = V ? Vec16<E>::N : 1;
  const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
  const int per_row = p.d / W;
  const int64_t r0 = (int64_t)blockIdx.x * p.rows;
  const int64_t c0 = r0 * per_row;
  const int64_t c1 = (r0 + p.rows < p.T ? r0 + p.rows : p.T) * per_row;
  float coef[kBlendMax];
#pragma unroll
  for (int i = 0; i < kBlendMax; ++i) coef[i] = i < p.n ? p.coef[i * p.H + h] : 0.f;
  for (int64_t c = c0 + threadIdx.x; c < c1; c += 256) {
    const int64_t t = c / per_row;
    const int col = (int)(c - t * per_row) * W;
    float acc[W];
#pragma unroll
    for (int e = 0; e < W; ++e) acc[e] = 0.f;
#pragma unroll
    for (int i = 0; i < kBlendMax; ++i) {
      if (i < p.n) {
        const E* src = at<const E>(p.in[i], b, h, t) + col;
        if (V) {
          Vec16<E> v;
          v.raw = *(const uint4*)src;
#pragma unroll
          for (int e = 0; e < W; ++e) acc[e] += coef[i] * tof(v.e[e]);
        } else {
          acc[0] += coef[i] * tof(src[0]);
        }
      }
    }
    if (p.g.ptr) {
      // output gate: y *= silu(g + bias), in fp32 before the one rounding
      const E* gs = at<const E>(p.g, b, h, t) + col;
      float gv[W];
      if (V) {
        Vec16<E> v;
        v.raw = *(const uint4*)gs;
#pragma unroll
        for (int e = 0; e < W; ++e) gv[e] = tof(v.e[e]);
      } else {
        gv[0] = tof(gs[0]);
      }
#pragma unroll
      for (int e = 0; e < W; ++e) {
        const float z = gv[e] + (p.gb ? p.gb[h * p.d + col + e] : 0.f);
        acc[e] *= z / (1.0f + __expf(-z));
      }
    }
    E* dst = at<E>(p.y, b, h, t) + col;
    if (V) {
      Vec16<E> v;
#pragma unroll
      for (int e = 0; e < W; ++e) v.e[e] = cvt<E>(acc[e]);
      *(uint4*)dst = v.raw;
    } else {
      dst[0] = cvt<E>(acc[0]);
    }
  }
}

template <typename E, bool V>
__global__ __launch_bounds__(256) void blend_bwd_kernel(BlendP p) {
  constexpr int W = V ? Vec16<E>::N : 1;
  __shared__ float red[4 * kBlendMax];
  const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
  const int per_row = p.d / W;
  const int64_t r0 = (int64_t)blockIdx.x * p.rows;
  const int64_t c0 = r0 * per_row;
  const int64_t c1 = (r0 + p.rows < p.T ? r0 + p.rows : p.T) * per_row;
  float coef[kBlendMax], dc[kBlendMax];
#pragma unroll
  for (int i = 0; i < kBlendMax; ++i) {
    coef[i] = i < p.n ? p.coef[i * p.H + h] : 0.f;
    dc[i] = 0.f;
  }
  for (int64_t c = c0 + threadIdx.x; c < c1; c += 256) {
    const int64_t t = c / per_row;
    const int col = (int)(c - t * per_row) * W;
    float g[W];
    const E* gsrc = at<const E>(p.dy, b, h, t) + col;
    if (V) {
      Vec16<E> v;
      v.raw = *(const uint4*)gsrc;
#pragma unroll
      for (int e = 0; e < W; ++e) g[e] = tof(v.e[e]);
    } else {
      g[0] = tof(gsrc[0]);
    }
#pragma unroll
    for (int i = 0; i < kBlendMax; ++i) {
      if (i < p.n) {
        const E* src = at<const E>(p.in[i], b, h, t) + col;
        if (V) {
          Vec16<E> v;
          v.raw = *(const uint4*)src;
#pragma unroll
          for (int e = 0; e < W; ++e) dc[i] += g[e] * tof(v.e[e]);
        } else {
          dc[i] += g[0] * tof(src[0]);
        }
        if (p.din[i].ptr) {
          E* dst = at<E>(p.din[i], b, h, t) + col;
          if (V) {
            Vec16<E> v;
#pragma unroll
            for (int e = 0; e < W; ++e) v.e[e] = cvt<E>(coef[i] * g[e]);
            *(uint4*)dst = v.raw;
          } else {
            dst[0] = cvt<E>(coef[i] * g[0]);
          }
        }
      }
    }
  }
  const float s = block_sums<kBlendMax>(dc, red);
  if (threadIdx.x < p.n)
    p.dpart[((int64_t)threadIdx.x * p.H + h) * p.B * p.tiles + (int64_t)b * p.tiles + blockIdx.x] = s;
}

}  // namespace ts

namespace {

using ts::fail;

int finish(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TS_OK;
}

// Rows of a [B,H,T,w] view can be read as 16-byte vectors.
bool vec_rows(const ts_strided& s, int width, int esize) {
  const int v = 16 / esize;
  return ((uintptr_t)s.ptr & 15u) == 0 && width % v == 0 && s.sb % v == 0 && s.sh % v == 0 && s.st % v == 0;
}

int check_spline(const ts_bspline_desc* d) {
  if (!d) return fail(TS_ERR_VALUE, "bspline: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0 || d->P < 1) return fail(TS_ERR_VALUE, "bspline: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "bspline: unknown dtype");
  if (d->degree < 0) return fail(TS_ERR_VALUE, "B-spline degree must be non-negative");
  if (d->n_basis <= d->degree) return fail(TS_ERR_VALUE, "B-spline basis count must exceed its degree");
  if (!(d->bound > 0.f)) return fail(TS_ERR_VALUE, "B-spline bound must be positive");
  if (d->n_basis > 32 || d->degree > 7)
    return fail(TS_ERR_NOT_IMPLEMENTED, "bspline: at most 32 basis functions of degree <= 7");
  if ((int64_t)d->B * d->H > 65535) return fail(TS_ERR_NOT_IMPLEMENTED, "bspline: B*H above 65535");
  return TS_OK;
}

int spline_tiles(const ts_bspline_desc* d) {
  return (int)(((int64_t)d->T * d->P + ts::kSplineTile - 1) / ts::kSplineTile);
}

int spline_nb_bucket(int nb) { return nb <= 8 ? 8 : nb <= 16 ? 16 : 32; }
int spline_deg_bucket(int deg) { return deg <= 3 ? 3 : 7; }

// Knot vector and reciprocal spans (kernel_features.py:166-199) in the table
// layout of the (nb bucket, degree bucket) kernel.  The interior knots follow
// torch.linspace(-bound, bound, n_inner + 2) in fp32: the first half counts up
// from the start, the second half down from the end.
void fill_spline(const ts_bspline_desc* d, const float* scale_h, ts::SplineP& p) {
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.P = d->P;
  p.nb = d->n_basis; p.deg = d->degree;
  p.tiles = spline_tiles(d);
  p.scale = d->scale; p.bound = d->bound;
  p.hi = nextafterf(d->bound, -INFINITY);
  p.inv_p = 1.0f / (float)d->P;
  p.scale_h = scale_h;
  const int deg = d->degree, n_inner = d->n_basis - deg - 1, K = d->n_basis + deg + 1;
  const int dmax = spline_deg_bucket(deg), ni = spline_nb_bucket(d->n_basis) + dmax;
  float kn[48];
  int k = 0;
  for (int i = 0; i <= deg; ++i) kn[k++] = -d->bound;
  if (n_inner > 0) {
    const int steps = n_inner + 2;
    const float step = (d->bound - (-d->bound)) / (float)(steps - 1);
    const int half = steps / 2;
    for (int i = 1; i <= n_inner; ++i)
      kn[k++] = i < half ? -d->bound + step * (float)i : d->bound - step * (float)(steps - i - 1);
  }
  for (int i = 0; i <= deg; ++i) kn[k++] = d->bound;
  while (k <= ni) kn[k++] = d->bound;  // padding past the last knot
  for (int i = 0; i <= ni; ++i) p.tab[i] = kn[i];
  for (int r = 1; r <= deg; ++r) {
    float* il = p.tab + ni + 1 + (r - 1) * ni;
    float* ir = p.tab + ni + 1 + (dmax + r - 1) * ni;
    for (int i = 0; i + r + 1 < K; ++i) {  // the K - r - 1 functions of order r
      const float ld = kn[i + r] - kn[i];
      const float rd = kn[i + r + 1] - kn[i + 1];
      il[i] = ld > 0.f ? 1.0f / ld : 0.f;
      ir[i] = rd > 0.f ? 1.0f / rd : 0.f;
    }
  }
}

typedef void (*SplineKernel)(ts::SplineP);

template <typename E, bool FWD, bool RMS>
SplineKernel spline_kernel(int nb, int deg) {
  const int nbb = spline_nb_bucket(nb);
  const bool lo = spline_deg_bucket(deg) == 3;
  if (FWD) {
    if (nbb == 8) return lo ? ts::bspline_fwd_kernel<E, 8, 3, RMS> : ts::bspline_fwd_kernel<E, 8, 7, RMS>;
    if (nbb == 16) return lo ? ts::bspline_fwd_kernel<E, 16, 3, RMS> : ts::bspline_fwd_kernel<E, 16, 7, RMS>;
    return lo ? ts::bspline_fwd_kernel<E, 32, 3, RMS> : ts::bspline_fwd_kernel<E, 32, 7, RMS>;
  }
  if (nbb == 8) return lo ? ts::bspline_bwd_kernel<E, 8, 3, RMS> : ts::bspline_bwd_kernel<E, 8, 7, RMS>;
  if (nbb == 16) return lo ? ts::bspline_bwd_kernel<E, 16, 3, RMS> : ts::bspline_bwd_kernel<E, 16, 7, RMS>;
  return lo ? ts::bspline_bwd_kernel<E, 32, 3, RMS> : ts::bspline_bwd_kernel<E, 32, 7, RMS>;
}

template <bool RMS>
SplineKernel pick_spline(const ts_bspline_desc* d, bool fwd) {
  if (d->dtype == TS_BF16)
    return fwd ? spline_kernel<ts::bf16, true, RMS>(d->n_basis, d->degree)
               : spline_kernel<ts::bf16, false, RMS>(d->n_basis, d->degree);
  return fwd ? spline_kernel<float, true, RMS>(d->n_basis, d->degree)
             : spline_kernel<float, false, RMS>(d->n_basis, d->degree);
}

int launch_spline(const ts_bspline_desc* d, ts::SplineP& p, bool fwd, bool rms, hipStream_t stream) {
  if (d->T == 0) return TS_OK;
  const dim3 grid((unsigned)p.tiles, (unsigned)(d->B * d->H));
  SplineKernel k = rms ? pick_spline<true>(d, fwd) : pick_spline<false>(d, fwd);
  hipLaunchKernelGGL(k, grid, dim3(256), 0, stream, p);
  return finish(fwd ? "bspline" : "bspline bwd");
}

int check_blend(const ts_blend_desc* d, const ts_strided* in) {
  if (!d || !in) return fail(TS_ERR_VALUE, "blend: null arguments");
  if (d->B < 1 || d->H < 1 || d->T < 0 || d->d < 1) return fail(TS_ERR_VALUE, "blend: bad shape");
  if (d->n_in < 1 || d->n_in > ts::kBlendMax) return fail(TS_ERR_VALUE, "blend: 1 to 8 inputs");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "blend: unknown dtype");
  if ((int64_t)d->B * d->H > 65535) return fail(TS_ERR_NOT_IMPLEMENTED, "blend: B*H above 65535");
  for (int i = 0; i < d->n_in; ++i)
    if (!in[i].ptr) return fail(TS_ERR_VALUE, "blend: missing input %d", i);
  return TS_OK;
}

int blend_tiles(const ts_blend_desc* d) {
  const int rows = ts::blend_rows(d->d);
  return (int)(((int64_t)d->T + rows - 1) / rows);
}

// 16-byte chunks when every tensor allows them.
bool blend_vec(const ts_blend_desc* d, const ts_strided* in, const ts_strided* extra, int n_extra) {
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  for (int i = 0; i < d->n_in; ++i)
    if (!vec_rows(in[i], d->d, es)) return false;
  for (int i = 0; i < n_extra; ++i)
    if (extra[i].ptr && !vec_rows(extra[i], d->d, es)) return false;
  return true;
}

}  // namespace

extern "C" {

int ts_bspline_parts(const ts_bspline_desc* d, int32_t* nparts) {
  int rc = check_spline(d);
  if (rc) return rc;
  if (!nparts) return fail(TS_ERR_VALUE, "bspline: null output");
  *nparts = d->B * spline_tiles(d);
  return TS_OK;
}

int ts_bspline_fwd(const ts_bspline_desc* d, ts_strided pre, const float* scale_h, ts_strided out,
                   hipStream_t stream) {
  int rc = check_spline(d);
  if (rc) return rc;
  if (!pre.ptr || !out.ptr) return fail(TS_ERR_VALUE, "bspline: missing tensors");
  ts::SplineP p;
  fill_spline(d, scale_h, p);
  p.pre = pre;
  p.out = out;
  p.vec = vec_rows(out, d->P * d->n_basis, d->dtype == TS_BF16 ? 2 : 4) &&
          d->n_basis % (d->dtype == TS_BF16 ? 8 : 4) == 0;
  return launch_spline(d, p, true, false, stream);
}

int ts_bspline_bwd(const ts_bspline_desc* d, ts_strided pre, const float* scale_h, ts_strided dout,
                   ts_strided dpre, float* dscale_part, hipStream_t stream) {
  int rc = check_spline(d);
  if (rc) return rc;
  if (!pre.ptr || !dout.ptr || !dpre.ptr) return fail(TS_ERR_VALUE, "bspline bwd: missing tensors");
  if (scale_h && !dscale_part) return fail(TS_ERR_VALUE, "bspline bwd: missing scale partials");
  ts::SplineP p;
  fill_spline(d, scale_h, p);
  p.pre = pre;
  p.dout = dout;
  p.dpre = dpre;
  p.dscale_part = scale_h ? dscale_part : nullptr;
  p.vec = vec_rows(dout, d->P * d->n_basis, d->dtype == TS_BF16 ? 2 : 4) &&
          d->n_basis % (d->dtype == TS_BF16 ? 8 : 4) == 0;
  return launch_spline(d, p, false, false, stream);
}

int ts_blend_parts(const ts_blend_desc* d, int32_t* nparts) {
  if (!d || !nparts || d->B < 1 || d->T < 0 || d->d < 1) return fail(TS_ERR_VALUE, "blend: bad arguments");
  *nparts = d->B * blend_tiles(d);
  return TS_OK;
}

// The B-spline map of RMS-normalized inputs: P must be a power of two up to 64.
static int check_spline_norm(const ts_bspline_desc* d, float eps) {
  int rc = check_spline(d);
  if (rc) return rc;
  if (d->P > 64 || (d->P & (d->P - 1))) return fail(TS_ERR_NOT_IMPLEMENTED, "bspline norm: %d projections (a power of two up to 64)", d->P);
  if (!(eps > 0.f)) return fail(TS_ERR_VALUE, "bspline norm: eps must be positive");
  return TS_OK;
}

int ts_bspline_norm_fwd(const ts_bspline_desc* d, ts_strided a, const float* shift, float eps, const float* scale_h,
                        ts_strided out, hipStream_t stream) {
  int rc = check_spline_norm(d, eps);
  if (rc) return rc;
  if (!a.ptr || !out.ptr) return fail(TS_ERR_VALUE, "bspline norm: missing tensors");
  ts::SplineP p;
  fill_spline(d, scale_h, p);
  p.pre = a;
  p.out = out;
  p.eps = eps;
  p.shift = shift;
  p.vec = vec_rows(out, d->P * d->n_basis, d->dtype == TS_BF16 ? 2 : 4) &&
          d->n_basis % (d->dtype == TS_BF16 ? 8 : 4) == 0;
  return launch_spline(d, p, true, true, stream);
}

int ts_bspline_norm_bwd(const ts_bspline_desc* d, ts_strided a, const float* shift, float eps, const float* scale_h,
                        ts_strided dout, ts_strided da, float* dscale_part, float* dshift_part, hipStream_t stream) {
  int rc = check_spline_norm(d, eps);
  if (rc) return rc;
  if (!a.ptr || !dout.ptr || !da.ptr) return fail(TS_ERR_VALUE, "bspline norm bwd: missing tensors");
  if (scale_h && !dscale_part) return fail(TS_ERR_VALUE, "bspline norm bwd: missing scale partials");
  if (dshift_part && !shift) return fail(TS_ERR_VALUE, "bspline norm bwd: gradient of an absent shift");
  ts::SplineP p;
  fill_spline(d, scale_h, p);
  p.pre = a;
  p.dout = dout;
  p.dpre = da;
  p.eps = eps;
  p.shift = shift;
  p.dscale_part = scale_h ? dscale_part : nullptr;
  p.dshift_part = dshift_part;
  p.vec = vec_rows(dout, d->P * d->n_basis, d->dtype == TS_BF16 ? 2 : 4) &&
          d->n_basis % (d->dtype == TS_BF16 ? 8 : 4) == 0;
  return launch_spline(d, p, false, true, stream);
}

int ts_blend_gated_fwd(const ts_blend_desc* d, const ts_strided* in, const float* coef, ts_strided g,
                       const float* g_bias, ts_strided y, hipStream_t stream) {
  int rc = check_blend(d, in);
  if (rc) return rc;
  if (!coef || !y.ptr) return fail(TS_ERR_VALUE, "blend: missing coefficients or output");
  if (d->T == 0) return TS_OK;
  ts::BlendP p;
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.d = d->d; p.n = d->n_in;
  p.coef = coef;
  for (int i = 0; i < d->n_in; ++i) p.in[i] = in[i];
  p.y = y;
  p.g = g;
  p.gb = g.ptr ? g_bias : nullptr;
  const ts_strided outs[2] = {y, g};
  const bool vec = blend_vec(d, in, outs, 2);
  p.tiles = blend_tiles(d);
  p.rows = ts::blend_rows(d->d);
  const dim3 grid((unsigned)p.tiles, (unsigned)(d->B * d->H));
  if (d->dtype == TS_BF16) {
    if (vec) hipLaunchKernelGGL((ts::blend_fwd_kernel<ts::bf16, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((ts::blend_fwd_kernel<ts::bf16, false>), grid, dim3(256), 0, stream, p);
  } else {
    if (vec) hipLaunchKernelGGL((ts::blend_fwd_kernel<float, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((ts::blend_fwd_kernel<float, false>), grid, dim3(256), 0, stream, p);
  }
  return finish("blend");
}

int ts_blend_fwd(const ts_blend_desc* d, const ts_strided* in, const float* coef, ts_strided y,
                 hipStream_t stream) {
  const ts_strided none = {nullptr, 0, 0, 0};
  return ts_blend_gated_fwd(d, in, coef, none, nullptr, y, stream);
}

int ts_blend_bwd(const ts_blend_desc* d, const ts_strided* in, const float* coef, ts_strided dy,
                 const ts_strided* din, float* dcoef_part, hipStream_t stream) {
  int rc = check_blend(d, in);
  if (rc) return rc;
  if (!coef || !dy.ptr || !din || !dcoef_part) return fail(TS_ERR_VALUE, "blend bwd: missing tensors");
  if (d->T == 0) return TS_OK;
  ts::BlendP p;
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.d = d->d; p.n = d->n_in;
  p.coef = coef;
  ts_strided extra[ts::kBlendMax + 1];
  for (int i = 0; i < d->n_in; ++i) {
    p.in[i] = in[i];
    p.din[i] = din[i];
    extra[i] = din[i];
  }
  extra[d->n_in] = dy;
  p.dy = dy;
  p.dpart = dcoef_part;
  const bool vec = blend_vec(d, in, extra, d->n_in + 1);
  p.tiles = blend_tiles(d);
  p.rows = ts::blend_rows(d->d);
  const dim3 grid((unsigned)p.tiles, (unsigned)(d->B * d->H));
  if (d->dtype == TS_BF16) {
    if (vec) hipLaunchKernelGGL((ts::blend_bwd_kernel<ts::bf16, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((ts::blend_bwd_kernel<ts::bf16, false>), grid, dim3(256), 0, stream, p);
  } else {
    if (vec) hipLaunchKernelGGL((ts::blend_bwd_kernel<float, true>), grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((ts::blend_bwd_kernel<float, false>), grid, dim3(256), 0, stream, p);
  }
  return finish("blend bwd");
}

}  // extern "C"
