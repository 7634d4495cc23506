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


// Work mapping of the read kernels: block (x, y) covers rows
// x * RPB .. x * RPB + RPB - 1 of the (b, h) = y slice.  A row (one token) is
// CPR 16-byte chunks held by CPR consecutive lanes, so a pass of 256 threads
// covers 256 / CPR consecutive rows of one head, a contiguous run of a
// head-major [B, H, T, d] stream (measured faster than spreading a pass over
// every head of a few tokens, which breaks head-major streams into short runs
// half a MiB apart).  A thread makes RPT passes (its loads are all issued
// before any arithmetic) and keeps the same chunk in each; a row reduction is
// a log2(CPR)-step butterfly.  CPR is the row's chunk count rounded up to a
// power of two; lanes past the row's last chunk only join the butterfly.
// Two passes per thread: at B8 T4096 H8 d64 the forward and backward read
// take 34.7 / 54.1 us with two, 38.6 / 61.9 us with four, 45.5 / 88.8 us
// with eight and 33.8 / 57.1 us with one.
constexpr int kReadRPT = 2;

template <int CPR>
__host__ __device__ constexpr int read_rows_per_block() { return kReadRPT * (256 / CPR); }

template <typename E>
__device__ __forceinline__ const E* slice_of(const ts_strided& s, int b, int h) {
  return (const E*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh;
}

template <typename E, int N>
__device__ __forceinline__ void unpack(const uint4& raw, float* out) {
  Vec16<E> v;
  v.raw = raw;
#pragma unroll
  for (int e = 0; e < N; ++e) out[e] = tof(v.e[e]);
}
template <typename E, int N>
__device__ __forceinline__ uint4 pack(const float* in) {
  Vec16<E> v;
#pragma unroll
  for (int e = 0; e < N; ++e) v.e[e] = cvt<E>(in[e]);
  return v.raw;
}

// sigma(x) from the hardware exp2 and reciprocal (a relative error of a few
// ulp of fp32, far below the bf16 rounding of the outputs)
__device__ __forceinline__ float fast_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// y = (resid + s * num / (mass + eps)) * silu(g + g_bias)     (engine.py:440-442, 526-528; gates.py:34-40)
template <typename E, int CPR>
__global__ __launch_bounds__(256) void read_fwd_kernel(ReadP p) {
  constexpr int N = Vec16<E>::N;
  constexpr int RP = 256 / CPR;  // rows per pass
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int c = ((int)threadIdx.x % CPR) * N;
  const bool colok = c < p.d;
  const int r0 = blockIdx.x * read_rows_per_block<CPR>() + (int)threadIdx.x / CPR;
  const E* num = slice_of<E>(p.num, b, h) + c;
  const E* res = p.resid.ptr ? slice_of<E>(p.resid, b, h) + c : nullptr;
  const E* gp = p.gate ? slice_of<E>(p.g, b, h) + c : nullptr;
  const float* mass = p.normalize ? slice_of<float>(p.mass, b, h) : nullptr;
  E* y = (E*)slice_of<E>(p.y, b, h) + c;
  uint4 rn[kReadRPT], rr[kReadRPT], rg[kReadRPT];
  float ms[kReadRPT];
#pragma unroll
  for (int i = 0; i < kReadRPT; ++i) {
    const int t = r0 + i * RP;
    if (t < p.T && colok) {
      rn[i] = *(const uint4*)(num + (int64_t)t * p.num.st);
      if (res) rr[i] = *(const uint4*)(res + (int64_t)t * p.resid.st);
      if (gp) rg[i] = *(const uint4*)(gp + (int64_t)t * p.g.st);
      if (mass) ms[i] = mass[(int64_t)t * p.mass.st];
    }
  }
  float gb[N];
#pragma unroll
  for (int e = 0; e < N; ++e) gb[e] = p.gbias && colok ? p.gbias[h * p.d + c + e] : 0.0f;
#pragma unroll
  for (int i = 0; i < kReadRPT; ++i) {
    const int t = r0 + i * RP;
    if (t >= p.T || !colok) continue;
    const float scale = mass ? p.s * __builtin_amdgcn_rcpf(ms[i] + p.eps) : p.s;
    float nv[N], rv[N], gv[N], out[N];
    unpack<E, N>(rn[i], nv);
    if (res) unpack<E, N>(rr[i], rv);
    if (gp) unpack<E, N>(rg[i], gv);
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float v = (res ? rv[e] : 0.0f) + scale * nv[e];
      if (gp) {
        const float x = gv[e] + gb[e];
        out[e] = v * x * fast_sigmoid(x);
      } else {
        out[e] = v;
      }
    }
    *(uint4*)(y + (int64_t)t * p.y.st) = pack<E, N>(out);
  }
}

// Backward of read_fwd; with `dgb_part` also the per-block sums of dg over
// tokens (the gate-bias gradient before the sum over blocks):
// parts[b * gridDim.x + blockIdx.x][h * d + col].  Each thread sums its own
// rows in registers, then each column adds the 256 / CPR row lanes in lane
// order through LDS: the result is reproducible bit for bit.
template <typename E, int CPR>
__global__ __launch_bounds__(256) void read_bwd_kernel(ReadP p, float* dgb_part) {
  constexpr int N = Vec16<E>::N;
  constexpr int RP = 256 / CPR;
  __shared__ float red[256 * N];
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int c = ((int)threadIdx.x % CPR) * N;
  const bool colok = c < p.d;
  const int r0 = blockIdx.x * read_rows_per_block<CPR>() + (int)threadIdx.x / CPR;
  const E* num = slice_of<E>(p.num, b, h) + c;
  const E* dyp = slice_of<E>(p.dy, b, h) + c;
  const E* res = p.resid.ptr ? slice_of<E>(p.resid, b, h) + c : nullptr;
  const E* gp = p.gate ? slice_of<E>(p.g, b, h) + c : nullptr;
  const float* mass = p.normalize ? slice_of<float>(p.mass, b, h) : nullptr;
  E* dnum = (E*)slice_of<E>(p.dnum, b, h) + c;
  E* dres = p.dresid.ptr ? (E*)slice_of<E>(p.dresid, b, h) + c : nullptr;
  E* dg = p.gate ? (E*)slice_of<E>(p.dg, b, h) + c : nullptr;
  float* dmass = p.normalize ? (float*)slice_of<float>(p.dmass, b, h) : nullptr;
  uint4 rn[kReadRPT], rd[kReadRPT], rr[kReadRPT], rg[kReadRPT];
  float ms[kReadRPT];
#pragma unroll
  for (int i = 0; i < kReadRPT; ++i) {
    const int t = r0 + i * RP;
    if (t < p.T && mass) ms[i] = mass[(int64_t)t * p.mass.st];
    if (t < p.T && colok) {
      rn[i] = *(const uint4*)(num + (int64_t)t * p.num.st);
      rd[i] = *(const uint4*)(dyp + (int64_t)t * p.dy.st);
      if (res) rr[i] = *(const uint4*)(res + (int64_t)t * p.resid.st);
      if (gp) rg[i] = *(const uint4*)(gp + (int64_t)t * p.g.st);
    }
  }
  float gb[N], colsum[N];
#pragma unroll
  for (int e = 0; e < N; ++e) {
    gb[e] = p.gbias && colok ? p.gbias[h * p.d + c + e] : 0.0f;
    colsum[e] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < kReadRPT; ++i) {
    const int t = r0 + i * RP;
    const bool live = t < p.T;  // dead rows and columns still join the row butterfly (with zeros)
    const float denom = mass && live ? ms[i] + p.eps : 1.0f;
    const float inv = __builtin_amdgcn_rcpf(denom);
    const float scale = mass ? p.s * inv : p.s;
    float dot = 0.0f;
    if (live && colok) {
      float nv[N], dv[N], rv[N], gv[N], o_dnum[N], o_dg[N], o_dres[N];
      unpack<E, N>(rn[i], nv);
      unpack<E, N>(rd[i], dv);
      if (res) unpack<E, N>(rr[i], rv);
      if (gp) unpack<E, N>(rg[i], gv);
#pragma unroll
      for (int e = 0; e < N; ++e) {
        float dpre = dv[e];
        if (gp) {
          const float x = gv[e] + gb[e];
          const float sg = fast_sigmoid(x);
          const float ypre = (res ? rv[e] : 0.0f) + scale * nv[e];
          o_dg[e] = dv[e] * ypre * (sg * (1.0f + x * (1.0f - sg)));
          colsum[e] += o_dg[e];
          dpre = dv[e] * x * sg;
        }
        o_dnum[e] = scale * dpre;
        o_dres[e] = dpre;
        dot += dpre * nv[e];
      }
      *(uint4*)(dnum + (int64_t)t * p.dnum.st) = pack<E, N>(o_dnum);
      if (dres) *(uint4*)(dres + (int64_t)t * p.dresid.st) = pack<E, N>(o_dres);
      if (dg) *(uint4*)(dg + (int64_t)t * p.dg.st) = pack<E, N>(o_dg);
    }
    if (mass) {
#pragma unroll
      for (int o = 1; o < CPR; o <<= 1) dot += __shfl_xor(dot, o, 64);
      if (live && threadIdx.x % CPR == 0) dmass[(int64_t)t * p.dmass.st] = -p.s * dot * inv * inv;
    }
  }
  if (dgb_part) {
#pragma unroll
    for (int e = 0; e < N; ++e) red[threadIdx.x * N + e] = colsum[e];
    __syncthreads();
    // one output column per thread (the host checks d <= 256)
    const int j = threadIdx.x;
    if (j < p.d) {
      const int chunk = j / N, e = j - chunk * N;
      float v = 0.0f;
      for (int l = 0; l < RP; ++l) v += red[(l * CPR + chunk) * N + e];
      dgb_part[((int64_t)b * gridDim.x + blockIdx.x) * (p.H * p.d) + h * p.d + j] = v;
    }
  }
}

// ---- query/key prologue: y = rope(x) / max(|rope(x)|, eps) per row
// (block.py:595-599 with rope.py:41-49 and norms.py:11-12), rows of strided
// [B,H,T,d] views in, contiguous rows out; same work mapping as the read
// kernels.  RoPE rotates pairs (2i, 2i+1) with i < rot / 2 by fp32 angles
// from [T, rot / 2] tables; a pair never straddles a 16-byte chunk.
struct NormP {
  int B, H, T, d, rot;
  float eps;
  ts_strided x, dy, y, dx;
  const float* cs;
  const float* sn;
};

template <int N>
__device__ __forceinline__ void rope_chunk(float* v, int c, int t, const NormP& p, bool inverse) {
#pragma unroll
  for (int e = 0; e < N; e += 2) {
    if (c + e < p.rot) {
      const int j = t * (p.rot >> 1) + ((c + e) >> 1);
      const float cs = p.cs[j];
      const float sn = inverse ? -p.sn[j] : p.sn[j];
      const float a = v[e], b = v[e + 1];
      v[e] = a * cs - b * sn;
      v[e + 1] = a * sn + b * cs;
    }
  }
}

template <typename E, int CPR>
__global__ __launch_bounds__(256) void qknorm_fwd_kernel(NormP p) {
  constexpr int N = Vec16<E>::N;
  constexpr int RP = 256 / CPR;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int c = ((int)threadIdx.x % CPR) * N;
  const bool colok = c < p.d;
  const int r0 = blockIdx.x * read_rows_per_block<CPR>() + (int)threadIdx.x / CPR;
  const E* x = slice_of<E>(p.x, b, h) + c;
  E* y = (E*)slice_of<E>(p.y, b, h) + c;
  uint4 rx[kReadRPT];
#pragma unroll
  for (int i = 0; i < kReadRPT; ++i) {
    const int t = r0 + i * RP;
    if (t < p.T && colok) rx[i] = *(const uint4*)(x + (int64_t)t * p.x.st);
  }
#pragma unroll
  for (int i = 0; i < kReadRPT; ++i) {
    const int t = r0 + i * RP;
    const bool live = t < p.T && colok;
    float v[N];
    float ss = 0.0f;
    if (live) {
      unpack<E, N>(rx[i], v);
      if (p.rot > 0) rope_chunk<N>(v, c, t, p, false);
#pragma unroll
      for (int e = 0; e < N; ++e) ss += v[e] * v[e];
    }
#pragma unroll
    for (int o = 1; o < CPR; o <<= 1) ss += __shfl_xor(ss, o, 64);
    if (live) {
      const float inv = 1.0f / fmaxf(sqrtf(ss), p.eps);
#pragma unroll
      for (int e = 0; e < N; ++e) v[e] *= inv;
      *(uint4*)(y + (int64_t)t * p.y.st) = pack<E, N>(v);
    }
  }
}

// dx = rope^T( n > eps ? (dy - y (y . dy)) / n : dy / eps ),  n = |rope(x)|
template <typename E, int CPR>
__global__ __launch_bounds__(256) void qknorm_bwd_kernel(NormP p) {
  constexpr int N = Vec16<E>::N;
  constexpr int RP = 256 / CPR;
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh - (bh / p.H) * p.H;
  const int c = ((int)threadIdx.x % CPR) * N;
  const bool colok = c < p.d;
  const int r0 = blockIdx.x * read_rows_per_block<CPR>() + (int)threadIdx.x / CPR;
  const E* x = slice_of<E>(p.x, b, h) + c;
  const E* dyp = slice_of<E>(p.dy, b, h) + c;
  E* dx = (E*)slice_of<E>(p.dx, b, h) + c;
  uint4 rx[kReadRPT], rd[kReadRPT];
#pragma unroll
  for (int i = 0; i < kReadRPT; ++i) {
    const int t = r0 + i * RP;
    if (t < p.T && colok) {
      rx[i] = *(const uint4*)(x + (int64_t)t * p.x.st);
      rd[i] = *(const uint4*)(dyp + (int64_t)t * p.dy.st);
    }
  }
#pragma unroll
  for (int i = 0; i < kReadRPT; ++i) {
    const int t = r0 + i * RP;
    const bool live = t < p.T && colok;
    float v[N], g[N];
    float ss = 0.0f, dot = 0.0f;
    if (live) {
      unpack<E, N>(rx[i], v);
      unpack<E, N>(rd[i], g);
      if (p.rot > 0) rope_chunk<N>(v, c, t, p, false);
#pragma unroll
      for (int e = 0; e < N; ++e) {
        ss += v[e] * v[e];
        dot += v[e] * g[e];
      }
    }
#pragma unroll
    for (int o = 1; o < CPR; o <<= 1) {
      ss += __shfl_xor(ss, o, 64);
      dot += __shfl_xor(dot, o, 64);
    }
    if (live) {
      const float n = sqrtf(ss);
      const bool big = n > p.eps;
      const float inv = 1.0f / (big ? n : p.eps);
      const float yd = dot * inv * inv;  // y . dy / n
#pragma unroll
      for (int e = 0; e < N; ++e) g[e] = big ? (g[e] - v[e] * yd) * inv : g[e] * inv;
      if (p.rot > 0) rope_chunk<N>(g, c, t, p, true);
      *(uint4*)(dx + (int64_t)t * p.dx.st) = pack<E, N>(g);
    }
  }
}

// z_t = a_t z_{t-1} + x_t  over T for every (b, h, feature).
// Decayed prefix z_u = a_u z_{u-1} + x_u along the scan order u (t = u, or
// t = T-1-u for an anti-causal scan), parallel over time: the order is cut
// into S segments of L steps.
//   wcumsum_summary_kernel : each thread folds one (b, h, segment, feature)
//                            from a zero state and stores only the segment's
//                            last value and (feature 0) its decay product
//                            P = prod a_u;
//   wcumsum_main_kernel    : each thread folds the earlier segments' (P, last)
//                            into its entering state C_j (C_{j+1} = P_j C_j +
//                            last_j, in segment order), then walks its
//                            segment from C_j and stores every z_u once.
// x is read twice and z written once (the local-then-correct form wrote z
// twice and read it back once).  Consecutive threads take consecutive
// features, so every access is a coalesced row.  Step decays: static
// exp(log_alpha[h]); a stream's a_u is exp(decay[t]) causally and
// exp(decay[t+1]) anti-causally (the decay of the token the state steps out
// of), 1 past the end.
struct WcumsumP {
  int B, H, T, F, S, L, ret, reverse;
  ts_strided x, out, decay;
  const float* log_alpha;
  float* tot;   // [B*H, S, F] last local value of each segment
  float* prod;  // [B*H, S]    decay product of each segment
};

__device__ __forceinline__ float wcumsum_step(const WcumsumP& p, const float* db, float a_static, int u) {
  if (p.ret == TS_RET_STATIC) return a_static;
  if (p.ret != TS_RET_STREAM) return 1.0f;
  const int tp = p.reverse ? p.T - 1 - u : u;
  const int src = p.reverse ? tp + 1 : tp;
  return src < p.T ? expf(db[(int64_t)src * p.decay.st]) : 1.0f;
}

// V consecutive features per thread (V = 4: 16-byte accesses where the rows
// allow them).
template <int V>
struct WVec;
template <>
struct WVec<1> {
  typedef float T;
  static __device__ __forceinline__ T zero() { return 0.f; }
};
template <>
struct WVec<4> {
  typedef floatx4 T;
  static __device__ __forceinline__ T zero() { return floatx4{0.f, 0.f, 0.f, 0.f}; }
};

struct WcumsumThread {
  int f, seg, b, h;
  int64_t r;
  const float* xb;
  const float* db;
  float a_static;
};

template <int V>
__device__ __forceinline__ bool wcumsum_thread(const WcumsumP& p, WcumsumThread& w) {
  const int FV = p.F / V;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)p.B * p.H * p.S * FV) return false;
  w.f = (int)(idx % FV) * V;
  w.r = idx / FV;
  w.seg = (int)(w.r % p.S);
  const int bh = (int)(w.r / p.S);
  w.b = bh / p.H;
  w.h = bh % p.H;
  w.xb = (const float*)p.x.ptr + (int64_t)w.b * p.x.sb + (int64_t)w.h * p.x.sh + w.f;
  w.db = p.ret == TS_RET_STREAM
             ? (const float*)p.decay.ptr + (int64_t)w.b * p.decay.sb + (int64_t)w.h * p.decay.sh
             : nullptr;
  w.a_static = p.ret == TS_RET_STATIC ? expf(p.log_alpha[w.h]) : 1.0f;
  return true;
}

template <int V>
__global__ __launch_bounds__(256) void wcumsum_summary_kernel(WcumsumP p) {
  typedef typename WVec<V>::T T;
  WcumsumThread w;
  if (!wcumsum_thread<V>(p, w)) return;
  const int u0 = w.seg * p.L;
  const int u1 = min(u0 + p.L, p.T);
  T z = WVec<V>::zero();
  float P = 1.0f;
#pragma unroll 8
  for (int u = u0; u < u1; ++u) {
    const int tp = p.reverse ? p.T - 1 - u : u;
    const float a = wcumsum_step(p, w.db, w.a_static, u);
    z = (u == u0 ? WVec<V>::zero() : a * z) + *(const T*)(w.xb + (int64_t)tp * p.x.st);
    P *= a;
  }
  *(T*)(p.tot + w.r * p.F + w.f) = z;
  if (w.f == 0) p.prod[w.r] = P;
}

template <int V>
__global__ __launch_bounds__(256) void wcumsum_main_kernel(WcumsumP p) {
  typedef typename WVec<V>::T T;
  WcumsumThread w;
  if (!wcumsum_thread<V>(p, w)) return;
  const int64_t row0 = (w.r / p.S) * p.S;
  T z = WVec<V>::zero();  // the state entering this segment
  for (int j = 0; j < w.seg; ++j) z = p.prod[row0 + j] * z + *(const T*)(p.tot + (row0 + j) * p.F + w.f);
  float* ob = (float*)p.out.ptr + (int64_t)w.b * p.out.sb + (int64_t)w.h * p.out.sh + w.f;
  const int u0 = w.seg * p.L;
  const int u1 = min(u0 + p.L, p.T);
#pragma unroll 8
  for (int u = u0; u < u1; ++u) {
    const int tp = p.reverse ? p.T - 1 - u : u;
    const float a = wcumsum_step(p, w.db, w.a_static, u);
    z = (u == 0 ? WVec<V>::zero() : a * z) + *(const T*)(w.xb + (int64_t)tp * p.x.st);
    *(T*)(ob + (int64_t)tp * p.out.st) = z;
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

// The same sum over 16-byte columns: a block is (256 / R) columns of four
// outputs x R slot rows; row r adds slots r, r + R, ... (four loads in flight
// per step), and the R rows of a column combine through LDS in row order, so
// the result does not depend on timing.  R grows with the slot count when
// there are few columns, so a wide sum and a tall one both fill the chip.
template <int R>
__device__ __forceinline__ void sum_slots_block(const float* a, int na, const float* b, int nb, int64_t nv, void* out,
                                                int out_bf16, float scale, int64_t blk, floatx4* red) {
  constexpr int CPB = 256 / R;
  const int tid = threadIdx.x;
  const int cl = tid % CPB, r = tid / CPB;
  const int64_t v = blk * CPB + cl;
  const int total = na + nb;
  floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0, acc2 = acc0, acc3 = acc0;
  if (v < nv) {
    const floatx4* av = (const floatx4*)a;
    const floatx4* bv = (const floatx4*)b;
    auto slot = [&](int t) -> floatx4 { return t < na ? av[(int64_t)t * nv + v] : bv[(int64_t)(t - na) * nv + v]; };
    int t = r;
    for (; t + 3 * R < total; t += 4 * R) {
      const floatx4 x0 = slot(t), x1 = slot(t + R), x2 = slot(t + 2 * R), x3 = slot(t + 3 * R);
      acc0 += x0;
      acc1 += x1;
      acc2 += x2;
      acc3 += x3;
    }
    for (; t < total; t += R) acc0 += slot(t);
  }
  red[tid] = (acc0 + acc1) + (acc2 + acc3);
  __syncthreads();
  if (r == 0 && v < nv) {
    floatx4 sum = red[cl];
#pragma unroll
    for (int k = 1; k < R; ++k) sum += red[k * CPB + cl];
    sum *= scale;
    if (out_bf16) {
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (bf16)sum[e];
      ((bf16x4*)out)[v] = o;
    } else {
      ((floatx4*)out)[v] = sum;
    }
  }
}

template <int R>
__global__ __launch_bounds__(256) void sum_slots_vec_kernel(const float* a, int na, const float* b, int nb,
                                                            int64_t nv, void* out, int out_bf16, float scale) {
  __shared__ floatx4 red[256];
  sum_slots_block<R>(a, na, b, nb, nv, out, out_bf16, scale, blockIdx.x, red);
}

// Several slot sums in one launch: block ranges [first[j], first[j+1]) belong
// to job j, which runs the one-launch kernel's code with its own R, so each
// result equals that of a separate ts_sum_slots call bit for bit.
struct SlotJobs {
  const float* a[kMaxSlotJobs];
  const float* b[kMaxSlotJobs];
  void* out[kMaxSlotJobs];
  int64_t nv[kMaxSlotJobs];
  int na[kMaxSlotJobs], nb[kMaxSlotJobs], R[kMaxSlotJobs], ob[kMaxSlotJobs];
  float scale[kMaxSlotJobs];
  int first[kMaxSlotJobs + 1];
  int n;
};

__global__ __launch_bounds__(256) void sum_slots_multi_kernel(SlotJobs J) {
  __shared__ floatx4 red[256];
  int j = 0;
  while (j + 1 < J.n && (int)blockIdx.x >= J.first[j + 1]) ++j;  // uniform per block
  const int64_t blk = (int64_t)blockIdx.x - J.first[j];
  switch (J.R[j]) {
    case 1: sum_slots_block<1>(J.a[j], J.na[j], J.b[j], J.nb[j], J.nv[j], J.out[j], J.ob[j], J.scale[j], blk, red); break;
    case 2: sum_slots_block<2>(J.a[j], J.na[j], J.b[j], J.nb[j], J.nv[j], J.out[j], J.ob[j], J.scale[j], blk, red); break;
    case 4: sum_slots_block<4>(J.a[j], J.na[j], J.b[j], J.nb[j], J.nv[j], J.out[j], J.ob[j], J.scale[j], blk, red); break;
    case 8: sum_slots_block<8>(J.a[j], J.na[j], J.b[j], J.nb[j], J.nv[j], J.out[j], J.ob[j], J.scale[j], blk, red); break;
    case 16: sum_slots_block<16>(J.a[j], J.na[j], J.b[j], J.nb[j], J.nv[j], J.out[j], J.ob[j], J.scale[j], blk, red); break;
    case 32: sum_slots_block<32>(J.a[j], J.na[j], J.b[j], J.nb[j], J.nv[j], J.out[j], J.ob[j], J.scale[j], blk, red); break;
    default: sum_slots_block<64>(J.a[j], J.na[j], J.b[j], J.nb[j], J.nv[j], J.out[j], J.ob[j], J.scale[j], blk, red); break;
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

// dst[b][t][s][h][:] = src_s[b][h][t][:]: grid x walks the [T][H][d/VEC]
// vectors of one (stream s = blockIdx.y, batch b = blockIdx.z), so the
// source descriptor is uniform per block; each thread moves 16 bytes.  Reads
// are whole source rows (d * sizeof(E) contiguous bytes), writes one
// contiguous [H*d] run per token.
struct StackP {
  int B, H, T, d, n;
  ts_strided src[4];
  void* dst;
};

template <typename E>
__global__ __launch_bounds__(256) void stack_heads_kernel(StackP p) {
  constexpr int VEC = 16 / (int)sizeof(E);
  const int s = blockIdx.y, b = blockIdx.z;
  const int dv = p.d / VEC;
  const int64_t per = (int64_t)p.T * p.H * dv;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= per) return;
  const int c = (int)(i % dv);
  const int64_t r = i / dv;
  const int h = (int)(r % p.H);
  const int t = (int)(r / p.H);
  const ts_strided src = p.src[s];
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (src.ptr)
    v = *(const uint4*)((const E*)src.ptr + (int64_t)b * src.sb + (int64_t)h * src.sh + (int64_t)t * src.st + c * VEC);
  E* dst = (E*)p.dst + (((int64_t)b * p.T + t) * p.n + s) * (int64_t)p.H * p.d + (int64_t)h * p.d + c * VEC;
  *(uint4*)dst = v;
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

// Chunks of 16 bytes per row rounded up to a power of two (<= 64).
int chunks_p2(const ts_read_desc* d) {
  const int chunks = d->d / (d->dtype == TS_BF16 ? 8 : 4);
  int p2 = 1;
  while (p2 < chunks) p2 <<= 1;
  return p2;
}

int rows_per_block(int cpr) { return ts::kReadRPT * (256 / cpr); }

// (T blocks, B*H) grid of the read kernels; false when it cannot be launched
bool read_grid(const ts_read_desc* d, dim3* grid) {
  const int rpb = rows_per_block(chunks_p2(d));
  *grid = dim3((unsigned)((d->T + rpb - 1) / rpb), (unsigned)(d->B * d->H));
  return (int64_t)d->B * d->H <= 65535;
}

template <typename E, int CPR>
void launch_read_fwd(dim3 grid, hipStream_t stream, const ts::ReadP& p) {
  hipLaunchKernelGGL((ts::read_fwd_kernel<E, CPR>), grid, dim3(256), 0, stream, p);
}
template <typename E, int CPR>
void launch_read_bwd(dim3 grid, hipStream_t stream, const ts::ReadP& p, float* parts) {
  hipLaunchKernelGGL((ts::read_bwd_kernel<E, CPR>), grid, dim3(256), 0, stream, p, parts);
}

template <typename E>
void dispatch_read(int cpr, dim3 grid, hipStream_t stream, const ts::ReadP& p, bool bwd, float* parts) {
  switch (cpr) {
#define TS_CASE(K)                                                              \
  case K:                                                                       \
    if (bwd) launch_read_bwd<E, K>(grid, stream, p, parts);                     \
    else launch_read_fwd<E, K>(grid, stream, p);                                \
    break;
    TS_CASE(1)
    TS_CASE(2)
    TS_CASE(4)
    TS_CASE(8)
    TS_CASE(16)
    TS_CASE(32)
    TS_CASE(64)
#undef TS_CASE
  }
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

template <typename E, int CPR>
void launch_qknorm(dim3 grid, hipStream_t stream, const ts::NormP& p, bool bwd) {
  if (bwd) hipLaunchKernelGGL((ts::qknorm_bwd_kernel<E, CPR>), grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL((ts::qknorm_fwd_kernel<E, CPR>), grid, dim3(256), 0, stream, p);
}

template <typename E>
void dispatch_qknorm(int cpr, dim3 grid, hipStream_t stream, const ts::NormP& p, bool bwd) {
  switch (cpr) {
    case 1: launch_qknorm<E, 1>(grid, stream, p, bwd); break;
    case 2: launch_qknorm<E, 2>(grid, stream, p, bwd); break;
    case 4: launch_qknorm<E, 4>(grid, stream, p, bwd); break;
    case 8: launch_qknorm<E, 8>(grid, stream, p, bwd); break;
    case 16: launch_qknorm<E, 16>(grid, stream, p, bwd); break;
    case 32: launch_qknorm<E, 32>(grid, stream, p, bwd); break;
    default: launch_qknorm<E, 64>(grid, stream, p, bwd); break;
  }
}

int qknorm_launch(const ts_qknorm_desc* d, ts_strided x, ts_strided dy, ts_strided out, const float* cs,
                  const float* sn, bool bwd, hipStream_t stream) {
  if (!d) return fail(TS_ERR_VALUE, "qknorm: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0 || d->d < 1) return fail(TS_ERR_VALUE, "qknorm: bad shape");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "qknorm: unknown dtype");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  if (d->d % vec || d->d / vec > 64) return fail(TS_ERR_VALUE, "qknorm: width %d must be a multiple of 16 bytes, at most 64 of them", d->d);
  if (d->rot < 0 || d->rot > d->d || d->rot % 2) return fail(TS_ERR_VALUE, "qknorm: rotated width %d", d->rot);
  if (d->rot > 0 && (!cs || !sn)) return fail(TS_ERR_VALUE, "qknorm: missing RoPE tables");
  if (!x.ptr || !out.ptr || (bwd && !dy.ptr)) return fail(TS_ERR_VALUE, "qknorm: missing tensors");
  for (const ts_strided* t : {&x, &dy, &out})
    if (t->ptr && (((uintptr_t)t->ptr & 15u) || t->st % vec || t->sh % vec || t->sb % vec))
      return fail(TS_ERR_VALUE, "qknorm: rows must be 16-byte aligned");
  if ((int64_t)d->B * d->H * d->T == 0) return TS_OK;
  const ts_read_desc rd = {d->B, d->H, d->T, d->d, d->dtype, 0, 0, 1.0f, d->eps};
  dim3 grid;
  if (!read_grid(&rd, &grid)) return fail(TS_ERR_NOT_IMPLEMENTED, "qknorm: more than 65535 (batch, head) slices");
  ts::NormP p;
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.d = d->d; p.rot = d->rot; p.eps = d->eps;
  p.x = x; p.dy = dy; p.cs = cs; p.sn = sn;
  if (bwd) p.dx = out;
  else p.y = out;
  if (d->dtype == TS_BF16) dispatch_qknorm<ts::bf16>(chunks_p2(&rd), grid, stream, p, bwd);
  else dispatch_qknorm<float>(chunks_p2(&rd), grid, stream, p, bwd);
  return finish(bwd ? "qknorm bwd" : "qknorm");
}

}  // namespace

namespace ts {

// Slot rows per column of the vectorised sum: enough threads to fill the chip
// (about 2^18 of them), at most one slot per row step.
static int slot_rows(int64_t nv, int total) {
  int R = 1;
  while (R < 64 && R < total && nv * R < 262144) R <<= 1;
  return R;
}

static bool slot_vec_ok(const float* a, const float* b, int64_t n, const void* out, int32_t out_dtype) {
  return n % 4 == 0 && !((uintptr_t)a & 15u) && !((uintptr_t)b & 15u) &&
         !((uintptr_t)out & (out_dtype == TS_BF16 ? 7u : 15u));
}

int sum_slots_batch(const SlotSum* jobs, int njobs, hipStream_t stream) {
  SlotJobs J;
  memset(&J, 0, sizeof(J));
  bool batch = njobs <= kMaxSlotJobs;
  for (int i = 0; i < njobs && batch; ++i) {
    const SlotSum& s = jobs[i];
    batch = s.n > 0 && s.na + s.nb > 0 && (s.na == 0 || s.a) && (s.nb == 0 || s.b) && s.out &&
            (s.out_dtype == TS_BF16 || s.out_dtype == TS_F32) && slot_vec_ok(s.a, s.b, s.n, s.out, s.out_dtype);
  }
  if (!batch) {
    for (int i = 0; i < njobs; ++i) {
      const SlotSum& s = jobs[i];
      const int rc = ts_sum_slots(s.a, s.na, s.b, s.nb, s.n, s.out, s.out_dtype, s.scale, stream);
      if (rc) return rc;
    }
    return TS_OK;
  }
  int blocks = 0;
  for (int i = 0; i < njobs; ++i) {
    const SlotSum& s = jobs[i];
    J.a[i] = s.a; J.b[i] = s.b; J.out[i] = s.out; J.na[i] = s.na; J.nb[i] = s.nb;
    J.nv[i] = s.n / 4;
    J.R[i] = slot_rows(J.nv[i], s.na + s.nb);
    J.ob[i] = s.out_dtype == TS_BF16 ? 1 : 0;
    J.scale[i] = s.scale;
    J.first[i] = blocks;
    blocks += (int)((J.nv[i] + 256 / J.R[i] - 1) / (256 / J.R[i]));
  }
  J.first[njobs] = blocks;
  J.n = njobs;
  if (blocks == 0) return TS_OK;
  hipLaunchKernelGGL(sum_slots_multi_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, J);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "sum_slots: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

}  // namespace ts

extern "C" {

int ts_read_fwd(const ts_read_desc* d, const ts_read_io* io, hipStream_t stream) {
  int rc = check_read(d);
  if (rc) return rc;
  if (!io || !io->num.ptr || !io->y.ptr) return fail(TS_ERR_VALUE, "read: missing tensors");
  if (d->normalize && !io->mass.ptr) return fail(TS_ERR_VALUE, "read: missing mass");
  if (d->gate && !io->g.ptr) return fail(TS_ERR_VALUE, "read: missing gate");
  if ((int64_t)d->B * d->H * d->T == 0) return TS_OK;
  dim3 grid;
  if (!read_grid(d, &grid)) return fail(TS_ERR_NOT_IMPLEMENTED, "read: more than 65535 (batch, head) slices");
  ts::ReadP p;
  fill_read(d, p);
  p.num = io->num; p.mass = io->mass; p.resid = io->resid; p.g = io->g; p.y = io->y;
  p.gbias = io->g_bias;
  if (d->dtype == TS_BF16) dispatch_read<ts::bf16>(chunks_p2(d), grid, stream, p, false, nullptr);
  else dispatch_read<float>(chunks_p2(d), grid, stream, p, false, nullptr);
  return finish("read");
}

int ts_read_bwd_parts(const ts_read_desc* d, int32_t* parts) {
  int rc = check_read(d);
  if (rc) return rc;
  dim3 grid;
  read_grid(d, &grid);
  if (parts) *parts = (int32_t)(d->B * (int)grid.x);
  return TS_OK;
}

int ts_read_bwd(const ts_read_desc* d, const ts_read_bwd_io* io, hipStream_t stream) {
  int rc = check_read(d);
  if (rc) return rc;
  if (!io || !io->num.ptr || !io->dy.ptr || !io->dnum.ptr) return fail(TS_ERR_VALUE, "read bwd: missing tensors");
  if (d->normalize && (!io->mass.ptr || !io->dmass.ptr)) return fail(TS_ERR_VALUE, "read bwd: missing mass");
  if (d->gate && (!io->g.ptr || !io->dg.ptr)) return fail(TS_ERR_VALUE, "read bwd: missing gate");
  if (io->dg_bias_part && (!d->gate || d->d > 256))
    return fail(TS_ERR_VALUE, "read bwd: gate-bias partials need the gate and a width of at most 256");
  if ((int64_t)d->B * d->H * d->T == 0) return TS_OK;
  dim3 grid;
  if (!read_grid(d, &grid)) return fail(TS_ERR_NOT_IMPLEMENTED, "read bwd: more than 65535 (batch, head) slices");
  ts::ReadP p;
  fill_read(d, p);
  p.num = io->num; p.mass = io->mass; p.resid = io->resid; p.g = io->g; p.dy = io->dy;
  p.dnum = io->dnum; p.dmass = io->dmass; p.dresid = io->dresid; p.dg = io->dg;
  p.gbias = io->g_bias;
  if (d->dtype == TS_BF16) dispatch_read<ts::bf16>(chunks_p2(d), grid, stream, p, true, io->dg_bias_part);
  else dispatch_read<float>(chunks_p2(d), grid, stream, p, true, io->dg_bias_part);
  return finish("read bwd");
}

int ts_qknorm_fwd(const ts_qknorm_desc* d, ts_strided x, ts_strided y, const float* rope_cos, const float* rope_sin,
                  hipStream_t stream) {
  return qknorm_launch(d, x, ts_strided{nullptr, 0, 0, 0}, y, rope_cos, rope_sin, false, stream);
}

int ts_qknorm_bwd(const ts_qknorm_desc* d, ts_strided x, ts_strided dy, ts_strided dx, const float* rope_cos,
                  const float* rope_sin, hipStream_t stream) {
  return qknorm_launch(d, x, dy, dx, rope_cos, rope_sin, true, stream);
}

int ts_sum_slots(const float* a, int32_t na, const float* b, int32_t nb, int64_t n, void* out, int32_t out_dtype,
                 float scale, hipStream_t stream) {
  if (n < 0 || na < 0 || nb < 0) return fail(TS_ERR_VALUE, "sum_slots: bad sizes");
  if ((na && !a) || (nb && !b) || !out) return fail(TS_ERR_VALUE, "sum_slots: missing buffers");
  if (out_dtype != TS_BF16 && out_dtype != TS_F32) return fail(TS_ERR_VALUE, "sum_slots: unknown dtype");
  if (n == 0) return TS_OK;
  const int total = na + nb;
  const bool vec = ts::slot_vec_ok(a, b, n, out, out_dtype);
  if (vec && total > 0) {
    // slot rows per column: enough threads to fill the chip, at most one slot per row step
    const int64_t nv = n / 4;
    const int R = ts::slot_rows(nv, total);
    const int cpb = 256 / R;
    const dim3 grid((unsigned)((nv + cpb - 1) / cpb));
    const int ob = out_dtype == TS_BF16 ? 1 : 0;
    switch (R) {
      case 1: hipLaunchKernelGGL(ts::sum_slots_vec_kernel<1>, grid, dim3(256), 0, stream, a, na, b, nb, nv, out, ob, scale); break;
      case 2: hipLaunchKernelGGL(ts::sum_slots_vec_kernel<2>, grid, dim3(256), 0, stream, a, na, b, nb, nv, out, ob, scale); break;
      case 4: hipLaunchKernelGGL(ts::sum_slots_vec_kernel<4>, grid, dim3(256), 0, stream, a, na, b, nb, nv, out, ob, scale); break;
      case 8: hipLaunchKernelGGL(ts::sum_slots_vec_kernel<8>, grid, dim3(256), 0, stream, a, na, b, nb, nv, out, ob, scale); break;
      case 16: hipLaunchKernelGGL(ts::sum_slots_vec_kernel<16>, grid, dim3(256), 0, stream, a, na, b, nb, nv, out, ob, scale); break;
      case 32: hipLaunchKernelGGL(ts::sum_slots_vec_kernel<32>, grid, dim3(256), 0, stream, a, na, b, nb, nv, out, ob, scale); break;
      default: hipLaunchKernelGGL(ts::sum_slots_vec_kernel<64>, grid, dim3(256), 0, stream, a, na, b, nb, nv, out, ob, scale); break;
    }
    return finish("sum_slots");
  }
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

int ts_stack_heads(const ts_stack_desc* d, const ts_strided* src, void* dst, hipStream_t stream) {
  if (!d || !src || !dst || d->B < 0 || d->H < 1 || d->T < 0 || d->d < 1 || d->n < 1 || d->n > 4)
    return fail(TS_ERR_VALUE, "stack_heads: bad arguments");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "stack_heads: unknown dtype");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  if (d->d % vec || ((uintptr_t)dst & 15u)) return fail(TS_ERR_VALUE, "stack_heads: rows must be 16-byte aligned");
  ts::StackP p;
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.d = d->d; p.n = d->n; p.dst = dst;
  for (int s = 0; s < d->n; ++s) {
    const ts_strided& x = src[s];
    if (x.ptr && (((uintptr_t)x.ptr & 15u) || x.sb % vec || x.sh % vec || x.st % vec))
      return fail(TS_ERR_VALUE, "stack_heads: source %d rows must be 16-byte aligned", s);
    p.src[s] = x;
  }
  const int64_t per = (int64_t)d->T * d->H * (d->d / vec);
  if (d->B == 0 || per == 0) return TS_OK;
  if ((per + 255) / 256 > 0x7fffffff || d->B > 65535) return fail(TS_ERR_NOT_IMPLEMENTED, "stack_heads: too large");
  const dim3 grid((unsigned)((per + 255) / 256), (unsigned)d->n, (unsigned)d->B);
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL(ts::stack_heads_kernel<ts::bf16>, grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL(ts::stack_heads_kernel<float>, grid, dim3(256), 0, stream, p);
  return finish("stack_heads");
}

// Segments of the scan order: enough (b, h, segment, feature) threads to
// fill the chip (about 2^19), at least 16 steps per segment.
static void wcumsum_segments(const ts_wcumsum_desc* d, int* S, int* L) {
  const int64_t lanes = (int64_t)d->B * d->H * d->F;
  int64_t want = ((int64_t)1 << 19) / (lanes > 0 ? lanes : 1);
  const int64_t most = (d->T + 15) / 16;
  if (want > most) want = most;
  if (want < 1) want = 1;
  *L = (int)((d->T + want - 1) / want);
  if (*L < 1) *L = 1;
  *S = (d->T + *L - 1) / *L;
}

int ts_wcumsum_workspace_bytes(const ts_wcumsum_desc* d, size_t* bytes) {
  if (!d || d->B < 1 || d->H < 1 || d->T < 0 || d->F < 1) return fail(TS_ERR_VALUE, "wcumsum: bad shape");
  int S = 0, L = 0;
  wcumsum_segments(d, &S, &L);
  if (bytes) *bytes = d->T == 0 ? 0 : (size_t)d->B * d->H * S * ((size_t)d->F + 1) * sizeof(float) + 256;
  return TS_OK;
}

int ts_wcumsum(const ts_wcumsum_desc* d, ts_strided x, ts_strided out, const float* log_alpha,
               ts_strided decay, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!d || d->B < 1 || d->H < 1 || d->T < 0 || d->F < 1) return fail(TS_ERR_VALUE, "wcumsum: bad shape");
  if (d->retention < TS_RET_NONE || d->retention > TS_RET_STREAM) return fail(TS_ERR_VALUE, "wcumsum: bad retention");
  if (d->T == 0) return TS_OK;
  if (!x.ptr || !out.ptr) return fail(TS_ERR_VALUE, "wcumsum: missing tensors");
  if (d->retention == TS_RET_STATIC && !log_alpha) return fail(TS_ERR_VALUE, "wcumsum: missing log_alpha");
  if (d->retention == TS_RET_STREAM && !decay.ptr) return fail(TS_ERR_VALUE, "wcumsum: missing decay");
  size_t need = 0;
  int rc = ts_wcumsum_workspace_bytes(d, &need);
  if (rc) return rc;
  if (!workspace || workspace_bytes < need)
    return fail(TS_ERR_VALUE, "wcumsum: workspace too small (%zu < %zu bytes)", workspace_bytes, need);
  if ((uintptr_t)workspace & 15u) return fail(TS_ERR_VALUE, "wcumsum: workspace is not 16-byte aligned");
  ts::WcumsumP p;
  p.B = d->B; p.H = d->H; p.T = d->T; p.F = d->F;
  wcumsum_segments(d, &p.S, &p.L);
  p.ret = d->retention; p.reverse = d->reverse;
  p.x = x; p.out = out; p.decay = decay; p.log_alpha = log_alpha;
  p.tot = (float*)workspace;
  p.prod = p.tot + (size_t)d->B * d->H * p.S * d->F;
  // four features per thread when every row start is 16-byte aligned
  const bool v4 = d->F % 4 == 0 && !((uintptr_t)x.ptr & 15u) && !((uintptr_t)out.ptr & 15u) && x.sb % 4 == 0 &&
                  x.sh % 4 == 0 && x.st % 4 == 0 && out.sb % 4 == 0 && out.sh % 4 == 0 && out.st % 4 == 0;
  const int V = v4 ? 4 : 1;
  const int64_t n = (int64_t)d->B * d->H * p.S * (d->F / V);
  const dim3 grid((unsigned)((n + 255) / 256));
  if (p.S > 1) {
    if (v4) hipLaunchKernelGGL(ts::wcumsum_summary_kernel<4>, grid, dim3(256), 0, stream, p);
    else hipLaunchKernelGGL(ts::wcumsum_summary_kernel<1>, grid, dim3(256), 0, stream, p);
    if ((rc = finish("wcumsum summary"))) return rc;
  }
  if (v4) hipLaunchKernelGGL(ts::wcumsum_main_kernel<4>, grid, dim3(256), 0, stream, p);
  else hipLaunchKernelGGL(ts::wcumsum_main_kernel<1>, grid, dim3(256), 0, stream, p);
  return finish("wcumsum");
}

}  // extern "C"
