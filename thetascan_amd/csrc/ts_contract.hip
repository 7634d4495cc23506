// Token contractions for gfx950: out[g] = sum_n a[g, n, :]^T b[g, n, :] in fp32
// for token-major tiles a [G, N, p] and b [G, N, q] (p, q multiples of 16 up to
// 128).  These are the weight gradients of the GN fast network (dW1 = da^T x,
// dW2 = lam^T dz + ...), formed from per-token tiles written by the GN backward
// kernels.
//
// Workgroup (slice s, group g) contracts tokens [s * span, (s + 1) * span) in
// 64-token tiles: both tiles are staged in LDS (rows fetched with 16-byte
// loads one tile ahead), and wave w accumulates the 16 x 16 output blocks of
// rows 16 * (w + 4 j) with MFMAs whose token-axis operands come from the
// transposing LDS read (the same fragments as the feature backward's weight
// gradients).  Every slice writes an fp32 partial [p, q]; ts_sum_slots adds
// the partials in slice order, so the result does not depend on timing.

#include "ts_common.h"
#include "ts_tokens.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct ContractP {
  int G, N, p, q, span;
  const void* a;
  const void* b;
  int64_t a_sg, a_sn, b_sg, b_sn;  // element strides: group, token
  float* parts;                    // [S][G][p][q]
};

// a / b tile rows fetched one tile ahead (16-byte vectors, rows past the
// slice's end load as zero).
template <typename E>
struct ContractTile {
  static constexpr int VEC = 16 / (int)sizeof(E);
  static constexpr int SLOTS = (TT * 128 / VEC + 255) / 256;
  uint4 r[SLOTS];
  __device__ __forceinline__ void fetch(const E* base, int64_t sn, int width, int n0, int n1, int tid) {
    const int per_row = width / VEC;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / per_row;
      r[i] = make_uint4(0u, 0u, 0u, 0u);
      if (idx < TT * per_row && n0 + row < n1)
        r[i] = *(const uint4*)(base + (int64_t)(n0 + row) * sn + (idx - row * per_row) * VEC);
    }
  }
  __device__ __forceinline__ void store(E* dst, int pitch, int width, int tid) const {
    const int per_row = width / VEC;
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) {
      const int idx = tid + i * 256;
      if (idx < TT * per_row) {
        const int row = idx / per_row;
        *(uint4*)(dst + row * pitch + (idx - row * per_row) * VEC) = r[i];
      }
    }
  }
};

template <typename E>
__global__ __launch_bounds__(256) void contract_kernel(ContractP P) {
  typedef TokFrag<E> TF;
  constexpr int VEC = 16 / (int)sizeof(E);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15, g4 = lane >> 4;
  const int s = blockIdx.x, grp = blockIdx.y;
  const int pitch_a = P.p + VEC, pitch_b = P.q + VEC;
  extern __shared__ __align__(16) unsigned char smem[];
  E* As = (E*)smem;
  E* Bs = As + TT * pitch_a;
  const E* a = (const E*)P.a + grp * P.a_sg;
  const E* b = (const E*)P.b + grp * P.b_sg;
  const int n0 = s * P.span;
  const int n1 = min(n0 + P.span, P.N);
  const int npb = P.p / 16, nqb = P.q / 16;

  floatx4 acc[2][8];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int qb = 0; qb < 8; ++qb) acc[j][qb] = floatx4{0.f, 0.f, 0.f, 0.f};

  ContractTile<E> la, lb;
  la.fetch(a, P.a_sn, P.p, n0, n1, tid);
  lb.fetch(b, P.b_sn, P.q, n0, n1, tid);
  for (int t0 = n0; t0 < n1; t0 += TT) {
    __syncthreads();  // the previous tile is no longer read
    la.store(As, pitch_a, P.p, tid);
    lb.store(Bs, pitch_b, P.q, tid);
    if (t0 + TT < n1) {
      la.fetch(a, P.a_sn, P.p, t0 + TT, n1, tid);
      lb.fetch(b, P.b_sn, P.q, t0 + TT, n1, tid);
    }
    __syncthreads();
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int pb = w + 4 * j;
        if (pb >= npb) break;
        const auto fa = TF::get(As, pitch_a, pb * 16, kp, lane);
#pragma unroll
        for (int qb = 0; qb < 8; ++qb) {
          if (qb >= nqb) break;
          acc[j][qb] = mma32(fa, TF::get(Bs, pitch_b, qb * 16, kp, lane), acc[j][qb]);
        }
      }
    }
  }
  // acc[j][qb] lane (l16, g4) holds rows pb*16 + 4*g4 + i, column qb*16 + l16
  float* out = P.parts + ((size_t)s * P.G + grp) * (size_t)P.p * P.q;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int pb = w + 4 * j;
    if (pb >= npb) break;
#pragma unroll
    for (int qb = 0; qb < 8; ++qb) {
      if (qb >= nqb) break;
#pragma unroll
      for (int i = 0; i < 4; ++i) out[(size_t)(pb * 16 + 4 * g4 + i) * P.q + qb * 16 + l16] = acc[j][qb][i];
    }
  }
}

}  // namespace ts

namespace {

using ts::fail;

struct ContractPlan {
  int S, span;
  size_t lds, parts_bytes;
};

int plan_contract(const ts_contract_desc* d, ContractPlan* P) {
  if (!d) return fail(TS_ERR_VALUE, "contract: null descriptor");
  if (d->G < 1 || d->N < 0 || d->p < 16 || d->q < 16) return fail(TS_ERR_VALUE, "contract: bad shape");
  if (d->p % 16 || d->q % 16 || d->p > 128 || d->q > 128)
    return fail(TS_ERR_NOT_IMPLEMENTED, "contract: widths %d x %d must be multiples of 16 up to 128", d->p, d->q);
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "contract: unknown dtype");
  // slices: about two workgroups per CU (256 CUs), at least two tiles each
  const int tiles = (d->N + ts::TT - 1) / ts::TT;
  int S = 1;
  while ((long)S * 2 * d->G <= 512 && tiles >= 4 * S) S *= 2;
  const int tiles_per = (tiles + S - 1) / S;
  P->span = tiles_per * ts::TT;
  P->S = tiles > 0 ? (tiles + tiles_per - 1) / tiles_per : 1;
  const int es = d->dtype == TS_BF16 ? 2 : 4;
  const int vec = 16 / es;
  P->lds = (size_t)ts::TT * (d->p + vec + d->q + vec) * es;
  P->parts_bytes = (size_t)P->S * d->G * d->p * d->q * sizeof(float);
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_contract_workspace_bytes(const ts_contract_desc* d, size_t* bytes) {
  ContractPlan P;
  int rc = plan_contract(d, &P);
  if (rc) return rc;
  if (bytes) *bytes = P.parts_bytes;
  return TS_OK;
}

int ts_contract_tokens(const ts_contract_desc* d, const void* a, int64_t a_sg, int64_t a_sn, const void* b,
                       int64_t b_sg, int64_t b_sn, float* out, void* workspace, size_t ws_bytes, hipStream_t stream) {
  ContractPlan P;
  int rc = plan_contract(d, &P);
  if (rc) return rc;
  if (!a || !b || !out) return fail(TS_ERR_VALUE, "contract: missing tensors");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  if (((uintptr_t)a & 15u) || ((uintptr_t)b & 15u) || a_sn % vec || b_sn % vec || a_sg % vec || b_sg % vec)
    return fail(TS_ERR_VALUE, "contract: rows must be 16-byte aligned");
  if (!workspace || ws_bytes < P.parts_bytes)
    return fail(TS_ERR_VALUE, "contract: workspace needs %zu bytes", P.parts_bytes);
  ts::ContractP p;
  memset(&p, 0, sizeof(p));
  p.G = d->G; p.N = d->N; p.p = d->p; p.q = d->q; p.span = P.span;
  p.a = a; p.b = b; p.a_sg = a_sg; p.a_sn = a_sn; p.b_sg = b_sg; p.b_sn = b_sn;
  p.parts = (float*)workspace;
  const dim3 grid((unsigned)P.S, (unsigned)d->G);
  const void* fn = d->dtype == TS_BF16 ? (const void*)ts::contract_kernel<ts::bf16> : (const void*)ts::contract_kernel<float>;
  if (P.lds > 65536) {
    hipError_t e = ts::ensure_lds_limit(fn, (int)P.lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "contract: LDS request failed: %s", hipGetErrorString(e));
  }
  if (d->dtype == TS_BF16)
    hipLaunchKernelGGL(ts::contract_kernel<ts::bf16>, grid, dim3(256), P.lds, stream, p);
  else
    hipLaunchKernelGGL(ts::contract_kernel<float>, grid, dim3(256), P.lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "contract: launch failed: %s", hipGetErrorString(e));
  return ts_sum_slots(p.parts, P.S, nullptr, 0, (int64_t)d->G * d->p * d->q, out, TS_F32, 1.0f, stream);
}

}  // extern "C"
