// Output projection fused with the normalized read (gfx950, bf16).
//
// Forward:   y   = (resid + s * num / (mass + eps)) * silu(g + g_bias)
//            out = y W^T                      (W [N, K], K = H * d)
// Backward:  dy  = dout W                     (through W^T [K, N])
//            dnum, dmass, dresid, dg (and the gate-bias partials) from dy
//
// Both directions are one GEMM C[row][token] = sum_k A[row][k] Bt[token][k]
// over a tile of 64 tokens of one batch row:
//   forward  rows = output features (A = W,   Bt = y, built from the read's
//            inputs in the prologue), epilogue: store out;
//   backward rows = read features   (A = W^T, Bt = dout, loaded in the
//            prologue), epilogue: the read backward on the rows it owns.
// y (forward) and dy (backward) therefore never round-trip HBM; the forward
// may still store y for the caller's weight-gradient GEMM.
//
// Layout of one workgroup (4 waves, 64 tokens): the Bt tile [64][K] bf16
// sits in LDS (written once by the prologue, read by every wave); wave w owns
// 16 * NB consecutive rows and all 64 tokens, i.e. NB x 4 accumulator blocks
// of 16 x 16 (128 registers at NB = 8).  The A fragments come straight from
// global memory (the weights stay in L2; the next contraction step's
// fragments are in flight while the current step's MFMAs run).  The A rows
// of the block pair (2P, 2P+1) are interleaved so that lane group g of the
// pair's accumulators holds rows 32P + 8g .. 32P + 8g + 7 of one token:
// eight consecutive outputs per lane, one 16-byte access per token in the
// epilogues.
//
// Reference chain: src/thetascan/_core/modules/block.py:718-724 (output gate,
// reshape, proj_out), src/thetascan/_core/modules/gates.py:34-40 (OutGate)
// and src/thetascan/_core/ops/engine.py:440-442, 526-528 (normalized read).

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

constexpr int kTokTile = 64;  // tokens per workgroup

struct ReadOutP {
  int B, H, T, d, N, K, normalize, gate, nslices;
  float s, eps;
  ts_strided num, mass, resid, g;  // [B,H,T,d] read inputs
  ts_strided dnum, dmass, dresid, dg;
  const float* gbias;              // [H*d] or null
  const bf16* a;                   // fwd: W [N][K]; bwd: W^T [K][N]
  const bf16* bt;                  // bwd: dout rows (b*T + t) of N
  int64_t bt_ld;
  bf16* out;                       // fwd: out rows (b*T + t) of N
  int64_t out_ld;
  bf16* y;                         // fwd: y rows (b*T + t) of K (or null)
  int64_t y_ld;
  float* dgb_part;                 // bwd: [slots][K] (or null)
};

__device__ __forceinline__ float ro_sigmoid(float x) {
  // the read kernels' sigmoid: hardware exp2 and reciprocal
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

__device__ __forceinline__ void unpack8(const uint4& raw, float* out) {
  const bf16x8 v = __builtin_bit_cast(bf16x8, raw);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = (float)v[e];
}
__device__ __forceinline__ uint4 pack8(const float* in) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (bf16)in[e];
  return __builtin_bit_cast(uint4, v);
}

template <typename T>
__device__ __forceinline__ T* slice_at(const ts_strided& s, int b, int h, int t) {
  return (T*)s.ptr + (int64_t)b * s.sb + (int64_t)h * s.sh + (int64_t)t * s.st;
}

// The contraction: acc[nb][mb] (rows row(nb, .), tokens 16 mb + .) over K.
// Row of A for lane row i of block nb: row0 + 32 (nb/2) + 8 (i/4) + 4 (nb%2) + i%4.
template <int NB>
__device__ __forceinline__ void readout_gemm(const bf16* __restrict__ a, int64_t lda, int row0, int K,
                                             const bf16* bs, int kp, floatx4 (&acc)[NB][4]) {
  const int lane = threadIdx.x & 63, g = lane >> 4, l16 = lane & 15;
  const int rsub = 8 * (l16 >> 2) + (l16 & 3);
  const bf16* arow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) arow[nb] = a + (int64_t)(row0 + 32 * (nb >> 1) + 4 * (nb & 1) + rsub) * lda + 8 * g;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) acc[nb][mb] = floatx4{0.f, 0.f, 0.f, 0.f};
  // two register sets of A fragments, alternating (K / 32 is even), so that
  // no register copy waits for the loads in flight
  const int ks_n = K / 32;
  uint4 fa[NB], fb[NB];
  const bf16* brow = bs + l16 * kp + 8 * g;
  auto load = [&](uint4 (&f)[NB], int ks) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) f[nb] = *(const uint4*)(arow[nb] + 32 * ks);
  };
  auto step = [&](const uint4 (&f)[NB], int ks) {
    bf16x8 bf[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) bf[mb] = __builtin_bit_cast(bf16x8, *(const uint4*)(brow + 16 * mb * kp + 32 * ks));
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const bf16x8 af = __builtin_bit_cast(bf16x8, f[nb]);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) acc[nb][mb] = mma32(af, bf[mb], acc[nb][mb]);
    }
  };
  load(fa, 0);
  for (int ks = 0; ks < ks_n; ks += 2) {
    load(fb, ks + 1);
    step(fa, ks);
    if (ks + 2 < ks_n) load(fa, ks + 2);
    step(fb, ks + 1);
  }
}

// One tile of the forward's y [64][K] into LDS (and to global y when kept,
// by slice 0 only), by the workgroup's 256 threads `pt`: thread (token r,
// chunk lane c4) handles 16-byte chunks c4 + 4 i of every head row, in
// batches of items (head, chunk) whose loads are all issued first.  The
// gate bias comes from the LDS copy gb_s (zeros without a bias).
__device__ __forceinline__ void readout_produce(const ReadOutP& p, int pt, int b, int t0, int slice, bf16* bs,
                                                int kp, const float* gb_s) {
  const int r = pt >> 2, c4 = pt & 3;
  const int t = t0 + r;
  const bool live = t < p.T;
  const int per_head = p.d >> 5;  // chunks per thread per head (d / 32)
  const int items = p.H * per_head;
  constexpr int IB = 8;
  for (int i0 = 0; i0 < items; i0 += IB) {
    uint4 rn[IB], rr[IB], rg[IB];
    float ms[IB];
#pragma unroll
    for (int j = 0; j < IB; ++j) {
      const int it = i0 + j;
      const int h = it / per_head, c = c4 + 4 * (it - h * per_head);
      rn[j] = rr[j] = rg[j] = uint4{0u, 0u, 0u, 0u};
      ms[j] = 0.0f;
      if (it < items && live) {
        rn[j] = *(const uint4*)(slice_at<const bf16>(p.num, b, h, t) + 8 * c);
        if (p.resid.ptr) rr[j] = *(const uint4*)(slice_at<const bf16>(p.resid, b, h, t) + 8 * c);
        if (p.gate) rg[j] = *(const uint4*)(slice_at<const bf16>(p.g, b, h, t) + 8 * c);
        if (p.normalize) ms[j] = *slice_at<const float>(p.mass, b, h, t);
      }
    }
#pragma unroll
    for (int j = 0; j < IB; ++j) {
      const int it = i0 + j;
      if (it >= items) break;
      const int h = it / per_head, c = c4 + 4 * (it - h * per_head);
      const int col = h * p.d + 8 * c;
      float o[8];
      if (live) {
        const float scale = p.normalize ? p.s * __builtin_amdgcn_rcpf(ms[j] + p.eps) : p.s;
        float nv[8], rv[8], gv[8];
        unpack8(rn[j], nv);
        unpack8(rr[j], rv);
        unpack8(rg[j], gv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float v = (p.resid.ptr ? rv[e] : 0.0f) + scale * nv[e];
          if (p.gate) {
            const float x = gv[e] + gb_s[col + e];
            o[e] = v * x * ro_sigmoid(x);
          } else {
            o[e] = v;
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = 0.0f;
      }
      const uint4 packed = pack8(o);
      *(uint4*)(bs + r * kp + col) = packed;
      if (live && p.y && slice == 0) *(uint4*)(p.y + ((int64_t)b * p.T + t) * p.y_ld + col) = packed;
    }
  }
}

// Forward.  grid (ceil(T / 64), B * nslices); slice = N / (64 NB) rows.
// One tile per workgroup of 4 waves (two workgroups per CU): every thread
// builds its share of the y tile, then the waves contract it.
template <int NB>
__global__ __launch_bounds__(256, 2) void readout_fwd_flat_kernel(ReadOutP p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int kp = p.K + 8;
  bf16* bs = (bf16*)smem;
  float* gb_s = (float*)(bs + kTokTile * kp);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, l16 = lane & 15;
  const int t0 = blockIdx.x * kTokTile;
  const int b = blockIdx.y / p.nslices;
  const int slice = blockIdx.y - b * p.nslices;
  for (int i = tid; i < p.K; i += blockDim.x) gb_s[i] = p.gbias ? p.gbias[i] : 0.0f;
  __syncthreads();
  readout_produce(p, tid, b, t0, slice, bs, kp, gb_s);
  __syncthreads();
  const int row0 = slice * 64 * NB + w * 16 * NB;
  floatx4 acc[NB][4];
  readout_gemm<NB>(p.a, p.K, row0, p.K, bs, kp, acc);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int t = t0 + 16 * mb + l16;
    if (t >= p.T) continue;
    bf16* orow = p.out + ((int64_t)b * p.T + t) * p.out_ld;
#pragma unroll
    for (int pr = 0; pr < NB / 2; ++pr) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = acc[2 * pr][mb][e];
        o[4 + e] = acc[2 * pr + 1][mb][e];
      }
      *(uint4*)(orow + row0 + 32 * pr + 8 * g) = pack8(o);
    }
  }
}

// Backward.  grid (ceil(T / 64), B * nslices); slice = K / (64 NB) read
// features (whole heads per wave: 16 NB is a multiple of d).
template <int NB>
__global__ __launch_bounds__(256, 2) void readout_bwd_kernel(ReadOutP p) {
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* bs = (bf16*)smem;
  const int kp = p.N + 8;
  float* gb_s = (float*)(bs + kTokTile * kp);  // the gate bias (zeros without one)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, l16 = lane & 15;
  const int t0 = blockIdx.x * kTokTile;
  const int b = blockIdx.y / p.nslices;
  const int slice = blockIdx.y - b * p.nslices;
  for (int i = tid; i < p.K; i += blockDim.x) gb_s[i] = p.gbias ? p.gbias[i] : 0.0f;

  // ---- prologue: dout tile [64][N] into LDS
  {
    const int r = tid >> 2, c4 = tid & 3;
    const int t = t0 + r;
    const bool live = t < p.T;
    const bf16* src = p.bt + ((int64_t)b * p.T + (live ? t : 0)) * p.bt_ld;
    const int per = p.N >> 5;  // chunks per thread
    constexpr int IB = 16;
    for (int i0 = 0; i0 < per; i0 += IB) {
      uint4 v[IB];
#pragma unroll
      for (int j = 0; j < IB; ++j) {
        v[j] = uint4{0u, 0u, 0u, 0u};
        if (i0 + j < per && live) v[j] = *(const uint4*)(src + 8 * (c4 + 4 * (i0 + j)));
      }
#pragma unroll
      for (int j = 0; j < IB; ++j)
        if (i0 + j < per) *(uint4*)(bs + r * kp + 8 * (c4 + 4 * (i0 + j))) = v[j];
    }
  }
  __syncthreads();

  const int row0 = slice * 64 * NB + w * 16 * NB;
  floatx4 acc[NB][4];
  readout_gemm<NB>(p.a, p.N, row0, p.N, bs, kp, acc);

  // ---- epilogue: the read backward on rows row0 + 32 pr + 8 g .. + 7
  const int d = p.d;
  const int ppr = d >> 5;  // pairs (32 rows) per head
  float colsum[NB / 2][8];
#pragma unroll
  for (int pr = 0; pr < NB / 2; ++pr)
#pragma unroll
    for (int e = 0; e < 8; ++e) colsum[pr][e] = 0.0f;
  // per token block: every pair's loads first (no store of an earlier pair
  // sits between them and the arithmetic), then the pairs in order
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int t = t0 + 16 * mb + l16;
    const bool live = t < p.T;
    const int tc = live ? t : 0;
    uint4 rn[NB / 2], rr[NB / 2], rg[NB / 2];
    float ms[NB / 2];
#pragma unroll
    for (int pr = 0; pr < NB / 2; ++pr) {
      const int j = row0 + 32 * pr + 8 * g;
      const int h = j / d, c = j - h * d;
      rn[pr] = rr[pr] = rg[pr] = uint4{0u, 0u, 0u, 0u};
      ms[pr] = 0.0f;
      if (live) {
        rn[pr] = *(const uint4*)(slice_at<const bf16>(p.num, b, h, tc) + c);
        if (p.resid.ptr) rr[pr] = *(const uint4*)(slice_at<const bf16>(p.resid, b, h, tc) + c);
        if (p.gate) rg[pr] = *(const uint4*)(slice_at<const bf16>(p.g, b, h, tc) + c);
        if (p.normalize) ms[pr] = *slice_at<const float>(p.mass, b, h, tc);
      }
    }
    float dot = 0.0f;
#pragma unroll
    for (int pr = 0; pr < NB / 2; ++pr) {
      const int j = row0 + 32 * pr + 8 * g;
      const int h = j / d, c = j - h * d;
      const float denom = p.normalize && live ? ms[pr] + p.eps : 1.0f;
      const float inv = __builtin_amdgcn_rcpf(denom);
      const float scale = p.normalize ? p.s * inv : p.s;
      float dv[8], nv[8], rv[8], gv[8], o_dnum[8], o_dg[8], o_dres[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dv[e] = acc[2 * pr][mb][e];
        dv[4 + e] = acc[2 * pr + 1][mb][e];
      }
      unpack8(rn[pr], nv);
      unpack8(rr[pr], rv);
      unpack8(rg[pr], gv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float dye = live ? dv[e] : 0.0f;  // dy stays fp32 (never stored)
        float dpre = dye;
        o_dg[e] = 0.0f;
        if (p.gate) {
          const float x = gv[e] + gb_s[j + e];
          const float sg = ro_sigmoid(x);
          const float ypre = (p.resid.ptr ? rv[e] : 0.0f) + scale * nv[e];
          o_dg[e] = dye * ypre * (sg * (1.0f + x * (1.0f - sg)));
          dpre = dye * x * sg;
        }
        o_dnum[e] = scale * dpre;
        o_dres[e] = dpre;
        dot += dpre * nv[e];
        colsum[pr][e] += o_dg[e];
      }
      if (live) {
        *(uint4*)(slice_at<bf16>(p.dnum, b, h, t) + c) = pack8(o_dnum);
        if (p.dresid.ptr) *(uint4*)(slice_at<bf16>(p.dresid, b, h, t) + c) = pack8(o_dres);
        if (p.gate) *(uint4*)(slice_at<bf16>(p.dg, b, h, t) + c) = pack8(o_dg);
      }
      if (p.normalize && (pr % ppr) == ppr - 1) {
        // the head's rows: this lane's pairs of the head, then the four lane groups
        float tot = dot + __shfl_xor(dot, 16, 64);
        tot += __shfl_xor(tot, 32, 64);
        if (live && g == 0) *slice_at<float>(p.dmass, b, h, t) = -p.s * tot * inv * inv;
        dot = 0.0f;
      } else if ((pr % ppr) == ppr - 1) {
        dot = 0.0f;
      }
    }
  }
  if (p.dgb_part) {
    // sum over the 16 token lanes of each lane group, in lane order
    float* dst = p.dgb_part + ((int64_t)b * gridDim.x + blockIdx.x) * p.K;
#pragma unroll
    for (int pr = 0; pr < NB / 2; ++pr)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = colsum[pr][e];
        v += __shfl_xor(v, 1, 64);
        v += __shfl_xor(v, 2, 64);
        v += __shfl_xor(v, 4, 64);
        v += __shfl_xor(v, 8, 64);
        colsum[pr][e] = v;
      }
    if (l16 == 0) {
#pragma unroll
      for (int pr = 0; pr < NB / 2; ++pr) {
        floatx4 lo = {colsum[pr][0], colsum[pr][1], colsum[pr][2], colsum[pr][3]};
        floatx4 hi = {colsum[pr][4], colsum[pr][5], colsum[pr][6], colsum[pr][7]};
        float* o = dst + row0 + 32 * pr + 8 * g;
        *(floatx4*)o = lo;
        *(floatx4*)(o + 4) = hi;
      }
    }
  }
}

}  // namespace ts

namespace {

using ts::fail;

int ro_finish(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TS_OK;
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Rows per workgroup (64 NB): the largest NB in {8, 4, 2} that divides `rows`
// (and, backward, whose 16 NB rows per wave hold whole heads of width d).
int pick_nb(int rows, int d, bool bwd) {
  for (int nb = 8; nb >= 2; nb >>= 1) {
    if (rows % (64 * nb)) continue;
    if (bwd && (16 * nb) % d) continue;
    return nb;
  }
  return 0;
}

int check_ro(const ts_read_out_desc* d, bool bwd, int* nb) {
  if (!d) return fail(TS_ERR_VALUE, "read_out: null descriptor");
  const ts_read_desc& r = d->read;
  if (r.B < 1 || r.H < 1 || r.T < 0 || r.d < 1 || d->n < 1) return fail(TS_ERR_VALUE, "read_out: bad shape");
  if (r.dtype != TS_BF16) return fail(TS_ERR_NOT_IMPLEMENTED, "read_out: bf16 only");
  if (r.d % 32 || r.d > 128) return fail(TS_ERR_NOT_IMPLEMENTED, "read_out: head width %d (needs 32, 64, 96 or 128)", r.d);
  const int K = r.H * r.d;
  if (K % 128 || d->n % 128) return fail(TS_ERR_NOT_IMPLEMENTED, "read_out: widths %d, %d need multiples of 128", K, d->n);
  // the forward double-buffers y tiles of 64 x (K + 8) bf16 in LDS
  if (K > 512 || d->n > 1024) return fail(TS_ERR_NOT_IMPLEMENTED, "read_out: widths %d, %d beyond 512, 1024", K, d->n);
  *nb = bwd ? pick_nb(K, r.d, true) : pick_nb(d->n, r.d, false);
  if (!*nb) return fail(TS_ERR_NOT_IMPLEMENTED, "read_out: no row tiling for widths %d, %d", K, d->n);
  return TS_OK;
}

void fill_ro(const ts_read_out_desc* d, ts::ReadOutP& p) {
  memset(&p, 0, sizeof(p));
  p.B = d->read.B; p.H = d->read.H; p.T = d->read.T; p.d = d->read.d; p.N = d->n; p.K = d->read.H * d->read.d;
  p.normalize = d->read.normalize ? 1 : 0; p.gate = d->read.gate ? 1 : 0;
  p.s = d->read.scale; p.eps = d->read.eps;
}

template <typename K>
int ro_launch(K kern, const char* what, int nb, int width_lds, const ts::ReadOutP& p, hipStream_t stream) {
  const int lds = ts::kTokTile * (width_lds + 8) * 2 + p.K * 4;
  hipError_t e = ts::ensure_lds_limit((const void*)kern, lds);
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "%s: LDS limit: %s", what, hipGetErrorString(e));
  const dim3 grid((unsigned)((p.T + ts::kTokTile - 1) / ts::kTokTile), (unsigned)(p.B * p.nslices));
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, stream, p);
  (void)nb;
  return ro_finish(what);
}

}  // namespace

extern "C" {

int ts_read_out_fwd(const ts_read_out_desc* d, const ts_read_out_io* io, hipStream_t stream) {
  int nb = 0;
  int rc = check_ro(d, false, &nb);
  if (rc) return rc;
  if (!io || !io->num.ptr || !io->w || !io->out) return fail(TS_ERR_VALUE, "read_out: missing tensors");
  if (d->read.normalize && !io->mass.ptr) return fail(TS_ERR_VALUE, "read_out: missing mass");
  if (d->read.gate && !io->g.ptr) return fail(TS_ERR_VALUE, "read_out: missing gate");
  if (io->out_ld < d->n || (io->y && io->y_ld < d->read.H * d->read.d))
    return fail(TS_ERR_VALUE, "read_out: row strides below the row widths");
  if (!al16(io->w) || !al16(io->out) || (io->out_ld % 8) || (io->y && (!al16(io->y) || io->y_ld % 8)) ||
      !al16(io->num.ptr) || (io->resid.ptr && !al16(io->resid.ptr)) || (io->g.ptr && !al16(io->g.ptr)))
    return fail(TS_ERR_VALUE, "read_out: rows must be 16-byte aligned");
  if (d->read.B * (int64_t)d->read.T == 0) return TS_OK;
  ts::ReadOutP p;
  fill_ro(d, p);
  p.nslices = d->n / (64 * nb);
  p.num = io->num; p.mass = io->mass; p.resid = io->resid; p.g = io->g; p.gbias = io->g_bias;
  p.a = (const ts::bf16*)io->w;
  p.out = (ts::bf16*)io->out; p.out_ld = io->out_ld;
  p.y = (ts::bf16*)io->y; p.y_ld = io->y_ld;
  switch (nb) {
    case 8: return ro_launch(ts::readout_fwd_flat_kernel<8>, "read_out fwd", nb, p.K, p, stream);
    case 4: return ro_launch(ts::readout_fwd_flat_kernel<4>, "read_out fwd", nb, p.K, p, stream);
    default: return ro_launch(ts::readout_fwd_flat_kernel<2>, "read_out fwd", nb, p.K, p, stream);
  }
}

int ts_read_out_bwd_parts(const ts_read_out_desc* d, int32_t* parts) {
  int nb = 0;
  int rc = check_ro(d, true, &nb);
  if (rc) return rc;
  if (parts) *parts = (int32_t)(d->read.B * ((d->read.T + ts::kTokTile - 1) / ts::kTokTile));
  return TS_OK;
}

int ts_read_out_bwd(const ts_read_out_desc* d, const ts_read_out_bwd_io* io, hipStream_t stream) {
  int nb = 0;
  int rc = check_ro(d, true, &nb);
  if (rc) return rc;
  if (!io || !io->num.ptr || !io->w_t || !io->dout || !io->dnum.ptr)
    return fail(TS_ERR_VALUE, "read_out bwd: missing tensors");
  if (d->read.normalize && (!io->mass.ptr || !io->dmass.ptr)) return fail(TS_ERR_VALUE, "read_out bwd: missing mass");
  if (d->read.gate && (!io->g.ptr || !io->dg.ptr)) return fail(TS_ERR_VALUE, "read_out bwd: missing gate");
  if (io->dg_bias_part && !d->read.gate) return fail(TS_ERR_VALUE, "read_out bwd: gate-bias partials need the gate");
  if (io->dout_ld < d->n) return fail(TS_ERR_VALUE, "read_out bwd: row stride below the row width");
  if (!al16(io->w_t) || !al16(io->dout) || (io->dout_ld % 8) || !al16(io->num.ptr) || !al16(io->dnum.ptr) ||
      (io->resid.ptr && !al16(io->resid.ptr)) || (io->g.ptr && !al16(io->g.ptr)) ||
      (io->dresid.ptr && !al16(io->dresid.ptr)) || (io->dg.ptr && !al16(io->dg.ptr)) ||
      (io->dg_bias_part && !al16(io->dg_bias_part)))
    return fail(TS_ERR_VALUE, "read_out bwd: rows must be 16-byte aligned");
  if (d->read.B * (int64_t)d->read.T == 0) return TS_OK;
  const int K = d->read.H * d->read.d;
  if ((int64_t)d->read.B * (K / (64 * nb)) > 65535) return fail(TS_ERR_NOT_IMPLEMENTED, "read_out bwd: batch too large");
  ts::ReadOutP p;
  fill_ro(d, p);
  p.nslices = K / (64 * nb);
  p.num = io->num; p.mass = io->mass; p.resid = io->resid; p.g = io->g; p.gbias = io->g_bias;
  p.dnum = io->dnum; p.dmass = io->dmass; p.dresid = io->dresid; p.dg = io->dg;
  p.a = (const ts::bf16*)io->w_t;
  p.bt = (const ts::bf16*)io->dout; p.bt_ld = io->dout_ld;
  p.dgb_part = io->dg_bias_part;
  switch (nb) {
    case 8: return ro_launch(ts::readout_bwd_kernel<8>, "read_out bwd", nb, p.N, p, stream);
    case 4: return ro_launch(ts::readout_bwd_kernel<4>, "read_out bwd", nb, p.N, p, stream);
    default: return ro_launch(ts::readout_bwd_kernel<2>, "read_out bwd", nb, p.N, p, stream);
  }
}

}  // extern "C"
