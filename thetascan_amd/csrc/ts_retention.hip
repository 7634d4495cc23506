// Gradient of a causal scan with respect to a static per-head retention
// (gfx950).
//
// A scan with static retention alpha = exp(log_alpha[h]),
//   o_t = sum_{i<=t} alpha^(t-i) (q_t . k_i) v_i   (+ the key-mass column),
// has the exact derivative
//   dL/dlog_alpha = sum_t sum_{i<=t} (t-i) alpha^(t-i) (q_t . k_i) (dO_t . v_i + dm_t),
// where dm is the gradient of the mass column (v_i = 1; dm enters as two
// bf16 columns hi + lo against two unit columns).  This is the
// retention gradient the reference's autograd forms through the chunk
// backend's tile weights (scan_chunk.py:102-155, 246-339).  Written as
// sum_t t dL_t with dL_t = q_t . dq_t - k_t . dk_t, it is a small difference
// of terms about T / (1 - alpha) times larger, which bf16 scans cannot
// resolve; this kernel sums the pair terms themselves instead.
//
// A workgroup walks one segment of seg_tiles 64-token tiles of one (b, h);
// wave w owns value block w (16 columns; the last block of a call with a mass
// column holds that column).  Per tile:
//   * pairs inside the tile: S = Q K^T and G = D V_w^T on MFMA (fp32 from the
//     bf16 inputs), summed with the weights d alpha^d, d = t - i >= 0;
//   * pairs with i in earlier tiles of the segment, through the states
//     M = sum_{i<t0} alpha^(t0-1-i) k_i v_i^T and M' = sum (t0-1-i) alpha^(..) k_i v_i^T:
//     sum_t alpha^(tau+1) [(tau+1) q_t^T M dO_t + q_t^T M' dO_t], tau = t - t0.
// Operands formed inside the kernel (the state copies and the weighted value
// and gradient rows) enter the MFMAs as bf16 pairs hi + lo, hi = bf16(x),
// lo = bf16(x - hi): with the bf16 inputs exact, every product then carries
// about 16 bits, as the fp32 sums need.
// Pairs across segments need the state entering the segment, which is not
// known here; each segment therefore also leaves its own forward summaries
// M_s, M'_s and the query-side sums A_s = sum_t (n+1) alpha^(n+1) q_t dO_t^T,
// B_s = sum_t alpha^(n+1) q_t dO_t^T (n = t - segment start), and a combine
// kernel adds <M_in, A_s> + <M'_in, B_s> with M_in, M'_in the prefix of the
// summaries (M'_in composes as alpha^L (M'_in + L M_in) + M'_s).

#include "ts_common.h"
#include "ts_scan_impl.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

struct RetP {
  int B, H, T, dk, dv, nvr, has_mass, seg_tiles, nseg, vw;  // nvr: real value blocks; vw: padded width
  ts_strided q, k, v, dout, dm;
  uint32_t q_rec, k_rec, v_rec, o_rec, dm_rec;
  const float* log_alpha;
  float* part;  // [BH][nseg]
  float* sums;  // [BH][nseg][4][dk][vw]: M, M', A, B
};

struct RetLayout {
  int qp, vp, mp;
  int qs, ks, vs, ds, ms;  // element offsets (E)
  int fbase;               // float offset of pw[65], dpw[65], red[8]
  int bytes;
};

__host__ __device__ inline RetLayout ret_layout(int DK, int vw, int nw) {
  RetLayout L{};
  L.qp = DK + 8;
  L.vp = vw + 8;
  L.mp = DK + 8;
  L.qs = 0;
  L.ks = L.qs + C * L.qp;
  L.vs = L.ks + C * L.qp;
  L.ds = L.vs + C * L.vp;
  L.ms = L.ds + C * L.vp;                       // [nw][4][16][mp]: M hi, M lo, M' hi, M' lo
  const int e_end = L.ms + nw * 4 * 16 * L.mp;
  const int e_bytes = (e_end * 2 + 15) / 16 * 16;
  L.fbase = e_bytes / 4;
  L.bytes = e_bytes + (65 + 65 + 8) * 4;
  return L;
}

// x = hi + lo to about 16 bits: hi = bf16(x), lo = bf16(x - hi).
template <typename H>
__device__ __forceinline__ void split(float x, H& hi, H& lo) {
  hi = (bf16)x;
  lo = (bf16)(x - tof((bf16)hi));
}

template <int DK>
__global__ __launch_bounds__(512) void retention_grad_kernel(RetP p) {
  typedef bf16 E;
  typedef LdsIO<E> IO;
  typedef Tok<E> TK;
  constexpr int NK32 = DK / 32;
  constexpr bool KTAIL = (DK % 32) != 0;
  constexpr int NKB = DK / 16;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, l16 = lane & 15;
  const int nw = blockDim.x >> 6;
  const int seg = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int bh = b * p.H + h;
  const int vw = p.vw;
  const RetLayout L = ret_layout(DK, vw, nw);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* Qs = base + L.qs;
  E* Ks = base + L.ks;
  E* Vs = base + L.vs;
  E* Ds = base + L.ds;
  E* Mw = base + L.ms + w * 4 * 16 * L.mp;   // this wave's M^T [16][mp] (hi, lo), then M'^T (hi, lo)
  E* Mlw = Mw + 16 * L.mp;
  E* Mpw = Mw + 32 * L.mp;
  E* Mplw = Mw + 48 * L.mp;
  float* fb = (float*)smem + L.fbase;
  float* pw = fb;        // alpha^d, d = 0..64
  float* dpw = fb + 65;  // d alpha^d
  float* red = fb + 130;

  const float la = p.log_alpha[h];
  if (tid < 65) {
    const float a = expf(la * (float)tid);
    pw[tid] = a;
    dpw[tid] = (float)tid * a;
  }

  const int nchunks = (p.T + C - 1) / C;
  const int c0 = seg * p.seg_tiles;
  const int c1 = min(c0 + p.seg_tiles, nchunks);
  const int q_st = (int)p.q.st * 2, k_st = (int)p.k.st * 2, v_st = (int)p.v.st * 2, o_st = (int)p.dout.st * 2;
  const rsrc_t q_rs = make_rsrc(bh_base(p.q, b, h, 2), p.q_rec);
  const rsrc_t k_rs = make_rsrc(bh_base(p.k, b, h, 2), p.k_rec);
  const rsrc_t v_rs = make_rsrc(bh_base(p.v, b, h, 2), p.v_rec);
  const rsrc_t o_rs = make_rsrc(bh_base(p.dout, b, h, 2), p.o_rec);
  const int vr = p.nvr * 16;  // real (padded) value columns; the mass block follows

  floatx4 M[NKB], Mp[NKB], A[NKB], Bq[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) M[kb] = Mp[kb] = A[kb] = Bq[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
  float acc = 0.f;

  for (int c = c0; c < c1; ++c) {
    const int t0 = c * C;
    const int len = min(C, p.T - t0);
    __syncthreads();  // the previous tile's operands are consumed
    // ---- tiles: Q, K [64][DK]; V, D [64][vw] (real columns, zero padding,
    // then the mass block: V column of ones, D column of dm)
    for (int idx = tid; idx < C * (DK / 8); idx += blockDim.x) {
      const int row = idx / (DK / 8), col = (idx % (DK / 8)) * 8;
      const uint32_t oq = col < p.dk ? (uint32_t)((t0 + row) * q_st + col * 2) : kOOB;
      const uint32_t ok = col < p.dk ? (uint32_t)((t0 + row) * k_st + col * 2) : kOOB;
      *(uint4*)(Qs + row * L.qp + col) = bld16(q_rs, oq);
      *(uint4*)(Ks + row * L.qp + col) = bld16(k_rs, ok);
    }
    for (int idx = tid; idx < C * (vw / 8); idx += blockDim.x) {
      const int row = idx / (vw / 8), col = (idx % (vw / 8)) * 8;
      uint4 vv = make_uint4(0u, 0u, 0u, 0u), dd = vv;
      if (col < vr) {
        const uint32_t ov = col < p.dv ? (uint32_t)((t0 + row) * v_st + col * 2) : kOOB;
        const uint32_t oo = col < p.dv ? (uint32_t)((t0 + row) * o_st + col * 2) : kOOB;
        vv = bld16(v_rs, ov);
        dd = bld16(o_rs, oo);
      } else if (col == vr && p.has_mass) {
        const bool valid = t0 + row < p.T;
        const float dmv = valid ? bldf(make_rsrc(bh_base(p.dm, b, h, 4), p.dm_rec),
                                      (uint32_t)((t0 + row) * (int)p.dm.st * 4)) : 0.f;
        // dm (fp32) as two bf16 columns hi + lo against two unit columns
        Vec16<E> a, d;
        a.raw = vv;
        d.raw = dd;
        a.e[0] = a.e[1] = valid ? (E)1.0f : (E)0.0f;
        E hi, lo;
        split(dmv, hi, lo);
        d.e[0] = hi;
        d.e[1] = lo;
        vv = a.raw;
        dd = d.raw;
      }
      *(uint4*)(Vs + row * L.vp + col) = vv;
      *(uint4*)(Ds + row * L.vp + col) = dd;
    }
    __syncthreads();

    const E* Dw = Ds + w * 16;
    const E* Vw = Vs + w * 16;
    // ---- pairs inside the tile
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
#pragma unroll
      for (int ib = 0; ib <= tb; ++ib) {
        floatx4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NK32; ++j)
          s = mma32(frow8<E>(Qs, L.qp, tb * 16 + l16, j, g), frow8<E>(Ks, L.qp, ib * 16 + l16, j, g), s);
        if (KTAIL) s = mma16(frow4<E>(Qs, L.qp, tb * 16 + l16, NK32, g), frow4<E>(Ks, L.qp, ib * 16 + l16, NK32, g), s);
        floatx4 gg = {0.f, 0.f, 0.f, 0.f};
        gg = mma16(frow4<E>(Dw, L.vp, tb * 16 + l16, 0, g), frow4<E>(Vw, L.vp, ib * 16 + l16, 0, g), gg);
        // accumulator layout: rows (queries) tb*16 + 4g + i, columns (keys) ib*16 + l16
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = (tb - ib) * 16 + 4 * g + i - l16;
          acc += (d >= 0 ? dpw[max(d, 0)] : 0.f) * s[i] * gg[i];
        }
      }
    }
    // ---- pairs with keys in earlier tiles of the segment
    if (c > c0) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        floatx4 qm = {0.f, 0.f, 0.f, 0.f}, qmp = qm;
#pragma unroll
        for (int j = 0; j < NK32; ++j) {
          const auto qf = frow8<E>(Qs, L.qp, tb * 16 + l16, j, g);
          qm = mma32(qf, frow8<E>(Mw, L.mp, l16, j, g), qm);
          qm = mma32(qf, frow8<E>(Mlw, L.mp, l16, j, g), qm);
          qmp = mma32(qf, frow8<E>(Mpw, L.mp, l16, j, g), qmp);
          qmp = mma32(qf, frow8<E>(Mplw, L.mp, l16, j, g), qmp);
        }
        if (KTAIL) {
          const auto qf = frow4<E>(Qs, L.qp, tb * 16 + l16, NK32, g);
          qm = mma16(qf, frow4<E>(Mw, L.mp, l16, NK32, g), qm);
          qm = mma16(qf, frow4<E>(Mlw, L.mp, l16, NK32, g), qm);
          qmp = mma16(qf, frow4<E>(Mpw, L.mp, l16, NK32, g), qmp);
          qmp = mma16(qf, frow4<E>(Mplw, L.mp, l16, NK32, g), qmp);
        }
        // rows: queries tau = tb*16 + 4g + i; columns: value l16 of this block
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int tau = tb * 16 + 4 * g + i;
          const float dv = tof(Dw[tau * L.vp + l16]);
          acc += pw[tau + 1] * ((float)(tau + 1) * qm[i] + qmp[i]) * dv;
        }
      }
    }
    // ---- query-side sums A, B (weights relative to the segment start)
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) {
      const bf16x8 d8 = TK::col8(Dw, L.vp, 0, kp, lane);
      bf16x8 dA, dAl, dB, dBl;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = 32 * kp + (e < 4 ? 4 * g + e : 12 + 4 * g + e);
        const float n1 = (float)((c - c0) * C + tok + 1);
        const float wb = expf(la * n1);
        const float x = tof(d8[e]);
        E h0, l0, h1, l1;
        split(x * n1 * wb, h0, l0);
        split(x * wb, h1, l1);
        dA[e] = h0; dAl[e] = l0; dB[e] = h1; dBl[e] = l1;
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const auto qc = TK::col8(Qs, L.qp, kb * 16, kp, lane);
        A[kb] = mma32(qc, dA, A[kb]);
        A[kb] = mma32(qc, dAl, A[kb]);
        Bq[kb] = mma32(qc, dB, Bq[kb]);
        Bq[kb] = mma32(qc, dBl, Bq[kb]);
      }
    }
    // ---- forward states after this tile (relative to its last token)
    {
      const float dec = pw[len];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          Mp[kb][i] = dec * (Mp[kb][i] + (float)len * M[kb][i]);
          M[kb][i] *= dec;
        }
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        const bf16x8 v8 = TK::col8(Vw, L.vp, 0, kp, lane);
        bf16x8 va, val, vb, vbl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int tok = 32 * kp + (e < 4 ? 4 * g + e : 12 + 4 * g + e);
          const int d = len - 1 - tok;
          const float x = tof(v8[e]);
          E h0, l0, h1, l1;
          split(d >= 0 ? x * pw[max(d, 0)] : 0.f, h0, l0);
          split(d >= 0 ? x * dpw[max(d, 0)] : 0.f, h1, l1);
          va[e] = h0; val[e] = l0; vb[e] = h1; vbl[e] = l1;
        }
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const auto kc = TK::col8(Ks, L.qp, kb * 16, kp, lane);
          M[kb] = mma32(kc, va, M[kb]);
          M[kb] = mma32(kc, val, M[kb]);
          Mp[kb] = mma32(kc, vb, Mp[kb]);
          Mp[kb] = mma32(kc, vbl, Mp[kb]);
        }
      }
      // bf16 hi / lo copies (transposed: [value][key]) for the next tile's queries
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        E hi[4], lo[4], phi[4], plo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          split(M[kb][i], hi[i], lo[i]);
          split(Mp[kb][i], phi[i], plo[i]);
        }
        const int o = l16 * L.mp + kb * 16 + 4 * g;
        IO::st4(Mw + o, tof(hi[0]), tof(hi[1]), tof(hi[2]), tof(hi[3]));
        IO::st4(Mlw + o, tof(lo[0]), tof(lo[1]), tof(lo[2]), tof(lo[3]));
        IO::st4(Mpw + o, tof(phi[0]), tof(phi[1]), tof(phi[2]), tof(phi[3]));
        IO::st4(Mplw + o, tof(plo[0]), tof(plo[1]), tof(plo[2]), tof(plo[3]));
      }
    }
  }

  // ---- this segment's pair sum and summaries
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) acc += __shfl_xor(acc, o, 64);
  if (lane == 0) red[w] = acc;
  __syncthreads();
  if (tid == 0) {
    float s = 0.f;
    for (int i = 0; i < nw; ++i) s += red[i];
    p.part[(size_t)bh * p.nseg + seg] = s;
  }
  const size_t nel = (size_t)p.dk * vw;
  float* out = p.sums + ((size_t)bh * p.nseg + seg) * 4 * nel;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const size_t e = (size_t)(kb * 16 + 4 * g + i) * vw + w * 16 + l16;
      out[e] = M[kb][i];
      out[nel + e] = Mp[kb][i];
      out[2 * nel + e] = A[kb][i];
      out[3 * nel + e] = Bq[kb][i];
    }
}

__global__ void retention_zero_kernel(float* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

// Cross-segment pairs: <M_in, A_s> + <M'_in, B_s> with the running prefix of
// the segment summaries, plus the segments' own pair sums -> out[b][h].
__global__ __launch_bounds__(256) void retention_combine_kernel(RetP p, float* out) {
  const int bh = blockIdx.x;
  const int h = bh % p.H;
  const float la = p.log_alpha[h];
  const size_t nel = (size_t)p.dk * p.vw;
  const int seg_len = p.seg_tiles * C;
  float acc = 0.f;
  for (size_t e = threadIdx.x; e < nel; e += blockDim.x) {
    float m = 0.f, mp = 0.f;
    for (int s = 0; s < p.nseg; ++s) {
      const float* base = p.sums + ((size_t)bh * p.nseg + s) * 4 * nel;
      if (s > 0) acc += m * base[2 * nel + e] + mp * base[3 * nel + e];
      const int len = min(seg_len, p.T - s * seg_len);
      const float aL = expf(la * (float)len);
      mp = aL * (mp + (float)len * m) + base[nel + e];
      m = aL * m + base[e];
    }
  }
  __shared__ float red[4];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) acc += __shfl_xor(acc, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = red[0] + red[1] + red[2] + red[3];
    for (int i = 0; i < p.nseg; ++i) s += p.part[(size_t)bh * p.nseg + i];
    out[bh] = s;
  }
}

}  // namespace ts

namespace {

using ts::fail;

typedef void (*RetFn)(ts::RetP);

RetFn pick_ret(int dk) {
  switch (dk) {
    case 16: return ts::retention_grad_kernel<16>;
    case 32: return ts::retention_grad_kernel<32>;
    case 48: return ts::retention_grad_kernel<48>;
    case 64: return ts::retention_grad_kernel<64>;
    case 80: return ts::retention_grad_kernel<80>;
    case 96: return ts::retention_grad_kernel<96>;
    case 112: return ts::retention_grad_kernel<112>;
    case 128: return ts::retention_grad_kernel<128>;
  }
  return nullptr;
}

struct RetPlan {
  int dkp, nvr, vw, nw, seg_tiles, nseg;
  size_t part_bytes, sums_bytes;
};

int ret_plan(const ts_retention_desc* d, RetPlan* P) {
  if (!d) return fail(TS_ERR_VALUE, "retention grad: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0 || d->dk < 1 || d->dv < 1)
    return fail(TS_ERR_VALUE, "retention grad: bad shape");
  if (d->dtype != TS_BF16) return fail(TS_ERR_NOT_IMPLEMENTED, "retention grad: bf16 streams only");
  if (d->dk > 128 || d->dk % 16 || d->dv % 8)
    return fail(TS_ERR_NOT_IMPLEMENTED,
                "retention grad: dk a multiple of 16 up to 128, dv a multiple of 8 (split wider keys)");
  P->dkp = d->dk;
  P->nvr = (d->dv + 15) / 16;
  P->vw = (P->nvr + (d->has_mass ? 1 : 0)) * 16;
  P->nw = P->vw / 16;
  if (P->nw > 8) return fail(TS_ERR_NOT_IMPLEMENTED, "retention grad: at most 8 value blocks per call (split wider values)");
  if (ts::ret_layout(P->dkp, P->vw, P->nw).bytes > ts::kLdsPerCU)
    return fail(TS_ERR_NOT_IMPLEMENTED, "retention grad: tiles of dk=%d and %d value columns exceed LDS (split the values)",
                P->dkp, P->vw);
  const int tiles = (d->T + ts::C - 1) / ts::C;
  int st = d->seg_tiles;
  if (st <= 0) {
    // about 512 workgroups, segments of at least two tiles
    st = 2;
    while (st < tiles && (long)d->B * d->H * ((tiles + st - 1) / st) > 512) st *= 2;
  }
  P->seg_tiles = st;
  P->nseg = tiles > 0 ? (tiles + st - 1) / st : 0;
  P->part_bytes = (size_t)d->B * d->H * P->nseg * sizeof(float);
  P->sums_bytes = (size_t)d->B * d->H * P->nseg * 4 * (size_t)P->dkp * P->vw * sizeof(float);
  return TS_OK;
}

uint32_t span_bytes(const ts_strided& s, int T, int width, int es) {
  if (!s.ptr || T == 0) return 0;
  return (uint32_t)(((int64_t)(T - 1) * s.st + width) * es);
}

}  // namespace

extern "C" {

int ts_retention_workspace_bytes(const ts_retention_desc* d, size_t* bytes) {
  RetPlan P;
  int rc = ret_plan(d, &P);
  if (rc) return rc;
  if (bytes) *bytes = P.part_bytes + 256 + P.sums_bytes;
  return TS_OK;
}

int ts_retention_grad(const ts_retention_desc* d, const ts_retention_io* io, float* out, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
  RetPlan P;
  int rc = ret_plan(d, &P);
  if (rc) return rc;
  if (!io || !out || !io->log_alpha || !io->q.ptr || !io->k.ptr || !io->v.ptr || !io->dout.ptr)
    return fail(TS_ERR_VALUE, "retention grad: missing tensors");
  if (d->has_mass && !io->dmass.ptr) return fail(TS_ERR_VALUE, "retention grad: missing dmass");
  for (const ts_strided* s : {&io->q, &io->k, &io->v, &io->dout})
    if (((uintptr_t)s->ptr & 15u) || s->st % 8 || s->sh % 8 || s->sb % 8)
      return fail(TS_ERR_VALUE, "retention grad: streams need 16-byte aligned rows");
  const size_t need = P.part_bytes + 256 + P.sums_bytes;
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 15u))
    return fail(TS_ERR_VALUE, "retention grad: workspace needs %zu bytes, 16-byte aligned", need);
  const int bh = d->B * d->H;
  if (d->T == 0) {
    hipLaunchKernelGGL(ts::retention_zero_kernel, dim3((bh + 255) / 256), dim3(256), 0, stream, out, bh);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TS_OK : fail(TS_ERR_RUNTIME, "retention grad: launch failed: %s", hipGetErrorString(e));
  }
  ts::RetP p;
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.dk = P.dkp; p.dv = d->dv; p.nvr = P.nvr; p.has_mass = d->has_mass;
  p.seg_tiles = P.seg_tiles; p.nseg = P.nseg; p.vw = P.vw;
  p.q = io->q; p.k = io->k; p.v = io->v; p.dout = io->dout; p.dm = io->dmass;
  p.q_rec = span_bytes(io->q, d->T, d->dk, 2);
  p.k_rec = span_bytes(io->k, d->T, d->dk, 2);
  p.v_rec = span_bytes(io->v, d->T, d->dv, 2);
  p.o_rec = span_bytes(io->dout, d->T, d->dv, 2);
  p.dm_rec = span_bytes(io->dmass, d->T, 1, 4);
  p.log_alpha = io->log_alpha;
  p.part = (float*)workspace;
  p.sums = (float*)((char*)workspace + (P.part_bytes + 255) / 256 * 256);
  RetFn fn = pick_ret(P.dkp);
  if (!fn) return fail(TS_ERR_NOT_IMPLEMENTED, "retention grad: no kernel for dk=%d", P.dkp);
  const ts::RetLayout L = ts::ret_layout(P.dkp, P.vw, P.nw);
  if (L.bytes > 65536) {
    hipError_t e = ts::ensure_lds_limit((const void*)fn, L.bytes);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "retention grad: LDS request failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(fn, dim3(P.nseg, d->H, d->B), dim3(64 * P.nw), (size_t)L.bytes, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "retention grad: launch failed: %s", hipGetErrorString(e));
  hipLaunchKernelGGL(ts::retention_combine_kernel, dim3(bh), dim3(256), 0, stream, p, out);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "retention grad: combine launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

}  // extern "C"
