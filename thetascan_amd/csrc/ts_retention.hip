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
//   * pairs inside the tile: the ten causal 16x16 blocks of S = Q K^T, each
//     formed once by one wave on MFMA, against G = D V^T of every value
//     block, summed with the weights d alpha^d, d = t - i >= 0;
//   * pairs with i in earlier tiles of the segment, through the states
//     M = sum_{i<t0} alpha^(t0-1-i) k_i v_i^T and M' = sum (t0-1-i) alpha^(..) k_i v_i^T:
//     sum_t alpha^(tau+1) [(tau+1) q_t^T M dO_t + q_t^T M' dO_t], tau = t - t0.
//     Each wave holds its value block of M and M' in MFMA accumulators, and
//     they enter the next MFMAs from registers (the accumulator rows are the
//     contraction order of the query fragments), with no LDS copy.
// Operands formed inside the kernel (the states and the weighted value and
// gradient rows) enter the MFMAs as bf16 pairs hi + lo, hi = bf16(x),
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
  int B, H, T, dk, dv, nvr, has_mass, seg_tiles, nseg, vw, nw;  // nvr: real value blocks; vw: padded width
  ts_strided q, k, v, dout, dm;
  uint32_t q_rec, k_rec, v_rec, o_rec, dm_rec;
  const float* log_alpha;
  float* part;  // [BH][nseg]
  float* sums;  // [BH][nseg][4][dk][vw]: M, M', A, B
};

// LDS of one workgroup: the four bf16 tiles, then fp32 weight tables.
struct RetLayout {
  int qp, vp;
  int qs, ks, vs, ds;  // element offsets (bf16)
  int fbase;           // float offset of the tables
  int bytes;
};
// table offsets (floats from fbase)
constexpr int kTabD = 0;      // [128] at 64 + d: d alpha^d for d >= 0, 0 for d < 0
constexpr int kTabRA = 128;   // [64] (tau+1) alpha^(tau+1)
constexpr int kTabRB = 192;   // [64] alpha^(tau+1)
constexpr int kTabPow = 256;  // [68] alpha^d, d = 0..64
constexpr int kTabWM = 324;   // [64] this tile's alpha^(len-1-tok), 0 past len
constexpr int kTabWMp = 388;  // [64] (len-1-tok) alpha^(len-1-tok)
constexpr int kTabWA = 452;   // [64] (n+1) alpha^(n+1), n from the segment start
constexpr int kTabWB = 516;   // [64] alpha^(n+1)
constexpr int kTabRed = 580;  // [8]
constexpr int kTabFloats = 588;

__host__ __device__ inline RetLayout ret_layout(int DK, int vw) {
  RetLayout L{};
  L.qp = DK + 8;
  L.vp = vw + 8;
  L.qs = 0;
  L.ks = L.qs + C * L.qp;
  L.vs = L.ks + C * L.qp;
  L.ds = L.vs + C * L.vp;
  const int e_end = L.ds + C * L.vp;
  const int e_bytes = (e_end * 2 + 15) / 16 * 16;
  L.fbase = e_bytes / 4;
  L.bytes = e_bytes + kTabFloats * 4;
  return L;
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// Two floats rounded to bf16 (RNE) in one dword, a in the low half.
__device__ __forceinline__ uint32_t pk2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(floatx2{a, b}, bf16x2));
}

// x = hi + lo to about 16 bits for eight values: hi = bf16(x), lo = bf16(x - hi).
__device__ __forceinline__ void split8(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = pk2(x[2 * j], x[2 * j + 1]);
    l[j] = pk2(x[2 * j] - __uint_as_float(h[j] << 16), x[2 * j + 1] - __uint_as_float(h[j] & 0xffff0000u));
  }
  hi = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
  lo = __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]));
}

// Accumulator fragments a, b (the eight k-values of one lane) as hi + lo.
__device__ __forceinline__ void split_acc(floatx4 a, floatx4 b, bf16x8& hi, bf16x8& lo) {
  const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  split8(x, hi, lo);
}
__device__ __forceinline__ void split_acc4(floatx4 a, bf16x4& hi, bf16x4& lo) {
  const uint32_t h0 = pk2(a[0], a[1]), h1 = pk2(a[2], a[3]);
  const uint32_t l0 = pk2(a[0] - __uint_as_float(h0 << 16), a[1] - __uint_as_float(h0 & 0xffff0000u));
  const uint32_t l1 = pk2(a[2] - __uint_as_float(h1 << 16), a[3] - __uint_as_float(h1 & 0xffff0000u));
  hi = __builtin_bit_cast(bf16x4, make_uint2(h0, h1));
  lo = __builtin_bit_cast(bf16x4, make_uint2(l0, l1));
}

// bf16 element e of a fragment as float
__device__ __forceinline__ float elt(bf16x8 v, int e) { return tof(v[e]); }

// Eight table entries at the tokens of a col8 fragment (kp, lane group g).
__device__ __forceinline__ void tab8(const float* t, int kp, int g, float (&w)[8]) {
  const floatx4 a = *(const floatx4*)(t + 32 * kp + 4 * g);
  const floatx4 b = *(const floatx4*)(t + 32 * kp + 16 + 4 * g);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w[i] = a[i];
    w[4 + i] = b[i];
  }
}

// (query block, key block) pairs of the causal tile, key block <= query block
__constant__ int kPairs[10][2] = {{0, 0}, {1, 0}, {1, 1}, {2, 0}, {2, 1}, {2, 2}, {3, 0}, {3, 1}, {3, 2}, {3, 3}};

template <int DK>
__global__ __launch_bounds__(512) void retention_grad_kernel(RetP p) {
  typedef bf16 E;
  typedef Tok<E> TK;
  constexpr int NK32 = DK / 32;
  constexpr bool KTAIL = (DK % 32) != 0;
  constexpr int NKB = DK / 16;
  constexpr int QC = DK / 8;  // 16-byte chunks per key row
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, l16 = lane & 15;
  const int bd = blockDim.x, nwave = bd >> 6;
  const int seg = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int bh = b * p.H + h;
  const int vw = p.vw, nw = p.nw;
  const bool owner = w < nw;  // owns value block w; later waves only load and form tile pairs
  const RetLayout L = ret_layout(DK, vw);
  extern __shared__ __align__(16) unsigned char smem[];
  E* base = (E*)smem;
  E* Qs = base + L.qs;
  E* Ks = base + L.ks;
  E* Vs = base + L.vs;
  E* Ds = base + L.ds;
  float* tab = (float*)smem + L.fbase;

  const float la = p.log_alpha[h];
  for (int i = tid; i < 128; i += bd) {
    const int d = i - 64;
    tab[kTabD + i] = d >= 0 ? (float)d * expf(la * (float)d) : 0.f;
  }
  for (int i = tid; i < 65; i += bd) tab[kTabPow + i] = expf(la * (float)i);
  for (int i = tid; i < 64; i += bd) {
    const float a = expf(la * (float)(i + 1));
    tab[kTabRA + i] = (float)(i + 1) * a;
    tab[kTabRB + i] = a;
  }

  const int nchunks = (p.T + C - 1) / C;
  const int c0 = seg * p.seg_tiles;
  const int c1 = min(c0 + p.seg_tiles, nchunks);
  const int q_st = (int)p.q.st * 2, k_st = (int)p.k.st * 2, v_st = (int)p.v.st * 2, o_st = (int)p.dout.st * 2;
  const rsrc_t q_rs = make_rsrc(bh_base(p.q, b, h, 2), p.q_rec);
  const rsrc_t k_rs = make_rsrc(bh_base(p.k, b, h, 2), p.k_rec);
  const rsrc_t v_rs = make_rsrc(bh_base(p.v, b, h, 2), p.v_rec);
  const rsrc_t o_rs = make_rsrc(bh_base(p.dout, b, h, 2), p.o_rec);
  const rsrc_t dm_rs = make_rsrc(bh_base(p.dm, b, h, 4), p.dm_rec);
  const int vr = p.nvr * 16;  // real (padded) value columns; the mass block follows

  // tile loads: at most two 16-byte chunks of each tile per thread (the host
  // launches max(value blocks, DK/16) waves); rows and columns fixed per tile
  int v_row[2], v_col[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = tid + r * bd;
    v_row[r] = idx < C * (vw / 8) ? idx / (vw / 8) : -1;
    v_col[r] = idx < C * (vw / 8) ? (idx % (vw / 8)) * 8 : 0;
  }

  // this wave's value block w: the states and query-side sums, rows (keys)
  // kb*16 + 4g + i, column (value) w*16 + l16
  floatx4 M[NKB], Mp[NKB], A[NKB], Bq[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) M[kb] = Mp[kb] = A[kb] = Bq[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
  float acc = 0.f;

  // tile c's loads go to registers while tile c - 1 is computed
  uint4 rq[2], rk[2], rv[2], rd[2];
  float rdm[2];
  auto fetch = [&](int c) {
    const int t0 = c * C;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int idx = tid + r * bd;
      rq[r] = rk[r] = rv[r] = rd[r] = make_uint4(0u, 0u, 0u, 0u);
      rdm[r] = 0.f;
      if (idx < C * QC) {
        const int row = idx / QC, col = (idx % QC) * 8;
        rq[r] = bld16(q_rs, (uint32_t)((t0 + row) * q_st + col * 2));
        rk[r] = bld16(k_rs, (uint32_t)((t0 + row) * k_st + col * 2));
      }
      const int row = v_row[r], col = v_col[r];
      if (row >= 0 && col < vr) {
        const uint32_t ov = col < p.dv ? (uint32_t)((t0 + row) * v_st + col * 2) : kOOB;
        const uint32_t oo = col < p.dv ? (uint32_t)((t0 + row) * o_st + col * 2) : kOOB;
        rv[r] = bld16(v_rs, ov);
        rd[r] = bld16(o_rs, oo);
      } else if (row >= 0 && col == vr && p.has_mass && t0 + row < p.T) {
        rdm[r] = bldf(dm_rs, (uint32_t)((t0 + row) * (int)p.dm.st * 4));
      }
    }
  };
  if (c0 < c1) fetch(c0);

  for (int c = c0; c < c1; ++c) {
    const int t0 = c * C;
    const int len = min(C, p.T - t0);
    __syncthreads();  // the previous tile's operands and tables are consumed
    {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int idx = tid + r * bd;
        if (idx < C * QC) {
          const int row = idx / QC, col = (idx % QC) * 8;
          *(uint4*)(Qs + row * L.qp + col) = rq[r];
          *(uint4*)(Ks + row * L.qp + col) = rk[r];
        }
        const int row = v_row[r], col = v_col[r];
        if (row >= 0) {
          uint4 vv = rv[r], dd = rd[r];
          if (col == vr && p.has_mass) {
            // two unit V columns against dm as bf16 hi + lo
            const bool valid = t0 + row < p.T;
            const uint32_t one = valid ? 0x3f803f80u : 0u;  // bf16 1.0 twice
            const uint32_t dh = pk2(rdm[r], 0.f);
            const float hi = __uint_as_float(dh << 16);
            vv = make_uint4(one, 0u, 0u, 0u);
            dd = make_uint4(pk2(hi, rdm[r] - hi), 0u, 0u, 0u);
          }
          *(uint4*)(Vs + row * L.vp + col) = vv;
          *(uint4*)(Ds + row * L.vp + col) = dd;
        }
      }
      // this tile's weights
      if (tid < 64) {
        const int tok = tid, d = len - 1 - tok;
        const float pw = d >= 0 ? tab[kTabPow + max(d, 0)] : 0.f;
        tab[kTabWM + tok] = pw;
        tab[kTabWMp + tok] = (float)d * pw;
        const float n1 = (float)((c - c0) * C + tok + 1);
        const float a = expf(la * n1);
        tab[kTabWA + tok] = n1 * a;
        tab[kTabWB + tok] = a;
      }
    }
    __syncthreads();
    if (c + 1 < c1) fetch(c + 1);

    // ---- pairs inside the tile: each score block once, against every value block
    for (int pi = w; pi < 10; pi += nwave) {
      const int tb = kPairs[pi][0], ib = kPairs[pi][1];
      floatx4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NK32; ++j)
        sc = mma32(frow8<E>(Qs, L.qp, tb * 16 + l16, j, g), frow8<E>(Ks, L.qp, ib * 16 + l16, j, g), sc);
      if (KTAIL) sc = mma16(frow4<E>(Qs, L.qp, tb * 16 + l16, NK32, g), frow4<E>(Ks, L.qp, ib * 16 + l16, NK32, g), sc);
      // rows (queries) tb*16 + 4g + i, columns (keys) ib*16 + l16; d = t - i
      const float* dt = tab + kTabD + 64 + (tb - ib) * 16 + 4 * g - l16;
      float wd[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) wd[i] = dt[i] * sc[i];
      // value blocks four at a time: their operand reads and products issue
      // together before the sums consume them
      for (int vb0 = 0; vb0 < nw; vb0 += 4) {
        floatx4 gg[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          gg[u] = floatx4{0.f, 0.f, 0.f, 0.f};
          const int vb = vb0 + u;
          if (vb < nw)
            gg[u] = mma16(frow4<E>(Ds + vb * 16, L.vp, tb * 16 + l16, 0, g),
                          frow4<E>(Vs + vb * 16, L.vp, ib * 16 + l16, 0, g), gg[u]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc += wd[i] * gg[u][i];
      }
    }

    if (owner) {
      const E* Dw = Ds + w * 16;
      const E* Vw = Vs + w * 16;
      bf16x8 d8[2];
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) d8[kp] = TK::col8(Dw, L.vp, 0, kp, lane);
      // ---- pairs with keys in earlier tiles of the segment, through the
      // states (B operand from the accumulators: column = value, contraction
      // over keys in the accumulator order), as bf16 hi + lo
      if (c > c0) {
        // rows of the products: queries tau = tb*16 + 4g + i; the gradient
        // entries of those rows in this value column are d8[tb / 2] elements
        // (tb % 2)*4 + i
        auto add_rows = [&](int tb, floatx4 qm, floatx4 qmp) {
          const floatx4 ra = *(const floatx4*)(tab + kTabRA + tb * 16 + 4 * g);
          const floatx4 rb = *(const floatx4*)(tab + kTabRB + tb * 16 + 4 * g);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc += (ra[i] * qm[i] + rb[i] * qmp[i]) * elt(d8[tb >> 1], (tb & 1) * 4 + i);
        };
        bf16x4 th, tl, tph, tpl;
        if (KTAIL) {
          split_acc4(M[NKB - 1], th, tl);
          split_acc4(Mp[NKB - 1], tph, tpl);
        }
        if constexpr (NK32 <= 2) {
          // narrow keys: every state fragment split once, one query block at a time
          constexpr int NJ = NK32 > 0 ? NK32 : 1;
          bf16x8 mh[NJ], ml[NJ], mph[NJ], mpl[NJ];
#pragma unroll
          for (int j = 0; j < NK32; ++j) {
            split_acc(M[2 * j], M[2 * j + 1], mh[j], ml[j]);
            split_acc(Mp[2 * j], Mp[2 * j + 1], mph[j], mpl[j]);
          }
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            floatx4 qm = {0.f, 0.f, 0.f, 0.f}, qmp = qm;
#pragma unroll
            for (int j = 0; j < NK32; ++j) {
              const auto qf = frow8<E>(Qs, L.qp, tb * 16 + l16, j, g);
              qm = mma32(qf, mh[j], qm);
              qm = mma32(qf, ml[j], qm);
              qmp = mma32(qf, mph[j], qmp);
              qmp = mma32(qf, mpl[j], qmp);
            }
            if (KTAIL) {
              const auto qf = frow4<E>(Qs, L.qp, tb * 16 + l16, NK32, g);
              qm = mma16(qf, th, qm);
              qm = mma16(qf, tl, qm);
              qmp = mma16(qf, tph, qmp);
              qmp = mma16(qf, tpl, qmp);
            }
            add_rows(tb, qm, qmp);
          }
        } else {
          // wide keys: one state fragment split at a time, all query blocks
          floatx4 qm[4], qmp[4];
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) qm[tb] = qmp[tb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < NK32; ++j) {
            bf16x8 mh, ml, mph, mpl;
            split_acc(M[2 * j], M[2 * j + 1], mh, ml);
            split_acc(Mp[2 * j], Mp[2 * j + 1], mph, mpl);
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
              const auto qf = frow8<E>(Qs, L.qp, tb * 16 + l16, j, g);
              qm[tb] = mma32(qf, mh, qm[tb]);
              qm[tb] = mma32(qf, ml, qm[tb]);
              qmp[tb] = mma32(qf, mph, qmp[tb]);
              qmp[tb] = mma32(qf, mpl, qmp[tb]);
            }
          }
          if (KTAIL) {
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
              const auto qf = frow4<E>(Qs, L.qp, tb * 16 + l16, NK32, g);
              qm[tb] = mma16(qf, th, qm[tb]);
              qm[tb] = mma16(qf, tl, qm[tb]);
              qmp[tb] = mma16(qf, tph, qmp[tb]);
              qmp[tb] = mma16(qf, tpl, qmp[tb]);
            }
          }
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) add_rows(tb, qm[tb], qmp[tb]);
        }
      }
      // ---- query-side sums A, B
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        float wa[8], wb[8], xa[8], xb[8];
        tab8(tab + kTabWA, kp, g, wa);
        tab8(tab + kTabWB, kp, g, wb);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = elt(d8[kp], e);
          xa[e] = x * wa[e];
          xb[e] = x * wb[e];
        }
        bf16x8 ah, al, bh8, bl8;
        split8(xa, ah, al);
        split8(xb, bh8, bl8);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const auto qc = TK::col8(Qs, L.qp, kb * 16, kp, lane);
          A[kb] = mma32(qc, ah, A[kb]);
          A[kb] = mma32(qc, al, A[kb]);
          Bq[kb] = mma32(qc, bh8, Bq[kb]);
          Bq[kb] = mma32(qc, bl8, Bq[kb]);
        }
      }
      // ---- states after this tile (relative to its last token)
      const float dec = tab[kTabPow + len];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          Mp[kb][i] = dec * (Mp[kb][i] + (float)len * M[kb][i]);
          M[kb][i] *= dec;
        }
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        float wm[8], wmp[8], xa[8], xb[8];
        tab8(tab + kTabWM, kp, g, wm);
        tab8(tab + kTabWMp, kp, g, wmp);
        const bf16x8 v8 = TK::col8(Vw, L.vp, 0, kp, lane);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = elt(v8, e);
          xa[e] = x * wm[e];
          xb[e] = x * wmp[e];
        }
        bf16x8 mh, ml, mph, mpl;
        split8(xa, mh, ml);
        split8(xb, mph, mpl);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const auto kc = TK::col8(Ks, L.qp, kb * 16, kp, lane);
          M[kb] = mma32(kc, mh, M[kb]);
          M[kb] = mma32(kc, ml, M[kb]);
          Mp[kb] = mma32(kc, mph, Mp[kb]);
          Mp[kb] = mma32(kc, mpl, Mp[kb]);
        }
      }
    }
  }

  // ---- this segment's pair sum and summaries
  float* red = tab + kTabRed;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) acc += __shfl_xor(acc, o, 64);
  if (lane == 0) red[w] = acc;
  __syncthreads();
  if (tid == 0) {
    float s = 0.f;
    for (int i = 0; i < nwave; ++i) s += red[i];
    p.part[(size_t)bh * p.nseg + seg] = s;
  }
  if (owner) {
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
}

__global__ void retention_zero_kernel(float* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = 0.f;
}

// Cross-segment pairs: <M_in, A_s> + <M'_in, B_s> with the running prefix of
// the segment summaries.  Block (x, bh) takes elements x*256 .. +255 of the
// [dk][vw] states and writes its partial sum; the finish kernel adds the
// partials and the segments' own pair sums -> out[b][h].
__global__ __launch_bounds__(256) void retention_combine_kernel(RetP p, float* partials) {
  const int bh = blockIdx.y;
  const int h = bh % p.H;
  const float la = p.log_alpha[h];
  const size_t nel = (size_t)p.dk * p.vw;
  const size_t e = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int seg_len = p.seg_tiles * C;
  float acc = 0.f;
  if (e < nel) {
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
  if (threadIdx.x == 0) partials[(size_t)bh * gridDim.x + blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(64) void retention_finish_kernel(RetP p, const float* partials, int nparts, float* out) {
  const int bh = blockIdx.x;
  float s = 0.f;
  for (int i = threadIdx.x; i < nparts; i += 64) s += partials[(size_t)bh * nparts + i];
  for (int i = threadIdx.x; i < p.nseg; i += 64) s += p.part[(size_t)bh * p.nseg + i];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) s += __shfl_xor(s, o, 64);
  if (threadIdx.x == 0) out[bh] = s;
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
  int dkp, nvr, vw, nw, waves, seg_tiles, nseg;
  int ncomb;  // combine blocks per (b, h): 256 state elements each
  size_t part_bytes, sums_bytes, comb_bytes;
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
  // enough waves that every thread loads at most two chunks of each tile
  P->waves = P->nw > d->dk / 16 ? P->nw : d->dk / 16;
  if (ts::ret_layout(P->dkp, P->vw).bytes > ts::kLdsPerCU)
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
  P->ncomb = (P->dkp * P->vw + 255) / 256;
  P->comb_bytes = (size_t)d->B * d->H * P->ncomb * sizeof(float);
  return TS_OK;
}

// workspace: [part | pad to 256 | sums | pad to 256 | combine partials]
size_t ws_bytes(const RetPlan& P) {
  return (P.part_bytes + 255) / 256 * 256 + (P.sums_bytes + 255) / 256 * 256 + P.comb_bytes;
}

// Bytes spanned by one (batch, head) slice of a [.., T, width] stream (the
// range of its buffer loads), or an error if the rows the kernel addresses --
// up to T rounded up to whole tiles, plus one tile -- could not be reached with
// 31-bit offsets (the tile offsets are computed in 32-bit integers).
int span_bytes(const char* name, const ts_strided& s, int T, int width, int es, uint32_t* out) {
  *out = 0;
  if (!s.ptr || T == 0) return TS_OK;
  if (s.st < 0) return fail(TS_ERR_VALUE, "retention grad: negative time stride of %s", name);
  const int64_t rows = ((int64_t)T + ts::C - 1) / ts::C * ts::C + ts::C;
  const int64_t reach = rows * s.st * es + (int64_t)width * es;
  if (reach >= ((int64_t)1 << 31))
    return fail(TS_ERR_NOT_IMPLEMENTED, "retention grad: one (batch, head) slice of %s spans more than 2 GiB", name);
  *out = (uint32_t)(((int64_t)(T - 1) * s.st + width) * es);
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_retention_workspace_bytes(const ts_retention_desc* d, size_t* bytes) {
  RetPlan P;
  int rc = ret_plan(d, &P);
  if (rc) return rc;
  if (bytes) *bytes = ws_bytes(P);
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
  // every slice must be addressable with 31-bit offsets (checked before any launch)
  uint32_t rec[5];
  if ((rc = span_bytes("q", io->q, d->T, d->dk, 2, &rec[0])) || (rc = span_bytes("k", io->k, d->T, d->dk, 2, &rec[1])) ||
      (rc = span_bytes("v", io->v, d->T, d->dv, 2, &rec[2])) ||
      (rc = span_bytes("dout", io->dout, d->T, d->dv, 2, &rec[3])) ||
      (rc = span_bytes("dmass", io->dmass, d->T, 1, 4, &rec[4])))
    return rc;
  const size_t need = ws_bytes(P);
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
  p.seg_tiles = P.seg_tiles; p.nseg = P.nseg; p.vw = P.vw; p.nw = P.nw;
  p.q = io->q; p.k = io->k; p.v = io->v; p.dout = io->dout; p.dm = io->dmass;
  p.q_rec = rec[0]; p.k_rec = rec[1]; p.v_rec = rec[2]; p.o_rec = rec[3]; p.dm_rec = rec[4];
  p.log_alpha = io->log_alpha;
  p.part = (float*)workspace;
  p.sums = (float*)((char*)workspace + (P.part_bytes + 255) / 256 * 256);
  RetFn fn = pick_ret(P.dkp);
  if (!fn) return fail(TS_ERR_NOT_IMPLEMENTED, "retention grad: no kernel for dk=%d", P.dkp);
  const ts::RetLayout L = ts::ret_layout(P.dkp, P.vw);
  if (L.bytes > 65536) {
    hipError_t e = ts::ensure_lds_limit((const void*)fn, L.bytes);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "retention grad: LDS request failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(fn, dim3(P.nseg, d->H, d->B), dim3(64 * P.waves), (size_t)L.bytes, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "retention grad: launch failed: %s", hipGetErrorString(e));
  float* comb = (float*)((char*)p.sums + (P.sums_bytes + 255) / 256 * 256);
  hipLaunchKernelGGL(ts::retention_combine_kernel, dim3(P.ncomb, bh), dim3(256), 0, stream, p, comb);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "retention grad: combine launch failed: %s", hipGetErrorString(e));
  hipLaunchKernelGGL(ts::retention_finish_kernel, dim3(bh), dim3(64), 0, stream, p, (const float*)comb, P.ncomb, out);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "retention grad: finish launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

}  // extern "C"
