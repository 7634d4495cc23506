// Chunked exact linear-attention scan for gfx950 (MI355X).
//
// One view of the reference's chunk backend
// (src/thetascan/_core/ops/scan_chunk.py:246-339): the sequence is cut into
// 64-token tiles; inside a tile the causal score block is a bf16 (or fp32)
// MFMA contraction with fp32 accumulation, and across tiles an fp32
// [dk, dv] state carries everything already written.
//
// Work decomposition (one workgroup per (batch*head, segment)):
//   1. summary kernel : each segment of `seg_chunks` tiles folds its own
//                       writes into a local state U_p (no queries needed);
//   2. prefix kernel  : exclusive scan of U_p over segments with the decay
//                       of each segment -> the state entering every segment;
//   3. main kernel    : each segment re-walks its tiles from that incoming
//                       state and writes the outputs.
// This turns B*H sequential scans (64 at the benchmark shape) into B*H*nseg
// independent workgroups so the whole chip is busy.
//
// Inside a workgroup wave w owns value block w (16 value columns): it holds
// the state S[:, 16w:16w+16] in registers (MFMA accumulator layout) and
// produces out[:, 16w:16w+16].  The score tile is computed once and shared
// through LDS.  Orientation (O^T = S^T Q^T + V^T P^T, S += K_w^T V) is chosen
// so the register state feeds the next MFMA directly as an operand, with the
// contraction index permuted consistently in both operands.

#include "ts_common.h"
#include "thetascan_hip.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace ts {

constexpr int C = 64;  // tokens per tile

// (query block, key block) pairs of the score tile, 2 bits each: the 10
// causal 16x16 blocks, then the two upper blocks read by the 32-key
// contractions of query blocks 0 and 2 (stored as zeros).
constexpr int kScoreBlocks = 12;
constexpr unsigned pack_blocks(const int (&a)[kScoreBlocks]) {
  unsigned r = 0;
  for (int i = 0; i < kScoreBlocks; ++i) r |= (unsigned)a[i] << (2 * i);
  return r;
}
constexpr int kBq[kScoreBlocks] = {0, 1, 1, 2, 2, 2, 3, 3, 3, 3, 0, 2};
constexpr int kBk[kScoreBlocks] = {0, 0, 1, 0, 1, 2, 0, 1, 2, 3, 1, 3};
constexpr unsigned kBlockQ = pack_blocks(kBq);
constexpr unsigned kBlockK = pack_blocks(kBk);

struct ScanP {
  int B, H, T, dk, dv, dvp;
  int nchunks, seg_chunks, nseg;
  int ret, reverse;
  int q_ext, k_ext, v_ext;
  int out_mode;
  float out_scale;
  ts_strided q, k, v, qe, ke, ve, decay, out, oe;
  const float* log_alpha;
  float* seg;     // [BH][nseg][DKP][dvp]
  float* segdec;  // [BH][nseg]
  int nsum;       // segments that run the summary kernel
};

__device__ __forceinline__ int phys_t(const ScanP& p, int t) { return p.reverse ? p.T - 1 - t : t; }

// Load a [C, wpad] tile of rows t0..t0+63 (zero padded past T and past
// `width`; column `width` carries the optional ext column) into LDS, row-major
// at `rowdst` and/or transposed at `tdst`.
template <typename E>
__device__ __forceinline__ void load_tile(const ScanP& p, const ts_strided& src, int ext_mode,
                                          const ts_strided& ext, int width, int wpad, int b,
                                          int h, int t0, E* rowdst, int rpitch, E* tdst,
                                          int tpitch, int tid, int nthreads) {
  constexpr int VEC = 16 / (int)sizeof(E);
  const int nvec = wpad / VEC;
  const E* base = (const E*)src.ptr + (int64_t)b * src.sb + (int64_t)h * src.sh;
  for (int idx = tid; idx < C * nvec; idx += nthreads) {
    const int r = idx / nvec;
    const int c0 = (idx - r * nvec) * VEC;
    const int t = t0 + r;
    Vec16<E> val;
    val.raw = make_uint4(0u, 0u, 0u, 0u);
    if (t < p.T) {
      const int tp = phys_t(p, t);
      if (c0 < width) {
        val.raw = *(const uint4*)(base + (int64_t)tp * src.st + c0);
      } else if (c0 == width && ext_mode != TS_EXT_NONE) {
        float x = 1.0f;
        if (ext_mode == TS_EXT_ARRAY)
          x = ((const float*)ext.ptr)[(int64_t)b * ext.sb + (int64_t)h * ext.sh + (int64_t)tp * ext.st];
        val.e[0] = cvt<E>(x);
      }
    }
    if (rowdst) *(uint4*)(rowdst + r * rpitch + c0) = val.raw;
    if (tdst) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) tdst[(c0 + e) * tpitch + r] = val.e[e];
    }
  }
}

// Per-tile retention tables (wave 0).  Matches scan_chunk._static_weights
// (scan_chunk.py:102-119) and _tile_weights (scan_chunk.py:122-155): phases
// are formed in fp32, exponents of the intra-tile weight are clamped to <= 0.
//   carry[i] : weight of the incoming state at local position i
//   wk[j]    : weight of key j in the state leaving the tile (after `len` steps)
//   pw[d]    : static weight alpha^d;  lloc[i] : stream tile-local cum. log
//   misc[0]  : log-decay of the whole tile (len steps)
__device__ __forceinline__ void tile_decay(const ScanP& p, int b, int h, int t0, int len, int lane,
                                          float* carry, float* wk, float* pw, float* lloc,
                                          float* misc) {
  if (p.ret == TS_RET_STATIC) {
    const float la = p.log_alpha[h];
    pw[lane] = expf(la * (float)lane);
    carry[lane] = expf(la * (float)(lane + 1));
    wk[lane] = lane < len ? expf(la * (float)(len - 1 - lane)) : 0.0f;
    if (lane == 0) misc[0] = la * (float)len;
  } else {
    // a(s): decay applied when stepping into logical position s.  Reversed
    // scans step from physical s+1 down to s, so they use the decay of the
    // physical successor.
    const int s = t0 + lane;
    float a = 0.0f;
    if (s < p.T) {
      int src = s;
      if (p.reverse) src = (p.T - 1 - s) + 1;
      if (src < p.T)
        a = ((const float*)p.decay.ptr)[(int64_t)b * p.decay.sb + (int64_t)h * p.decay.sh +
                                        (int64_t)src * p.decay.st];
    }
    float x = a;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      float y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    lloc[lane] = x;
    const float last = __shfl(x, len - 1, 64);
    carry[lane] = expf(x);
    wk[lane] = lane < len ? expf(last - x) : 0.0f;
    if (lane == 0) misc[0] = last;
  }
}

template <typename E, int DKP, bool MAIN>
__global__ __launch_bounds__(1024) void scan_kernel(ScanP p) {
  typedef typename Frag<E>::f8 F8;
  typedef typename Frag<E>::f4 F4;
  typedef LdsIO<E> IO;
  constexpr int VEC = 16 / (int)sizeof(E);
  constexpr int QP = DKP + VEC;  // row pitch of Qs / Ks (elements)
  constexpr int TP = C + VEC;    // row pitch of KTs / VTs / Ps
  constexpr int NKB = DKP / 16;  // 16-row key-feature blocks of the state
  constexpr int NK32 = DKP / 32; // full 32-wide contraction blocks over dk
  constexpr bool KTAIL = (DKP % 32) != 0;

  const int dvp = p.dvp;
  const int NW = dvp / 16;
  const int NT = NW * 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int seg = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  extern __shared__ __align__(16) unsigned char smem[];
  E* Qs = (E*)smem;
  E* Ks = Qs + (MAIN ? C * QP : 0);
  E* KTs = Ks + (MAIN ? C * QP : 0);
  E* VTs = KTs + DKP * TP;
  E* Ps = VTs + dvp * TP;
  float* s_carry = (float*)(Ps + (MAIN ? C * TP : 0));
  float* s_wk = s_carry + C;
  float* s_pw = s_wk + C;
  float* s_lloc = s_pw + C;
  float* s_misc = s_lloc + C;

  floatx4 S[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) S[kb] = floatx4{0.f, 0.f, 0.f, 0.f};
  bool state_zero = true;
  if (MAIN && seg > 0) {
    const float* src = p.seg + ((size_t)bh * p.nseg + seg) * (size_t)(DKP * dvp);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[kb][i] = src[(kb * 16 + 4 * g + i) * dvp + w * 16 + l16];
    state_zero = false;
  }

  const int c_begin = seg * p.seg_chunks;
  const int c_end = min(c_begin + p.seg_chunks, p.nchunks);
  float seg_log = 0.0f;

  for (int c = c_begin; c < c_end; ++c) {
    const int t0 = c * C;
    const int len = min(C, p.T - t0);
    __syncthreads();  // LDS of the previous tile is no longer read
    if (p.ret != TS_RET_NONE && w == 0)
      tile_decay(p, b, h, t0, len, lane, s_carry, s_wk, s_pw, s_lloc, s_misc);
    if (MAIN) {
      load_tile<E>(p, p.q, p.q_ext, p.qe, p.dk, DKP, b, h, t0, Qs, QP, nullptr, 0, tid, NT);
      load_tile<E>(p, p.k, p.k_ext, p.ke, p.dk, DKP, b, h, t0, Ks, QP, KTs, TP, tid, NT);
    } else {
      load_tile<E>(p, p.k, p.k_ext, p.ke, p.dk, DKP, b, h, t0, nullptr, 0, KTs, TP, tid, NT);
    }
    load_tile<E>(p, p.v, p.v_ext, p.ve, p.dv, dvp, b, h, t0, nullptr, 0, VTs, TP, tid, NT);
    __syncthreads();

    if (MAIN) {
      // ---- causal score tile P[query][key] = w(q,k) <q, k>, shared via LDS.
      // 10 lower-triangular 16x16 blocks plus the two upper blocks that the
      // 32-key contraction of query blocks 0 and 2 reads (written as zero).
      for (int bi = w; bi < kScoreBlocks; bi += NW) {
        const int qb = (kBlockQ >> (2 * bi)) & 3;
        const int kb = (kBlockK >> (2 * bi)) & 3;
        const int query = qb * 16 + l16;
        const int key0 = kb * 16 + 4 * g;
        float pv[4] = {0.f, 0.f, 0.f, 0.f};
        if (bi < 10) {
          floatx4 acc = {0.f, 0.f, 0.f, 0.f};
          const E* krow = Ks + (kb * 16 + l16) * QP;
          const E* qrow = Qs + query * QP;
#pragma unroll
          for (int kk = 0; kk < NK32; ++kk)
            acc = mma32(IO::ld8(krow + kk * 32 + 8 * g), IO::ld8(qrow + kk * 32 + 8 * g), acc);
          if (KTAIL)
            acc = mma16(IO::ld4(krow + NK32 * 32 + 4 * g), IO::ld4(qrow + NK32 * 32 + 4 * g), acc);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = key0 + i;
            float wt = 1.0f;
            if (p.ret == TS_RET_STATIC)
              wt = s_pw[max(query - key, 0)];
            else if (p.ret == TS_RET_STREAM)
              wt = expf(fminf(s_lloc[query] - s_lloc[key], 0.0f));
            pv[i] = key <= query ? acc[i] * wt : 0.0f;
          }
        }
        IO::st4(Ps + query * TP + key0, pv[0], pv[1], pv[2], pv[3]);
      }
      __syncthreads();
    }

    // ---- value block of this wave
    F8 av[2];
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) av[kp] = IO::ld8(VTs + (w * 16 + l16) * TP + kp * 32 + 8 * g);

    if (MAIN) {
#pragma unroll
      for (int qb = 0; qb < 4; ++qb) {
        const int query = qb * 16 + l16;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        if (!state_zero) {
          const E* qrow = Qs + query * QP;
#pragma unroll
          for (int j = 0; j < NK32; ++j)
            acc = mma32(IO::from_acc(S[2 * j], S[2 * j + 1]),
                        IO::cat(IO::ld4(qrow + 32 * j + 4 * g), IO::ld4(qrow + 32 * j + 16 + 4 * g)),
                        acc);
          if (KTAIL) acc = mma16(IO::from_acc4(S[NKB - 1]), IO::ld4(qrow + NK32 * 32 + 4 * g), acc);
          if (p.ret != TS_RET_NONE) {
            const float cw = s_carry[query];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] *= cw;
          }
        }
#pragma unroll
        for (int kp = 0; kp <= qb / 2; ++kp)
          acc = mma32(av[kp], IO::ld8(Ps + query * TP + kp * 32 + 8 * g), acc);

        const int t = t0 + query;
        if (t < p.T) {
          const int tp = phys_t(p, t);
          const int dvb = w * 16 + 4 * g;
          const int64_t ooff = (int64_t)b * p.out.sb + (int64_t)h * p.out.sh + (int64_t)tp * p.out.st;
          if (p.out_mode == TS_OUT_STORE) {
            E* o = (E*)p.out.ptr + ooff + dvb;
            if (dvb + 4 <= p.dv) {
              IO::st4(o, acc[0], acc[1], acc[2], acc[3]);
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (dvb + i < p.dv) o[i] = cvt<E>(acc[i]);
            }
          } else {
            float* o = (float*)p.out.ptr + ooff + dvb;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (dvb + i < p.dv) {
                const float val = p.out_scale * acc[i];
                o[i] = p.out_mode == TS_OUT_ACCUM_F32 ? o[i] + val : val;
              }
            }
          }
          if (p.oe.ptr && dvb <= p.dv && p.dv < dvb + 4) {
            float* oe = (float*)p.oe.ptr + (int64_t)b * p.oe.sb + (int64_t)h * p.oe.sh + (int64_t)tp * p.oe.st;
            const float val = (p.out_mode == TS_OUT_STORE ? 1.0f : p.out_scale) * acc[p.dv - dvb];
            *oe = p.out_mode == TS_OUT_ACCUM_F32 ? *oe + val : val;
          }
        }
      }
    }

    // ---- state update: S = decay(tile) * S + K_w^T V
    if (p.ret != TS_RET_NONE) {
      const float cdec = expf(s_misc[0]);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[kb][i] *= cdec;
      if (tid == 0) seg_log += s_misc[0];
    }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int kp = 0; kp < 2; ++kp) {
        F8 ak = IO::ld8(KTs + (kb * 16 + l16) * TP + kp * 32 + 8 * g);
        if (p.ret != TS_RET_NONE) {
#pragma unroll
          for (int e = 0; e < 8; ++e) ak[e] = cvt<E>(tof(ak[e]) * s_wk[kp * 32 + 8 * g + e]);
        }
        S[kb] = mma32(ak, av[kp], S[kb]);
      }
    }
    state_zero = false;
  }

  if (!MAIN) {
    float* dst = p.seg + ((size_t)bh * p.nseg + seg) * (size_t)(DKP * dvp);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[(kb * 16 + 4 * g + i) * dvp + w * 16 + l16] = S[kb][i];
    if (tid == 0) p.segdec[(size_t)bh * p.nseg + seg] = seg_log;
  }
}

// Exclusive scan of the segment summaries:  seg[p] <- state entering segment p.
__global__ void scan_prefix_kernel(float* seg, const float* segdec, float* final_state, int nseg,
                                   int nsum, int nelem) {
  const int bh = blockIdx.y;
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nelem) return;
  float* base = seg + (size_t)bh * nseg * nelem + e;
  float carry = 0.0f;
  for (int s = 0; s < nseg; ++s) {
    float u = 0.0f;
    if (s < nsum) u = base[(size_t)s * nelem];
    base[(size_t)s * nelem] = carry;
    if (s < nsum) carry = expf(segdec[(size_t)bh * nseg + s]) * carry + u;
  }
  if (final_state) final_state[(size_t)bh * nelem + e] = carry;
}

}  // namespace ts

// ============================================================== host side
namespace ts {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace ts

namespace {

using ts::fail;

const int kDkPads[] = {32, 64, 80, 128, 144};

int pick_dkp(int need) {
  for (int v : kDkPads)
    if (need <= v) return v;
  return -1;
}

struct Layout {
  int dkp, dvp, nchunks, seg_chunks, nseg, nsum;
  size_t ws_bytes;
};

int compute_layout(const ts_scan_desc* d, Layout* L) {
  if (!d) return fail(TS_ERR_VALUE, "scan: null descriptor");
  if (d->B < 1 || d->H < 1 || d->T < 0) return fail(TS_ERR_VALUE, "scan: bad shape");
  if (d->dk < 1 || d->dv < 1) return fail(TS_ERR_VALUE, "scan: feature widths must be >= 1");
  if (d->dtype != TS_BF16 && d->dtype != TS_F32) return fail(TS_ERR_VALUE, "scan: unknown dtype");
  if (d->retention < TS_RET_NONE || d->retention > TS_RET_STREAM)
    return fail(TS_ERR_VALUE, "scan: unknown retention kind");
  const int vec = d->dtype == TS_BF16 ? 8 : 4;
  if (d->dk % vec || d->dv % vec)
    return fail(TS_ERR_VALUE, "scan: feature widths must be multiples of 16 bytes (dk=%d dv=%d)",
                d->dk, d->dv);
  const int dk_eff = d->dk + ((d->q_ext != TS_EXT_NONE || d->k_ext != TS_EXT_NONE) ? 1 : 0);
  L->dkp = pick_dkp(dk_eff);
  if (L->dkp < 0) return fail(TS_ERR_NOT_IMPLEMENTED, "scan: key width %d exceeds 144", dk_eff);
  L->dvp = ((d->dv + (d->v_ext != TS_EXT_NONE ? 1 : 0)) + 15) / 16 * 16;
  if (L->dvp > 256) return fail(TS_ERR_NOT_IMPLEMENTED, "scan: value width %d exceeds 256", L->dvp);
  L->nchunks = (d->T + ts::C - 1) / ts::C;
  const int bh = d->B * d->H;
  if (d->seg_chunks > 0) {
    L->seg_chunks = d->seg_chunks;
  } else {
    // Enough workgroups to fill 256 CUs a few times over.
    int want = 768 / (bh > 0 ? bh : 1);
    if (want < 1) want = 1;
    L->seg_chunks = (L->nchunks + want - 1) / want;
    if (L->seg_chunks < 1) L->seg_chunks = 1;
  }
  L->nseg = L->nchunks > 0 ? (L->nchunks + L->seg_chunks - 1) / L->seg_chunks : 0;
  L->nsum = d->want_final ? L->nseg : (L->nseg > 0 ? L->nseg - 1 : 0);
  L->ws_bytes = 0;
  if (L->nsum > 0)
    L->ws_bytes = (size_t)bh * L->nseg * (size_t)L->dkp * L->dvp * sizeof(float) +
                  (size_t)bh * L->nseg * sizeof(float) + 256;
  return TS_OK;
}

size_t lds_bytes(int esize, int dkp, int dvp, bool main_kernel) {
  const int vec = 16 / esize;
  const int qp = dkp + vec, tp = ts::C + vec;
  size_t elems = (size_t)dkp * tp + (size_t)dvp * tp;
  if (main_kernel) elems += 2 * (size_t)ts::C * qp + (size_t)ts::C * tp;
  return elems * esize + 5 * ts::C * sizeof(float);
}

typedef void (*KernelFn)(ts::ScanP);

template <typename E>
KernelFn pick_kernel(int dkp, bool main_kernel) {
  switch (dkp) {
#define TS_CASE(D)                                                                           \
  case D:                                                                                    \
    return main_kernel ? (KernelFn)ts::scan_kernel<E, D, true> : (KernelFn)ts::scan_kernel<E, D, false>;
    TS_CASE(32)
    TS_CASE(64)
    TS_CASE(80)
    TS_CASE(128)
    TS_CASE(144)
#undef TS_CASE
  }
  return nullptr;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_stream(const char* name, const ts_strided& s, int vec, bool required) {
  if (!s.ptr) return required ? fail(TS_ERR_VALUE, "scan: missing tensor %s", name) : TS_OK;
  if (!aligned16(s.ptr)) return fail(TS_ERR_VALUE, "scan: tensor %s is not 16-byte aligned", name);
  if (s.st % vec || s.sh % vec || s.sb % vec)
    return fail(TS_ERR_VALUE, "scan: strides of %s must be multiples of 16 bytes", name);
  return TS_OK;
}

int launch(KernelFn fn, dim3 grid, dim3 block, size_t lds, hipStream_t stream, const ts::ScanP& p) {
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: LDS request failed: %s", hipGetErrorString(e));
  }
  hipLaunchKernelGGL(fn, grid, block, lds, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: launch failed: %s", hipGetErrorString(e));
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_abi_version(void) { return TS_ABI_VERSION; }

const char* ts_last_error(void) { return ts::g_err; }

int ts_scan_layout(const ts_scan_desc* desc, int32_t* dk_pad, int32_t* dv_pad, int32_t* n_segments) {
  Layout L;
  int rc = compute_layout(desc, &L);
  if (rc) return rc;
  if (dk_pad) *dk_pad = L.dkp;
  if (dv_pad) *dv_pad = L.dvp;
  if (n_segments) *n_segments = L.nseg;
  return TS_OK;
}

int ts_scan_workspace_bytes(const ts_scan_desc* desc, size_t* bytes) {
  Layout L;
  int rc = compute_layout(desc, &L);
  if (rc) return rc;
  if (bytes) *bytes = L.ws_bytes;
  return TS_OK;
}

int ts_scan_fwd(const ts_scan_desc* d, const ts_scan_io* io, void* workspace, size_t ws_bytes,
                hipStream_t stream) {
  Layout L;
  int rc = compute_layout(d, &L);
  if (rc) return rc;
  if (!io) return fail(TS_ERR_VALUE, "scan: null io");
  if (d->T == 0) return TS_OK;
  const int esize = d->dtype == TS_BF16 ? 2 : 4;
  const int vec = 16 / esize;
  if ((rc = check_stream("q", io->q, vec, true))) return rc;
  if ((rc = check_stream("k", io->k, vec, true))) return rc;
  if ((rc = check_stream("v", io->v, vec, true))) return rc;
  const int out_vec = d->out_mode == TS_OUT_STORE ? vec : 4;
  if (!io->out.ptr) return fail(TS_ERR_VALUE, "scan: missing output");
  if (((uintptr_t)io->out.ptr & 7u) || io->out.st % out_vec || io->out.sh % out_vec || io->out.sb % out_vec)
    return fail(TS_ERR_VALUE, "scan: output rows must be aligned");
  if (d->q_ext == TS_EXT_ARRAY && !io->q_ext.ptr) return fail(TS_ERR_VALUE, "scan: missing q ext column");
  if (d->k_ext == TS_EXT_ARRAY && !io->k_ext.ptr) return fail(TS_ERR_VALUE, "scan: missing k ext column");
  if (d->v_ext == TS_EXT_ARRAY && !io->v_ext.ptr) return fail(TS_ERR_VALUE, "scan: missing v ext column");
  if (d->retention == TS_RET_STATIC && !io->log_alpha) return fail(TS_ERR_VALUE, "scan: missing log_alpha");
  if (d->retention == TS_RET_STREAM && !io->decay.ptr) return fail(TS_ERR_VALUE, "scan: missing decay stream");
  if (d->want_final && !io->final_state) return fail(TS_ERR_VALUE, "scan: missing final_state buffer");
  if (L.ws_bytes > 0 && (!workspace || ws_bytes < L.ws_bytes))
    return fail(TS_ERR_VALUE, "scan: workspace too small (%lld < %lld bytes)", (long long)ws_bytes,
                (long long)L.ws_bytes);

  ts::ScanP p;
  memset(&p, 0, sizeof(p));
  p.B = d->B; p.H = d->H; p.T = d->T; p.dk = d->dk; p.dv = d->dv; p.dvp = L.dvp;
  p.nchunks = L.nchunks; p.seg_chunks = L.seg_chunks; p.nseg = L.nseg; p.nsum = L.nsum;
  p.ret = d->retention; p.reverse = d->reverse;
  p.q_ext = d->q_ext; p.k_ext = d->k_ext; p.v_ext = d->v_ext;
  p.out_mode = d->out_mode; p.out_scale = d->out_scale;
  p.q = io->q; p.k = io->k; p.v = io->v;
  p.qe = io->q_ext; p.ke = io->k_ext; p.ve = io->v_ext;
  p.decay = io->decay; p.out = io->out; p.oe = io->out_ext;
  p.log_alpha = io->log_alpha;
  if (L.ws_bytes > 0) {
    p.seg = (float*)workspace;
    p.segdec = p.seg + (size_t)d->B * d->H * L.nseg * (size_t)L.dkp * L.dvp;
  }

  const int bh = d->B * d->H;
  const dim3 block(L.dvp / 16 * 64);
  KernelFn fsum = d->dtype == TS_BF16 ? pick_kernel<ts::bf16>(L.dkp, false) : pick_kernel<float>(L.dkp, false);
  KernelFn fmain = d->dtype == TS_BF16 ? pick_kernel<ts::bf16>(L.dkp, true) : pick_kernel<float>(L.dkp, true);
  const size_t lds_sum = lds_bytes(esize, L.dkp, L.dvp, false);
  const size_t lds_main = lds_bytes(esize, L.dkp, L.dvp, true);
  if (lds_main > 160 * 1024)
    return fail(TS_ERR_NOT_IMPLEMENTED, "scan: tile of %lld bytes exceeds LDS (dk_pad=%d)",
                (long long)lds_main, L.dkp);

  if (L.nsum > 0) {
    if ((rc = launch(fsum, dim3(L.nsum, bh), block, lds_sum, stream, p))) return rc;
    const int nelem = L.dkp * L.dvp;
    hipLaunchKernelGGL(ts::scan_prefix_kernel, dim3((nelem + 255) / 256, bh), dim3(256), 0, stream, p.seg,
                       p.segdec, d->want_final ? io->final_state : nullptr, L.nseg, L.nsum, nelem);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "scan: prefix launch failed: %s", hipGetErrorString(e));
  }
  return launch(fmain, dim3(L.nseg, bh), block, lds_main, stream, p);
}

}  // extern "C"
