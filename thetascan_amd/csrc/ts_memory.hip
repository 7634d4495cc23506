// Depth-1 kernel memory as two host calls (forward, backward).
//
// The host side of the fused mixer submits, per step, two feature maps, a
// scan and a read in the forward and a read backward, three scans, two
// feature backwards and up to five small reductions in the backward.  Each
// of those is a few microseconds of host work in C but tens of microseconds
// through a Python binding, and the forward is host-bound at the benchmark
// shape.  These two entry points run the same kernels (through the same
// entry points) from one call each; every intermediate lives in two
// caller-provided byte buffers whose layout is fixed here:
//
//   saved   (forward -> backward): phi_q, phi_k [B,H,T,m]; resid, num
//           [B,H,T,d]; mass fp32 [B,H,T]; tau, g_bias as fp32; the forward
//           scan's segment states (read transposed by the dq scan)
//   scratch (backward only): dnum, dresid [B,H,T,d]; dmass fp32 [B,H,T];
//           dphi_q, dphi_k [B,H,T,m]; the reverse scans' segment states;
//           per-workgroup weight-gradient slots; gate-bias column partials
//
// Reference chain: block.py:593-724 (between proj_qkv and proj_out) and
// engine.py:260-544 for a depth-1 kernel memory (feature map, plain-sum
// scan, key-mass read, output gate).

#include "ts_common.h"
#include "thetascan_hip.h"

#include <string.h>

namespace ts {

// fp32 copies of the small parameters the kernels read (tau[H], g_bias[H*d]).
__global__ void params_f32_kernel(const void* a, int na, const void* b, int nb, int bf16_in, float* oa, float* ob) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < na) oa[i] = bf16_in ? (float)((const bf16*)a)[i] : ((const float*)a)[i];
  else if (i < na + nb) ob[i - na] = bf16_in ? (float)((const bf16*)b)[i - na] : ((const float*)b)[i - na];
}

}  // namespace ts

namespace {

using ts::fail;

constexpr size_t kAlign = 256;

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Byte offsets of every region of the two buffers, and the descriptors of
// the calls, for one desc.
struct MemPlan {
  int es;
  size_t n_bhtd, n_bhtm, n_bht;  // element counts
  // saved
  size_t o_phq, o_phk, o_res, o_num, o_mass, o_tau, o_gb, o_wsf, saved;
  size_t ws_f;  // forward scan workspace bytes
  // scratch
  size_t o_dnum, o_dres, o_dmass, o_dphq, o_dphk, o_wsb, o_w1k, o_tk, o_w1q, o_w2q, o_tq, o_col, scratch;
  size_t ws_b;
  bool reuse;  // m == d with kept segment states: dq reads the forward's, dv reads dk's
  int pk, pq, col_slices;
  ts_scan_desc sf, sdq, sdk, sdv;
};

ts_scan_desc scan_desc(const ts_memory_desc* d, int dk, int dv, int reverse, int qe, int ke, int ve) {
  ts_scan_desc s;
  memset(&s, 0, sizeof(s));
  s.B = d->feat.B; s.H = d->feat.H; s.T = d->feat.T;
  s.dk = dk; s.dv = dv; s.dtype = d->feat.dtype; s.retention = TS_RET_NONE; s.reverse = reverse;
  s.q_ext = qe; s.k_ext = ke; s.v_ext = ve;
  s.out_mode = TS_OUT_STORE; s.out_scale = 1.0f; s.seg_chunks = d->seg_chunks;
  return s;
}

int plan_memory(const ts_memory_desc* d, MemPlan* P) {
  if (!d) return fail(TS_ERR_VALUE, "memory: null descriptor");
  const ts_feature_desc& f = d->feat;
  if (d->param_dtype != TS_BF16 && d->param_dtype != TS_F32) return fail(TS_ERR_VALUE, "memory: unknown param dtype");
  if (d->has_g_bias && !d->gate) return fail(TS_ERR_VALUE, "memory: a gate bias needs the gate");
  int rc;
  // feature backward: fused weight-gradient kernels for both streams, weights staged in LDS
  int32_t pk = 0, pq = 0, tk = 1, tq = 1;
  if ((rc = ts_feature_bwd_parts(&f, 0, &pk)) || (rc = ts_feature_bwd_parts(&f, 1, &pq))) return rc;
  if (pk <= 0 || pq <= 0) return fail(TS_ERR_NOT_IMPLEMENTED, "memory: no fused feature backward for d=%d m=%d", f.d, f.m);
  if ((rc = ts_feature_bwd_transposed(&f, 0, 1, &tk)) || (rc = ts_feature_bwd_transposed(&f, 1, 1, &tq))) return rc;
  if (tk || tq) return fail(TS_ERR_NOT_IMPLEMENTED, "memory: weights of d=%d m=%d do not fit in LDS", f.d, f.m);
  P->pk = pk;
  P->pq = pq;
  const int norm = d->normalize ? 1 : 0;
  const int ones = norm ? TS_EXT_ONES : TS_EXT_NONE;
  const int arr = norm ? TS_EXT_ARRAY : TS_EXT_NONE;
  P->sf = scan_desc(d, f.m, f.d, 0, TS_EXT_NONE, TS_EXT_NONE, ones);
  P->sdq = scan_desc(d, f.d, f.m, 0, arr, ones, TS_EXT_NONE);
  P->sdk = scan_desc(d, f.d, f.m, 1, ones, arr, TS_EXT_NONE);
  P->sdv = scan_desc(d, f.m, f.d, 1, TS_EXT_NONE, TS_EXT_NONE, TS_EXT_NONE);
  size_t wf = 0, wq = 0, wk = 0, wv = 0;
  if ((rc = ts_scan_workspace_bytes(&P->sf, &wf)) || (rc = ts_scan_workspace_bytes(&P->sdk, &wk))) return rc;
  P->reuse = f.m == f.d && wf > 0 && wk > 0;
  if (P->reuse) {
    P->sdq.states_in = 2;
    P->sdv.states_in = 2;
  }
  if ((rc = ts_scan_workspace_bytes(&P->sdq, &wq)) || (rc = ts_scan_workspace_bytes(&P->sdv, &wv))) return rc;
  P->ws_f = wf;
  P->ws_b = wk;
  if (!P->reuse) P->ws_b = wk > wq ? (wk > wv ? wk : wv) : (wq > wv ? wq : wv);

  const int es = f.dtype == TS_BF16 ? 2 : 4;
  P->es = es;
  const size_t bht = (size_t)f.B * f.H * f.T;
  P->n_bht = bht;
  P->n_bhtd = bht * f.d;
  P->n_bhtm = bht * f.m;
  size_t o = 0;
  P->o_phq = o; o = align_up(o + P->n_bhtm * es);
  P->o_phk = o; o = align_up(o + P->n_bhtm * es);
  P->o_res = o; o = align_up(o + P->n_bhtd * es);
  P->o_num = o; o = align_up(o + P->n_bhtd * es);
  P->o_mass = o; o = align_up(o + (norm ? bht * 4 : 0));
  P->o_tau = o; o = align_up(o + (f.has_tau ? (size_t)f.H * 4 : 0));
  P->o_gb = o; o = align_up(o + (d->has_g_bias ? (size_t)f.H * f.d * 4 : 0));
  P->o_wsf = o; o = align_up(o + wf);
  P->saved = o;

  const int hd = f.H * f.d;
  P->col_slices = 0;
  if (d->has_g_bias) {
    // gate-bias gradient: per-workgroup column partials written by the read backward
    if (f.d > 256) return fail(TS_ERR_NOT_IMPLEMENTED, "memory: gate-bias gradient of head width %d", f.d);
    ts_read_desc rd = {f.B, f.H, f.T, f.d, f.dtype, d->normalize ? 1 : 0, 1, f.resid_scale, f.eps};
    int32_t parts = 0;
    if ((rc = ts_read_bwd_parts(&rd, &parts))) return rc;
    P->col_slices = parts;
  }
  o = 0;
  P->o_dnum = o; o = align_up(o + P->n_bhtd * es);
  P->o_dres = o; o = align_up(o + P->n_bhtd * es);
  P->o_dmass = o; o = align_up(o + (norm ? bht * 4 : 0));
  P->o_dphq = o; o = align_up(o + P->n_bhtm * es);
  P->o_dphk = o; o = align_up(o + P->n_bhtm * es);
  P->o_wsb = o; o = align_up(o + P->ws_b);
  const size_t hmd = (size_t)f.H * f.m * f.d;
  P->o_w1k = o; o = align_up(o + (size_t)pk * hmd * 4);
  P->o_tk = o; o = align_up(o + (f.has_tau ? (size_t)pk * f.H * 4 : 0));
  P->o_w1q = o; o = align_up(o + (size_t)pq * hmd * 4);
  P->o_w2q = o; o = align_up(o + (size_t)pq * hmd * 4);
  P->o_tq = o; o = align_up(o + (f.has_tau ? (size_t)pq * f.H * 4 : 0));
  P->o_col = o; o = align_up(o + (size_t)P->col_slices * hd * 4);
  P->scratch = o;
  return TS_OK;
}

// Whether the forward scan's segment summaries come from the key feature
// kernel (ts_feature_fwd_summary): bf16, d = m = 64, and a scan with kept
// segment states (more than one segment).
bool summaries_from_features(const ts_feature_desc& f, const MemPlan& P) {
  return f.dtype == TS_BF16 && f.d == 64 && f.m == 64 && P.ws_f > 0;
}

// Contiguous [B,H,T,w] stream at byte offset `off` of `base`.
ts_strided bhtw(const void* base, size_t off, const ts_feature_desc& f, int w) {
  return ts_strided{(const char*)base + off, (int64_t)f.H * f.T * w, (int64_t)f.T * w, (int64_t)w};
}
ts_strided none() { return ts_strided{nullptr, 0, 0, 0}; }

int check_view(const char* name, const ts_strided& s, bool required) {
  if (!s.ptr) return required ? fail(TS_ERR_VALUE, "memory: missing %s", name) : TS_OK;
  return TS_OK;
}

}  // namespace

extern "C" {

int ts_memory_bytes(const ts_memory_desc* desc, size_t* saved_bytes, size_t* scratch_bytes) {
  MemPlan P;
  int rc = plan_memory(desc, &P);
  if (rc) return rc;
  if (saved_bytes) *saved_bytes = P.saved;
  if (scratch_bytes) *scratch_bytes = P.scratch;
  return TS_OK;
}

int ts_memory_fwd(const ts_memory_desc* d, const ts_memory_io* io, ts_strided y, void* saved, size_t saved_bytes,
                  hipStream_t stream) {
  MemPlan P;
  int rc = plan_memory(d, &P);
  if (rc) return rc;
  if (!io) return fail(TS_ERR_VALUE, "memory: null io");
  const ts_feature_desc& f = d->feat;
  if ((rc = check_view("q", io->q, true)) || (rc = check_view("k", io->k, true)) ||
      (rc = check_view("v", io->v, true)) || (rc = check_view("g", io->g, d->gate != 0)) ||
      (rc = check_view("y", y, true)))
    return rc;
  if (!io->w1 || !io->w2) return fail(TS_ERR_VALUE, "memory: missing weights");
  if (f.has_tau && !io->tau) return fail(TS_ERR_VALUE, "memory: missing tau");
  if (d->has_g_bias && !io->g_bias) return fail(TS_ERR_VALUE, "memory: missing gate bias");
  if (!saved || saved_bytes < P.saved || ((uintptr_t)saved & (kAlign - 1)))
    return fail(TS_ERR_VALUE, "memory: saved buffer needs %zu bytes, 256-byte aligned", P.saved);
  if (f.T == 0) return TS_OK;
  char* sv = (char*)saved;
  float* tau32 = f.has_tau ? (float*)(sv + P.o_tau) : nullptr;
  float* gb32 = d->has_g_bias ? (float*)(sv + P.o_gb) : nullptr;
  const int na = f.has_tau ? f.H : 0, nb = d->has_g_bias ? f.H * f.d : 0;
  if (na + nb > 0) {
    hipLaunchKernelGGL(ts::params_f32_kernel, dim3((unsigned)((na + nb + 255) / 256)), dim3(256), 0, stream, io->tau,
                       na, io->g_bias, nb, d->param_dtype == TS_BF16 ? 1 : 0, tau32, gb32);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TS_ERR_RUNTIME, "memory: launch failed: %s", hipGetErrorString(e));
  }
  const ts_strided phq = bhtw(sv, P.o_phq, f, f.m), phk = bhtw(sv, P.o_phk, f, f.m);
  const ts_strided res = bhtw(sv, P.o_res, f, f.d), num = bhtw(sv, P.o_num, f, f.d);
  const ts_strided mass = d->normalize ? bhtw(sv, P.o_mass, f, 1) : none();

  // The key features' kernel also writes the forward scan's segment
  // summaries (64-wide bf16 features with kept segment states), so the scan
  // runs its prefix and main passes only.
  void* wsf = P.ws_f ? sv + P.o_wsf : nullptr;
  const bool summ = summaries_from_features(f, P);
  ts_feature_io fk = {io->k, io->w1, nullptr, tau32, io->in_cos, io->in_sin, io->f_cos, io->f_sin, phk, none()};
  if (summ) rc = ts_feature_fwd_summary(&f, &fk, io->v, &P.sf, wsf, P.ws_f, stream);
  else rc = ts_feature_fwd(&f, &fk, stream);
  if (rc) return rc;
  ts_feature_io fq = {io->q, io->w1, io->w2, tau32, io->in_cos, io->in_sin, io->f_cos, io->f_sin, phq, res};
  if ((rc = ts_feature_fwd(&f, &fq, stream))) return rc;

  ts_scan_io s;
  memset(&s, 0, sizeof(s));
  s.q = phq; s.k = phk; s.v = io->v; s.out = num; s.out_ext = mass;
  ts_scan_desc sf = P.sf;
  if (summ) sf.states_in = 3;
  if ((rc = ts_scan_fwd(&sf, &s, wsf, P.ws_f, stream))) return rc;

  ts_read_desc rd = {f.B, f.H, f.T, f.d, f.dtype, d->normalize ? 1 : 0, d->gate ? 1 : 0, f.resid_scale, f.eps};
  ts_read_io ri = {num, mass, res, d->gate ? io->g : none(), y, gb32};
  return ts_read_fwd(&rd, &ri, stream);
}

int ts_memory_bwd(const ts_memory_desc* d, const ts_memory_io* io, const ts_memory_grads* gr, const void* saved,
                  size_t saved_bytes, void* scratch, size_t scratch_bytes, hipStream_t stream) {
  MemPlan P;
  int rc = plan_memory(d, &P);
  if (rc) return rc;
  if (!io || !gr) return fail(TS_ERR_VALUE, "memory: null io");
  const ts_feature_desc& f = d->feat;
  if ((rc = check_view("q", io->q, true)) || (rc = check_view("k", io->k, true)) ||
      (rc = check_view("v", io->v, true)) || (rc = check_view("g", io->g, d->gate != 0)) ||
      (rc = check_view("dy", gr->dy, true)) || (rc = check_view("dq", gr->dq, true)) ||
      (rc = check_view("dk", gr->dk, true)) || (rc = check_view("dv", gr->dv, true)) ||
      (rc = check_view("dg", gr->dg, d->gate != 0)))
    return rc;
  if (!io->w1 || !io->w2) return fail(TS_ERR_VALUE, "memory: missing weights");
  if (!saved || saved_bytes < P.saved) return fail(TS_ERR_VALUE, "memory: saved buffer too small");
  if (!scratch || scratch_bytes < P.scratch || ((uintptr_t)scratch & (kAlign - 1)))
    return fail(TS_ERR_VALUE, "memory: scratch buffer needs %zu bytes, 256-byte aligned", P.scratch);
  if ((gr->dtau && !f.has_tau) || (gr->dg_bias && !d->has_g_bias))
    return fail(TS_ERR_VALUE, "memory: gradient of an absent parameter");
  if (f.T == 0) return TS_OK;
  const char* sv = (const char*)saved;
  char* sc = (char*)scratch;
  const float* tau32 = f.has_tau ? (const float*)(sv + P.o_tau) : nullptr;
  const float* gb32 = d->has_g_bias ? (const float*)(sv + P.o_gb) : nullptr;
  const ts_strided phq = bhtw(sv, P.o_phq, f, f.m), phk = bhtw(sv, P.o_phk, f, f.m);
  const ts_strided res = bhtw(sv, P.o_res, f, f.d), num = bhtw(sv, P.o_num, f, f.d);
  const ts_strided mass = d->normalize ? bhtw(sv, P.o_mass, f, 1) : none();
  const ts_strided dnum = bhtw(sc, P.o_dnum, f, f.d), dres = bhtw(sc, P.o_dres, f, f.d);
  const ts_strided dmass = d->normalize ? bhtw(sc, P.o_dmass, f, 1) : none();
  const ts_strided dphq = bhtw(sc, P.o_dphq, f, f.m), dphk = bhtw(sc, P.o_dphk, f, f.m);

  // read backward
  ts_read_desc rd = {f.B, f.H, f.T, f.d, f.dtype, d->normalize ? 1 : 0, d->gate ? 1 : 0, f.resid_scale, f.eps};
  float* gb_parts = gr->dg_bias ? (float*)(sc + P.o_col) : nullptr;
  ts_read_bwd_io rb = {num, mass, res, d->gate ? io->g : none(), gr->dy, dnum, dmass, dres,
                       d->gate ? gr->dg : none(), gb32, gb_parts};
  if ((rc = ts_read_bwd(&rd, &rb, stream))) return rc;

  // dphi_q = scan(dnum, v, phi_k): its segment states are the forward's, transposed
  void* wsb = P.ws_b ? sc + P.o_wsb : nullptr;
  ts_scan_io s;
  memset(&s, 0, sizeof(s));
  s.q = dnum; s.k = io->v; s.v = phk; s.q_ext = dmass; s.out = dphq;
  if (P.reuse) rc = ts_scan_fwd(&P.sdq, &s, (void*)(sv + P.o_wsf), P.ws_f, stream);
  else rc = ts_scan_fwd(&P.sdq, &s, wsb, P.ws_b, stream);
  if (rc) return rc;
  // dphi_k = reverse scan(v, dnum, phi_q); dv = reverse scan(phi_k, phi_q, dnum)
  // reads its segment states transposed (sum_i dnum_i phi_q_i^T)
  if (f.d == 64 && f.m == 64 && f.dtype == TS_BF16) {
    // both in one pass over dnum and phi_q (the state updated once per tile;
    // the key-mass read adds dmass to the dk scan's scores)
    const ts_scan_pair_io pio = {io->v, dnum, phq, phk, dphk, gr->dv, dmass};
    if ((rc = ts_scan_pair_fwd(&P.sdk, &pio, wsb, P.ws_b, stream))) return rc;
  } else {
    memset(&s, 0, sizeof(s));
    s.q = io->v; s.k = dnum; s.v = phq; s.k_ext = dmass; s.out = dphk;
    if ((rc = ts_scan_fwd(&P.sdk, &s, wsb, P.ws_b, stream))) return rc;
    memset(&s, 0, sizeof(s));
    s.q = phk; s.k = phq; s.v = dnum; s.out = gr->dv;
    if ((rc = ts_scan_fwd(&P.sdv, &s, wsb, P.ws_b, stream))) return rc;
  }


  // feature backwards with per-workgroup weight-gradient slots
  const bool want_k = gr->dw1 || gr->dtau;
  const bool want_q = want_k || gr->dw2;
  float* w1k = (float*)(sc + P.o_w1k);
  float* tk = f.has_tau ? (float*)(sc + P.o_tk) : nullptr;
  float* w1q = (float*)(sc + P.o_w1q);
  float* w2q = (float*)(sc + P.o_w2q);
  float* tq = f.has_tau ? (float*)(sc + P.o_tq) : nullptr;
  ts_feature_bwd_io bk;
  memset(&bk, 0, sizeof(bk));
  bk.x = io->k; bk.w1 = io->w1; bk.tau = tau32;
  bk.in_cos = io->in_cos; bk.in_sin = io->in_sin; bk.f_cos = io->f_cos; bk.f_sin = io->f_sin;
  bk.dphi = dphk; bk.dx = gr->dk;
  if (want_k) { bk.dw1_part = w1k; bk.dtau_part = tk; }
  if ((rc = ts_feature_bwd(&f, &bk, stream))) return rc;
  ts_feature_bwd_io bq = bk;
  bq.x = io->q; bq.dphi = dphq; bq.dresid = dres; bq.dx = gr->dq; bq.w2 = io->w2;
  bq.dw1_part = bq.dw2_part = nullptr; bq.dtau_part = nullptr;
  if (want_q) { bq.dw1_part = w1q; bq.dw2_part = w2q; bq.dtau_part = tq; }
  if ((rc = ts_feature_bwd(&f, &bq, stream))) return rc;

  // every weight-gradient sum (gate bias, W1, W2, tau) in one launch
  const int64_t hmd = (int64_t)f.H * f.m * f.d;
  ts::SlotSum jobs[ts::kMaxSlotJobs];
  int njobs = 0;
  if (gb_parts) jobs[njobs++] = {gb_parts, P.col_slices, nullptr, 0, (int64_t)f.H * f.d, gr->dg_bias, d->param_dtype, 1.0f};
  if (gr->dw1) jobs[njobs++] = {w1k, P.pk, w1q, P.pq, hmd, gr->dw1, d->param_dtype, 1.0f};
  if (gr->dw2) jobs[njobs++] = {w2q, P.pq, nullptr, 0, hmd, gr->dw2, d->param_dtype, 1.0f};
  if (gr->dtau) jobs[njobs++] = {tk, P.pk, tq, P.pq, f.H, gr->dtau, d->param_dtype, 1.0f};
  return ts::sum_slots_batch(jobs, njobs, stream);
}

}  // extern "C"
