/*
 * thetascan_hip.h -- C ABI of the MI355X (gfx950) ThetaScan scan hot path.
 *
 * One shared library, libthetascan_hip.so, exports every entry point below.
 * All pointers are device pointers owned by the caller; every call is
 * asynchronous on the caller's hipStream_t and returns a status code
 * (TS_OK on success).  ts_last_error() returns a thread-local message for the
 * last failing call.  Status codes map onto the reference's exception types:
 *
 *   TS_ERR_VALUE           -> ValueError          (bad sizes, chunk < 1, ...)
 *   TS_ERR_NOT_IMPLEMENTED -> NotImplementedError (per-channel decay, ...)
 *   TS_ERR_RUNTIME         -> RuntimeError        (HIP launch failure, ...)
 *
 * Tensors are described by a base pointer plus element strides for the
 * (batch, head, time) axes; the innermost (feature) axis must be contiguous.
 * Row base addresses must be 16-byte aligned and feature widths a multiple of
 * 16 bytes / element size: callers pad otherwise (the Python binding does).
 */
#ifndef THETASCAN_HIP_H
#define THETASCAN_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TS_ABI_VERSION 1

enum ts_status {
  TS_OK = 0,
  TS_ERR_VALUE = 1,
  TS_ERR_NOT_IMPLEMENTED = 2,
  TS_ERR_RUNTIME = 3,
};

enum ts_dtype { TS_BF16 = 0, TS_F32 = 1 };

/* Retention (temporal weighting) of one scan view.  Mirrors the three
 * retention forms accepted by scan_chunk.linattn_views
 * (src/thetascan/_core/ops/scan_chunk.py:246-291):
 *   NONE   -- plain causal sum                          (retention None)
 *   STATIC -- per-head log-retention log_alpha[H]       (retention [H])
 *   STREAM -- per-token log-retention decay[B,H,T]      (retention [B,H,T,1]) */
enum ts_retention { TS_RET_NONE = 0, TS_RET_STATIC = 1, TS_RET_STREAM = 2 };

/* Extra column appended after the last feature of q, k or v. */
enum ts_ext { TS_EXT_NONE = 0, TS_EXT_ONES = 1, TS_EXT_ARRAY = 2 };

/* Output handling. */
enum ts_out_mode {
  TS_OUT_STORE = 0,      /* out (input dtype) = result                     */
  TS_OUT_STORE_F32 = 1,  /* out (fp32) = scale * result                    */
  TS_OUT_ACCUM_F32 = 2,  /* out (fp32) += scale * result                   */
};

typedef struct ts_strided {
  const void* ptr;
  int64_t sb, sh, st; /* element strides of batch, head and time */
} ts_strided;

typedef struct ts_scan_desc {
  int32_t B, H, T;
  int32_t dk, dv;       /* feature widths of q/k and v, without ext columns  */
  int32_t dtype;        /* ts_dtype of q, k, v (and out for TS_OUT_STORE)    */
  int32_t retention;    /* ts_retention                                      */
  int32_t reverse;      /* 1: anti-causal scan (time axis read backwards)    */
  int32_t q_ext, k_ext, v_ext; /* ts_ext of an extra column at index dk/dv   */
  int32_t out_mode;     /* ts_out_mode                                       */
  float out_scale;      /* scale for the fp32 output modes                   */
  int32_t seg_chunks;   /* 64-token tiles per workgroup segment; 0 = auto    */
  int32_t want_final;   /* 1: write the final [dk_pad, dv_pad] state          */
} ts_scan_desc;

typedef struct ts_scan_io {
  ts_strided q, k, v;
  ts_strided q_ext, k_ext, v_ext; /* fp32 [B,H,T] columns for TS_EXT_ARRAY     */
  const float* log_alpha;         /* [H] for TS_RET_STATIC                     */
  ts_strided decay;               /* fp32 [B,H,T] for TS_RET_STREAM            */
  ts_strided out;                 /* [B,H,T,dv]                                */
  ts_strided out_ext;             /* fp32 [B,H,T]: result column dv (or NULL) */
  float* final_state;             /* fp32 [B*H, dk_pad, dv_pad] (or NULL)      */
} ts_scan_io;

/* ABI version (TS_ABI_VERSION). */
int ts_abi_version(void);

/* Message for the last failing call on this thread. */
const char* ts_last_error(void);

/* Padded widths and workgroup segmentation the scan uses for `desc`;
 * final_state is laid out with these padded widths.  Any output pointer may
 * be NULL. */
int ts_scan_layout(const ts_scan_desc* desc, int32_t* dk_pad, int32_t* dv_pad,
                   int32_t* n_segments);

/* Device workspace (bytes) ts_scan_fwd needs for `desc`. */
int ts_scan_workspace_bytes(const ts_scan_desc* desc, size_t* bytes);

/* Causal (or anti-causal, desc->reverse) linear-attention scan of one view:
 *
 *   out_t = sum_{i<=t} w(t,i) <q_t, k_i> v_i,   w(t,i) = prod_{i<j<=t} alpha_j
 *
 * with q, k, v extended by their optional ext columns.  Replaces one
 * retention slot of scan_chunk.linattn_views
 * (src/thetascan/_core/ops/scan_chunk.py:246-339) and one call of
 * scan_naive.linattn (src/thetascan/_core/ops/scan_naive.py:5-18), whose
 * recurrence it computes exactly, in 64-token tiles with an fp32 carried
 * state.  The extra v column TS_EXT_ONES with out_ext set is the key-mass
 * denominator of the normalized read (src/thetascan/_core/ops/engine.py:419-442). */
int ts_scan_fwd(const ts_scan_desc* desc, const ts_scan_io* io,
                void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* THETASCAN_HIP_H */
