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

/* 8: the scan entry points require a 16-byte aligned workspace (a sub-
 *    allocated workspace at an odd offset was accepted by version 7).
 * 9: ts_wcumsum takes a workspace (ts_wcumsum_workspace_bytes).
 * 10: the GN descriptors carry the hidden nonlinearity (and the write its
 *     damping);
 * 11: ts_scan_pair_io carries scan A's key-side ext column (k_ext);
 * 12: ts_retention_grad.
 * 13: ts_scan_pair_io gains log_alpha (after k_ext): ts_scan_pair_fwd takes
 *     a static retention and the fp32 store / accumulate output modes; a
 *     ts_retention_grad slice that reaches 2 GiB is refused with
 *     TS_ERR_NOT_IMPLEMENTED.
 * 14: ts_read_out_fwd / ts_read_out_bwd / ts_read_out_bwd_parts (the read
 *     fused with the output projection), ts_kmap_*, ts_anchor_*,
 *     ts_bspline_norm_*, ts_feature_fwd_summary, ts_scan_desc.states_in = 3,
 *     TS_GN_SILU, ts_gn_act_* and ts_abs_mass_*; nothing earlier changed.
 * 15: ts_rownorm_fwd / ts_rownorm_bwd; nothing earlier changed.
 * 16: ts_stack_heads; nothing earlier changed.
 * 17: ts_scale_add_fwd / ts_scale_add_bwd / ts_scale_add_parts, ts_relu2_fwd /
 *     ts_relu2_bwd, ts_softcap_xent_fwd / ts_softcap_xent_bwd, ts_blend_gated_fwd;
 *     nothing earlier changed. */
#define TS_ABI_VERSION 17

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
  int32_t value_split;  /* value columns per workgroup (16, 32, 64 or 128,
                           dividing dv_pad); 0 = the whole width             */
  int32_t states_in;    /* 0: compute the segment states; 1: the workspace
                           already holds them (from an earlier call of this
                           scan's keys and values); 2: it holds those of the
                           swapped scan (keys and values exchanged, same
                           segments and retention), read transposed; a key-side
                           ext row u is then the swapped scan's value-side ext
                           state.  Skips the summary and prefix passes.  No
                           value-side ext column (nor key-side with 1).      */
                        /* 3: it holds this scan's segment summaries (as
                           ts_feature_fwd_summary writes them): the summary
                           pass is skipped, the prefix and main passes run.
                           Plain sum, no key-side ext columns, no final
                           state, one value slice.                           */
  int32_t init_state;   /* 1: io->init_state holds the state entering the first
                           token (a continued sequence; 0 = a zero state).
                           The first token's decay applies to it, so a scan
                           of x[T0:] from the final state of x[:T0] equals
                           the tail of the scan of x (a reversed scan's first
                           step carries no per-token decay: its caller
                           applies the decay linking the pieces).  Not with
                           states_in.                                        */
} ts_scan_desc;

typedef struct ts_scan_io {
  ts_strided q, k, v;
  ts_strided q_ext, k_ext, v_ext; /* fp32 [B,H,T] columns for TS_EXT_ARRAY     */
  const float* log_alpha;         /* [H] for TS_RET_STATIC                     */
  ts_strided decay;               /* fp32 [B,H,T] for TS_RET_STREAM            */
  ts_strided out;                 /* [B,H,T,dv]                                */
  ts_strided out_ext;             /* fp32 [B,H,T]: result column dv (or NULL) */
  float* final_state;             /* fp32 [B*H, dk_pad, dv_pad] (or NULL)      */
  const float* init_state;        /* fp32 [B*H, dk_pad, dv_pad] (init_state)   */
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

/* Device workspace (bytes) ts_scan_fwd and ts_scan_pair_fwd need for `desc`.
 * The workspace base must be 16-byte aligned (the summaries are read and
 * written as 16-byte vectors); a misaligned base is refused with
 * TS_ERR_VALUE.  Its contents need no initialisation. */
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

/* ts_scan_fwd without a workspace argument and without any device allocation
 * (no counterpart in the reference: for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The segment summaries live in a library-owned device
 * buffer of TS_SCAN_NOALLOC_MAX_WORKSPACE bytes, one per GPU, held until the
 * process ends; a scan whose ts_scan_workspace_bytes() exceeds it returns
 * TS_ERR_VALUE, and states_in (kept segment states) is refused.  Every call on
 * one GPU shares that buffer: calls that overlap on one GPU (several streams,
 * several host threads) race and must be serialised by the caller.  Results
 * equal ts_scan_fwd's with the same desc and io.  The first call on a device
 * looks up the buffer's address and sets the kernels' LDS limits: make one
 * call on each device outside a stream capture before capturing calls into a
 * graph (the captured calls then make no runtime query). */
#define TS_SCAN_NOALLOC_MAX_WORKSPACE (32u * 1024u * 1024u)

int ts_scan_fwd_noalloc(const ts_scan_desc* desc, const ts_scan_io* io, hipStream_t stream);

/* Two plain scans over the same keys and values up to a swap, in one pass:
 *
 *   out_a_t = sum_{i<=t} <qa_t, k_i> v_i,   out_b_t = sum_{i<=t} <qb_t, v_i> k_i
 *
 * (anti-causal with desc->reverse).  These are the backward's dk and dv scans
 * of a kernel memory (scan_hip._ScanViews.backward; the reference's autograd
 * of scan_chunk.linattn_views, scan_chunk.py:246-339): k = dnum, v = phi(q),
 * qa = v, qb = phi(k).  K and V are read once and the state is updated once
 * per tile; each output equals its own ts_scan_fwd call.  desc describes
 * scan A (q = qa): bf16, no retention, TS_OUT_STORE, dk == dv == 64, no
 * value-side ext column; with q_ext = TS_EXT_ONES and k_ext = TS_EXT_ARRAY
 * scan A is the key-mass read's backward, out_a_t = sum_i (<qa_t, k_i> +
 * k_ext_i) v_i (scan B has no ext column); workspace from
 * ts_scan_workspace_bytes(desc), 16-byte aligned. */
typedef struct ts_scan_pair_io {
  ts_strided qa, k, v, qb;
  ts_strided out_a;               /* [B,H,T,dv] (bf16, or fp32 in the fp32
                                     output modes, stored or accumulated)     */
  ts_strided out_b;               /* [B,H,T,dk] (same)                         */
  ts_strided k_ext;               /* fp32 [B,H,T] key-side ext of scan A (desc
                                     q_ext ones, k_ext array), else NULL       */
  const float* log_alpha;         /* [H] static log-retention of both scans
                                     (desc retention TS_RET_STATIC), else NULL */
} ts_scan_pair_io;

int ts_scan_pair_fwd(const ts_scan_desc* desc, const ts_scan_pair_io* io,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------ retention gradient */

/* dL/dlog_alpha[h] of one causal scan with a static per-head retention,
 *   o_t = sum_{i<=t} alpha^(t-i) <q_t, k_i> v_i  (+ the key-mass column),
 * for upstream gradients dout (and dmass of the mass column):
 *   out[b][h] = sum_t sum_{i<=t} (t-i) alpha^(t-i) <q_t, k_i> (<dout_t, v_i> + dmass_t).
 * Summed pair by pair (bf16 operands, fp32 accumulation), not as
 * sum_t t (q_t.dq_t - k_t.dk_t), whose terms cancel.  Replaces the retention
 * gradient autograd forms through scan_chunk.py:102-155 (_static_weights /
 * _tile_weights) for a learned static retention (block.py:647-681, the
 * bank's fade_alpha).  Parallel over segments of seg_tiles 64-token tiles
 * (0: automatic) with a combine pass for pairs across segments. */
typedef struct ts_retention_desc {
  int32_t B, H, T;
  int32_t dk;           /* multiple of 16, <= 128 (split wider keys: the sum is additive) */
  int32_t dv;           /* multiple of 8; value blocks + mass block <= 8 x 16 */
  int32_t dtype;        /* TS_BF16 */
  int32_t has_mass;     /* dmass given: the read's key-mass column */
  int32_t seg_tiles;
} ts_retention_desc;

typedef struct ts_retention_io {
  ts_strided q, k;      /* [B,H,T,dk] */
  ts_strided v, dout;   /* [B,H,T,dv] */
  ts_strided dmass;     /* fp32 [B,H,T] or NULL */
  const float* log_alpha;  /* fp32 [H] */
} ts_retention_io;

/* Device workspace ts_retention_grad needs (16-byte aligned). */
int ts_retention_workspace_bytes(const ts_retention_desc* desc, size_t* bytes);

/* out: fp32 [B][H]. */
int ts_retention_grad(const ts_retention_desc* desc, const ts_retention_io* io, float* out, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------ several retentions */

#define TS_MAX_VIEWS 3

typedef struct ts_scan_views_desc {
  int32_t B, H, T;
  int32_t dk, dv;       /* feature widths: dk <= 128, dv <= 64 (multiples of 8) */
  int32_t dtype;        /* TS_BF16                                             */
  int32_t n_views;      /* 2 .. TS_MAX_VIEWS                                   */
  int32_t mass;         /* 1: v carries a unit ext column; each view also
                           returns its key mass (out_ext)                      */
  int32_t seg_chunks;   /* 64-token tiles per workgroup segment; 0 = auto      */
} ts_scan_views_desc;

typedef struct ts_scan_views_io {
  ts_strided q, k, v;
  const float* log_alpha[TS_MAX_VIEWS]; /* [H] static retention of view j;
                                           NULL: no retention (plain sum)     */
  ts_strided out[TS_MAX_VIEWS];         /* [B,H,T,dv] in the input dtype      */
  ts_strided out_ext[TS_MAX_VIEWS];     /* fp32 [B,H,T] key mass (mass = 1)   */
} ts_scan_views_io;

/* Device workspace (bytes) ts_scan_views_fwd needs for `desc` (16-byte
 * aligned base, contents need no initialisation). */
int ts_scan_views_workspace_bytes(const ts_scan_views_desc* desc, size_t* bytes);

/* The forward causal scans of n_views retentions (none or static [H]) over
 * the same q, k, v in one pass: the multi-view call of
 * scan_chunk.linattn_views (src/thetascan/_core/ops/scan_chunk.py:246-339,
 * whose score tile S = Q K^T is shared by every view), as called by
 * interface.scan_views for a temporal bank (interface.py:173-182).  q, k and
 * v are read once per pass, the score tile is formed once per 64-token tile,
 * and each view keeps its own fp32 state.  Results equal n_views calls of
 * ts_scan_fwd with the same segmentation. */
int ts_scan_views_fwd(const ts_scan_views_desc* desc, const ts_scan_views_io* io,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);


/* ------------------------------------------------------------------ write */

enum ts_feature_kind { TS_FEAT_RELU2 = 0, TS_FEAT_SOFTMAX = 1 };

typedef struct ts_feature_desc {
  int32_t B, H, T;
  int32_t d;            /* head width: 16, 32, 64 or 128                        */
  int32_t m;            /* feature width: 16, 32, 64, 128 or 256                */
  int32_t dtype;        /* ts_dtype of x, weights and bf16/fp32 outputs        */
  int32_t kind;         /* ts_feature_kind                                      */
  int32_t in_rot;       /* input-RoPE rotated channels of x (0 or 4k <= d)     */
  int32_t feat_rot;     /* feature-RoPE rotated channels of phi (0 or 4k <= m) */
  int32_t has_tau;      /* relu2: subtract the per-head threshold tau[H]       */
  float gain;           /* softmax: logit gain                                 */
  float resid_scale;    /* s = 1/sqrt(depth) of the residual read              */
  float eps;            /* 1e-6 in the reference                               */
} ts_feature_desc;

typedef struct ts_feature_io {
  ts_strided x;                    /* [B,H,T,d] raw keys or queries            */
  const void* w1;                  /* [H,m,d] effective W1                     */
  const void* w2;                  /* [H,d,m] effective W2 (resid only)        */
  const float* tau;                /* [H]                                      */
  const float* in_cos;             /* [T, in_rot/2]                            */
  const float* in_sin;
  const float* f_cos;              /* [T, feat_rot/2]                          */
  const float* f_sin;
  ts_strided phi;                  /* out [B,H,T,m]: rotated features          */
  ts_strided resid;                /* out [B,H,T,d]: xn + s*W2 h  (or NULL)    */
} ts_feature_io;

/* Fused write-side feature map for one stream (keys, or queries):
 *   xn  = l2norm(rope_in(x));  a = W1 xn;  pre = rmsnorm(a) - tau
 *   h   = relu2_ridge(pre) | softmax(gain * pre);  phi = rope_feat(h)
 *   resid = xn + s * W2 h   (queries only)
 * Replaces block.py:595-618 (input RoPE, L2 norm, feature-RoPE table),
 * engine.py:117-158 (_block_forward), kernel_features.py:73-135 (feature
 * maps), engine.py:74-86 (_hrot_stream) and the base term of
 * engine.py:522-528. */
int ts_feature_fwd(const ts_feature_desc* desc, const ts_feature_io* io, hipStream_t stream);

typedef struct ts_feature_bwd_io {
  ts_strided x;                    /* [B,H,T,d] forward input                  */
  const void* w1;                  /* [H,m,d]                                  */
  const void* w1t;                 /* [H,d,m] (W1 transposed), or NULL         */
  const void* w2t;                 /* [H,m,d] (W2 transposed; resid), or NULL  */
  const float* tau;
  const float* in_cos;
  const float* in_sin;
  const float* f_cos;
  const float* f_sin;
  ts_strided dphi;                 /* [B,H,T,m]: grad of phi                   */
  ts_strided dresid;               /* [B,H,T,d]: grad of resid (or NULL)       */
  ts_strided dx;                   /* out [B,H,T,d]: grad of x                 */
  ts_strided da;                   /* out [B,H,T,m]: grad of a = W1 xn (NULL ok) */
  ts_strided xn;                   /* out [B,H,T,d]: xn (NULL ok)              */
  ts_strided h;                    /* out [B,H,T,m]: unrotated h (NULL ok)     */
  ts_strided dtau;                 /* out fp32 [B,H,T]: -sum_j dpre_j (NULL ok) */
  float* dw1_part;                 /* out fp32 [P,H,m,d]: partial sums of da^T xn        */
  float* dw2_part;                 /* out fp32 [P,H,d,m]: partial sums of s dresid^T h   */
  float* dtau_part;                /* out fp32 [P,H]: partial sums of -sum_j dpre_j      */
  const void* w2;                  /* [H,d,m] (resid; read when w2t is NULL)   */
} ts_feature_bwd_io;

/* ts_feature_fwd for keys that also writes the segment summaries of the scan
 * `scan` (plain sum, keys = these features, values = v [B,H,T,64], with or
 * without its value-side ones column) into that scan's workspace, exactly as
 * the scan's own summary pass computes them (same MFMA sequence): a
 * following ts_scan_fwd of `scan` with states_in = 3 then skips the pass that
 * would read the features and values a second time.  bf16, d = m = 64.
 * No counterpart in the reference (a fusion of two of its steps). */
int ts_feature_fwd_summary(const ts_feature_desc* desc, const ts_feature_io* io, ts_strided v,
                           const ts_scan_desc* scan, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

/* Whether ts_feature_bwd needs the transposed weights w1t / w2t for `desc`
 * (weights too large to stage in LDS).  Otherwise they may be NULL: the
 * kernel transposes W1 (and W2 from `w2`) while staging them. */
int ts_feature_bwd_transposed(const ts_feature_desc* desc, int32_t has_dresid, int32_t fused_wgrad,
                              int32_t* needed);

/* Backward of ts_feature_fwd (recomputes the forward tile in registers/LDS).
 * Two ways to obtain the weight gradients of W1, W2 and tau:
 *   fused    -- dw1_part != NULL: every workgroup contracts its tokens'
 *               da^T xn (and s dresid^T h, and the tau gradient) into one of
 *               P partial slots, P from ts_feature_bwd_parts(); the caller
 *               sums the slots.  da/xn/h/dtau are then ignored.
 *   per-token -- dw1_part == NULL: da, xn, h, dtau are written per token
 *               (any may be NULL) for the caller's own GEMMs.
 * Replaces the autograd backward of the chain ts_feature_fwd replaces. */
int ts_feature_bwd(const ts_feature_desc* desc, const ts_feature_bwd_io* io, hipStream_t stream);

/* Number P of partial weight-gradient slots ts_feature_bwd fills for `desc`
 * (with or without a dresid input), or 0 when no fused weight-gradient kernel
 * covers the shape (the per-token outputs must be used). */
int ts_feature_bwd_parts(const ts_feature_desc* desc, int32_t has_dresid, int32_t* parts);

/* ------------------------------------------------------------------- read */

typedef struct ts_read_desc {
  int32_t B, H, T, d;
  int32_t dtype;        /* of num, resid, gate and y                           */
  int32_t normalize;    /* 1: mem = num / (mass + eps)                         */
  int32_t gate;         /* 1: y *= silu(g)                                     */
  float scale;          /* s = 1/sqrt(depth)                                   */
  float eps;
} ts_read_desc;

typedef struct ts_read_io {
  ts_strided num;                  /* [B,H,T,d] scan numerator                 */
  ts_strided mass;                 /* fp32 [B,H,T] key mass (normalize)        */
  ts_strided resid;                /* [B,H,T,d] xn + s*W2 h                    */
  ts_strided g;                    /* gate pre-activation, [B,H,T,d] view      */
  ts_strided y;                    /* out [B,H,T,d] view (e.g. of [B,T,H*d])   */
  const float* g_bias;             /* fp32 [H,d] added to g before silu (NULL) */
} ts_read_io;

/* Normalized read epilogue:  y = (resid + s * num / (mass + eps)) * silu(g + g_bias).
 * Replaces engine.py:440-442, 526-528 and the output gate of
 * block.py:721-722 (gates.py:34-40). */
int ts_read_fwd(const ts_read_desc* desc, const ts_read_io* io, hipStream_t stream);

typedef struct ts_read_bwd_io {
  ts_strided num, mass, resid, g;  /* forward inputs                           */
  ts_strided dy;                   /* grad of y                                */
  ts_strided dnum;                 /* out [B,H,T,d] (desc dtype)               */
  ts_strided dmass;                /* out fp32 [B,H,T] (normalize)             */
  ts_strided dresid;               /* out [B,H,T,d] (desc dtype; NULL ok)      */
  ts_strided dg;                   /* out [B,H,T,d] (gate)                     */
  const float* g_bias;             /* as in ts_read_io                         */
  float* dg_bias_part;             /* out fp32 [P, H*d] per-workgroup sums of dg
                                      over tokens (gate, d <= 256; NULL ok): the
                                      gate-bias gradient is their sum over P,
                                      P from ts_read_bwd_parts (ts_sum_slots)  */
} ts_read_bwd_io;

/* Backward of ts_read_fwd: dnum, dmass, dresid, dg and optionally the
 * gate-bias gradient partials.  Replaces the autograd backward of the same
 * chain (engine.py:440-442, 526-528; gates.py:34-40, with the bias gradient
 * summed over every token). */
int ts_read_bwd(const ts_read_desc* desc, const ts_read_bwd_io* io, hipStream_t stream);

/* Number P of gate-bias partial rows ts_read_bwd writes for `desc`. */
int ts_read_bwd_parts(const ts_read_desc* desc, int32_t* parts);

/* ------------------------------------ kernel feature maps with controls */

enum ts_kmap_kind { TS_KMAP_SOFTMAX = 0, TS_KMAP_RELU2 = 1 };
enum ts_kmap_sparsity { TS_SPARSE_NONE = 0, TS_SPARSE_SOFT = 1, TS_SPARSE_ST = 2, TS_SPARSE_ST_BLEND = 3 };

typedef struct ts_kmap_desc {
  int32_t B, H, T;
  int32_t m;            /* feature width: 16, 32, 48 or 64                     */
  int32_t dtype;        /* ts_dtype of a, phi, dphi, da                         */
  int32_t kind;         /* ts_kmap_kind                                         */
  int32_t rms;          /* 1: a is the raw W1 product and is RMS-normalized
                           first; 0: a is the normalized pre-activation        */
  int32_t gain_mode;    /* softmax gain: 0 the scalar `gain`, 1 per head [H],
                           2 per feature [H, m] (positive values)              */
  int32_t sparsity;     /* ts_kmap_sparsity (softmax only)                      */
  float gain;
  float temperature;    /* relative-threshold temperature                      */
  float eps;
} ts_kmap_desc;

typedef struct ts_kmap_params {
  const float* shift;   /* [H, m] added after the RMSNorm: score bias minus the
                           learned thresholds (NULL: none)                      */
  const float* gain;    /* [H] or [H, m] (gain_mode 1, 2)                        */
  const float* rho;     /* [H] relative threshold in (0, 1) (sparsity)          */
  const float* alpha;   /* [H] sparse blend in [0, 1] (TS_SPARSE_ST_BLEND)      */
} ts_kmap_params;

/* Number P of per-workgroup partial rows of the control gradients. */
int ts_kmap_parts(const ts_kmap_desc* desc, const ts_kmap_params* params, int32_t* parts);

/* phi [B,H,T,m] = map(rmsnorm(a) + shift) (or map(a + shift)), the softmax
 * partition with its gain, score bias and relative-to-max sparsity (soft,
 * straight-through, straight-through blend) or the ReLU^2 ridge.  Replaces
 * kernel_features.py:43-135 (with the RMSNorm of engine.py:117-158). */
int ts_kmap_fwd(const ts_kmap_desc* desc, const ts_kmap_params* params, ts_strided a, ts_strided phi,
                hipStream_t stream);

typedef struct ts_kmap_grads {
  ts_strided da;        /* out [B,H,T,m]: grad of a                              */
  float* dshift_part;   /* out fp32 [P, H, m] (NULL: not wanted)                 */
  float* dgain_part;    /* out fp32 [P, H] or [P, H, m] (NULL: not wanted)       */
  float* drho_part;     /* out fp32 [P, H] (NULL: not wanted)                    */
  float* dalpha_part;   /* out fp32 [P, H] (NULL: not wanted)                    */
} ts_kmap_grads;

/* Backward of ts_kmap_fwd: da and partial sums (over each workgroup's tokens)
 * of the gradients of shift, gain, rho and alpha; the straight-through gates
 * differentiate through their sigmoid, the clamp of rho and the floor of the
 * sparse sum pass no gradient, and the max's gradient is shared equally by
 * the maximal logits (torch's amax rule). */
int ts_kmap_bwd(const ts_kmap_desc* desc, const ts_kmap_params* params, ts_strided a, ts_strided dphi,
                const ts_kmap_grads* grads, hipStream_t stream);

/* ---------------------------------------------------- value-anchor deposit */

typedef struct ts_anchor_desc {
  int32_t B, H, T;
  int32_t d;            /* value width: 16, 32, 64 or 128                      */
  int32_t V;            /* anchors in the codebook: 2 .. 64                    */
  int32_t c_heads;      /* codebook heads: 1 (shared by every head) or H       */
  int32_t dtype;        /* ts_dtype of v, r, dr, dv and the dls rows           */
  float gain;           /* softmax gain (the configured scalar sharpness)      */
  float eps;            /* norm floor (1e-6 in the reference)                  */
} ts_anchor_desc;

/* Padded anchor width VP (16, 32 or 64) of the backward's dls rows. */
int ts_anchor_width(const ts_anchor_desc* desc, int32_t* vp);

/* r [B,H,T,V] = softmax(gain * C (v / max(||v||, eps))), C = codebook fp32
 * [c_heads, V, d]: the value-anchor deposit of a kernel memory.  Replaces
 * engine.py:284-296 (the value_centers branch of write_streams). */
int ts_anchor_fwd(const ts_anchor_desc* desc, ts_strided v, const float* codebook, ts_strided r,
                  hipStream_t stream);

/* Backward of ts_anchor_fwd: dv [B,H,T,d] from dr [B,H,T,V], and dls
 * [H, B*T, VP] (head-major rows, zero past V) = dlogits / max(||v||, eps),
 * so that the codebook gradient is sum over tokens of dls^T v (per head; summed
 * over heads for a shared codebook). */
int ts_anchor_bwd(const ts_anchor_desc* desc, ts_strided v, const float* codebook, ts_strided dr,
                  ts_strided dv, void* dls, hipStream_t stream);

/* ------------------------------------- read fused with the output projection */

typedef struct ts_read_out_desc {
  ts_read_desc read;    /* B, H, T, d (32, 64, 96, 128), bf16 only, normalize,
                           gate, scale, eps -- as for ts_read_fwd            */
  int32_t n;            /* output width N (d_model); N and H*d are multiples
                           of 128, H*d at most 512 and N at most 1024        */
} ts_read_out_desc;

typedef struct ts_read_out_io {
  ts_strided num, mass, resid, g;  /* as ts_read_io (resid may be NULL)      */
  const float* g_bias;             /* fp32 [H*d] or NULL                     */
  const void* w;                   /* [N, H*d] output projection weight      */
  void* out;                       /* out rows b*T + t of N elements         */
  int64_t out_ld;                  /* row stride of out (elements)           */
  void* y;                         /* out rows b*T + t of H*d elements: the
                                      read output y (NULL: not kept)         */
  int64_t y_ld;
} ts_read_out_io;

/* out = y W^T with y = (resid + s * num / (mass + eps)) * silu(g + g_bias)
 * formed in the GEMM's prologue (y is bit-identical to ts_read_fwd's and
 * never read back from HBM).  Replaces block.py:721-724 (the output gate,
 * the reshape and proj_out) together with what ts_read_fwd replaces.
 * TS_ERR_NOT_IMPLEMENTED for shapes outside the descriptor's limits. */
int ts_read_out_fwd(const ts_read_out_desc* desc, const ts_read_out_io* io, hipStream_t stream);

typedef struct ts_read_out_bwd_io {
  ts_strided num, mass, resid, g;  /* forward inputs                         */
  const float* g_bias;
  const void* w_t;                 /* [H*d, N]: the weight transposed        */
  const void* dout;                /* rows b*T + t of N: grad of out         */
  int64_t dout_ld;
  ts_strided dnum, dmass, dresid, dg;  /* outputs as for ts_read_bwd          */
  float* dg_bias_part;             /* out fp32 [P, H*d] gate-bias partials
                                      (P from ts_read_out_bwd_parts; NULL ok) */
} ts_read_out_bwd_io;

/* Backward of ts_read_out_fwd except the weight gradient (dout^T y, which
 * the caller contracts from the y the forward kept): dy = dout W is formed
 * in registers and consumed by the read backward (dnum, dmass, dresid, dg).
 * Replaces the input-gradient product of proj_out (block.py:724) and the
 * autograd backward ts_read_bwd replaces.  Needs head widths 32, 64 or 128. */
int ts_read_out_bwd(const ts_read_out_desc* desc, const ts_read_out_bwd_io* io, hipStream_t stream);

/* Number P of gate-bias partial rows ts_read_out_bwd writes for `desc`. */
int ts_read_out_bwd_parts(const ts_read_out_desc* desc, int32_t* parts);

/* ------------------------------------------------- query/key prologue */

typedef struct ts_qknorm_desc {
  int32_t B, H, T, d;
  int32_t dtype;        /* of x, y, dy, dx                                     */
  int32_t rot;          /* RoPE width (even, <= d; 0 = none)                   */
  float eps;
} ts_qknorm_desc;

/* y = rope(x) / max(|rope(x)|, eps) per [B,H,T,d] row, RoPE on pairs
 * (2i, 2i+1), i < rot / 2, with fp32 angles from rope_cos/rope_sin [T, rot/2].
 * Replaces the input RoPE and the query/key L2 norm of the mixer prologue
 * (block.py:595-599; rope.py:41-49; norms.py:11-12). */
int ts_qknorm_fwd(const ts_qknorm_desc* desc, ts_strided x, ts_strided y, const float* rope_cos,
                  const float* rope_sin, hipStream_t stream);

/* Backward of ts_qknorm_fwd: dx from x and dy. */
int ts_qknorm_bwd(const ts_qknorm_desc* desc, ts_strided x, ts_strided dy, ts_strided dx, const float* rope_cos,
                  const float* rope_sin, hipStream_t stream);

/* -------------------------------------------------------- GN write payloads */

/* Hidden nonlinearity sigma of a GN fast network. */
enum ts_gn_act {
  TS_GN_RELU2 = 0,  /* sigma = relu(pre)^2, sigma' = 2 relu(pre)   (engine.py nonlin relu2) */
  TS_GN_TANH = 1,   /* sigma = tanh(pre), sigma' = 1 - tanh(pre)^2 (no counterpart in the
                       reference, whose nonlinearities are relu2 and silu, nonlin.py:28-31) */
  TS_GN_SILU = 2,   /* sigma = pre sigmoid(pre), sigma' = sg (1 + pre (1 - sg))
                       (engine.py nonlin silu, nonlin.py:18-24)                          */
};

/* Damped Gauss-Newton write of a one-hidden-layer fast network
 * (engine.py:117-158 _block_forward, 180-195 _g_from_lambda, 215-255
 * _lambda_solve and the write streams of 260-340), per token x (key) and v:
 *   a = W1 x;  pre = a rsqrt(mean a^2 + eps) - tau;  h = sigma(pre)
 *   r = v - x - s W2 h
 *   lam = r / ((|h|^2 + |x|^2 (W2 o W2)(sigma'(pre) rinv)^2) * inv_depth + damping)
 *   g = s sigma'(pre) (W2^T lam) rinv
 * Outputs h [.,m] (LA2 keys), s*lam [.,d] (LA2 values), g [.,m] (LA1 values).
 * Depth-1 memories (s = inv_depth = 1) with relu2, relu2_threshold, silu or tanh.
 * The reference's damping is eps (engine.py:255). */
typedef struct ts_gn_desc {
  int32_t B, H, T;
  int32_t d;            /* head width: 16, 32, 64 or 128                        */
  int32_t m;            /* hidden width: a multiple of 16 up to 128, or 256     */
  int32_t dtype;        /* ts_dtype of every stream and weight                  */
  int32_t has_tau;      /* relu2_threshold: subtract tau [H, m]                 */
  float s;              /* 1/sqrt(depth)                                        */
  float inv_depth;      /* 1/depth: the Jacobi diagonal averages the levels     */
  float eps;            /* 1e-6 in the reference (RMSNorm)                      */
  int32_t act;          /* ts_gn_act                                            */
  float damping;        /* > 0: the Jacobi diagonal's damping (the reference: eps) */
} ts_gn_desc;

typedef struct ts_gn_io {
  ts_strided x, v;      /* [B,H,T,d] keys (as written) and values               */
  const void* w1;       /* [H,m,d]                                              */
  const void* w2;       /* [H,d,m]                                              */
  const void* w2t;      /* [H,m,d] transposed copy of w2                        */
  const float* tau;     /* [H,m] or NULL                                        */
  ts_strided h, lam, g; /* out: h [.,m], s*lam [.,d], g [.,m]                   */
} ts_gn_io;

int ts_gn_write_fwd(const ts_gn_desc* desc, const ts_gn_io* io, hipStream_t stream);

typedef struct ts_gn_bwd_io {
  ts_strided x, v;
  const void* w1, *w2;
  const void* w1t;      /* [H,d,m] transposed copy of w1                        */
  const void* w2t;
  const float* tau;
  ts_strided dh, dlam, dg; /* gradients of the three outputs (NULL = zero)     */
  ts_strided dx_in;     /* added into dx (NULL = zero)                          */
  ts_strided dx, dv;    /* out [B,H,T,d]                                        */
  void* tiles_m;        /* out [4 (+1 with tau), H, B*T, m]: dz, h, da, s2 (, dpre) */
  void* tiles_d;        /* out [4, H, B*T, d]: lam, du, x, drq                  */
} ts_gn_bwd_io;

/* Backward of ts_gn_write_fwd: dx, dv, and the token tiles whose contractions
 * give the weight gradients: dW1 = da^T x, dW2 = lam^T dz + du^T h
 * + 2 W2 o (drq^T s2), dtau = -sum_tokens dpre. */
int ts_gn_write_bwd(const ts_gn_desc* desc, const ts_gn_bwd_io* io, hipStream_t stream);

/* One stage of the GN read (engine.py:467-506), per query q [.,d]:
 *   a = W1 q + c,  c = 0 | num | num / (mass + eps)      (corr = 0 | 1 | 2)
 *   h = sigma(a rsqrt(mean a^2 + eps) - tau)             -> h [.,m]
 *   resid = q + s W2 h                                   -> resid [.,d]
 * Stage 1 of the two-stage normalized read is corr 0 without resid (the
 * queries of the feature-mass scan, engine.py:475-480); stage 2 adds the
 * normalized stage-1 read (corr 2, engine.py:481-487) and gives the queries of
 * the memory scan and the residual of y = q + s (W2 h + mem).  corr 1 is the
 * unnormalized LA1 correction of engine.py:488-500. */
typedef struct ts_gn_read_desc {
  int32_t B, H, T, d, m;
  int32_t dtype;
  int32_t has_tau;      /* subtract tau [H, m]                                  */
  int32_t corr;         /* 0, 1 or 2 as above                                   */
  int32_t want_resid;
  float s;              /* 1/sqrt(depth)                                        */
  float eps;
  int32_t act;          /* ts_gn_act of h (stage 1 of the two-stage read: relu2) */
} ts_gn_read_desc;

typedef struct ts_gn_read_io {
  ts_strided q;
  const void* w1;       /* [H,m,d]                                              */
  const void* w2;       /* [H,d,m] (want_resid)                                 */
  const float* tau;     /* [H,m] or NULL                                        */
  ts_strided num;       /* [B,H,T,m] (corr 1, 2)                                */
  ts_strided mass;      /* fp32 [B,H,T] (corr 2)                                */
  ts_strided h, resid;  /* out                                                  */
} ts_gn_read_io;

int ts_gn_read_fwd(const ts_gn_read_desc* desc, const ts_gn_read_io* io, hipStream_t stream);

typedef struct ts_gn_read_bwd_io {
  ts_strided q;
  const void* w1;
  const void* w1t;      /* [H,d,m] transposed copy of w1                        */
  const void* w2t;      /* [H,m,d] transposed copy of w2 (want_resid)           */
  const float* tau;
  ts_strided num, mass;
  ts_strided dh, dresid;   /* gradients of h and resid (NULL = zero)           */
  ts_strided dq;        /* out [.,d]                                            */
  ts_strided dnum;      /* out [.,m] (corr 1, 2)                                */
  float* dmass;         /* out fp32, laid out like mass (corr 2)                */
  void* tiles_m;        /* out [2 (+1 with tau), H, B*T, m]: da, h (, dpre)     */
  void* tiles_d;        /* out [2, H, B*T, d]: q, s*dresid                      */
} ts_gn_read_bwd_io;

/* Backward of ts_gn_read_fwd: dq, dnum, dmass and the token tiles of
 * dW1 = da^T q, dW2 = (s dresid)^T h, dtau = -sum_tokens dpre. */
int ts_gn_read_bwd(const ts_gn_read_desc* desc, const ts_gn_read_bwd_io* io, hipStream_t stream);

/* Per-row GN hidden activation with its Jacobian scales, the nonlinear core
 * of any GN block (engine.py:117-158 _block_forward, with the per-feature
 * scales that _g_from_lambda / _w2s / _lambda_solve multiply W2 by,
 * engine.py:180-255): for a = W1 x (and the SwiGLU gate pre-activation
 * b = Wg x) of one token,
 *   elementwise act:  z = a ra - tau, h = sigma(z), sa = sigma'(z) ra
 *   TS_GN_SWIGLU:     za = a ra, zb = b rb, h = silu(zb) za,
 *                     sa = silu(zb) ra, sb = za silu'(zb) rb
 * with ra, rb the inverse RMS of a, b.  The GEMMs around it (W1 x, W2 h,
 * W2^T lam, (W2 o W2) sa^2) stay with the caller, which is what lets one
 * kernel serve any depth and both Gauss-Newton steps. */
enum { TS_GN_SWIGLU = 3 };
typedef struct ts_gn_act_desc {
  int32_t B, H, T;
  int32_t m;            /* hidden width, a multiple of 8 (bf16) or 4 (fp32)     */
  int32_t dtype;        /* of every row                                         */
  int32_t act;          /* ts_gn_act or TS_GN_SWIGLU                            */
  int32_t has_tau;      /* elementwise acts: subtract tau [H, m] (fp32)         */
  float eps;            /* RMSNorm eps (1e-6 in the reference)                  */
} ts_gn_act_desc;

/* h, and when their pointers are set sa (and sb for SwiGLU); rows [B,H,T,m]
 * with 16-byte aligned rows; b only for SwiGLU. */
int ts_gn_act_fwd(const ts_gn_act_desc* desc, ts_strided a, ts_strided b, const float* tau, ts_strided h,
                  ts_strided sa, ts_strided sb, hipStream_t stream);

/* Backward of ts_gn_act_fwd: da (and db) from dh, dsa, dsb (a null pointer
 * reads as zeros); dz, when set, receives dz = d(a ra - tau) per row, whose
 * negated token sum is dtau. */
int ts_gn_act_bwd(const ts_gn_act_desc* desc, ts_strided a, ts_strided b, const float* tau, ts_strided dh,
                  ts_strided dsa, ts_strided dsb, ts_strided da, ts_strided db, ts_strided dz, hipStream_t stream);

/* ------------------------------------------------------ B-spline features */

/* Projected open-uniform B-spline feature map
 * (src/thetascan/_core/ops/kernel_features.py:138-230):
 *   c = clamp(scale_h * pre[b,h,t,p], -bound, nextafter(bound, -inf))
 *   out[b,h,t, p*n_basis + j] = N_j(c) / sum_i N_i(c) / P
 * N_j are the n_basis Cox-de Boor functions of `degree` on the clamped knot
 * vector (degree+1 copies of -bound and of +bound around n_basis-degree-1
 * uniform interior knots).  n_basis <= 32, degree <= 7.  scale_h is an fp32
 * [H] array (learned per-head scale) or NULL for the constant `scale`. */
typedef struct ts_bspline_desc {
  int32_t B, H, T, P;   /* pre [B,H,T,P]; out [B,H,T,P*n_basis]               */
  int32_t n_basis, degree;
  int32_t dtype;        /* of pre, out, dout and dpre                          */
  float bound;
  float scale;          /* used when scale_h is NULL                           */
} ts_bspline_desc;

int ts_bspline_fwd(const ts_bspline_desc* desc, ts_strided pre, const float* scale_h, ts_strided out,
                   hipStream_t stream);

/* Number of fp32 partial sums per head that ts_bspline_bwd writes to
 * dscale_part ([H][nparts]; their sum over the last axis is dL/dscale_h). */
int ts_bspline_parts(const ts_bspline_desc* desc, int32_t* nparts);

/* dpre = (d out / d pre)^T dout, and when scale_h is set the partial sums of
 * (d out / d scale_h)^T dout.  Differentiates the clamp, the recursion, the
 * clamp at zero and the renormalisation exactly as written above. */
int ts_bspline_bwd(const ts_bspline_desc* desc, ts_strided pre, const float* scale_h, ts_strided dout,
                   ts_strided dpre, float* dscale_part, hipStream_t stream);

/* The same map of z = rmsnorm(a) + shift, where a [B,H,T,P] is the raw W1
 * product (the RMS over each token's P projections, eps inside the root, as
 * the reference's RMSNorm) and shift an fp32 [H, P] array (minus the learned
 * threshold; NULL: none).  P is a power of two up to 64.  Replaces the
 * RMSNorm and threshold of engine.py:117-158 around kernel_features.py:208-230
 * for a projected B-spline memory. */
int ts_bspline_norm_fwd(const ts_bspline_desc* desc, ts_strided a, const float* shift, float eps,
                        const float* scale_h, ts_strided out, hipStream_t stream);

/* Backward of ts_bspline_norm_fwd: da, the scale partials as ts_bspline_bwd,
 * and fp32 partial sums of dL/dshift [H][nparts][P] (nparts from
 * ts_bspline_parts; NULL: not wanted). */
int ts_bspline_norm_bwd(const ts_bspline_desc* desc, ts_strided a, const float* shift, float eps,
                        const float* scale_h, ts_strided dout, ts_strided da, float* dscale_part,
                        float* dshift_part, hipStream_t stream);

/* ------------------------------------------------------------ bank blend */

/* Temporal-bank blend of n_in (<= 8) read views (block.py:667-718):
 *   y[b,h,t,:] = sum_i coef[i*H + h] * in_i[b,h,t,:]
 * Fast bank:  coef = (1 - sum_j eta_j, eta_1 .. eta_J) over (R_0, R_1 .. R_J);
 * stale bank: coef = (1, -eta_1 .. -eta_J, sum_j eta_j) over
 * (R_0, R_stale_1 .. R_stale_J, R_null). */
typedef struct ts_blend_desc {
  int32_t B, H, T, d;
  int32_t n_in;
  int32_t dtype;        /* of every input, y, dy and din                       */
} ts_blend_desc;

int ts_blend_fwd(const ts_blend_desc* desc, const ts_strided* in, const float* coef, ts_strided y,
                 hipStream_t stream);

/* ts_blend_fwd followed by the output gate (block.py:721-722, gates.py:34-40):
 *   y = (sum_i coef[i*H + h] * in_i) * silu(g + g_bias)
 * with g the gate's pre-activation x W_g^T as a [B,H,T,d] view (of the
 * rows' dtype) and g_bias fp32 [H*d] (NULL: none); g.ptr NULL is
 * ts_blend_fwd.  Forward only (inference): a training step keeps the gate as
 * its own autograd product. */
int ts_blend_gated_fwd(const ts_blend_desc* desc, const ts_strided* in, const float* coef, ts_strided g,
                       const float* g_bias, ts_strided y, hipStream_t stream);

/* Number of fp32 partial sums per (input, head) that ts_blend_bwd writes to
 * dcoef_part ([n_in][H][nparts]). */
int ts_blend_parts(const ts_blend_desc* desc, int32_t* nparts);

/* din_i = coef[i*H + h] * dy (din entries may be NULL to skip an input) and
 * partial sums of dL/dcoef[i*H + h] = sum dy * in_i. */
int ts_blend_bwd(const ts_blend_desc* desc, const ts_strided* in, const float* coef, ts_strided dy,
                 const ts_strided* din, float* dcoef_part, hipStream_t stream);

/* --------------------------------------------------------------- prefixes */

/* Decayed prefix sum along T of an fp32 [B,H,T,F] stream:
 *   z_t = a_t z_{t-1} + x_t   (a = exp(log_alpha[h]) static, or exp(decay[b,h,t]),
 *   or 1 for the plain prefix), optionally anti-causal (reverse).
 * Parallel over time: segments of the time axis scan from a zero state, then
 * each adds the decayed state entering it (two launches).  The workspace
 * (ts_wcumsum_workspace_bytes, 16-byte aligned, no initialisation) holds one
 * state and one decay product per segment.
 * Replaces interface.ema_cumsum / causal_prefix_sum / Accumulator.mass_cum
 * (src/thetascan/_core/ops/interface.py:58-107, 216-230). */
typedef struct ts_wcumsum_desc {
  int32_t B, H, T, F;
  int32_t retention;    /* ts_retention                                        */
  int32_t reverse;
} ts_wcumsum_desc;

int ts_wcumsum_workspace_bytes(const ts_wcumsum_desc* desc, size_t* bytes);

int ts_wcumsum(const ts_wcumsum_desc* desc, ts_strided x, ts_strided out, const float* log_alpha,
               ts_strided decay, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Mass of absolute features: the normalizer num / (mass + eps) of a read whose
 * features can be negative (a tanh GN fast network), so that |num| / mass <=
 * max |value|:
 *   mass_t = sum_j |q_tj| C_tj,   C_t = a_t C_{t-1} + |k_t|   (C_-1 = 0)
 * for q, k [B,H,T,F] (ts_dtype `dtype`, F = 4, 8, 16, ... 256, rows aligned to
 * four features) and the view's retention (as ts_wcumsum: none, static
 * exp(log_alpha[h]) or exp(decay[b,h,t])); mass is fp32 [B,H,T] (element
 * strides in ts_strided, the feature stride unused).  The backward forms
 * dq = dmass sign(q) C and dk = sign(k) R, R the anti-causal decayed prefix of
 * dmass |q| (either output may be NULL).  Neither stores the [B,H,T,F]
 * prefix.  Replaces the composed path's absolute-feature key mass (a torch
 * chain of abs, casts, a decayed prefix, product and row sum); the
 * reference's features are nonnegative, so its unit column
 * (engine.py:440-442) is this mass for them. */
typedef struct ts_abs_mass_desc {
  int32_t B, H, T, F;
  int32_t dtype;        /* of q, k, dq, dk                                     */
  int32_t retention;    /* ts_retention                                        */
} ts_abs_mass_desc;

int ts_abs_mass_workspace_bytes(const ts_abs_mass_desc* desc, size_t* bytes);

int ts_abs_mass_fwd(const ts_abs_mass_desc* desc, ts_strided q, ts_strided k, const float* log_alpha,
                    ts_strided decay, ts_strided mass, void* workspace, size_t workspace_bytes, hipStream_t stream);

int ts_abs_mass_bwd(const ts_abs_mass_desc* desc, ts_strided q, ts_strided k, ts_strided dmass,
                    const float* log_alpha, ts_strided decay, ts_strided dq, ts_strided dk, void* workspace,
                    size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------- row norm of the host LM */

/* RMS-normed rows with an optional half-split rotary turn and per-head gain,
 * for the hybrid language model around the ThetaScan layers (config 5's
 * attention prologue q, k = rotate(rms_norm(q)) * gain and its residual-stream
 * norms, written with F.rms_norm and torch elementwise ops in the upstream
 * training script, which this build does not have):
 *   r = (mean(x^2) + eps)^-1/2,  y = gain[h] * R_t(x r)
 * R_t turns the halves (n1, n2) of a row to (n1 c + n2 s, n2 c - n1 s) with
 * c = cos[t], s = sin[t] (fp32 [T, W/2]) when desc->rope, else is the
 * identity; gain (fp32 [H]) may be NULL.  x is a [B,H,T,W] view (rows 16-byte
 * aligned), y a contiguous [B,H,T,W] tensor of the same dtype, rstd fp32
 * [B*H*T] (kept for the backward).  W = 8, 16, 32, ... 512 (16 or more with
 * the turn).  The backward writes dx (contiguous [B,H,T,W]) and, when dg_row
 * is given, each row's <dy, R_t(x r)> (fp32 [B*H*T]; the gain's gradient is
 * their sum over a head's rows).  fp32 arithmetic, one rounding per output. */
typedef struct ts_rownorm_desc {
  int32_t B, H, T, W;
  int32_t dtype;        /* of x, y, dy, dx                                     */
  int32_t rope;         /* 1: apply the rotary turn                            */
  float eps;
} ts_rownorm_desc;

int ts_rownorm_fwd(const ts_rownorm_desc* desc, ts_strided x, const float* cos, const float* sin,
                   const float* gain, void* y, float* rstd, hipStream_t stream);

int ts_rownorm_bwd(const ts_rownorm_desc* desc, ts_strided x, ts_strided dy, const float* cos, const float* sin,
                   const float* gain, const float* rstd, void* dx, float* dg_row, hipStream_t stream);

/* ------------------------------------------------ host LM row glue */

/* Contiguous [rows, W] tensors of ts_dtype `dtype` (W a multiple of 8, every
 * pointer 16-byte aligned). */
typedef struct ts_rows_desc {
  int64_t rows;
  int32_t W, dtype;
} ts_rows_desc;

/* y = a (.) x + b (.) u with per-column factors a, b [W] of ts_dtype `dtype`
 * (NULL: 1), in fp32 with one rounding: the residual-stream mixes and scaled
 * residual adds
 * of the hybrid language model's blocks (x = mix0 x + mix1 x0 and
 * x + scale (.) f(x), written with torch elementwise ops in the upstream
 * training script, which this build does not have). */
int ts_scale_add_fwd(const ts_rows_desc* desc, const void* x, const void* u, const void* a, const void* b,
                     void* y, hipStream_t stream);

/* Number P of fp32 column-sum partials [P][W] that ts_scale_add_bwd writes
 * (W at most 2048). */
int ts_scale_add_parts(const ts_rows_desc* desc, int32_t* parts);

/* Backward of ts_scale_add_fwd for the output gradient g: dx = a (.) g and
 * du = b (.) g (NULL: not wanted), and partials [P][W] of the column sums
 * sum_rows g (.) x (da_part) and g (.) u (db_part) (NULL: not wanted), whose
 * sum over P (ts_sum_slots) is the gradient of a and of b. */
int ts_scale_add_bwd(const ts_rows_desc* desc, const void* g, const void* x, const void* u, const void* a,
                     const void* b, void* dx, void* du, float* da_part, float* db_part, hipStream_t stream);

/* h = relu(z)^2 and its backward dz = 2 relu(z) g: the MLP activation of the
 * hybrid language model's blocks (relu(fc(x)).square()). */
int ts_relu2_fwd(const ts_rows_desc* desc, const void* z, void* h, hipStream_t stream);
int ts_relu2_bwd(const ts_rows_desc* desc, const void* z, const void* g, void* dz, hipStream_t stream);

/* Softcapped cross entropy of the host LM's logits z [rows, W] (W at most
 * 512, or a multiple of 512 up to 4096) against int64 targets in [0, W):
 *   c = cap tanh(z / cap),  lse_r = log sum_j exp(c_rj),  loss_r = lse_r - c_r,target
 * (fp32 loss and lse [rows]; a target outside [0, W) gives a NaN loss and
 * gradient row); the backward writes
 *   dz = g g_scale (softmax(c_r) - onehot(target_r)) (1 - (c / cap)^2)
 * for the scalar gradient *g (device fp32) of sum_r loss_r g_scale (g_scale =
 * 1 / rows for the mean), recomputing c from z and lse.  The logit soft-cap
 * and cross entropy of the upstream training script (torch's tanh and
 * F.cross_entropy over fp32 logits). */
int ts_softcap_xent_fwd(const ts_rows_desc* desc, const void* z, const int64_t* target, float cap, float* loss,
                        float* lse, hipStream_t stream);
int ts_softcap_xent_bwd(const ts_rows_desc* desc, const void* z, const int64_t* target, float cap, const float* lse,
                        const float* g, float g_scale, void* dz, hipStream_t stream);

/* ------------------------------------------ stacked projection gradient */

/* dst[b, t, s, h, :] = src[s][b, h, t, :] for s < n (1 <= n <= 4); a source
 * whose ptr is NULL contributes zeros.  dst is a contiguous [B, T, n, H, d]
 * tensor of ts_dtype `dtype`; each source is a [B,H,T,d] view (unit feature
 * stride) whose rows and base are 16-byte aligned.  This is the backward of
 * the split of a stacked q/k/v projection (block.py:593-594: one GEMM for the
 * three streams): the three stream gradients gathered into the layout that
 * the projection's input- and weight-gradient GEMMs read, in one pass. */
typedef struct ts_stack_desc {
  int32_t B, H, T, d, n;
  int32_t dtype;
} ts_stack_desc;

int ts_stack_heads(const ts_stack_desc* desc, const ts_strided* src, void* dst, hipStream_t stream);

/* out[i] = scale * (sum_{s<na} a[s*n + i] + sum_{s<nb} b[s*n + i]) for i < n,
 * written as ts_dtype out_dtype: sums the partial weight-gradient slots of
 * one or two ts_feature_bwd calls (keys and queries) into the gradient of W1,
 * W2 or tau.  With ts_feature_bwd it replaces the autograd reductions of the
 * weight gradients of engine.py:117-158 (summed over every token). */
int ts_sum_slots(const float* a, int32_t na, const float* b, int32_t nb, int64_t n, void* out,
                 int32_t out_dtype, float scale, hipStream_t stream);

/* parts[s][c] = sum of x[r * row_stride + c] over the rows r of slice s
 * (rows split into `slices` equal runs), for a [rows, cols] matrix of
 * ts_dtype `dtype` with cols (at most 2048) and row_stride multiples of 8
 * and a 16-byte aligned base.  Followed by ts_sum_slots it is the bias gradient of the
 * output-gate projection (gates.py:34-40, summed over every token). */
int ts_col_sums(const void* x, int32_t dtype, int64_t rows, int32_t cols, int64_t row_stride, float* parts,
                int32_t slices, hipStream_t stream);

/* ------------------------------------------------- token contractions */

typedef struct ts_contract_desc {
  int32_t G, N;         /* groups (heads) and tokens                           */
  int32_t p, q;         /* widths of a and b (multiples of 16, at most 128)    */
  int32_t dtype;        /* of a and b                                          */
} ts_contract_desc;

/* Bytes of the fp32 partials ts_contract_tokens needs as its workspace. */
int ts_contract_workspace_bytes(const ts_contract_desc* desc, size_t* bytes);

/* out[g] = sum_n a[g, n, :]^T b[g, n, :] as fp32 [G, p, q], for token-major
 * tiles a[g, n, i] at a + g * a_sg + n * a_sn + i (and b alike).  The weight
 * gradients of the GN fast network (dW1, dW2) contracted over every token
 * (the autograd reductions of engine.py:117-158, 180-255). */
int ts_contract_tokens(const ts_contract_desc* desc, const void* a, int64_t a_sg, int64_t a_sn, const void* b,
                       int64_t b_sg, int64_t b_sn, float* out, void* workspace, size_t ws_bytes,
                       hipStream_t stream);

/* ------------------------------------------------ depth-1 kernel memory */

/* Everything between the input and the output projection of a depth-1
 * kernel-memory mixer, forward and backward, each as one call (the host
 * submits one call instead of four to eight):
 *   phi_k = feature(k);  phi_q, resid = feature(q)          ts_feature_fwd x2
 *   num [, mass] = scan(phi_q, phi_k, v [, ones])            ts_scan_fwd
 *   y = (resid + s num / (mass + eps)) * silu(g + g_bias)    ts_read_fwd
 * and the backward ts_read_bwd -> three scans -> ts_feature_bwd x2 -> slot
 * sums (weight gradients of W1, W2, tau and the gate bias).  Replaces
 * block.py:593-724 between proj_qkv and proj_out (block.py:598-599 q/k/v
 * split, gates.py:34-40 the gate) and engine.py:260-544 for a depth-1
 * kernel memory with a plain temporal sum.  Shapes whose feature backward has
 * no fused weight-gradient kernel, or whose weights are too wide to stage
 * in LDS, are reported as TS_ERR_NOT_IMPLEMENTED by ts_memory_bytes. */
typedef struct ts_memory_desc {
  ts_feature_desc feat;  /* B, H, T, head width d, feature width m, dtype, map */
  int32_t normalize;     /* key-mass read (the scan's value-side ones column)  */
  int32_t gate;          /* output gate g                                       */
  int32_t has_g_bias;    /* gate bias (gate only)                               */
  int32_t seg_chunks;    /* scan segments (0 = auto)                            */
  int32_t param_dtype;   /* ts_dtype of tau and g_bias as given, and of the
                            weight gradients written by ts_memory_bwd          */
} ts_memory_desc;

typedef struct ts_memory_io {
  ts_strided q, k, v, g;  /* [B,H,T,d] views of the input projection (desc dtype;
                             g NULL without gate)                              */
  const void* w1;         /* [H,m,d] effective W1 (desc dtype)                 */
  const void* w2;         /* [H,d,m] effective W2 (desc dtype)                 */
  const void* tau;        /* [H] threshold (param dtype; feat.has_tau)         */
  const void* g_bias;     /* [H*d] gate bias (param dtype; has_g_bias)         */
  const float* in_cos;    /* rope tables as for ts_feature_fwd                 */
  const float* in_sin;
  const float* f_cos;
  const float* f_sin;
} ts_memory_io;

/* Bytes of the `saved` buffer (written by the forward, read by the
 * backward: features, residual, numerator, mass, fp32 parameters and the
 * forward scan's segment states) and of the backward's `scratch` buffer. */
int ts_memory_bytes(const ts_memory_desc* desc, size_t* saved_bytes, size_t* scratch_bytes);

/* Forward: y [B,H,T,d] view (e.g. of [B,T,H*d]). */
int ts_memory_fwd(const ts_memory_desc* desc, const ts_memory_io* io, ts_strided y, void* saved,
                  size_t saved_bytes, hipStream_t stream);

typedef struct ts_memory_grads {
  ts_strided dy;          /* [B,H,T,d] grad of y                               */
  ts_strided dq, dk, dv;  /* out [B,H,T,d] views of the projection's gradient  */
  ts_strided dg;          /* out [B,H,T,d] (gate)                              */
  void* dw1;              /* out [H,m,d] param dtype, or NULL                  */
  void* dw2;              /* out [H,d,m] param dtype, or NULL                  */
  void* dtau;             /* out [H] param dtype, or NULL                      */
  void* dg_bias;          /* out [H*d] param dtype, or NULL; needs dg rows of
                             one [B*T, H*d] matrix (row stride dg.st)          */
} ts_memory_grads;

/* Backward of ts_memory_fwd with the same desc, io and saved buffer. */
int ts_memory_bwd(const ts_memory_desc* desc, const ts_memory_io* io, const ts_memory_grads* grads,
                  const void* saved, size_t saved_bytes, void* scratch, size_t scratch_bytes,
                  hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* THETASCAN_HIP_H */
