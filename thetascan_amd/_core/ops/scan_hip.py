"""The ``hip`` scan backend: chunked linear-attention scans on MI355X.

Same contract as the reference chunk backend
(``src/thetascan/_core/ops/scan_chunk.py:246-358``):

* :func:`linattn_views` ``(q, k, v, retentions, chunk) -> tuple`` scans one
  stream set through several temporal views.  ``None`` is the plain causal
  sum, a ``[H]`` tensor a static per-head log-retention, a ``[B,H,T,1]``
  tensor a per-token log-retention stream.
* :func:`linattn` is the one-view wrapper with the reference's ``decay`` /
  ``log_alpha`` keywords.

Inputs are ``[B,H,T,D]`` (any strides with a contiguous feature axis),
outputs are new tensors in the query dtype.  Everything is differentiable in
``q``, ``k``, ``v`` and the retention.  The arithmetic runs in the HIP kernels
of ``libthetascan_hip.so``; there is no CPU path -- CPU tensors raise.

Chunk semantics.  ``chunk`` is validated exactly like the reference
(``ValueError`` below 1).  The scan is exact for any tiling, so the kernel
always works in its own 64-token tiles; ``chunk`` therefore only changes the
reference's rounding, never the mathematical result.  Retention phases are
formed in fp32 per tile and the carried state is fp32, as the reference's
precision policy requires (``scan_chunk.py:89-99, 301``).

Backward.  The gradients of a causal scan are scans of the same form:

* ``dq = scan(dO, v, k)`` (causal),
* ``dk = scan(v, dO, q)`` and ``dv = scan(k, q, dO)`` (anti-causal),

all with the forward retention.  The key-mass column of the normalized read
(``engine.py:419-442``) rides along as ext columns (ones in ``v``, its
gradient in ``dO``).  Retention gradients follow from
``dL_t = q_t.dq_t - k_t.dk_t`` (gradient with respect to the cumulative log
at t): ``dlog_alpha = sum_t t dL_t`` for a static head retention and the
reverse cumulative sum of ``dL`` for a per-token stream.
"""
from __future__ import annotations

import ctypes

import torch

from ... import _lib
from . import stream
from .dispatch import HipOp

DEFAULT_CHUNK = 512   # reference default (scan_chunk.DEFAULT_CHUNK); validated only
TILE = 64             # the kernel's tile


# ------------------------------------------------------------------ launching

def _vec(dtype: torch.dtype) -> int:
    return 8 if dtype == torch.bfloat16 else 4


def _kernel_view(x: torch.Tensor, width: int | None = None) -> torch.Tensor:
    """Return ``x`` as a kernel-legal [B,H,T,F] view (padding/copying if needed)."""
    vec = _vec(x.dtype)
    feat = x.shape[-1]
    target = -(-feat // vec) * vec if width is None else width
    ok = (
        target == feat
        and x.stride(-1) == 1
        and all(s % vec == 0 for s in x.stride()[:3])
        and x.data_ptr() % 16 == 0
    )
    if ok:
        return x
    out = x.new_zeros(*x.shape[:3], target)
    out[..., :feat] = x
    return out


def _ext_arg(ext):
    """(mode, tensor) for an ext column: None, 'ones' or an fp32 [B,H,T] tensor."""
    if ext is None:
        return _lib.EXT_NONE, None
    if isinstance(ext, str):
        assert ext == "ones"
        return _lib.EXT_ONES, None
    return _lib.EXT_ARRAY, ext.to(torch.float32)


MAX_WIDTH = 128  # widest key / value width one kernel launch handles


def scan_launch(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    retention: int = _lib.RET_NONE,
    log_alpha: torch.Tensor | None = None,
    decay: torch.Tensor | None = None,
    reverse: bool = False,
    q_ext=None,
    k_ext=None,
    v_ext=None,
    out: torch.Tensor | None = None,
    out_mode: int = _lib.OUT_STORE,
    out_scale: float = 1.0,
    want_ext_out: bool = False,
    ext_out: torch.Tensor | None = None,
    want_final: bool = False,
    seg_chunks: int = 0,
    value_split: int = 0,
    workspace: torch.Tensor | None = None,
    states_in: int = 0,
    init_state: torch.Tensor | None = None,
    final_out: torch.Tensor | None = None,
):
    """One scan (several kernel launches when a width exceeds ``MAX_WIDTH``).

    Returns ``(out, ext_out, final_state)`` as :func:`_scan_once`.  The scan
    is linear in each operand, so wide values split into independent value
    chunks and wide keys into key chunks whose results add up.

    ``workspace`` (from :func:`workspace_for`) keeps the segment states of
    this scan after the call; ``states_in`` = 1 (2) reads the states an
    earlier call of the same (swapped) keys and values left there instead of
    recomputing them -- single-launch widths only.  ``final_out`` (fp32, the
    final state's shape) receives the final state; it may be ``init_state``
    itself (an in-place update: every entry is read before the same thread
    writes it).
    """
    dk, dv = q.shape[-1], v.shape[-1]
    if workspace is not None or states_in or init_state is not None or final_out is not None:
        if dk > MAX_WIDTH or dv > MAX_WIDTH:
            raise NotImplementedError("hip scan: kept segment states and initial states need widths up to 128")
    if dk <= MAX_WIDTH and dv <= MAX_WIDTH:
        return _scan_once(q, k, v, retention=retention, log_alpha=log_alpha, decay=decay, reverse=reverse,
                          q_ext=q_ext, k_ext=k_ext, v_ext=v_ext, out=out, out_mode=out_mode, out_scale=out_scale,
                          want_ext_out=want_ext_out, ext_out=ext_out, want_final=want_final,
                          seg_chunks=seg_chunks, value_split=value_split, workspace=workspace,
                          states_in=states_in, init_state=init_state, final_out=final_out)
    if want_final:
        raise NotImplementedError(f"hip scan: final state of widths dk={dk} dv={dv} above {MAX_WIDTH}")
    kw = dict(retention=retention, log_alpha=log_alpha, decay=decay, reverse=reverse, seg_chunks=seg_chunks,
              value_split=value_split)
    B, H, T = q.shape[:3]
    if dv > MAX_WIDTH:
        ext_res = ext_out
        full = out
        if full is None:
            if out_mode == _lib.OUT_ACCUM_F32:
                raise ValueError("accumulating scan needs an output tensor")
            # every value chunk writes its columns of one buffer (the last
            # chunk's padded to the kernel's vector width)
            vec = _vec(q.dtype)
            odt = q.dtype if out_mode == _lib.OUT_STORE else torch.float32
            full = torch.empty(B, H, T, -(-dv // vec) * vec, dtype=odt, device=q.device)
        for i, c0 in enumerate(range(0, dv, MAX_WIDTH)):
            vs = v[..., c0:c0 + MAX_WIDTH]
            o_i = full[..., c0:c0 + vs.shape[-1]] if out is not None else \
                full[..., c0:c0 + -(-vs.shape[-1] // _vec(q.dtype)) * _vec(q.dtype)]
            _, e, _ = scan_launch(q, k, vs, q_ext=q_ext, k_ext=k_ext, v_ext=v_ext if i == 0 else None,
                                  out=o_i, out_mode=out_mode, out_scale=out_scale,
                                  want_ext_out=want_ext_out and i == 0, ext_out=ext_out if i == 0 else None, **kw)
            if i == 0:
                ext_res = e
        return (out if out is not None else full[..., :dv]), ext_res, None
    # dk > MAX_WIDTH: fp32 partial scans over key chunks, the first stored
    # (or accumulated, for an accumulating call), the others accumulated
    target, eacc = (None, None) if out_mode == _lib.OUT_STORE else (out, ext_out)
    if target is None:
        target = torch.empty(B, H, T, -(-dv // _vec(q.dtype)) * _vec(q.dtype), dtype=torch.float32,
                             device=q.device)
    scale = out_scale if out_mode != _lib.OUT_STORE else 1.0
    first_mode = _lib.OUT_ACCUM_F32 if out_mode == _lib.OUT_ACCUM_F32 else _lib.OUT_STORE_F32
    for i, c0 in enumerate(range(0, dk, MAX_WIDTH)):
        first = i == 0
        target, e, _ = _scan_once(q[..., c0:c0 + MAX_WIDTH], k[..., c0:c0 + MAX_WIDTH], v,
                                  q_ext=q_ext if first else None, k_ext=k_ext if first else None, v_ext=v_ext,
                                  out=target, out_mode=first_mode if first else _lib.OUT_ACCUM_F32,
                                  out_scale=scale, want_ext_out=want_ext_out, ext_out=eacc, **kw)
        eacc = e if want_ext_out else None
    if out_mode != _lib.OUT_STORE:
        return (target if out is not None else target[..., :dv]), eacc, None
    result = target[..., :dv].to(q.dtype) if out is None else out.copy_(target[..., : out.shape[-1]])
    return result, eacc, None


def _scan_once(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    retention: int = _lib.RET_NONE,
    log_alpha: torch.Tensor | None = None,
    decay: torch.Tensor | None = None,
    reverse: bool = False,
    q_ext=None,
    k_ext=None,
    v_ext=None,
    out: torch.Tensor | None = None,
    out_mode: int = _lib.OUT_STORE,
    out_scale: float = 1.0,
    want_ext_out: bool = False,
    ext_out: torch.Tensor | None = None,
    want_final: bool = False,
    seg_chunks: int = 0,
    value_split: int = 0,
    workspace: torch.Tensor | None = None,
    states_in: int = 0,
    init_state: torch.Tensor | None = None,
    final_out: torch.Tensor | None = None,
):
    """One kernel launch.  Returns ``(out, ext_out, final_state)``.

    ``out`` is ``[B,H,T,dv]``; ``ext_out`` (fp32 ``[B,H,T]``) is the result
    column of the ``v`` ext column; ``final_state`` is the fp32
    ``[B,H,dk(+1),dv(+1)]`` state after the last token (ext rows/columns
    included when present).
    """
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    lib = _lib.load()
    dtype = q.dtype
    code = _lib.dtype_code(dtype)
    if k.dtype != dtype:
        k = k.to(dtype)
    if v.dtype != dtype:
        v = v.to(dtype)
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    if k.shape[:3] != (B, H, T) or v.shape[:3] != (B, H, T) or k.shape[-1] != dk:
        raise ValueError(f"hip scan: incompatible shapes q{tuple(q.shape)} k{tuple(k.shape)} v{tuple(v.shape)}")
    vec = _vec(dtype)
    dkw = -(-dk // vec) * vec
    dvw = -(-dv // vec) * vec
    qk = _kernel_view(q, dkw)
    kk = _kernel_view(k, dkw)
    vk = _kernel_view(v, dvw)
    qe_mode, qe = _ext_arg(q_ext)
    ke_mode, ke = _ext_arg(k_ext)
    ve_mode, ve = _ext_arg(v_ext)

    fields = (B, H, T, dkw, dvw, code, retention, int(reverse), qe_mode, ke_mode, ve_mode,
              out_mode, float(out_scale), int(seg_chunks), int(want_final), int(value_split), int(states_in),
              int(init_state is not None))
    desc = _lib.ScanDesc(*fields)
    plan = _PLANS.get(fields)
    if plan is None:
        c_dkp, c_dvp, c_nseg = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        _lib.check(lib.ts_scan_layout(ctypes.byref(desc), ctypes.byref(c_dkp), ctypes.byref(c_dvp),
                                      ctypes.byref(c_nseg)), "scan layout")
        c_ws = ctypes.c_size_t()
        _lib.check(lib.ts_scan_workspace_bytes(ctypes.byref(desc), ctypes.byref(c_ws)), "scan workspace")
        if len(_PLANS) > 256:
            _PLANS.clear()
        plan = _PLANS[fields] = (c_dkp.value, c_dvp.value, c_ws.value)
    dk_pad, dv_pad, ws_bytes = plan

    out_dtype = dtype if out_mode == _lib.OUT_STORE else torch.float32
    if out is None:
        if out_mode == _lib.OUT_ACCUM_F32:
            raise ValueError("accumulating scan needs an output tensor")
        out_buf = torch.empty(B, H, T, dvw, dtype=out_dtype, device=q.device)
    else:
        if out.dtype != out_dtype or out.shape[-1] != dvw or out.stride(-1) != 1:
            raise ValueError("hip scan: output buffer does not match the scan")
        out_buf = out
    if want_ext_out and ext_out is None:
        if out_mode == _lib.OUT_ACCUM_F32:
            raise ValueError("accumulating scan needs an ext output tensor")
        ext_out = torch.empty(B, H, T, dtype=torch.float32, device=q.device)
    init = None
    if init_state is not None:
        if tuple(init_state.shape[-2:]) != (dk_pad, dv_pad) or init_state.numel() != B * H * dk_pad * dv_pad:
            raise ValueError(f"hip scan: initial state of shape {tuple(init_state.shape)}, "
                             f"expected [{B}, {H}, {dk_pad}, {dv_pad}]")
        init = init_state.detach().to(device=q.device, dtype=torch.float32).contiguous()
    final = None
    if want_final:
        # every entry of the [dk(+1)][dv(+1)] layout is written except the
        # corner of a key ext row meeting a value ext column
        corner = qe_mode != _lib.EXT_NONE and ke_mode != _lib.EXT_NONE and ve_mode != _lib.EXT_NONE
        if final_out is not None:
            if (final_out.dtype != torch.float32 or not final_out.is_contiguous() or final_out.device != q.device
                    or tuple(final_out.shape[-2:]) != (dk_pad, dv_pad)
                    or final_out.numel() != B * H * dk_pad * dv_pad):
                raise ValueError("hip scan: final_out must be a contiguous fp32 tensor of the final state's shape")
            final = final_out.view(B * H, dk_pad, dv_pad)
            if corner and (init is None or init.data_ptr() != final.data_ptr()):
                final.zero_()
        else:
            final = (torch.zeros if corner else torch.empty)(B * H, dk_pad, dv_pad, dtype=torch.float32,
                                                              device=q.device)
    elif final_out is not None:
        raise ValueError("hip scan: final_out without want_final")
    if workspace is not None:
        if workspace.numel() * workspace.element_size() < ws_bytes:
            raise ValueError("hip scan: workspace too small")
    elif ws_bytes:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)

    la = None
    if retention == _lib.RET_STATIC:
        la = log_alpha.detach().to(device=q.device, dtype=torch.float32).reshape(H).contiguous()
    dec = None
    if retention == _lib.RET_STREAM:
        dec = decay.detach().to(dtype=torch.float32).reshape(B, H, T)

    io = _lib.ScanIO(
        _lib.strided(qk), _lib.strided(kk), _lib.strided(vk),
        _lib.strided(qe), _lib.strided(ke), _lib.strided(ve),
        la.data_ptr() if la is not None else None,
        _lib.strided(dec),
        _lib.strided(out_buf),
        _lib.strided(ext_out if want_ext_out else None),
        final.data_ptr() if final is not None else None,
        init.data_ptr() if init is not None else None,
    )
    def traffic():
        rw = 2 if out_mode == _lib.OUT_ACCUM_F32 else 1
        out_bytes = B * H * T * dv * out_buf.element_size() * rw
        return (_lib.nbytes(q, k, v, qe, ke, ve, dec) + out_bytes
                + (_lib.nbytes(ext_out) * rw if want_ext_out else 0))

    with _lib.timed("ts_scan_fwd", traffic):
        status = lib.ts_scan_fwd(
            ctypes.byref(desc), ctypes.byref(io),
            workspace.data_ptr() if workspace is not None else None,
            ws_bytes, _lib.stream_handle(q.device),
        )
    _lib.check(status, "ts_scan_fwd")
    result = out_buf if out is not None else out_buf[..., :dv]
    if final is not None:
        final = final.view(B, H, dk_pad, dv_pad)
    return result, ext_out, final


_PLANS: dict = {}


def pair_eligible(qa: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qb: torch.Tensor) -> bool:
    """Whether ts_scan_pair_fwd serves scan(qa, k, v) and scan(qb, v, k)."""
    return (qa.is_cuda and all(t.dtype == torch.bfloat16 for t in (qa, k, v, qb))
            and qa.shape[-1] == k.shape[-1] == v.shape[-1] == qb.shape[-1] == 64)


def scan_pair_launch(qa: torch.Tensor, k: torch.Tensor, v: torch.Tensor, qb: torch.Tensor, *, reverse: bool = False,
                     seg_chunks: int = 0, out_a: torch.Tensor | None = None, out_b: torch.Tensor | None = None,
                     k_ext: torch.Tensor | None = None, log_alpha: torch.Tensor | None = None,
                     out_mode: int = _lib.OUT_STORE, out_scale: float = 1.0):
    """scan(qa, k, v) and scan(qb, v, k) (bf16, 64-wide) in one pass over k
    and v; returns ``(out_a, out_b)``, each equal to its own scan_launch.
    ``k_ext`` (fp32 [B,H,T]) gives scan A the key-side ext pair of a
    normalized read's backward: scan_launch(qa, k, v, q_ext="ones", k_ext=k_ext).
    ``log_alpha`` ([H]) is a static retention of both scans; ``out_mode``
    OUT_STORE_F32 / OUT_ACCUM_F32 writes or adds ``out_scale`` x the results
    into fp32 outputs (both given for accumulation)."""
    lib = _lib.load()
    B, H, T, d = qa.shape
    views = [_kernel_view(t, 64) for t in (qa, k, v, qb)]
    odt = qa.dtype if out_mode == _lib.OUT_STORE else torch.float32
    if out_mode == _lib.OUT_ACCUM_F32 and (out_a is None or out_b is None):
        raise ValueError("scan pair: accumulation needs both outputs")
    if out_a is None:
        out_a = torch.empty(B, H, T, 64, dtype=odt, device=qa.device)
    if out_b is None:
        out_b = torch.empty(B, H, T, 64, dtype=odt, device=qa.device)
    if out_a.dtype != odt or out_b.dtype != odt:
        raise ValueError(f"scan pair: outputs must be {odt} for this output mode")
    ke = None if k_ext is None else k_ext.to(torch.float32).contiguous()
    la = None if log_alpha is None else log_alpha.detach().to(device=qa.device, dtype=torch.float32).reshape(H).contiguous()
    desc = _lib.ScanDesc(B, H, T, 64, 64, _lib.dtype_code(qa.dtype), _lib.RET_STATIC if la is not None else _lib.RET_NONE,
                         int(reverse), _lib.EXT_ONES if ke is not None else 0, _lib.EXT_ARRAY if ke is not None else 0, 0,
                         out_mode, float(out_scale), int(seg_chunks), 0, 0, 0, 0)
    c_ws = ctypes.c_size_t()
    _lib.check(lib.ts_scan_workspace_bytes(ctypes.byref(desc), ctypes.byref(c_ws)), "scan workspace")
    workspace = torch.empty(c_ws.value, dtype=torch.uint8, device=qa.device) if c_ws.value else None
    io = _lib.ScanPairIO(*[_lib.strided(t) for t in views], _lib.strided(out_a), _lib.strided(out_b),
                         _lib.strided(ke), la.data_ptr() if la is not None else None)
    with _lib.timed("ts_scan_pair_fwd", lambda: _lib.nbytes(*views, out_a, out_b, ke)):
        status = lib.ts_scan_pair_fwd(ctypes.byref(desc), ctypes.byref(io),
                                      workspace.data_ptr() if workspace is not None else None, c_ws.value,
                                      _lib.stream_handle(qa.device))
    _lib.check(status, "ts_scan_pair_fwd")
    return out_a, out_b


def retention_grad(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dout: torch.Tensor,
                   dmass: torch.Tensor | None, log_alpha: torch.Tensor, seg_tiles: int = 0) -> torch.Tensor:
    """dL/dlog_alpha [B,H] (fp32) of scan(q, k, v) with the static retention
    ``log_alpha`` [H] (and the key-mass column when ``dmass`` is given), summed
    pair by pair by ts_retention_grad; keys wider than 128 and values wider
    than one call split into independent calls whose sums add."""
    lib = _lib.load()
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    la = log_alpha.detach().to(torch.float32).reshape(H).contiguous()
    dm = None if dmass is None else dmass.detach().to(torch.float32).contiguous()
    total = torch.zeros(B, H, dtype=torch.float32, device=q.device)
    dkw = -(-dk // 16) * 16
    qk = [_kernel_view(q, dkw), _kernel_view(k.to(q.dtype), dkw)]
    vwidth = -(-dv // 8) * 8
    vv = _kernel_view(v.to(q.dtype), vwidth)
    do = _kernel_view(dout.to(q.dtype), vwidth)
    for k0 in range(0, dkw, 128):
        qs, ks = qk[0][..., k0:k0 + 128], qk[1][..., k0:k0 + 128]
        first = True
        v0 = 0
        while v0 < vwidth:
            mass = first and dm is not None
            # one wave per 16 value columns, at most eight per call
            blocks = 8
            width = min(vwidth - v0, 16 * (blocks - 1) if mass else 16 * blocks)
            vs, ds = vv[..., v0:v0 + width], do[..., v0:v0 + width]
            desc = _lib.RetentionDesc(B, H, T, qs.shape[-1], width, _lib.dtype_code(q.dtype), int(mass),
                                      int(seg_tiles))
            nbytes = ctypes.c_size_t()
            _lib.check(lib.ts_retention_workspace_bytes(ctypes.byref(desc), ctypes.byref(nbytes)),
                       "ts_retention_workspace_bytes")
            work = torch.empty(nbytes.value, dtype=torch.uint8, device=q.device)
            out = torch.empty(B, H, dtype=torch.float32, device=q.device)
            io = _lib.RetentionIO(_lib.strided(qs), _lib.strided(ks), _lib.strided(vs), _lib.strided(ds),
                                  _lib.strided(dm if mass else None), la.data_ptr())
            with _lib.timed("ts_retention_grad", lambda: _lib.nbytes(qs, ks, vs, ds)):
                status = lib.ts_retention_grad(ctypes.byref(desc), ctypes.byref(io), out.data_ptr(), work.data_ptr(),
                                               nbytes.value, _lib.stream_handle(q.device))
            _lib.check(status, "ts_retention_grad")
            total += out
            first = False
            v0 += width
    return total


def views_eligible(q: torch.Tensor, v: torch.Tensor, kinds) -> bool:
    """Whether ts_scan_views_fwd serves these views (bf16 on the GPU, 2..3
    retentions that are none or static, dk <= 128, dv <= 64)."""
    return (q.is_cuda and q.dtype == torch.bfloat16 and 2 <= len(kinds) <= _lib.MAX_VIEWS
            and all(k in (_lib.RET_NONE, _lib.RET_STATIC) for k in kinds)
            and q.shape[-1] <= 128 and v.shape[-1] <= 64)


def scan_views_launch(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, log_alphas, *, mass: bool,
                      seg_chunks: int = 0):
    """Forward causal scans of the same q, k, v under several retentions in one
    pass (``log_alphas``: a per-head fp32 log-retention, or None for the plain
    sum, per view).  Returns ``(outs, masses)`` (masses None without ``mass``);
    each equals :func:`scan_launch` of that retention bit for bit."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    lib = _lib.load()
    dtype = q.dtype
    k = k.to(dtype)
    v = v.to(dtype)
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    n = len(log_alphas)
    vec = _vec(dtype)
    dkw = -(-dk // vec) * vec
    dvw = -(-dv // vec) * vec
    qk, kk, vk = _kernel_view(q, dkw), _kernel_view(k, dkw), _kernel_view(v, dvw)
    desc = _lib.ScanViewsDesc(B, H, T, dkw, dvw, _lib.dtype_code(dtype), n, int(mass), int(seg_chunks))
    c_ws = ctypes.c_size_t()
    _lib.check(lib.ts_scan_views_workspace_bytes(ctypes.byref(desc), ctypes.byref(c_ws)), "scan views workspace")
    workspace = torch.empty(c_ws.value, dtype=torch.uint8, device=q.device) if c_ws.value else None
    outs = [torch.empty(B, H, T, dvw, dtype=dtype, device=q.device) for _ in range(n)]
    masses = [torch.empty(B, H, T, dtype=torch.float32, device=q.device) for _ in range(n)] if mass else None
    las = [None if la is None else la.detach().to(device=q.device, dtype=torch.float32).reshape(H).contiguous()
           for la in log_alphas]
    io = _lib.ScanViewsIO()
    io.q, io.k, io.v = _lib.strided(qk), _lib.strided(kk), _lib.strided(vk)
    for j in range(n):
        io.log_alpha[j] = las[j].data_ptr() if las[j] is not None else None
        io.out[j] = _lib.strided(outs[j])
        io.out_ext[j] = _lib.strided(masses[j] if mass else None)

    def traffic():
        return _lib.nbytes(q, k, v) + n * B * H * T * (dv * outs[0].element_size() + (4 if mass else 0))

    with _lib.timed("ts_scan_views_fwd", traffic):
        status = lib.ts_scan_views_fwd(ctypes.byref(desc), ctypes.byref(io),
                                       workspace.data_ptr() if workspace is not None else None, c_ws.value,
                                       _lib.stream_handle(q.device))
    _lib.check(status, "ts_scan_views_fwd")
    return [o[..., :dv] for o in outs], masses


def workspace_for(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, seg_chunks: int = 0,
                  retention: int = _lib.RET_NONE, reverse: bool = False, v_ext: bool = False,
                  kx: bool = False) -> torch.Tensor | None:
    """A workspace that keeps the segment states of ``scan_launch(q, k, v, ...)``
    for a later call with ``states_in`` (None when the scan has one segment).
    ``v_ext`` / ``kx`` describe the scan's value-side / key-side ext columns."""
    B, H, T, dk = q.shape
    nbytes = workspace_bytes(B, H, T, dk, v.shape[-1], q.dtype, seg_chunks=seg_chunks, retention=retention,
                             reverse=reverse, v_ext=v_ext, kx=kx)
    if not nbytes:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=q.device)


def workspace_bytes(B: int, H: int, T: int, dk: int, dv: int, dtype: torch.dtype, *, seg_chunks: int = 0,
                    retention: int = _lib.RET_NONE, reverse: bool = False, v_ext: bool = False,
                    kx: bool = False) -> int:
    """Bytes of the segment-state workspace of such a scan (a host query)."""
    lib = _lib.load()
    vec = _vec(dtype)
    ext = _lib.EXT_ONES
    desc = _lib.ScanDesc(B, H, T, -(-dk // vec) * vec, -(-dv // vec) * vec, _lib.dtype_code(dtype), retention,
                         int(reverse), ext if kx else 0, ext if kx else 0, ext if v_ext else 0, _lib.OUT_STORE, 1.0,
                         int(seg_chunks), 0, 0, 0)
    c_ws = ctypes.c_size_t()
    _lib.check(lib.ts_scan_workspace_bytes(ctypes.byref(desc), ctypes.byref(c_ws)), "scan workspace")
    return c_ws.value


# ------------------------------------------------------------------ retentions

def _classify(retention, q: torch.Tensor):
    """Validate one retention exactly like the reference (scan_chunk.py:277-291)."""
    heads = q.shape[1]
    if retention is None:
        return _lib.RET_NONE
    if retention.ndim == 4:
        if retention.shape[-1] != 1:
            raise NotImplementedError("chunk backend: scalar decay only (v1)")
        return _lib.RET_STREAM
    if retention.numel() != heads:
        raise ValueError(
            "chunk backend: a static retention needs one entry per head, "
            f"got {tuple(retention.shape)} for q {tuple(q.shape)}"
        )
    return _lib.RET_STATIC


def _ret_kwargs(kind: int, retention):
    if kind == _lib.RET_STATIC:
        return {"retention": kind, "log_alpha": retention}
    if kind == _lib.RET_STREAM:
        return {"retention": kind, "decay": retention}
    return {"retention": kind}


def _retention_grad(kind: int, retention: torch.Tensor, dL: torch.Tensor) -> torch.Tensor:
    """Gradient of a retention from dL[B,H,T] = q.dq - k.dk (per view).

    The sums cancel heavily (sum_t dL_t = 0), so they accumulate in float64."""
    dL = dL.double()
    if kind == _lib.RET_STATIC:
        t = torch.arange(dL.shape[2], device=dL.device, dtype=torch.float64)
        grad = (dL * t).sum(dim=(0, 2))
        return grad.to(retention.dtype).view_as(retention)
    # d a_j = sum_{t>=j} dL_t for j >= 1; position 0 never multiplies a stored term.
    grad = dL.flip(-1).cumsum(-1).flip(-1)
    grad[..., 0] = 0.0
    return grad.unsqueeze(-1).to(retention.dtype)


# ------------------------------------------------------------------ autograd

def _view_groups(n: int) -> list[range]:
    """Consecutive groups of at most MAX_VIEWS retentions, as even as possible
    (5 -> 3 + 2): one multi-view pass each."""
    count = -(-n // _lib.MAX_VIEWS)
    bounds = [n * i // count for i in range(count + 1)]
    return [range(a, b) for a, b in zip(bounds, bounds[1:])]


def _views_forward(q, k, v, with_mass: bool, retentions):
    """Forward scans of every retention -> (outs, masses)."""
    kinds = [_classify(r, q) for r in retentions]
    if len(kinds) >= 2 and views_eligible(q, v, kinds[:2]) and all(
            kd in (_lib.RET_NONE, _lib.RET_STATIC) for kd in kinds):
        # one pass per group of retentions: the score tile is formed once per
        # group (a bank of four rates and the plain sum: two passes)
        outs, masses = [], []
        for group in _view_groups(len(kinds)):
            if len(group) == 1:
                j = group[0]
                out, mass, _ = scan_launch(q, k, v, **_ret_kwargs(kinds[j], retentions[j]),
                                           v_ext="ones" if with_mass else None, want_ext_out=with_mass)
                outs.append(out)
                masses.extend([mass] if with_mass else [])
                continue
            g_outs, g_masses = scan_views_launch(q, k, v, [retentions[j] if kinds[j] == _lib.RET_STATIC else None
                                                           for j in group], mass=with_mass)
            outs.extend(g_outs)
            masses.extend(g_masses or [])
        return outs, masses
    outs, masses = [], []
    for kind, r in zip(kinds, retentions):
        out, mass, _ = scan_launch(q, k, v, **_ret_kwargs(kind, r), v_ext="ones" if with_mass else None,
                                   want_ext_out=with_mass)
        outs.append(out)
        if with_mass:
            masses.append(mass)
    return outs, masses


def _views_backward(q, k, v, retentions, d_outs, d_mass, need_q: bool, need_k: bool, need_v: bool, need_r):
    """Backward of :func:`_views_forward`: three scans per view (None entries
    of ``d_outs`` / ``d_mass`` are zero gradients) -> (gq, gk, gv, r_grads)."""
    n = len(retentions)
    kinds = [_classify(r, q) for r in retentions]
    B, H, T, dk = q.shape
    dv = v.shape[-1]
    if n == 1 and not (retentions[0] is not None and need_r[0]) and (d_outs[0] is not None or d_mass[0] is not None):
        # one view and no retention gradient: each gradient is one scan,
        # stored in the input dtype (the same single rounding as an fp32
        # accumulation cast at the end)
        kind, r = kinds[0], retentions[0]
        dO, dm = d_outs[0], d_mass[0]
        if dO is None:
            dO = torch.zeros(B, H, T, dv, dtype=q.dtype, device=q.device)
        dO = dO.to(q.dtype)
        rk = _ret_kwargs(kind, r)
        q_ext = None if dm is None else dm.to(torch.float32)
        gq = gk = gv = None
        if need_q:
            gq = scan_launch(dO, v, k, **rk, q_ext=q_ext, k_ext="ones" if dm is not None else None)[0][..., :dk]
        if need_k:
            gk = scan_launch(v, dO, q, **rk, reverse=True, q_ext="ones" if dm is not None else None,
                             k_ext=q_ext)[0][..., :dk]
        if need_v:
            gv = scan_launch(k, q, dO, **rk, reverse=True)[0][..., :dv]
        return gq, gk, gv, [None]
    # the first scan into each fp32 gradient stores, later ones accumulate;
    # a gradient no scan wrote is zeroed at the end
    dq = torch.empty(B, H, T, -(-dk // _vec(q.dtype)) * _vec(q.dtype), dtype=torch.float32, device=q.device)
    dkk = torch.empty_like(dq)
    dvv = torch.empty(B, H, T, -(-dv // _vec(q.dtype)) * _vec(q.dtype), dtype=torch.float32, device=q.device)
    written = {"q": False, "k": False, "v": False}

    def mode(name):
        m = _lib.OUT_ACCUM_F32 if written[name] else _lib.OUT_STORE_F32
        written[name] = True
        return m

    r_grads = []
    for j in range(n):
        kind, r = kinds[j], retentions[j]
        dO = d_outs[j]
        dm = d_mass[j]
        if dO is None and dm is None:
            r_grads.append(None)
            continue
        if dO is None:
            dO = torch.zeros(B, H, T, dv, dtype=q.dtype, device=q.device)
        dO = dO.to(q.dtype)
        rk = _ret_kwargs(kind, r)
        mass_ext = dm is not None
        q_ext = dm.to(torch.float32) if mass_ext else None
        want_r = r is not None and need_r[j]
        # a bf16 static retention's gradient is summed pair by pair
        # (ts_retention_grad: no cancellation); the other retention gradients
        # come from fp32 scans
        pairwise = want_r and kind == _lib.RET_STATIC and q.dtype == torch.bfloat16
        if want_r and not pairwise:
            # dL_t = q_t.dq_t - k_t.dk_t sums to zero over t, and the
            # retention gradient (sum_t t dL_t, or a suffix sum of dL) is a
            # small difference of large terms: bf16 rounding of the score
            # tiles inside the scans would be amplified by about T / (the
            # retention's window).  These two scans therefore run on fp32
            # operands (the bf16 values are exact in fp32).
            qs, ks, vs, dOs = q, k, v, dO
            if q.dtype != torch.float32:
                qs, ks, vs, dOs = q.float(), k.float(), v.float(), dO.float()
            dq_j, _, _ = scan_launch(dOs, vs, ks, **rk, q_ext=q_ext, k_ext="ones" if mass_ext else None,
                                     out_mode=_lib.OUT_STORE_F32)
            dk_j, _, _ = scan_launch(vs, dOs, qs, **rk, reverse=True, q_ext="ones" if mass_ext else None,
                                     k_ext=q_ext, out_mode=_lib.OUT_STORE_F32)
            dL = (qs * dq_j[..., :dk]).sum(-1) - (ks * dk_j[..., :dk]).sum(-1)
            r_grads.append(_retention_grad(kind, r, dL))
            for name, buf, part in (("q", dq, dq_j), ("k", dkk, dk_j)):
                if written[name]:
                    buf[..., : part.shape[-1]] += part
                else:
                    buf.zero_()[..., : part.shape[-1]] = part
                    written[name] = True
        else:
            r_grads.append(retention_grad(q, k, v, dO, dm, r).sum(0).to(r.dtype).view_as(r) if pairwise else None)
            if need_q:
                scan_launch(dO, v, k, **rk, q_ext=q_ext, k_ext="ones" if mass_ext else None,
                            out=dq, out_mode=mode("q"))
            if need_k and need_v and kind in (_lib.RET_NONE, _lib.RET_STATIC) and pair_eligible(v, dO, q, k) \
                    and written["k"] == written["v"]:
                # dk and dv share keys dO and values q: one pass over both
                m = mode("k")
                mode("v")
                scan_pair_launch(v, dO, q, k, reverse=True, k_ext=q_ext, out_a=dkk, out_b=dvv,
                                 log_alpha=r if kind == _lib.RET_STATIC else None, out_mode=m)
                continue
            if need_k:
                scan_launch(v, dO, q, **rk, reverse=True, q_ext="ones" if mass_ext else None,
                            k_ext=q_ext, out=dkk, out_mode=mode("k"))
        if need_v:
            scan_launch(k, q, dO, **rk, reverse=True, out=dvv, out_mode=mode("v"))
    for name, buf in (("q", dq), ("k", dkk), ("v", dvv)):
        if not written[name]:
            buf.zero_()
    gq = dq[..., :dk].to(q.dtype) if need_q else None
    gk = dkk[..., :dk].to(k.dtype) if need_k else None
    gv = dvv[..., :dv].to(v.dtype) if need_v else None
    return gq, gk, gv, r_grads


# The scan as an autograd node (dispatch.HipOp: a torch.library custom op
# under torch.compile, an autograd.Function in eager mode).  Absent retentions
# and absent gradients travel as empty placeholders.

def _placeholder(like: torch.Tensor) -> torch.Tensor:
    return like.new_empty(0)


def _or_none(t: torch.Tensor):
    return None if t.numel() == 0 and t.ndim == 1 else t


def _scan_views_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rets: list[torch.Tensor],
                        with_mass: bool) -> list[torch.Tensor]:
    outs, masses = _views_forward(q, k, v, with_mass, [_or_none(r) for r in rets])
    return outs + masses


def _scan_views_fake(q, k, v, rets, with_mass):
    B, H, T = q.shape[:3]
    outs = [q.new_empty(B, H, T, v.shape[-1]) for _ in rets]
    masses = [q.new_empty(B, H, T, dtype=torch.float32) for _ in rets] if with_mass else []
    return outs + masses


def _scan_views_backward_impl(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rets: list[torch.Tensor],
                              d_outs: list[torch.Tensor], d_mass: list[torch.Tensor], need: list[bool]
                              ) -> list[torch.Tensor]:
    retentions = [_or_none(r) for r in rets]
    gq, gk, gv, r_grads = _views_backward(q, k, v, retentions, [_or_none(g) for g in d_outs],
                                          [_or_none(g) for g in d_mass], need[0], need[1], need[2], need[3:])
    grads = [gq, gk, gv] + list(r_grads) + [None] * (len(rets) - len(r_grads))
    like = [q, k, v] + list(rets)
    return [_placeholder(x) if g is None else g for g, x in zip(grads, like)]


def _scan_views_backward_fake(q, k, v, rets, d_outs, d_mass, need):
    like = [q, k, v] + list(rets)
    return [torch.empty_like(x) if (w and _or_none(x) is not None) else _placeholder(x) for x, w in zip(like, need)]


def _scan_views_setup(ctx, inputs, output):
    q, k, v, rets, with_mass = inputs
    ctx.with_mass = with_mass
    ctx.need = [q.requires_grad, k.requires_grad, v.requires_grad] + [r.requires_grad for r in rets]
    ctx.save_for_backward(q, k, v, *rets)


def _scan_views_backward(ctx, grads, bwd):
    q, k, v, *rets = ctx.saved_tensors
    n = len(rets)
    d_outs = [_placeholder(q) if g is None else g for g in grads[:n]]
    d_mass = [_placeholder(q) if g is None else g for g in grads[n:]] if ctx.with_mass else \
        [_placeholder(q) for _ in range(n)]
    res = bwd(q, k, v, list(rets), d_outs, d_mass, ctx.need)
    out = [None if not w else _or_none(g) for g, w in zip(res, ctx.need)]
    return out[0], out[1], out[2], out[3:], None


_scan_views_op = HipOp("scan_views", forward=_scan_views_forward, forward_fake=_scan_views_fake,
                       backward_impl=_scan_views_backward_impl, backward_fake=_scan_views_backward_fake,
                       setup=_scan_views_setup, backward=_scan_views_backward)


def _carried_scan(q, k, v, kind, r, with_mass: bool, init):
    """One forward scan that starts from ``init`` (a list of fp32 state
    blocks, None: zero) and returns ``(out, mass, blocks)``.  Keys and values
    wider than one launch split into blocks of at most MAX_WIDTH columns; each
    block of the state N [dk, dv] (the mass column rides with the first value
    block) is carried by its own launch, and the outputs of key blocks add."""
    dk, dv = q.shape[-1], v.shape[-1]
    kcols = list(range(0, dk, MAX_WIDTH))
    vcols = list(range(0, dv, MAX_WIDTH))
    blocks = init if init is not None else [None] * (len(kcols) * len(vcols))
    if len(blocks) != len(kcols) * len(vcols):
        raise ValueError("streaming state does not match this scan's widths")
    rk = _ret_kwargs(kind, r)
    in_place = stream.updates_in_place()
    if len(blocks) == 1:
        out, mass, fin = scan_launch(q, k, v, **rk, v_ext="ones" if with_mass else None, want_ext_out=with_mass,
                                     want_final=True, init_state=blocks[0],
                                     final_out=blocks[0] if in_place else None)
        return out, mass, [fin]
    acc = torch.zeros(*q.shape[:3], dv, dtype=torch.float32, device=q.device)
    mass = torch.zeros(q.shape[:3], dtype=torch.float32, device=q.device) if with_mass else None
    finals = []
    i = 0
    for k0 in kcols:
        qs, ks = q[..., k0:k0 + MAX_WIDTH], k[..., k0:k0 + MAX_WIDTH]
        for j, v0 in enumerate(vcols):
            ext = with_mass and j == 0
            o, e, fin = scan_launch(qs, ks, v[..., v0:v0 + MAX_WIDTH], **rk, v_ext="ones" if ext else None,
                                    want_ext_out=ext, want_final=True, init_state=blocks[i],
                                    final_out=blocks[i] if in_place else None)
            acc[..., v0:v0 + o.shape[-1]] += o.float()
            if ext:
                mass += e
            finals.append(fin)
            i += 1
    return acc.to(q.dtype), mass, finals


def _views_carried(q, k, v, retentions, with_mass: bool, out_f32: bool, carry) -> list:
    """The forward scans of every retention continued from ``carry``."""
    if out_f32 and q.dtype != torch.float32:
        q, k, v = q.float(), k.float(), v.float()
    outs, masses = [], []
    for r in retentions:
        out, mass, finals = _carried_scan(q, k, v, _classify(r, q), r, with_mass, carry.take())
        carry.put(finals)
        outs.append(out)
        if with_mass:
            masses.append(mass)
    return outs + masses


def _run_views(q, k, v, retentions, chunk, with_mass, out_f32=False):
    if chunk < 1:
        raise ValueError("chunk backend: chunk must be >= 1")
    if not retentions:
        return ()
    for r in retentions:
        _classify(r, q)
    carry = stream.active()
    if carry is not None:
        return _views_carried(q, k, v, tuple(retentions), with_mass, out_f32, carry)
    if out_f32 and q.dtype != torch.float32:
        # A caller that subtracts views (a stale view is plain - fast, nearly
        # equal over recent tokens) gets scans on fp32 operands, forward and
        # backward: bf16 rounding inside each scan would be amplified by the
        # cancellation.  The bf16 values are exact in fp32; autograd casts the
        # gradients back.
        q, k, v = q.float(), k.float(), v.float()
    rets = [_placeholder(q) if r is None else r for r in retentions]
    return _scan_views_op(q, k, v, rets, bool(with_mass))


def linattn_views(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    retentions: tuple,
    chunk: int = DEFAULT_CHUNK,
    *,
    out_f32: bool = False,
) -> tuple:
    """Scan one stream set through several temporal views (scan_chunk.py:246-339).

    ``out_f32`` scans fp32 copies of the operands and returns fp32 outputs (for
    callers that combine views by subtraction); otherwise outputs are in the
    query dtype."""
    return tuple(_run_views(q, k, v, tuple(retentions), chunk, False, out_f32))


def linattn_views_mass(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    retentions: tuple,
    chunk: int = DEFAULT_CHUNK,
    *,
    out_f32: bool = False,
) -> tuple:
    """Like :func:`linattn_views` with an implicit unit value column.

    Returns ``((num_0, mass_0), (num_1, mass_1), ...)`` where ``mass`` is the
    fp32 ``[B,H,T]`` result of the unit column -- the same numbers the
    reference obtains from ``cat([v, ones])`` (``engine.py:430``), without
    materialising the augmented tensor.
    """
    res = _run_views(q, k, v, tuple(retentions), chunk, True, out_f32)
    n = len(retentions)
    return tuple((res[j], res[n + j]) for j in range(n))


def linattn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    decay: torch.Tensor | None = None,
    chunk: int = DEFAULT_CHUNK,
    log_alpha: torch.Tensor | None = None,
) -> torch.Tensor:
    """Inclusive causal scan (scan_chunk.py:342-358); ``log_alpha`` wins over ``decay``."""
    retention = log_alpha if log_alpha is not None else decay
    return linattn_views(q, k, v, (retention,), chunk)[0]


def final_state(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    retention=None,
    with_mass: bool = False,
) -> torch.Tensor:
    """fp32 state after the last token: ``N_T = sum_i w(T-1,i) k_i v_i^T``.

    With ``with_mass`` the last column is the key mass ``D_T = sum_i w k_i``.
    Shape ``[B,H,dk,dv(+1)]``.  Not differentiable (a streaming-decode cache).
    """
    kind = _classify(retention, q)
    _, _, fin = scan_launch(
        q.detach(), k.detach(), v.detach(), **_ret_kwargs(kind, retention),
        v_ext="ones" if with_mass else None, want_final=True,
    )
    dk = k.shape[-1]
    dv = v.shape[-1]
    vec = _vec(q.dtype)
    dvw = -(-dv // vec) * vec
    state = fin[:, :, :dk, :dv]
    if with_mass:
        state = torch.cat([state, fin[:, :, :dk, dvw:dvw + 1]], dim=-1)
    return state


def linattn_state(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, retention=None, state=None, *,
                  mass: bool = False):
    """Continue a causal scan from a carried state (forward only, for streaming).

    ``state`` is the fp32 ``[B, H, dk(+1), dv(+1)]`` state after the tokens
    already seen (None: a fresh sequence); ``retention`` is None, a static
    ``[H]`` log-retention or a per-token ``[B, H, T, 1]`` one for these tokens.
    With ``mass`` the value stream carries the unit column of the key-mass read
    (its row sums come back as ``mass`` and its column rides in the state).
    Returns ``(out, mass or None, new_state)``; feeding the pieces of a
    sequence through this in order gives exactly the scan of the whole
    sequence (``scan_naive.py:5-18``: S_t = a_t S_{t-1} + k_t v_t^T), so a
    decode step is a call with T = 1.
    """
    kind = _classify(retention, q)
    with torch.no_grad():
        out, ext, final = scan_launch(q, k, v, **_ret_kwargs(kind, retention), v_ext="ones" if mass else None,
                                      want_ext_out=mass, want_final=True, init_state=state)
    return out, ext, final

