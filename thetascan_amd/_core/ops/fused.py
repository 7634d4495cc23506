"""Fused HIP hot path of the kernel-family mixer (write -> scan -> read).

``kernel_mixer`` is one autograd node (a pair of torch.library custom ops)
covering a depth-1 kernel-memory mixer: the stacked qkv / output-gate
projection GEMM, then

    phi_k = feature(k)                 ts_feature_fwd   (keys)
    phi_q, resid = feature(q)          ts_feature_fwd   (queries, + W2 base)
    num, mass = scan(phi_q, phi_k, v)  ts_scan_fwd      (key-mass column)
    y = (resid + s*num/(mass+eps)) * silu(g)            ts_read_fwd

with q, k, v and the gate logits g read from that one projection, then the
output projection; and its backward (ts_read_bwd -> three scans -> ts_feature_bwd, then plain
GEMMs for the W1/W2 gradients).  Reference chain:
src/thetascan/_core/modules/block.py:593-724 and
src/thetascan/_core/ops/engine.py:260-544 for a depth-1 kernel memory.
"""
from __future__ import annotations

import ctypes
import math
import threading

import torch

from ... import _lib
from .dispatch import HipOp, eager_forward
from . import scan_hip, stream
from .linear import slot_sum, split_k_outer, weight_grad


_INV: dict = {}


def _rope_tables(T: int, rot: int, base: float, device, start=0) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin [T, rot/2] of positions start .. start+T-1 (rope.py:7-38
    phases, kept in fp32).  ``start`` may be an int64 device tensor (a
    captured decode step): the positions are the same exact fp32 integers."""
    if isinstance(start, torch.Tensor):
        # kept for the life of the process: a captured step reads them in place
        key = (rot, float(base), str(device))
        inv = _INV.get(key)
        if inv is None:
            inv = _INV[key] = 1.0 / (base ** (torch.arange(0, rot, 2, device=device, dtype=torch.float32) / rot))
        akey = ("offsets", T, str(device))
        offsets = _INV.get(akey)
        if offsets is None:
            offsets = _INV[akey] = torch.arange(T, device=device, dtype=torch.float32)
        # one launch: fp32 integers below 2^24 are exact, so these are the
        # values (start + arange(T)).float() would give
        pos = offsets + start
    else:
        inv = 1.0 / (base ** (torch.arange(0, rot, 2, device=device, dtype=torch.float32) / rot))
        pos = torch.arange(start, start + T, device=device, dtype=torch.float32)
    f = torch.outer(pos, inv)
    return f.cos().contiguous(), f.sin().contiguous()


_TABLES: dict = {}
# Continued sequences (decode steps) read their rows from tables of whole
# blocks of positions; rows of a block equal the directly formed ones bit for
# bit while positions are exact fp32 integers (below 2^24).
POSITION_BLOCK = 1024


def rope_tables(T: int, rot: int, base: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    """The tables of the current call's positions: 0 .. T-1, or, while a
    sequence is continued, from the number of tokens already seen."""
    dev_pos = stream.device_position()
    if dev_pos is not None:
        # a captured decode step: rows formed on the device once per call
        memo = stream.active().memo
        key = ("rope", T, rot, float(base), str(device))
        if key not in memo:
            memo[key] = _rope_tables(T, rot, base, device, dev_pos)
        return memo[key]
    start = stream.position()
    if start:
        b0 = start - start % POSITION_BLOCK
        if start + T > b0 + POSITION_BLOCK or b0 + POSITION_BLOCK > 1 << 24:
            return _rope_tables(T, rot, base, device, start)
        key = ("block", b0, rot, float(base), str(device))
        hit = _TABLES.get(key)
        if hit is None:
            if len(_TABLES) > 64:
                _TABLES.clear()
            hit = _TABLES[key] = _rope_tables(POSITION_BLOCK, rot, base, device, b0)
        return hit[0][start - b0:start - b0 + T], hit[1][start - b0:start - b0 + T]
    key = (T, rot, float(base), str(device))
    hit = _TABLES.get(key)
    if hit is None:
        if len(_TABLES) > 64:
            _TABLES.clear()
        hit = _TABLES[key] = _rope_tables(T, rot, base, device)
    return hit


class FeatureSpec:
    """Static description of one fused feature map."""

    def __init__(self, kind: int, m: int, gain: float, in_rot: int, feat_rot: int, rope_base: float,
                 resid_scale: float, eps: float = 1e-6):
        self.kind, self.m, self.gain = kind, m, gain
        self.in_rot, self.feat_rot, self.rope_base = in_rot, feat_rot, rope_base
        self.resid_scale, self.eps = resid_scale, eps

    def desc(self, x: torch.Tensor, has_tau: bool) -> _lib.FeatureDesc:
        B, H, T, d = x.shape
        return _lib.FeatureDesc(B, H, T, d, self.m, _lib.dtype_code(x.dtype), self.kind, self.in_rot,
                                self.feat_rot, int(has_tau), float(self.gain), float(self.resid_scale),
                                float(self.eps))

    def tables(self, T: int, device):
        ic = is_ = fc = fs = None
        if self.in_rot:
            ic, is_ = rope_tables(T, self.in_rot, self.rope_base, device)
        if self.feat_rot:
            fc, fs = rope_tables(T, self.feat_rot, self.rope_base, device)
        return ic, is_, fc, fs


def feature_fwd(spec: FeatureSpec, x, w1, w2, tau, want_resid: bool):
    lib = _lib.load()
    B, H, T, d = x.shape
    phi = torch.empty(B, H, T, spec.m, dtype=x.dtype, device=x.device)
    resid = torch.empty(B, H, T, d, dtype=x.dtype, device=x.device) if want_resid else None
    ic, is_, fc, fs = spec.tables(T, x.device)
    io = _lib.FeatureIO(_lib.strided(x), _lib.ptr(w1), _lib.ptr(w2), _lib.ptr(tau), _lib.ptr(ic),
                        _lib.ptr(is_), _lib.ptr(fc), _lib.ptr(fs), _lib.strided(phi), _lib.strided(resid))
    desc = spec.desc(x, tau is not None)
    with _lib.timed("ts_feature_fwd", lambda: _lib.nbytes(x, phi, resid)):
        status = lib.ts_feature_fwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(x.device))
    _lib.check(status, "ts_feature_fwd")
    return phi, resid


def summary_eligible(spec: FeatureSpec, x: torch.Tensor, ws) -> bool:
    """Whether a key feature forward also writes the segment summaries of the
    memory's forward scan (:func:`feature_fwd_summary`): bf16, d = m = 64 and
    a scan with kept segment states.  The one-call forward uses the same rule,
    so both paths compute the summaries in the same kernel."""
    return ws is not None and x.dtype == torch.bfloat16 and x.shape[-1] == 64 and spec.m == 64


def feature_fwd_summary(spec: FeatureSpec, x, w1, tau, v, normalize: bool, seg_chunks: int, ws):
    """Key features phi(x) that also write, into ``ws``, the segment summaries
    of the plain scan ``sum_i <q_t, phi_i> v_i`` (with its ones column when
    ``normalize``): a following :func:`scan_hip.scan_launch` with
    ``states_in=3`` and the same workspace skips its summary pass."""
    lib = _lib.load()
    B, H, T, d = x.shape
    phi = torch.empty(B, H, T, spec.m, dtype=x.dtype, device=x.device)
    ic, is_, fc, fs = spec.tables(T, x.device)
    io = _lib.FeatureIO(_lib.strided(x), _lib.ptr(w1), None, _lib.ptr(tau), _lib.ptr(ic), _lib.ptr(is_),
                        _lib.ptr(fc), _lib.ptr(fs), _lib.strided(phi), _lib.strided(None))
    desc = spec.desc(x, tau is not None)
    sdesc = _lib.ScanDesc(B, H, T, spec.m, v.shape[-1], _lib.dtype_code(x.dtype), _lib.RET_NONE, 0, 0, 0,
                          _lib.EXT_ONES if normalize else 0, _lib.OUT_STORE, 1.0, int(seg_chunks), 0, 0, 3, 0)
    with _lib.timed("ts_feature_fwd", lambda: _lib.nbytes(x, phi, v)):
        status = lib.ts_feature_fwd_summary(ctypes.byref(desc), ctypes.byref(io), _lib.strided(v),
                                            ctypes.byref(sdesc), ws.data_ptr(), ws.numel(),
                                            _lib.stream_handle(x.device))
    _lib.check(status, "ts_feature_fwd_summary")
    return phi


def _head_major(B, H, T, w, dtype, device):
    """[B,H,T,w] view of a head-major [H,B*T,w] buffer (GEMM-ready for weight grads)."""
    buf = torch.empty(H, B, T, w, dtype=dtype, device=device)
    return buf.transpose(0, 1), buf.view(H, B * T, w)


class Slots:
    """Partial weight-gradient slots [P, ...] (fp32) written by one fused backward."""

    def __init__(self, parts: torch.Tensor):
        self.parts = parts


def feature_bwd(spec: FeatureSpec, x, w1, tau, dphi, dresid, dx, w2=None, want_weights=True, w1t=None, w2t=None):
    """Backward of one stream; dx is written in place.

    Returns ``(dw1 [H,m,d], dw2 [H,d,m], dtau [H])`` -- this stream's
    contributions to the gradients of W1, W2 (queries only) and the threshold
    tau, each a :class:`Slots` of per-workgroup partial sums contracted inside
    the kernel (sum them with :func:`sum_grads`), or, for shapes without a
    fused kernel, an fp32 tensor from per-token tiles and split-K GEMMs
    (None where not applicable or not wanted).  ``w1t`` / ``w2t`` are the
    [H,d,m] / [H,m,d] transposes; they are only formed when the weights are too
    large for the kernel to transpose while staging them in LDS.
    """
    lib = _lib.load()
    B, H, T, d = x.shape
    m = spec.m
    dev = x.device
    desc = spec.desc(x, tau is not None)
    key = (B, H, T, d, m, x.dtype, spec.kind, dresid is not None, bool(want_weights))
    plan = _PARTS.get(key)
    if plan is None:
        parts, needed = ctypes.c_int32(0), ctypes.c_int32(1)
        if want_weights:
            _lib.check(lib.ts_feature_bwd_parts(ctypes.byref(desc), int(dresid is not None), ctypes.byref(parts)),
                       "ts_feature_bwd_parts")
        _lib.check(lib.ts_feature_bwd_transposed(ctypes.byref(desc), int(dresid is not None),
                                                 int(parts.value > 0), ctypes.byref(needed)),
                   "ts_feature_bwd_transposed")
        plan = _PARTS[key] = (parts.value, bool(needed.value))
    P, need_t = plan
    if need_t:
        if w1t is None:
            w1t = w1.transpose(1, 2).contiguous()
        if dresid is not None and w2t is None:
            w2t = w2.transpose(1, 2).contiguous()
    da = xn = h = da_v = xn_v = h_v = dtau_tok = None
    dw1p = dw2p = dtaup = None
    if want_weights and P > 0:
        dw1p = torch.empty(P, H, m, d, dtype=torch.float32, device=dev)
        if dresid is not None:
            dw2p = torch.empty(P, H, d, m, dtype=torch.float32, device=dev)
        if tau is not None:
            dtaup = torch.empty(P, H, dtype=torch.float32, device=dev)
    elif want_weights:
        da_v, da = _head_major(B, H, T, m, x.dtype, dev)
        xn_v, xn = _head_major(B, H, T, d, x.dtype, dev)
        if dresid is not None:
            h_v, h = _head_major(B, H, T, m, x.dtype, dev)
        if tau is not None:
            dtau_tok = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    ic, is_, fc, fs = spec.tables(T, dev)
    io = _lib.FeatureBwdIO(
        _lib.strided(x), _lib.ptr(w1), _lib.ptr(w1t), _lib.ptr(w2t), _lib.ptr(tau), _lib.ptr(ic),
        _lib.ptr(is_), _lib.ptr(fc), _lib.ptr(fs), _lib.strided(dphi), _lib.strided(dresid),
        _lib.strided(dx), _lib.strided(da_v), _lib.strided(xn_v), _lib.strided(h_v), _lib.strided(dtau_tok),
        _lib.ptr(dw1p), _lib.ptr(dw2p), _lib.ptr(dtaup), _lib.ptr(w2 if dresid is not None else None),
    )
    with _lib.timed("ts_feature_bwd", lambda: _lib.nbytes(x, dphi, dresid, dx, da, xn, h, dtau_tok, dw1p, dw2p,
                                                          dtaup)):
        status = lib.ts_feature_bwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(dev))
    _lib.check(status, "ts_feature_bwd")
    if not want_weights:
        return None, None, None
    if P > 0:
        return Slots(dw1p), None if dw2p is None else Slots(dw2p), None if dtaup is None else Slots(dtaup)
    dw1 = split_k_outer(da, xn)
    dw2 = None if h is None else split_k_outer(_head_major_of(dresid), h) * spec.resid_scale
    dtau = None if dtau_tok is None else dtau_tok.sum(dim=(0, 2))
    return dw1, dw2, dtau


_PARTS: dict = {}


def sum_grads(a, b, dtype: torch.dtype, shape):
    """Gradient of ``shape`` in ``dtype`` from one or two stream contributions
    (:class:`Slots` are summed by one ts_sum_slots launch)."""
    items = [x for x in (a, b) if x is not None]
    if not items:
        return None
    if all(isinstance(x, Slots) for x in items) and dtype in (torch.bfloat16, torch.float32):
        lib = _lib.load()
        first = items[0].parts
        n = first[0].numel()
        second = items[1].parts if len(items) > 1 else None
        out = torch.empty(shape, dtype=dtype, device=first.device)
        _lib.check(lib.ts_sum_slots(first.data_ptr(), first.shape[0], _lib.ptr(second),
                                    0 if second is None else second.shape[0], n, out.data_ptr(),
                                    _lib.dtype_code(dtype), 1.0, _lib.stream_handle(first.device)),
                   "ts_sum_slots")
        return out
    total = None
    for x in items:
        val = x.parts.sum(0) if isinstance(x, Slots) else x
        total = val if total is None else total + val
    return total.view(shape).to(dtype)


def _head_major_of(t: torch.Tensor) -> torch.Tensor:
    """[H, B*T, w] view (or copy) of a [B,H,T,w] tensor."""
    B, H, T, w = t.shape
    hm = t.transpose(0, 1)
    if not hm.is_contiguous():
        hm = hm.contiguous()
    return hm.view(H, B * T, w)


def read_fwd(num, mass, resid, g, y, scale: float, eps: float = 1e-6, gbias=None):
    lib = _lib.load()
    B, H, T, d = num.shape
    desc = _lib.ReadDesc(B, H, T, d, _lib.dtype_code(num.dtype), int(mass is not None), int(g is not None),
                         float(scale), float(eps))
    io = _lib.ReadIO(_lib.strided(num), _lib.strided(mass), _lib.strided(resid), _lib.strided(g),
                     _lib.strided(y), _lib.ptr(gbias))
    with _lib.timed("ts_read_fwd", lambda: _lib.nbytes(num, mass, resid, g, y)):
        status = lib.ts_read_fwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(num.device))
    _lib.check(status, "ts_read_fwd")
    return y


def read_bwd(num, mass, resid, g, dy, scale: float, eps: float = 1e-6, dg=None, gbias=None, gbias_grad=None):
    """Backward of :func:`read_fwd`; ``dg`` optionally names the [B,H,T,d]
    view the gate gradient is written to.  With ``gbias_grad`` (a dtype) the
    gate-bias gradient [H*d] is also formed, from per-workgroup column sums
    the kernel writes beside dg.

    Returns ``(dnum, dmass, (dresid, dresid_head_major), dg, dgbias)``."""
    lib = _lib.load()
    B, H, T, d = num.shape
    dnum = torch.empty_like(num)
    dmass = torch.empty(B, H, T, dtype=torch.float32, device=num.device) if mass is not None else None
    dresid, dresid_hm = _head_major(B, H, T, d, num.dtype, num.device)
    if g is not None and dg is None:
        dg = torch.empty(B, T, H, d, dtype=num.dtype, device=num.device).transpose(1, 2)
    desc = _lib.ReadDesc(B, H, T, d, _lib.dtype_code(num.dtype), int(mass is not None), int(g is not None),
                         float(scale), float(eps))
    parts = None
    if gbias_grad is not None and g is not None:
        n = ctypes.c_int32()
        _lib.check(lib.ts_read_bwd_parts(ctypes.byref(desc), ctypes.byref(n)), "ts_read_bwd_parts")
        parts = torch.empty(n.value, H * d, dtype=torch.float32, device=num.device)
    io = _lib.ReadBwdIO(_lib.strided(num), _lib.strided(mass), _lib.strided(resid), _lib.strided(g),
                        _lib.strided(dy), _lib.strided(dnum), _lib.strided(dmass), _lib.strided(dresid),
                        _lib.strided(dg), _lib.ptr(gbias), _lib.ptr(parts))
    with _lib.timed("ts_read_bwd", lambda: _lib.nbytes(num, mass, resid, g, dy, dnum, dmass, dresid, dg)):
        status = lib.ts_read_bwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(num.device))
    _lib.check(status, "ts_read_bwd")
    dgbias = None if parts is None else slot_sum(parts, gbias_grad, (H * d,))
    return dnum, dmass, (dresid, dresid_hm), dg, dgbias


def _read_out_desc(num, mass, g, n: int, scale: float, eps: float) -> _lib.ReadOutDesc:
    B, H, T, d = num.shape
    return _lib.ReadOutDesc(_lib.ReadDesc(B, H, T, d, _lib.dtype_code(num.dtype), int(mass is not None),
                                          int(g is not None), float(scale), float(eps)), int(n))


_READ_OUT_OK: dict = {}


def read_out_supported(B: int, H: int, T: int, d: int, n: int, dtype: torch.dtype) -> bool:
    """Whether ts_read_out_fwd / ts_read_out_bwd take this shape (a host query)."""
    key = (B, H, T, d, n, dtype)
    hit = _READ_OUT_OK.get(key)
    if hit is None:
        if dtype != torch.bfloat16:
            hit = False
        else:
            desc = _lib.ReadOutDesc(_lib.ReadDesc(B, H, T, d, _lib.TS_BF16, 0, 0, 1.0, 1e-6), int(n))
            hit = _lib.load().ts_read_out_bwd_parts(ctypes.byref(desc), None) == _lib.TS_OK
        if len(_READ_OUT_OK) > 256:
            _READ_OUT_OK.clear()
        _READ_OUT_OK[key] = hit
    return hit


def read_out_fwd(num, mass, resid, g, w_out, out, y, scale: float, eps: float = 1e-6, gbias=None):
    """``out`` [B*T, N] = read(num, mass, resid, g) @ w_out^T, the read
    formed in the GEMM's prologue; ``y`` [B*T, H*d] (or None) receives the
    read output for the weight gradient."""
    lib = _lib.load()
    n = w_out.shape[0]
    desc = _read_out_desc(num, mass, g, n, scale, eps)
    io = _lib.ReadOutIO(_lib.strided(num), _lib.strided(mass), _lib.strided(resid), _lib.strided(g),
                        _lib.ptr(gbias), w_out.data_ptr(), out.data_ptr(), out.stride(0),
                        _lib.ptr(y), 0 if y is None else y.stride(0))
    with _lib.timed("ts_read_out_fwd", lambda: _lib.nbytes(num, mass, resid, g, out, y)):
        status = lib.ts_read_out_fwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(num.device))
    _lib.check(status, "ts_read_out_fwd")
    return out


def read_out_bwd(num, mass, resid, g, w_out_t, dout, scale: float, eps: float = 1e-6, dg=None, gbias=None,
                 gbias_grad=None):
    """Backward of :func:`read_out_fwd` except the weight gradient: ``dout``
    [B*T, N] times the weight (``w_out_t`` = its [H*d, N] transpose) feeds
    the read backward in registers.  Returns what :func:`read_bwd` returns."""
    lib = _lib.load()
    B, H, T, d = num.shape
    n = dout.shape[-1]
    dnum = torch.empty_like(num)
    dmass = torch.empty(B, H, T, dtype=torch.float32, device=num.device) if mass is not None else None
    dresid, dresid_hm = _head_major(B, H, T, d, num.dtype, num.device)
    if g is not None and dg is None:
        dg = torch.empty(B, T, H, d, dtype=num.dtype, device=num.device).transpose(1, 2)
    desc = _read_out_desc(num, mass, g, n, scale, eps)
    parts = None
    if gbias_grad is not None and g is not None:
        cnt = ctypes.c_int32()
        _lib.check(lib.ts_read_out_bwd_parts(ctypes.byref(desc), ctypes.byref(cnt)), "ts_read_out_bwd_parts")
        parts = torch.empty(cnt.value, H * d, dtype=torch.float32, device=num.device)
    io = _lib.ReadOutBwdIO(_lib.strided(num), _lib.strided(mass), _lib.strided(resid), _lib.strided(g),
                           _lib.ptr(gbias), w_out_t.data_ptr(), dout.data_ptr(), dout.stride(0),
                           _lib.strided(dnum), _lib.strided(dmass), _lib.strided(dresid), _lib.strided(dg),
                           _lib.ptr(parts))
    with _lib.timed("ts_read_out_bwd", lambda: _lib.nbytes(num, mass, resid, g, dout, dnum, dmass, dresid, dg)):
        status = lib.ts_read_out_bwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(num.device))
    _lib.check(status, "ts_read_out_bwd")
    dgbias = None if parts is None else slot_sum(parts, gbias_grad, (H * d,))
    return dnum, dmass, (dresid, dresid_hm), dg, dgbias


def wcumsum(x: torch.Tensor, retention=None, reverse: bool = False) -> torch.Tensor:
    """Decayed prefix sum along T of a [B,H,T,F] stream (fp32 result).

    ``retention`` is None (plain prefix), a static [H] log-retention or a
    [B,H,T,1] per-token log-retention stream.
    """
    if not x.is_cuda:
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    lib = _lib.load()
    xf = x.to(torch.float32)
    if xf.stride(-1) != 1:
        xf = xf.contiguous()
    B, H, T, F = xf.shape
    out = torch.empty(B, H, T, F, dtype=torch.float32, device=x.device)
    kind, la, dec = _lib.RET_NONE, None, None
    if retention is not None:
        if retention.ndim == 4:
            kind = _lib.RET_STREAM
            dec = retention.detach().to(torch.float32).reshape(B, H, T)
        else:
            kind = _lib.RET_STATIC
            la = retention.detach().to(torch.float32).reshape(H).contiguous()
    desc = _lib.WcumsumDesc(B, H, T, F, kind, int(reverse))
    nbytes = ctypes.c_size_t()
    _lib.check(lib.ts_wcumsum_workspace_bytes(ctypes.byref(desc), ctypes.byref(nbytes)), "ts_wcumsum_workspace_bytes")
    work = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device=x.device)
    with _lib.timed("ts_wcumsum", lambda: _lib.nbytes(xf, out, dec)):
        status = lib.ts_wcumsum(ctypes.byref(desc), _lib.strided(xf), _lib.strided(out), _lib.ptr(la),
                                _lib.strided(dec), work.data_ptr(), nbytes.value, _lib.stream_handle(x.device))
    _lib.check(status, "ts_wcumsum")
    return out


def _retention_args(retention, B: int, H: int, T: int):
    """(ts_retention, static log-retention [H] or None, per-token log-retention [B,H,T] or None)."""
    if retention is None:
        return _lib.RET_NONE, None, None
    if retention.ndim == 4:
        return _lib.RET_STREAM, None, retention.detach().to(torch.float32).reshape(B, H, T)
    return _lib.RET_STATIC, retention.detach().to(torch.float32).reshape(H).contiguous(), None


def abs_mass_eligible(q: torch.Tensor, k: torch.Tensor, retention=None) -> bool:
    """Whether ts_abs_mass takes these features: the same dtype (bf16 / fp32)
    on the GPU, F = 4, 8, ... 256, and a retention that needs no gradient."""
    F = q.shape[-1]
    return (q.is_cuda and q.ndim == 4 and k.shape == q.shape and q.dtype == k.dtype
            and q.dtype in (torch.bfloat16, torch.float32) and F % 4 == 0 and (F // 4) & (F // 4 - 1) == 0
            and F // 4 <= 64 and (retention is None or not retention.requires_grad))


def _am_rows(t: torch.Tensor) -> torch.Tensor:
    ok = t.stride(-1) == 1 and t.data_ptr() % (4 * t.element_size()) == 0 and all(s % 4 == 0 for s in t.stride()[:3])
    return t if ok else t.contiguous()


def _am_desc(q, retention):
    B, H, T, F = q.shape
    kind, la, dec = _retention_args(retention, B, H, T)
    desc = _lib.AbsMassDesc(B, H, T, F, _lib.dtype_code(q.dtype), kind)
    lib = _lib.load()
    nbytes = ctypes.c_size_t()
    _lib.check(lib.ts_abs_mass_workspace_bytes(ctypes.byref(desc), ctypes.byref(nbytes)), "ts_abs_mass_workspace_bytes")
    work = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device=q.device)
    return lib, desc, la, dec, work, nbytes.value


def _abs_mass_forward(q: torch.Tensor, k: torch.Tensor, retention: torch.Tensor | None) -> torch.Tensor:
    q4, k4 = _am_rows(q), _am_rows(k)
    B, H, T, F = q4.shape
    lib, desc, la, dec, work, nb = _am_desc(q4, retention)
    mass = torch.empty(B, H, T, dtype=torch.float32, device=q.device)
    with _lib.timed("ts_abs_mass_fwd", lambda: _lib.nbytes(q4, k4, mass)):
        status = lib.ts_abs_mass_fwd(ctypes.byref(desc), _lib.strided(q4), _lib.strided(k4), _lib.ptr(la),
                                     _lib.strided(dec), _lib.strided(mass), work.data_ptr(), nb,
                                     _lib.stream_handle(q.device))
    _lib.check(status, "ts_abs_mass_fwd")
    return mass


def _abs_mass_fake(q, k, retention):
    return q.new_empty(q.shape[:3], dtype=torch.float32)


def _abs_mass_backward_impl(dmass: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                            retention: torch.Tensor | None) -> list[torch.Tensor]:
    q4, k4 = _am_rows(q), _am_rows(k)
    lib, desc, la, dec, work, nb = _am_desc(q4, retention)
    dm = dmass.to(torch.float32).contiguous()
    dq = torch.empty(q4.shape, dtype=q.dtype, device=q.device)
    dk = torch.empty(k4.shape, dtype=k.dtype, device=k.device)
    with _lib.timed("ts_abs_mass_bwd", lambda: _lib.nbytes(q4, k4, dm, dm, q4, k4, dq, dk)):
        status = lib.ts_abs_mass_bwd(ctypes.byref(desc), _lib.strided(q4), _lib.strided(k4), _lib.strided(dm),
                                     _lib.ptr(la), _lib.strided(dec), _lib.strided(dq), _lib.strided(dk),
                                     work.data_ptr(), nb, _lib.stream_handle(q.device))
    _lib.check(status, "ts_abs_mass_bwd")
    return [dq, dk]


def _abs_mass_backward_fake(dmass, q, k, retention):
    return [q.new_empty(q.shape), k.new_empty(k.shape)]


def _abs_mass_setup(ctx, inputs, output):
    q, k, retention = inputs
    ctx.save_for_backward(q, k, retention)


def _abs_mass_backward(ctx, dmass, bwd):
    q, k, retention = ctx.saved_tensors
    dq, dk = bwd(dmass, q, k, retention)
    return dq, dk, None


_abs_mass_op = HipOp("abs_mass", forward=_abs_mass_forward, forward_fake=_abs_mass_fake,
                     backward_impl=_abs_mass_backward_impl, backward_fake=_abs_mass_backward_fake,
                     setup=_abs_mass_setup, backward=_abs_mass_backward)


def abs_mass(q: torch.Tensor, k: torch.Tensor, retention=None) -> torch.Tensor:
    """mass_t = sum_j |q_tj| C_tj with C the decayed prefix of |k| along T
    (``retention``: None, a static [H] or a per-token [B,H,T,1] log-retention;
    it receives no gradient): fp32 [B,H,T], one ts_abs_mass_fwd call, and
    ts_abs_mass_bwd for dq and dk."""
    if not q.is_cuda:
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    return _abs_mass_op(q, k, None if retention is None else retention.detach())


def _stacked(w_qkv, w_g):
    """[W_qkv; W_g] (rebuilt every call: parameters may change in place in ways
    no version counter records, e.g. through ``.data``)."""
    return torch.cat([w_qkv.detach(), w_g.detach().to(w_qkv.dtype)], dim=0)


class _State:
    """What the kernel-memory backward needs from its forward.  The tensors of
    ``SAVED`` travel between the forward and backward ops; everything else is
    rebuilt from the op inputs (:func:`_restore`)."""

    SAVED = ("saved", "ws", "phi_q", "phi_k", "num", "mass", "resid")
    __slots__ = ("spec", "normalize", "seg_chunks", "heads", "d", "has_gate", "has_tau", "tau_dtype", "w_dtypes",
                 "b_dtype", "ws", "proj", "w1c", "w2c", "tauf", "gb", "phi_q", "phi_k", "num", "mass", "resid",
                 "native", "io", "saved", "tau", "b_g", "tables")


_MEMORY: dict = {}


def _memory_plan(spec: FeatureSpec, B, H, T, d, dtype, tau, b_g, w1, w2, normalize, has_gate, seg_chunks):
    """(desc, saved bytes, scratch bytes) of the one-call kernel memory
    (ts_memory_fwd / ts_memory_bwd), or None where it does not apply (a host
    query: no device work)."""
    pdt = w1.dtype
    if pdt not in (torch.bfloat16, torch.float32) or w2.dtype != pdt:
        return None
    if tau is not None and (tau.dtype != pdt or tau.numel() != H):
        return None
    if b_g is not None and (b_g.dtype != pdt or b_g.numel() != H * d):
        return None
    key = (B, H, T, d, spec.m, dtype, spec.kind, spec.in_rot, spec.feat_rot, spec.gain, spec.resid_scale, spec.eps,
           tau is not None, b_g is not None, bool(normalize), bool(has_gate), int(seg_chunks), pdt)
    hit = _MEMORY.get(key)
    if hit is None:
        lib = _lib.load()
        feat = _lib.FeatureDesc(B, H, T, d, spec.m, _lib.dtype_code(dtype), spec.kind, spec.in_rot, spec.feat_rot,
                                int(tau is not None), float(spec.gain), float(spec.resid_scale), float(spec.eps))
        desc = _lib.MemoryDesc(feat, int(normalize), int(has_gate), int(b_g is not None), int(seg_chunks),
                               _lib.dtype_code(pdt))
        sb, cb = ctypes.c_size_t(), ctypes.c_size_t()
        status = lib.ts_memory_bytes(ctypes.byref(desc), ctypes.byref(sb), ctypes.byref(cb))
        if status == _lib.TS_ERR_NOT_IMPLEMENTED:
            hit = False
        else:
            _lib.check(status, "ts_memory_bytes")
            hit = (desc, sb.value, cb.value)
        if len(_MEMORY) > 64:
            _MEMORY.clear()
        _MEMORY[key] = hit
    return hit or None


def _use_native(proj, tau, b_g) -> bool:
    """The one-call path runs unless launches are recorded per entry point or a
    parameter is not a contiguous vector."""
    return (not _lib.recording() and proj.is_contiguous() and (tau is None or tau.is_contiguous())
            and (b_g is None or b_g.is_contiguous()))


def _proj_view(base: int, es: int, col: int, T: int, P: int, d: int) -> _lib.Strided:
    """[B,H,T,d] view at column ``col`` of a [B,T,P] buffer at address ``base``."""
    return _lib.Strided(base + col * es, T * P, d, P)


def _split_proj(proj, H: int, d: int, has_gate: bool):
    """q, k, v (and the gate logits) as [B,H,T,d] views of the projection."""
    B, T, P = proj.shape
    qkv = proj[..., :3 * H * d].view(B, T, 3, H, d)
    gv = proj[..., 3 * H * d:].view(B, T, H, d).transpose(1, 2) if has_gate else None
    return qkv[:, :, 0].transpose(1, 2), qkv[:, :, 1].transpose(1, 2), qkv[:, :, 2].transpose(1, 2), gv


def _memory_forward(st: _State, proj, w1, w2, tau, b_g, spec: FeatureSpec, normalize: bool, seg_chunks: int,
                    heads: int, has_gate: bool):
    """Forward of the depth-1 kernel memory; fills ``st`` for the backward."""
    B, T, P = proj.shape
    H = heads
    d = P // (4 * H) if has_gate else P // (3 * H)
    _describe(st, proj, w1, w2, tau, b_g, spec, normalize, seg_chunks, H, d, has_gate)
    if _use_native(proj, tau, b_g):
        plan = _memory_plan(spec, B, H, T, d, proj.dtype, tau, b_g, w1, w2, normalize, has_gate, seg_chunks)
        if plan is not None:
            return _native_forward(st, plan, proj, w1, w2, tau, b_g, spec, H, d, has_gate)
    q, k, v, gv = _split_proj(proj, H, d, has_gate)
    dt = proj.dtype
    _weights_for(st, proj, w1, w2, tau, b_g)
    # The dq scan's segment states are the transpose of this scan's
    # (sum_i v_i phi_k_i^T; with the mass column its key-side row is this
    # scan's value-side sum_i phi_k_i), so the forward keeps them.
    ws = None
    if spec.m == d:
        ws = scan_hip.workspace_for(k, k, v, seg_chunks=seg_chunks, v_ext=normalize)
    summ = summary_eligible(spec, k, ws)
    if summ:
        phi_k = feature_fwd_summary(spec, k, st.w1c, st.tauf, v, normalize, seg_chunks, ws)
    else:
        phi_k, _ = feature_fwd(spec, k, st.w1c, None, st.tauf, False)
    phi_q, resid = feature_fwd(spec, q, st.w1c, st.w2c, st.tauf, True)
    num, mass, _ = scan_hip.scan_launch(
        phi_q, phi_k, v, v_ext="ones" if normalize else None, want_ext_out=normalize,
        seg_chunks=seg_chunks, workspace=ws, states_in=3 if summ else 0,
    )
    y = torch.empty(B, T, H, d, dtype=dt, device=proj.device)
    read_fwd(num, mass, resid, gv, y.transpose(1, 2), spec.resid_scale, spec.eps, gbias=st.gb)
    st.ws, st.phi_q, st.phi_k, st.num, st.mass, st.resid = ws, phi_q, phi_k, num, mass, resid
    return y.view(B, T, H * d)


def _describe(st: _State, proj, w1, w2, tau, b_g, spec, normalize, seg_chunks, H, d, has_gate):
    st.spec, st.normalize, st.seg_chunks, st.heads, st.d, st.has_gate = spec, normalize, seg_chunks, H, d, has_gate
    st.has_tau, st.tau_dtype = tau is not None, None if tau is None else tau.dtype
    st.w_dtypes, st.b_dtype = (w1.dtype, w2.dtype), None if b_g is None else b_g.dtype
    st.proj, st.tau, st.b_g = proj, None if tau is None else tau.detach(), None if b_g is None else b_g.detach()
    st.native = st.saved = st.ws = st.phi_q = st.phi_k = st.num = st.mass = st.resid = None


def _weights_for(st: _State, proj, w1, w2, tau, b_g):
    """Kernel-dtype copies of the memory weights (the per-entry-point path)."""
    dt = proj.dtype
    st.w1c = w1.detach().to(dt).contiguous()
    st.w2c = w2.detach().to(dt).contiguous()
    st.tauf = None if tau is None else tau.detach().to(torch.float32).contiguous()
    st.gb = None if b_g is None else b_g.detach().to(torch.float32).contiguous()


def _native_io(st: _State, proj, w1, w2, spec: FeatureSpec, H: int, d: int, has_gate: bool):
    """The ts_memory_io of ``proj``; every tensor it names is kept on ``st``."""
    B, T, P = proj.shape
    dt = proj.dtype
    st.w1c = w1.detach().to(dt).contiguous()
    st.w2c = w2.detach().to(dt).contiguous()
    # the io holds raw addresses that ts_memory_bwd reads again: the RoPE
    # tables stay referenced here even if the table cache drops them
    st.tables = spec.tables(T, proj.device)
    ic, is_, fc, fs = st.tables
    base, es, Hd = proj.data_ptr(), proj.element_size(), H * d
    st.io = _lib.MemoryIO(_proj_view(base, es, 0, T, P, d), _proj_view(base, es, Hd, T, P, d),
                          _proj_view(base, es, 2 * Hd, T, P, d),
                          _proj_view(base, es, 3 * Hd, T, P, d) if has_gate else _lib.Strided(None, 0, 0, 0),
                          st.w1c.data_ptr(), st.w2c.data_ptr(), _lib.ptr(st.tau), _lib.ptr(st.b_g), _lib.ptr(ic),
                          _lib.ptr(is_), _lib.ptr(fc), _lib.ptr(fs))
    return st.io


def _native_forward(st: _State, plan, proj, w1, w2, tau, b_g, spec: FeatureSpec, H: int, d: int, has_gate: bool):
    """The forward as one ts_memory_fwd call; intermediates stay in one
    ``saved`` buffer that only the library reads."""
    desc, saved_bytes, _ = plan
    B, T, P = proj.shape
    dev = proj.device
    lib = _lib.load()
    io = _native_io(st, proj, w1, w2, spec, H, d, has_gate)
    saved = torch.empty(saved_bytes, dtype=torch.uint8, device=dev)
    Hd = H * d
    y = torch.empty(B, T, Hd, dtype=proj.dtype, device=dev)
    status = lib.ts_memory_fwd(ctypes.byref(desc), ctypes.byref(io), _lib.Strided(y.data_ptr(), T * Hd, d, Hd),
                               saved.data_ptr(), saved_bytes, _lib.stream_handle(dev))
    _lib.check(status, "ts_memory_fwd")
    st.native, st.saved = plan, saved
    return y


def _restore(saved_tensors, proj, w1, w2, tau, b_g, spec: FeatureSpec, normalize: bool, seg_chunks: int, H: int,
             has_gate: bool) -> _State:
    """The forward's :class:`_State` from the op inputs and its saved tensors."""
    st = _State()
    B, T, P = proj.shape
    d = P // (4 * H) if has_gate else P // (3 * H)
    _describe(st, proj, w1, w2, tau, b_g, spec, normalize, seg_chunks, H, d, has_gate)
    vals = dict(zip(_State.SAVED, (None if t is None or (t.ndim == 1 and t.numel() == 0 and name != "saved")
                                   else t for name, t in zip(_State.SAVED, saved_tensors))))
    if vals["saved"] is not None and vals["saved"].numel() > 0:
        st.native = _memory_plan(spec, B, H, T, d, proj.dtype, st.tau, st.b_g, w1, w2, normalize, has_gate,
                                 seg_chunks)
        st.saved = vals["saved"]
        _native_io(st, proj, w1, w2, spec, H, d, has_gate)
        return st
    _weights_for(st, proj, w1, w2, tau, b_g)
    for name in _State.SAVED[1:]:
        setattr(st, name, vals[name])
    return st


def _native_backward(st: _State, dy, need_w1: bool, need_w2: bool, need_tau: bool, need_b: bool):
    desc, saved_bytes, scratch_bytes = st.native
    proj = st.proj
    B, T, P = proj.shape
    H, d = st.heads, st.d
    Hd = H * d
    dev = proj.device
    lib = _lib.load()
    dy = dy.to(proj.dtype)
    if not dy.is_contiguous():
        dy = dy.contiguous()
    dproj = torch.empty_like(proj)
    scratch = torch.empty(scratch_bytes, dtype=torch.uint8, device=dev)
    pdt = st.w_dtypes[0]
    dw1 = torch.empty(st.w1c.shape, dtype=pdt, device=dev) if need_w1 else None
    dw2 = torch.empty(st.w2c.shape, dtype=pdt, device=dev) if need_w2 else None
    dtau = torch.empty(H, dtype=pdt, device=dev) if (need_tau and st.has_tau) else None
    db = torch.empty(Hd, dtype=pdt, device=dev) if (need_b and st.b_dtype is not None) else None
    base, es = dproj.data_ptr(), dproj.element_size()
    grads = _lib.MemoryGrads(_lib.Strided(dy.data_ptr(), T * Hd, d, Hd), _proj_view(base, es, 0, T, P, d),
                             _proj_view(base, es, Hd, T, P, d), _proj_view(base, es, 2 * Hd, T, P, d),
                             _proj_view(base, es, 3 * Hd, T, P, d) if st.has_gate else _lib.Strided(None, 0, 0, 0),
                             _lib.ptr(dw1), _lib.ptr(dw2), _lib.ptr(dtau), _lib.ptr(db))
    status = lib.ts_memory_bwd(ctypes.byref(desc), ctypes.byref(st.io), ctypes.byref(grads), st.saved.data_ptr(),
                               saved_bytes, scratch.data_ptr(), scratch_bytes, _lib.stream_handle(dev))
    _lib.check(status, "ts_memory_bwd")
    if dtau is not None and st.tau is not None:
        dtau = dtau.view(st.tau.shape)
    if db is not None and st.b_g is not None:
        db = db.view(st.b_g.shape)
    return dproj, dw1, dw2, dtau, db


def _memory_backward(st: _State, dy, need_w1: bool, need_w2: bool, need_tau: bool, need_b: bool):
    """Backward of :func:`_memory_forward` -> (dproj, dW1, dW2, dtau, db_g)."""
    if st.native is not None:
        return _native_backward(st, dy, need_w1, need_w2, need_tau, need_b)
    spec, proj = st.spec, st.proj
    B, T, P = proj.shape
    H, d = st.heads, st.d
    dt = proj.dtype
    num, mass, resid, phi_q, phi_k = st.num, st.mass, st.resid, st.phi_q, st.phi_k
    q, k, v, gv = _split_proj(proj, H, d, st.has_gate)
    dproj = torch.empty_like(proj)
    dq, dk, dv, dgv = _split_proj(dproj, H, d, st.has_gate)
    dyv = dy.to(dt).view(B, T, H, d).transpose(1, 2)
    want_gb = st.gb is not None and need_b
    dnum, dmass, (dresid, _), _, db_g = read_bwd(num, mass, resid, gv, dyv, spec.resid_scale, spec.eps, dg=dgv,
                                                 gbias=st.gb, gbias_grad=st.b_dtype if want_gb else None)
    norm = st.normalize
    q_ext = dmass if norm else None
    ws_f = st.ws
    # dq = scan(dnum, v, phi_k): its segment states are the forward's, transposed
    dphi_q, _, _ = scan_hip.scan_launch(dnum, v, phi_k, q_ext=q_ext, k_ext="ones" if norm else None,
                                        seg_chunks=st.seg_chunks, workspace=ws_f,
                                        states_in=2 if ws_f is not None else 0)
    # dk = reverse scan(v, dnum, phi_q) and dv = reverse scan(phi_k, phi_q, dnum) share
    # their segment states up to a transpose (sum_i dnum_i phi_q_i^T)
    if scan_hip.pair_eligible(v, dnum, phi_q, phi_k):
        # both in one pass over dnum and phi_q (the key-mass read's dmass
        # joins the dk scan's scores)
        dphi_k, _ = scan_hip.scan_pair_launch(v, dnum, phi_q, phi_k, reverse=True, seg_chunks=st.seg_chunks,
                                              out_b=dv, k_ext=q_ext)
    else:
        ws_r = scan_hip.workspace_for(v, dnum, phi_q, seg_chunks=st.seg_chunks, reverse=True, kx=norm) \
            if ws_f is not None else None
        dphi_k, _, _ = scan_hip.scan_launch(v, dnum, phi_q, reverse=True, q_ext="ones" if norm else None,
                                            k_ext=q_ext, seg_chunks=st.seg_chunks, workspace=ws_r)
        scan_hip.scan_launch(phi_k, phi_q, dnum, reverse=True, out=dv, seg_chunks=st.seg_chunks,
                             workspace=ws_r, states_in=2 if ws_r is not None else 0)
    need_tau = st.has_tau and need_tau
    want_k = need_w1 or need_tau
    want_q = need_w1 or need_w2 or need_tau
    dw1_k, _, dtau_k = feature_bwd(spec, k, st.w1c, st.tauf, dphi_k, None, dk, want_weights=want_k)
    dw1_q, dw2_q, dtau_q = feature_bwd(spec, q, st.w1c, st.tauf, dphi_q, dresid, dq, w2=st.w2c,
                                       want_weights=want_q)
    dw1 = dw2 = dtau = None
    if need_w1:
        dw1 = sum_grads(dw1_k, dw1_q, st.w_dtypes[0], st.w1c.shape)
    if need_w2:
        dw2 = sum_grads(dw2_q, None, st.w_dtypes[1], st.w2c.shape)
    if need_tau:
        dtau = sum_grads(dtau_k, dtau_q, st.tau_dtype, (H,))
    return dproj, dw1, dw2, dtau, db_g


# The depth-1 kernel-memory mixer as one autograd node (dispatch.HipOp): the
# forward is the stacked qkv / gate projection GEMM, the kernel memory and the
# output projection (block.py:593-599, 721-724 around engine.py's read); the
# backward the split-K weight-gradient GEMMs around the memory backward.  The
# tensors the backward needs are outputs of the forward, placeholders (empty
# tensors) where absent.

def _spec_args(spec: FeatureSpec):
    return (int(spec.kind), int(spec.m), float(spec.gain), int(spec.in_rot), int(spec.feat_rot),
            float(spec.rope_base), float(spec.resid_scale), float(spec.eps))


def _kernel_mixer_forward(x: torch.Tensor, w_qkv: torch.Tensor, w_g: torch.Tensor | None, b_g: torch.Tensor | None,
                     w1: torch.Tensor, w2: torch.Tensor, tau: torch.Tensor | None, w_out: torch.Tensor, kind: int,
                     m: int, gain: float, in_rot: int, feat_rot: int, rope_base: float, resid_scale: float,
                     eps: float, normalize: bool, seg_chunks: int, heads: int) -> list[torch.Tensor]:
    spec = FeatureSpec(kind, m, gain, in_rot, feat_rot, rope_base, resid_scale, eps)
    weight = w_qkv if w_g is None else _stacked(w_qkv, w_g)
    proj = torch.nn.functional.linear(x, weight)
    st = _State()
    y = _memory_forward(st, proj, w1, w2, tau, b_g, spec, normalize, seg_chunks, heads, w_g is not None)
    out = torch.nn.functional.linear(y, w_out)
    # the stacked [W_qkv; W_g] travels to the backward's input-gradient GEMM
    stacked = weight if w_g is not None else x.new_empty(0)
    if eager_forward():
        _HANDOFF.state = (out, st)
    return [out, proj, y] + [x.new_empty(0) if getattr(st, n) is None else getattr(st, n)
                             for n in _State.SAVED] + [stacked]


def _kernel_mixer_fake(x, w_qkv, w_g, b_g, w1, w2, tau, w_out, kind, m, gain, in_rot, feat_rot, rope_base,
                       resid_scale, eps, normalize, seg_chunks, heads):
    spec = FeatureSpec(kind, m, gain, in_rot, feat_rot, rope_base, resid_scale, eps)
    B, T, _ = x.shape
    H = heads
    P = w_qkv.shape[0] + (0 if w_g is None else w_g.shape[0])
    d = w_qkv.shape[0] // (3 * H)
    dev, dt = x.device, x.dtype
    out = x.new_empty(B, T, w_out.shape[0])
    proj = x.new_empty(B, T, P)
    y = x.new_empty(B, T, H * d)
    plan = _memory_plan(spec, B, H, T, d, dt, tau, b_g, w1, w2, normalize, w_g is not None, seg_chunks) \
        if _use_native(proj, tau, b_g) else None
    stacked = x.new_empty(P, x.shape[-1]) if w_g is not None else x.new_empty(0)
    if plan is not None:
        return [out, proj, y, torch.empty(plan[1], dtype=torch.uint8, device=dev)] + \
            [x.new_empty(0) for _ in range(6)] + [stacked]
    ws = x.new_empty(0)
    if m == d:
        nbytes = scan_hip.workspace_bytes(B, H, T, m, d, dt, seg_chunks=seg_chunks, v_ext=normalize)
        if nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    mass = torch.empty(B, H, T, dtype=torch.float32, device=dev) if normalize else x.new_empty(0)
    return [out, proj, y, x.new_empty(0), ws, x.new_empty(B, H, T, m), x.new_empty(B, H, T, m),
            x.new_empty(B, H, T, d), mass, x.new_empty(B, H, T, d), stacked]


def _kernel_mixer_backward_impl(dout: torch.Tensor, x: torch.Tensor, w_qkv: torch.Tensor, w_g: torch.Tensor | None,
                         b_g: torch.Tensor | None, w1: torch.Tensor, w2: torch.Tensor, tau: torch.Tensor | None,
                         w_out: torch.Tensor, proj: torch.Tensor, y: torch.Tensor, saved: list[torch.Tensor],
                         kind: int, m: int, gain: float, in_rot: int, feat_rot: int, rope_base: float,
                         resid_scale: float, eps: float, normalize: bool, seg_chunks: int, heads: int,
                         need: list[bool]) -> list[torch.Tensor]:
    spec = FeatureSpec(kind, m, gain, in_rot, feat_rot, rope_base, resid_scale, eps)
    st = _restore(saved[:-1], proj, w1, w2, tau, b_g, spec, normalize, seg_chunks, heads, w_g is not None)
    return _kernel_mixer_grads(st, dout, x, w_qkv, w_g, w_out, y, saved[-1], need)


def _kernel_mixer_grads(st: _State, dout, x, w_qkv, w_g, w_out, y, stacked, need: list[bool],
                        own_storage: bool = True) -> list[torch.Tensor]:
    """The backward of the kernel-mixer op from its forward's state.  With
    ``own_storage`` False (an autograd function's backward) the W_qkv and W_g
    gradients are two views of one stacked gradient; a custom op's outputs
    must not share storage, so it gets a copy of the W_g rows."""
    has_gate = w_g is not None
    d2 = dout.reshape(-1, w_out.shape[0])
    dw_out = weight_grad(d2, y.reshape(-1, y.shape[-1]), w_out.dtype) if need[7] else None
    dy = (d2 @ w_out).view(y.shape)
    dproj, dw1, dw2, dtau, db_g = _memory_backward(st, dy, need[4], need[5], need[6], need[3])
    weight = w_qkv if w_g is None else stacked
    P = weight.shape[0]
    dp2 = dproj.view(-1, P)
    dx = (dp2 @ weight).view(x.shape) if need[0] else None
    dw_qkv = dw_g = None
    if need[1] or (has_gate and need[2]):
        same = not has_gate or w_qkv.dtype == w_g.dtype
        dw = weight_grad(dp2, x.reshape(-1, x.shape[-1]), w_qkv.dtype if same else torch.float32)
        dw_qkv = dw[:w_qkv.shape[0]].to(w_qkv.dtype)
        if has_gate:
            dw_g = dw[w_qkv.shape[0]:].to(w_g.dtype, copy=own_storage)
    grads = [dx, dw_qkv, dw_g, db_g, dw1, dw2, dtau, dw_out]
    return [x.new_empty(0) if g is None else g for g in grads]


def _kernel_mixer_backward_fake(dout, x, w_qkv, w_g, b_g, w1, w2, tau, w_out, proj, y, saved, kind, m, gain, in_rot,
                                feat_rot, rope_base, resid_scale, eps, normalize, seg_chunks, heads, need):
    like = [x, w_qkv, w_g, b_g, w1, w2, tau, w_out]
    return [t.new_empty(t.shape) if (t is not None and w) else x.new_empty(0) for t, w in zip(like, need)]


# Eager execution hands the forward's _State to its backward on the autograd
# context (the forward stores it here, keyed by its output, and the setup right
# after it on the same thread takes it), so the backward need not rebuild it
# from the saved tensors.  The compiled path's backward rebuilds it.
_HANDOFF = threading.local()


def _kernel_mixer_setup(ctx, inputs, output):
    x, w_qkv, w_g, b_g, w1, w2, tau, w_out, *args = inputs
    ctx.args = args
    tensors = [x, w_qkv, w_g, b_g, w1, w2, tau, w_out]
    ctx.need = [t is not None and t.requires_grad for t in tensors]
    ctx.save_for_backward(*tensors, *output[1:])
    handed = getattr(_HANDOFF, "state", None)
    _HANDOFF.state = None
    ctx.state = handed[1] if handed is not None and handed[0] is output[0] else None


def _kernel_mixer_backward(ctx, grads, bwd):
    x, w_qkv, w_g, b_g, w1, w2, tau, w_out, proj, y, *saved = ctx.saved_tensors
    st = getattr(ctx, "state", None)
    if st is not None:  # eager: the forward's own state (same launches as the rebuilt one)
        ctx.state = None
        res = _kernel_mixer_grads(st, grads[0], x, w_qkv, w_g, w_out, y, saved[-1], ctx.need, own_storage=False)
    else:
        res = bwd(grads[0], x, w_qkv, w_g, b_g, w1, w2, tau, w_out, proj, y, list(saved), *ctx.args, ctx.need)
    return (*[g if w else None for g, w in zip(res, ctx.need)], *([None] * len(ctx.args)))


_kernel_mixer_op = HipOp("kernel_mixer", forward=_kernel_mixer_forward, forward_fake=_kernel_mixer_fake,
                         backward_impl=_kernel_mixer_backward_impl, backward_fake=_kernel_mixer_backward_fake,
                         setup=_kernel_mixer_setup, backward=_kernel_mixer_backward)


def kernel_mixer(x, w_qkv, w_g, b_g, w1, w2, tau, w_out, spec: FeatureSpec, normalize: bool, heads: int,
                 seg_chunks: int = 0):
    """out = proj_out(kernel_memory(x [W_qkv; W_g]^T)) for the depth-1 kernel memory, one autograd node."""
    if not x.is_cuda:
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    if not x.is_contiguous():
        x = x.contiguous()
    return _kernel_mixer_op(x, w_qkv, w_g, b_g, w1, w2, tau, w_out, *_spec_args(spec), bool(normalize),
                            int(seg_chunks), int(heads))[0]
