"""GN-family write payloads on the GPU (ts_gn_write_fwd / ts_gn_write_bwd).

Replaces, for depth-1 ReLU^2 (and ReLU^2-threshold), SiLU or tanh GN memories with one
Jacobian step, the torch chain of src/thetascan/_core/ops/engine.py:117-158
(_block_forward), 180-195 (_g_from_lambda), 215-255 (_lambda_solve) and the
stream assembly of 260-340: one kernel produces the LA2 keys h, the LA2
values s*lam and the LA1 values g per token.  The backward kernel recomputes
the forward, writes dx and dv, and leaves slot-major token tiles
([slot, H, B*T, w]) that split-K batched GEMMs contract into dW1, dW2 and dtau.
"""
from __future__ import annotations

import ctypes

import torch

from ... import _lib
from .dispatch import HipOp

GN_HEAD_DIMS = (16, 32, 64, 128)
ACTS = {"relu2": _lib.GN_RELU2, "tanh": _lib.GN_TANH, "silu": _lib.GN_SILU}  # hidden nonlinearities the kernels take


def supported_width(m: int, dtype: torch.dtype | None = None, d: int | None = None) -> bool:
    """Hidden widths the GN kernels take: multiples of 16 up to 128, 192 and
    256 in any dtype, and 384 in bf16 at head widths 32 and 64."""
    if m == 384:
        return dtype == torch.bfloat16 and d in (32, 64)
    return m in (192, 256) or (16 <= m <= 128 and m % 16 == 0)


def eligible(cfg, weights, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Whether the HIP GN write covers this configuration and these streams."""
    if cfg.write_rule != "gn" or cfg.depth != 1 or cfg.write_iters != 1 or cfg.nonlin not in ACTS:
        return False
    if cfg.value_centers:
        return False
    if not (k.is_cuda and v.is_cuda) or k.dtype not in (torch.bfloat16, torch.float32) or v.dtype != k.dtype:
        return False
    W1, W2, _ = weights[0]
    d, m = k.shape[-1], W1.shape[-2]
    return d in GN_HEAD_DIMS and supported_width(m, k.dtype, d) and v.shape[-1] == d and W2.shape[-1] == m


def _rows(t: torch.Tensor) -> torch.Tensor:
    """A [B,H,T,w] view whose rows the kernel can read: contiguous last axis,
    16-byte aligned rows (else a contiguous copy)."""
    vec = 16 // t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % vec == 0 for s in t.stride()[:3])
    return t if ok else t.contiguous()


def _desc(x, m, has_tau, s, inv_depth, eps, act, damping):
    B, H, T, d = x.shape
    return _lib.GnDesc(B, H, T, d, m, _lib.dtype_code(x.dtype), int(has_tau), float(s), float(inv_depth),
                       float(eps), int(act), float(damping))


def contract_tokens(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """sum_n a[h, n, :]^T b[h, n, :] -> fp32 [H, p, q] for head-major token
    tiles a [H, N, p], b [H, N, q]: one ts_contract_tokens call (token
    slices contracted on MFMA into fp32 partials, summed in slice order) for
    widths that are multiples of 16 up to 128, else a split-K batched GEMM."""
    H, N, p = a.shape
    q = b.shape[-1]
    if (a.is_cuda and a.dtype == b.dtype and a.dtype in (torch.bfloat16, torch.float32) and p % 16 == 0
            and q % 16 == 0 and p <= 128 and q <= 128 and a.stride(-1) == 1 and b.stride(-1) == 1):
        vec = 16 // a.element_size()
        if (a.data_ptr() % 16 == 0 and b.data_ptr() % 16 == 0
                and all(x % vec == 0 for x in (a.stride(0), a.stride(1), b.stride(0), b.stride(1)))):
            lib = _lib.load()
            desc = _lib.ContractDesc(H, N, p, q, _lib.dtype_code(a.dtype))
            ws = ctypes.c_size_t()
            _lib.check(lib.ts_contract_workspace_bytes(ctypes.byref(desc), ctypes.byref(ws)), "contract workspace")
            work = torch.empty(ws.value, dtype=torch.uint8, device=a.device)
            out = torch.empty(H, p, q, dtype=torch.float32, device=a.device)
            with _lib.timed("ts_contract_tokens", lambda: _lib.nbytes(a, b, out)):
                status = lib.ts_contract_tokens(ctypes.byref(desc), a.data_ptr(), a.stride(0), a.stride(1),
                                                b.data_ptr(), b.stride(0), b.stride(1), out.data_ptr(),
                                                work.data_ptr(), ws.value, _lib.stream_handle(a.device))
            _lib.check(status, "ts_contract_tokens")
            return out
    S = 1
    while S < 64 and H * S < 512 and N % (2 * S) == 0 and N // (2 * S) >= 256:
        S *= 2
    parts = torch.bmm(a.reshape(H * S, N // S, p).transpose(1, 2), b.reshape(H * S, N // S, q))
    return parts.view(H, S, p, q).sum(1, dtype=torch.float32)


def _gn_write_forward(x: torch.Tensor, v: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, tau: torch.Tensor | None,
                 s: float, inv_depth: float, eps: float, act: int, damping: float) -> list[torch.Tensor]:
    lib = _lib.load()
    xk, vk = _rows(x), _rows(v)
    B, H, T, d = xk.shape
    m = w1.shape[1]
    dt = x.dtype
    w1c = w1.detach().to(dt).contiguous()
    w2c = w2.detach().to(dt).contiguous()
    w2t = w2c.transpose(1, 2).contiguous()
    tc = None if tau is None else tau.detach().to(torch.float32).contiguous()
    h = torch.empty(B, H, T, m, dtype=dt, device=x.device)
    lam = torch.empty(B, H, T, d, dtype=dt, device=x.device)
    g = torch.empty(B, H, T, m, dtype=dt, device=x.device)
    desc = _desc(xk, m, tc is not None, s, inv_depth, eps, act, damping)
    io = _lib.GnIO(_lib.strided(xk), _lib.strided(vk), w1c.data_ptr(), w2c.data_ptr(), w2t.data_ptr(),
                   _lib.ptr(tc), _lib.strided(h), _lib.strided(lam), _lib.strided(g))
    with _lib.timed("ts_gn_write_fwd", lambda: _lib.nbytes(xk, vk, h, lam, g)):
        status = lib.ts_gn_write_fwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(x.device))
    _lib.check(status, "ts_gn_write_fwd")
    return [h, lam, g]


def _gn_write_fake(x, v, w1, w2, tau, s, inv_depth, eps, act, damping):
    B, H, T, d = x.shape
    m = w1.shape[1]
    return [x.new_empty(B, H, T, m), x.new_empty(B, H, T, d), x.new_empty(B, H, T, m)]


def _gn_write_backward_impl(dh: torch.Tensor | None, dlam: torch.Tensor | None, dg: torch.Tensor | None, x: torch.Tensor,
                     v: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, tau: torch.Tensor | None, s: float,
                     inv_depth: float, eps: float, act: int, damping: float, need_tau: bool
                     ) -> list[torch.Tensor]:
    lib = _lib.load()
    xk, vk = _rows(x), _rows(v)
    B, H, T, d = xk.shape
    m = w1.shape[1]
    dt = xk.dtype
    N = B * T
    w1c = w1.detach().to(dt).contiguous()
    w2c = w2.detach().to(dt).contiguous()
    w2t = w2c.transpose(1, 2).contiguous()
    w1t = w1c.transpose(1, 2).contiguous()
    tc = None if tau is None else tau.detach().to(torch.float32).contiguous()
    has_tau = tc is not None

    def grad(t):
        return None if t is None else _rows(t.to(dt))

    dh, dlam, dg = grad(dh), grad(dlam), grad(dg)
    dx = torch.empty(B, H, T, d, dtype=dt, device=xk.device)
    dv = torch.empty(B, H, T, d, dtype=dt, device=xk.device)
    nsm = 5 if has_tau else 4
    tm = torch.empty(nsm, H, N, m, dtype=dt, device=xk.device)
    td = torch.empty(4, H, N, d, dtype=dt, device=xk.device)
    desc = _desc(xk, m, has_tau, s, inv_depth, eps, act, damping)
    io = _lib.GnBwdIO(_lib.strided(xk), _lib.strided(vk), w1c.data_ptr(), w2c.data_ptr(), w1t.data_ptr(),
                      w2t.data_ptr(), _lib.ptr(tc), _lib.strided(dh), _lib.strided(dlam), _lib.strided(dg),
                      _lib.strided(None), _lib.strided(dx), _lib.strided(dv), tm.data_ptr(), td.data_ptr())
    with _lib.timed("ts_gn_write_bwd", lambda: _lib.nbytes(xk, vk, dh, dlam, dg, dx, dv, tm, td)):
        status = lib.ts_gn_write_bwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(xk.device))
    _lib.check(status, "ts_gn_write_bwd")
    # dW1 = da^T x;  dW2 = lam^T dz + du^T h + 2 W2 o (drq^T s2);  dtau = -sum dpre
    dw1 = contract_tokens(tm[2], td[2])
    dw2 = contract_tokens(td[0], tm[0]) + contract_tokens(td[1], tm[1])
    dw2 = dw2 + 2.0 * w2c.to(torch.float32) * contract_tokens(td[3], tm[3])
    dtau = x.new_empty(0)
    if has_tau and need_tau:
        dtau = (-tm[4].sum(1, dtype=torch.float32)).to(tau.dtype)
    return [dx, dv, dw1.to(w1.dtype), dw2.to(w2.dtype), dtau]


def _gn_write_backward_fake(dh, dlam, dg, x, v, w1, w2, tau, s, inv_depth, eps, act, damping, need_tau):
    dtau = x.new_empty(0) if (tau is None or not need_tau) else tau.new_empty(tau.shape)
    return [x.new_empty(x.shape), x.new_empty(x.shape), w1.new_empty(w1.shape), w2.new_empty(w2.shape), dtau]


def _gn_write_setup(ctx, inputs, output):
    x, v, w1, w2, tau, s, inv_depth, eps, act, damping = inputs
    ctx.args = (s, inv_depth, eps, act, damping)
    ctx.need_tau = tau is not None and tau.requires_grad
    ctx.save_for_backward(x, v, w1, w2, tau)


def _gn_write_backward(ctx, grads, bwd):
    x, v, w1, w2, tau = ctx.saved_tensors
    dh, dlam, dg = grads
    dx, dv, dw1, dw2, dtau = bwd(dh, dlam, dg, x, v, w1, w2, tau, *ctx.args, ctx.need_tau)
    return dx, dv, dw1, dw2, (dtau if ctx.need_tau else None), None, None, None, None, None


_gn_write_op = HipOp("gn_write", forward=_gn_write_forward, forward_fake=_gn_write_fake,
                     backward_impl=_gn_write_backward_impl, backward_fake=_gn_write_backward_fake,
                     setup=_gn_write_setup, backward=_gn_write_backward)


def write(x, v, w1, w2, tau=None, *, s: float = 1.0, inv_depth: float = 1.0, eps: float = 1e-6,
          nonlin: str = "relu2", damping: float | None = None):
    """GN write payloads ``(h, s*lam, g)`` of keys ``x`` and values ``v``
    ([B,H,T,d]) for per-head weights ``w1`` [H,m,d], ``w2`` [H,d,m] (a leading
    1 broadcasts over heads) and an optional threshold ``tau`` [H,m].
    ``nonlin`` is the hidden nonlinearity (relu2, silu or tanh); ``damping`` the
    Jacobi diagonal's damping (None: ``eps``, as the reference)."""
    if not (x.is_cuda and v.is_cuda):
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    H = x.shape[1]
    if w1.shape[0] != H:
        w1 = w1.expand(H, -1, -1)
    if w2.shape[0] != H:
        w2 = w2.expand(H, -1, -1)
    if tau is not None and tau.shape != (H, w1.shape[1]):
        tau = tau.reshape(-1, w1.shape[1]).expand(H, -1)
    damp = float(eps if damping is None else damping)
    h, lam, g = _gn_write_op(x, v, w1, w2, tau, float(s), float(inv_depth), float(eps), ACTS[nonlin], damp)
    return h, lam, g


# ------------------------------------------------------------------ GN read

READ_NONE, READ_PLAIN, READ_NORMALIZED = 0, 1, 2


def _read_desc(q, m, has_tau, corr, want_resid, s, eps, act):
    B, H, T, d = q.shape
    return _lib.GnReadDesc(B, H, T, d, m, _lib.dtype_code(q.dtype), int(has_tau), int(corr), int(want_resid),
                           float(s), float(eps), int(act))


def _gn_read_forward(q: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor | None, tau: torch.Tensor | None,
                num: torch.Tensor | None, mass: torch.Tensor | None, corr: int, want_resid: bool, s: float,
                eps: float, act: int) -> list[torch.Tensor]:
    lib = _lib.load()
    qk = _rows(q)
    B, H, T, d = qk.shape
    m = w1.shape[1]
    dt = q.dtype
    w1c = w1.detach().to(dt).contiguous()
    w2c = w2.detach().to(dt).contiguous() if want_resid else None
    tc = None if tau is None else tau.detach().to(torch.float32).contiguous()
    nk = None if num is None else _rows(num.to(dt))
    mk = None if mass is None else mass.detach().to(torch.float32)
    h = torch.empty(B, H, T, m, dtype=dt, device=q.device)
    resid = torch.empty(B, H, T, d, dtype=dt, device=q.device) if want_resid else q.new_empty(0)
    desc = _read_desc(qk, m, tc is not None, corr, want_resid, s, eps, act)
    io = _lib.GnReadIO(_lib.strided(qk), w1c.data_ptr(), _lib.ptr(w2c), _lib.ptr(tc), _lib.strided(nk),
                       _lib.strided(mk), _lib.strided(h), _lib.strided(resid if want_resid else None))
    with _lib.timed("ts_gn_read_fwd", lambda: _lib.nbytes(qk, nk, mk, h, resid)):
        status = lib.ts_gn_read_fwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(q.device))
    _lib.check(status, "ts_gn_read_fwd")
    return [h, resid]


def _gn_read_fake(q, w1, w2, tau, num, mass, corr, want_resid, s, eps, act):
    B, H, T, d = q.shape
    return [q.new_empty(B, H, T, w1.shape[1]), q.new_empty(B, H, T, d) if want_resid else q.new_empty(0)]


def _gn_read_backward_impl(dh: torch.Tensor | None, dresid: torch.Tensor | None, q: torch.Tensor, w1: torch.Tensor,
                    w2: torch.Tensor | None, tau: torch.Tensor | None, num: torch.Tensor | None,
                    mass: torch.Tensor | None, corr: int, want_resid: bool, s: float, eps: float, act: int,
                    need_tau: bool) -> list[torch.Tensor]:
    lib = _lib.load()
    qk = _rows(q)
    B, H, T, d = qk.shape
    m = w1.shape[1]
    dt = qk.dtype
    N = B * T
    w1c = w1.detach().to(dt).contiguous()
    w1t = w1c.transpose(1, 2).contiguous()
    w2t = w2.detach().to(dt).transpose(1, 2).contiguous() if want_resid else None
    tc = None if tau is None else tau.detach().to(torch.float32).contiguous()
    nk = None if num is None else _rows(num.to(dt))
    mk = None if mass is None else mass.detach().to(torch.float32)
    dh = None if dh is None else _rows(dh.to(dt))
    dresid = None if (dresid is None or not want_resid) else _rows(dresid.to(dt))
    dq = torch.empty(B, H, T, d, dtype=dt, device=qk.device)
    dnum = torch.empty(B, H, T, m, dtype=dt, device=qk.device) if corr else None
    dmass = torch.empty(B, H, T, dtype=torch.float32, device=qk.device) if corr == READ_NORMALIZED else None
    has_tau = tc is not None
    tm = torch.empty(3 if has_tau else 2, H, N, m, dtype=dt, device=qk.device)
    td = torch.empty(2, H, N, d, dtype=dt, device=qk.device)
    desc = _read_desc(qk, m, has_tau, corr, want_resid, s, eps, act)
    io = _lib.GnReadBwdIO(_lib.strided(qk), w1c.data_ptr(), w1t.data_ptr(), _lib.ptr(w2t), _lib.ptr(tc),
                          _lib.strided(nk), _lib.strided(mk), _lib.strided(dh), _lib.strided(dresid),
                          _lib.strided(dq), _lib.strided(dnum), _lib.ptr(dmass), tm.data_ptr(), td.data_ptr())
    with _lib.timed("ts_gn_read_bwd", lambda: _lib.nbytes(qk, nk, mk, dh, dresid, dq, dnum, dmass, tm, td)):
        status = lib.ts_gn_read_bwd(ctypes.byref(desc), ctypes.byref(io), _lib.stream_handle(qk.device))
    _lib.check(status, "ts_gn_read_bwd")
    dw1 = contract_tokens(tm[0], td[0]).to(w1.dtype)
    dw2 = contract_tokens(td[1], tm[1]).to(w2.dtype) if want_resid else q.new_empty(0)
    dtau = (-tm[2].sum(1, dtype=torch.float32)).to(tau.dtype) if (has_tau and need_tau) else q.new_empty(0)
    dnum = q.new_empty(0) if dnum is None else dnum.to(num.dtype)
    dmass = q.new_empty(0) if dmass is None else dmass.to(mass.dtype)
    return [dq, dw1, dw2, dtau, dnum, dmass]


def _gn_read_backward_fake(dh, dresid, q, w1, w2, tau, num, mass, corr, want_resid, s, eps, act, need_tau):
    return [q.new_empty(q.shape), w1.new_empty(w1.shape), w2.new_empty(w2.shape) if want_resid else q.new_empty(0),
            tau.new_empty(tau.shape) if (tau is not None and need_tau) else q.new_empty(0),
            num.new_empty(num.shape) if corr else q.new_empty(0),
            mass.new_empty(mass.shape) if corr == READ_NORMALIZED else q.new_empty(0)]


def _gn_read_setup(ctx, inputs, output):
    q, w1, w2, tau, num, mass, corr, want_resid, s, eps, act = inputs
    ctx.args = (corr, want_resid, s, eps, act)
    ctx.need_tau = tau is not None and tau.requires_grad
    ctx.save_for_backward(q, w1, w2, tau, num, mass)


def _gn_read_backward(ctx, grads, bwd):
    q, w1, w2, tau, num, mass = ctx.saved_tensors
    corr, want_resid, s, eps, act = ctx.args
    dh, dresid = grads
    dq, dw1, dw2, dtau, dnum, dmass = bwd(dh, dresid if want_resid else None, q, w1, w2, tau, num, mass, corr,
                                          want_resid, s, eps, act, ctx.need_tau)
    return (dq, dw1, dw2 if want_resid else None, dtau if ctx.need_tau else None,
            dnum if corr else None, dmass if corr == READ_NORMALIZED else None, None, None, None, None, None)


_gn_read_op = HipOp("gn_read", forward=_gn_read_forward, forward_fake=_gn_read_fake,
                    backward_impl=_gn_read_backward_impl, backward_fake=_gn_read_backward_fake,
                    setup=_gn_read_setup, backward=_gn_read_backward)


def read_stage(q, w1, w2=None, tau=None, num=None, mass=None, *, corr: int = READ_NONE, want_resid: bool = False,
               s: float = 1.0, eps: float = 1e-6, nonlin: str = "relu2"):
    """One GN read stage: ``h = sigma(rmsnorm(W1 q + c) - tau)`` (sigma relu2
    or tanh) with ``c`` = 0, ``num`` or ``num / (mass + eps)`` and, with
    ``want_resid``, ``resid = q + s W2 h``.  Returns ``(h, resid or None)``."""
    if not q.is_cuda:
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    H = q.shape[1]
    if w1.shape[0] != H:
        w1 = w1.expand(H, -1, -1)
    if w2 is not None and w2.shape[0] != H:
        w2 = w2.expand(H, -1, -1)
    if tau is not None and tau.shape != (H, w1.shape[1]):
        tau = tau.reshape(-1, w1.shape[1]).expand(H, -1)
    h, resid = _gn_read_op(q, w1, w2, tau, num, mass, int(corr), bool(want_resid), float(s), float(eps),
                           ACTS[nonlin])
    return h, (resid if want_resid else None)


def _normalized_read_forward(num: torch.Tensor, mass: torch.Tensor | None, resid: torch.Tensor,
                             gate: torch.Tensor | None, gate_bias: torch.Tensor | None, s: float,
                             eps: float) -> torch.Tensor:
    """y = resid + s * num / (mass + eps)  (or + s * num without mass): the read
    epilogue of engine.py:440-442, 538-544 on ts_read_fwd.  An fp32 numerator (a
    difference of views) is read in fp32, then rounded once to the dtype of
    ``resid``.  With ``gate`` (the [B,H,T,d] view of the output gate's
    pre-activation x W_g^T, same dtype as num) y is also multiplied by
    silu(gate + gate_bias) (block.py:721-722, gates.py:34-40) and written
    token-major: a [B,H,T,d] view of [B,T,H,d] memory, which the output
    projection reads as [B,T,H*d] without a copy."""
    from . import fused

    nk, rk = _rows(num), _rows(resid.to(num.dtype))
    mk = None if mass is None else mass.detach().to(torch.float32)
    if gate is None:
        y = torch.empty_like(nk)
        fused.read_fwd(nk, mk, rk, None, y, s, eps)
        return y.to(resid.dtype)
    B, H, T, d = nk.shape
    y = torch.empty(B, T, H, d, dtype=nk.dtype, device=nk.device).transpose(1, 2)
    gb = None if gate_bias is None else gate_bias.detach().to(torch.float32).contiguous()
    fused.read_fwd(nk, mk, rk, _rows(gate), y, s, eps, gbias=gb)
    return y


def _normalized_read_fake(num, mass, resid, gate, gate_bias, s, eps):
    if gate is None:
        return resid.new_empty(num.shape)
    B, H, T, d = num.shape
    return num.new_empty(B, T, H, d).transpose(1, 2)


def _normalized_read_backward_impl(dy: torch.Tensor, num: torch.Tensor, mass: torch.Tensor | None,
                                   resid: torch.Tensor, gate: torch.Tensor | None, gate_bias: torch.Tensor | None,
                                   s: float, eps: float) -> list[torch.Tensor]:
    from . import fused

    nk, rk = _rows(num), _rows(resid.to(num.dtype))
    mk = None if mass is None else mass.detach().to(torch.float32)
    gk = None if gate is None else _rows(gate)
    gb = None if gate_bias is None else gate_bias.detach().to(torch.float32).contiguous()
    dnum, dmass, (dresid, _), dg, dgb = fused.read_bwd(
        nk, mk, rk, gk, _rows(dy.to(nk.dtype)), s, eps, gbias=gb,
        gbias_grad=None if gate_bias is None else gate_bias.dtype)
    dmass = num.new_empty(0) if dmass is None else dmass.to(mass.dtype)
    return [dnum, dmass, dresid.to(resid.dtype), num.new_empty(0) if dg is None else dg,
            num.new_empty(0) if dgb is None else dgb]


def _normalized_read_backward_fake(dy, num, mass, resid, gate, gate_bias, s, eps):
    B, H, T, d = num.shape
    return [num.new_empty(num.shape), num.new_empty(0) if mass is None else mass.new_empty(mass.shape),
            resid.new_empty(resid.shape),
            num.new_empty(0) if gate is None else num.new_empty(B, T, H, d).transpose(1, 2),
            num.new_empty(0) if gate_bias is None else gate_bias.new_empty(gate_bias.shape)]


def _normalized_read_setup(ctx, inputs, output):
    num, mass, resid, gate, gate_bias, s, eps = inputs
    ctx.args = (s, eps)
    ctx.need_bias = gate_bias is not None and gate_bias.requires_grad
    ctx.save_for_backward(num, mass, resid, gate, gate_bias)


def _normalized_read_backward(ctx, dy, bwd):
    num, mass, resid, gate, gate_bias = ctx.saved_tensors
    dnum, dmass, dresid, dg, dgb = bwd(dy, num, mass, resid, gate, gate_bias, *ctx.args)
    return (dnum, None if mass is None else dmass, dresid, None if gate is None else dg,
            dgb if ctx.need_bias else None, None, None)


_normalized_read_op = HipOp("normalized_read", forward=_normalized_read_forward,
                            forward_fake=_normalized_read_fake, backward_impl=_normalized_read_backward_impl,
                            backward_fake=_normalized_read_backward_fake, setup=_normalized_read_setup,
                            backward=_normalized_read_backward)


def normalized_read(num, mass, resid, *, s: float = 1.0, eps: float = 1e-6, gate=None, gate_bias=None):
    """Read epilogue of one view on the GPU (ts_read_fwd / ts_read_bwd),
    optionally with the output gate (see :func:`_normalized_read_forward`)."""
    return _normalized_read_op(num, mass, resid, gate, gate_bias, float(s), float(eps))


def read_eligible(cfg, weights, q: torch.Tensor) -> bool:
    """Whether the HIP GN read stages cover this configuration (depth-1
    ReLU^2 GN memories with one Jacobian step, no value anchors)."""
    if cfg.write_rule != "gn" or cfg.depth != 1 or cfg.write_iters != 1 or cfg.nonlin not in ACTS:
        return False
    if cfg.value_centers or not q.is_cuda or q.dtype not in (torch.bfloat16, torch.float32):
        return False
    if cfg.read_norm and cfg.read_norm_mode != "key_mass":
        return False
    W1, W2, _ = weights[0]
    return q.shape[-1] in GN_HEAD_DIMS and supported_width(W1.shape[-2], q.dtype, q.shape[-1])


# ------------------------------------------------------------------ per-row activation

ACT_ROWS = dict(ACTS, swiglu=_lib.GN_SWIGLU)  # ts_gn_act_* nonlinearities


def act_rows_eligible(a: torch.Tensor, nonlin: str) -> bool:
    """Whether ts_gn_act takes these pre-activations: [B,H,T,m] rows in bf16
    (m a multiple of 8) or fp32 (of 4) on the GPU, an elementwise nonlinearity
    or SwiGLU."""
    vec = 8 if a.dtype == torch.bfloat16 else 4
    return (nonlin in ACT_ROWS and a.is_cuda and a.ndim == 4 and a.dtype in (torch.bfloat16, torch.float32)
            and a.shape[-1] % vec == 0)


def _act_desc(a, act, has_tau, eps):
    B, H, T, m = a.shape
    return _lib.GnActDesc(B, H, T, m, _lib.dtype_code(a.dtype), int(act), int(has_tau), float(eps))


def _act_forward(a: torch.Tensor, b: torch.Tensor | None, tau: torch.Tensor | None, act: int, eps: float,
                 want_scales: bool) -> list[torch.Tensor]:
    lib = _lib.load()
    a4 = _rows(a)
    b4 = None if b is None else _rows(b.to(a.dtype))
    tauf = None if tau is None else tau.detach().to(torch.float32).contiguous()
    glu = act == _lib.GN_SWIGLU
    h = torch.empty(a4.shape, dtype=a.dtype, device=a.device)
    sa = torch.empty_like(h) if want_scales else None
    sb = torch.empty_like(h) if want_scales and glu else None
    desc = _act_desc(a4, act, tau is not None, eps)
    with _lib.timed("ts_gn_act_fwd", lambda: _lib.nbytes(a4, b4, h, sa, sb)):
        status = lib.ts_gn_act_fwd(ctypes.byref(desc), _lib.strided(a4), _lib.strided(b4), _lib.ptr(tauf),
                                   _lib.strided(h), _lib.strided(sa), _lib.strided(sb), _lib.stream_handle(a.device))
    _lib.check(status, "ts_gn_act_fwd")
    empty = a.new_empty(0)
    return [h, empty if sa is None else sa, empty if sb is None else sb]


def _act_fake(a, b, tau, act, eps, want_scales):
    glu = act == _lib.GN_SWIGLU
    return [a.new_empty(a.shape), a.new_empty(a.shape) if want_scales else a.new_empty(0),
            a.new_empty(a.shape) if want_scales and glu else a.new_empty(0)]


def _act_backward_impl(dh: torch.Tensor | None, dsa: torch.Tensor | None, dsb: torch.Tensor | None, a: torch.Tensor,
                       b: torch.Tensor | None, tau: torch.Tensor | None, act: int, eps: float,
                       need_tau: bool) -> list[torch.Tensor]:
    lib = _lib.load()
    a4 = _rows(a)
    b4 = None if b is None else _rows(b.to(a.dtype))
    tauf = None if tau is None else tau.detach().to(torch.float32).contiguous()
    glu = act == _lib.GN_SWIGLU
    g = lambda t: None if t is None or t.numel() == 0 else _rows(t.to(a.dtype))  # noqa: E731
    dh4, dsa4, dsb4 = g(dh), g(dsa), g(dsb)
    da = torch.empty(a4.shape, dtype=a.dtype, device=a.device)
    db = torch.empty_like(da) if glu else None
    dz = torch.empty_like(da) if need_tau and tau is not None else None
    desc = _act_desc(a4, act, tau is not None, eps)
    with _lib.timed("ts_gn_act_bwd", lambda: _lib.nbytes(a4, b4, dh4, dsa4, dsb4, da, db, dz)):
        status = lib.ts_gn_act_bwd(ctypes.byref(desc), _lib.strided(a4), _lib.strided(b4), _lib.ptr(tauf),
                                   _lib.strided(dh4), _lib.strided(dsa4), _lib.strided(dsb4), _lib.strided(da),
                                   _lib.strided(db), _lib.strided(dz), _lib.stream_handle(a.device))
    _lib.check(status, "ts_gn_act_bwd")
    empty = a.new_empty(0)
    dtau = empty if dz is None else (-dz.float().sum(dim=(0, 2))).to(tau.dtype)
    return [da, empty if db is None else db.to(b.dtype), dtau]


def _act_backward_fake(dh, dsa, dsb, a, b, tau, act, eps, need_tau):
    return [a.new_empty(a.shape), a.new_empty(0) if b is None else b.new_empty(b.shape),
            tau.new_empty(tau.shape) if need_tau and tau is not None else a.new_empty(0)]


def _act_setup(ctx, inputs, output):
    a, b, tau, act, eps, _want = inputs
    ctx.act, ctx.eps = act, eps
    ctx.need_tau = tau is not None and tau.requires_grad
    ctx.save_for_backward(a, b, tau)


def _act_backward(ctx, grads, bwd):
    dh, dsa, dsb = grads
    a, b, tau = ctx.saved_tensors
    da, db, dtau = bwd(dh, dsa, dsb, a, b, tau, ctx.act, ctx.eps, ctx.need_tau)
    return (da, db if b is not None else None, dtau if ctx.need_tau else None, None, None, None)


_act_op = HipOp("gn_act", forward=_act_forward, forward_fake=_act_fake, backward_impl=_act_backward_impl,
                backward_fake=_act_backward_fake, setup=_act_setup, backward=_act_backward)


def act_rows(a, b=None, tau=None, *, nonlin: str = "relu2", eps: float = 1e-6, want_scales: bool = True):
    """The GN block's hidden features and Jacobian scales of pre-activations
    ``a`` = W1 x ([B,H,T,m]; ``b`` = Wg x for SwiGLU) on the GPU
    (ts_gn_act_fwd / ts_gn_act_bwd):

    * elementwise nonlinearity: z = rmsnorm(a) - tau, h = sigma(z),
      sa = sigma'(z) / rms(a)  (engine.py:117-158, 180-255);
    * SwiGLU: h = silu(rmsnorm(b)) rmsnorm(a), sa = silu(rmsnorm(b)) / rms(a),
      sb = rmsnorm(a) silu'(rmsnorm(b)) / rms(b).

    Returns ``(h, sa, sb)`` (sa / sb None when not wanted or not SwiGLU)."""
    if not a.is_cuda:
        raise RuntimeError("hip backend: tensors must live on the GPU (no CPU fallback)")
    act = ACT_ROWS[nonlin]
    if (act == _lib.GN_SWIGLU) != (b is not None):
        raise ValueError("gn act: SwiGLU needs the gate pre-activation b, the other nonlinearities none")
    if tau is not None:
        H, m = a.shape[1], a.shape[-1]
        tau = tau.reshape(-1, m).expand(H, m) if tau.shape != (H, m) else tau
    h, sa, sb = _act_op(a, b, tau, int(act), float(eps), bool(want_scales))
    return h, (sa if want_scales else None), (sb if want_scales and b is not None else None)
