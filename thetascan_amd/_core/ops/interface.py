"""Scan-backend boundary of the MI355X build.

Mirrors the reference's plugin surface (src/thetascan/_core/ops/interface.py):
``_REGISTRY``, ``resolve_backend``, ``_fn``, ``scan_views``, the temporal
views ``Accumulator`` / ``FadeStale`` / ``FadeFast`` / ``NullAccumulator``,
and the mass helpers ``ema_cumsum`` / ``causal_prefix_sum``.  The only
backend this package ships is ``"hip"``; ``"auto"`` resolves to it.  The
reference's portable backends (naive/quad/chunk/cumsum/fla) are not part of
the product -- asking for one raises.
"""
from __future__ import annotations

from functools import partial

import torch

from . import fused, scan_hip, stream
from .dispatch import HipOp

_REGISTRY = {"hip": scan_hip.linattn}
PORTABLE = ("naive", "quad", "chunk", "cumsum", "fla")


def resolve_backend(
    name: str,
    decay_gate: str = "off",
    accumulation: str = "sum",
    device: torch.device | str | None = None,
    require_scalar_decay: bool = False,
) -> str:
    """``auto`` -> ``hip`` (interface.py:12-39 resolves ``auto`` -> ``chunk``)."""
    if name == "auto":
        return "hip"
    if name in PORTABLE:
        raise NotImplementedError(
            f"backend {name!r} is a portable reference backend; the MI355X build ships only 'hip'"
        )
    if name not in _REGISTRY:
        raise ValueError(f"unknown scan backend {name!r}")
    return name


def _fn(backend: str, chunk: int = scan_hip.DEFAULT_CHUNK):
    """Backend name -> ``linattn``-style callable (interface.py:42-47)."""
    if backend not in _REGISTRY:
        resolve_backend(backend)
    return partial(scan_hip.linattn, chunk=chunk)


def ema_cumsum(x: torch.Tensor, log_alpha: torch.Tensor, chunk: int = 64) -> torch.Tensor:
    """z_t = sum_{i<=t} alpha^(t-i) x_i with static alpha[H] (interface.py:58-93)."""
    return _prefix(x, log_alpha)


def causal_prefix_sum(x: torch.Tensor) -> torch.Tensor:
    """Prefix sum along T (interface.py:96-107)."""
    return _prefix(x, None)


def decayed_prefix(x: torch.Tensor, decay: torch.Tensor) -> torch.Tensor:
    """z_t = sum_{i<=t} prod_{i<j<=t} a_j x_i for a [B,H,T,1] log-decay stream
    (the unit query/key scan of interface.py:229-230)."""
    return _prefix(x, decay)


def _prefix(x: torch.Tensor, retention: torch.Tensor | None) -> torch.Tensor:
    carry = stream.active()
    if carry is None:
        return _wcumsum_op(x, retention, False).to(x.dtype)
    # continued from the previous call's last row c: z_t = local_t + w_t c,
    # w_t = 1 (plain), alpha^(t+1) (static) or prod_{j<=t} a_j (stream)
    z = fused.wcumsum(x, retention, False)
    c = carry.take()
    if c is not None:
        T = x.shape[2]
        if retention is None:
            w = torch.ones(1, 1, T, 1, dtype=torch.float32, device=x.device)
        elif retention.ndim == 4:
            w = retention.float().cumsum(2).exp()
        else:
            t1 = torch.arange(1, T + 1, dtype=torch.float32, device=x.device)
            w = (retention.float().view(1, -1, 1, 1) * t1.view(1, 1, T, 1)).exp()
        z = z + w * c.unsqueeze(2)
    if x.shape[2]:
        carry.put(z[:, :, -1].clone())
    else:
        carry.put(c if c is not None else z.new_zeros(*x.shape[:2], x.shape[-1]))
    return z.to(x.dtype)


# The decayed prefix as an autograd node (dispatch.HipOp) with its transposed
# (anti-causal) backward.  The forward returns the fp32 prefix; the caller
# casts.

def _wcumsum_forward(x: torch.Tensor, retention: torch.Tensor | None, reverse: bool) -> torch.Tensor:
    return fused.wcumsum(x, retention, reverse)


def _wcumsum_fake(x, retention, reverse):
    return x.new_empty(x.shape, dtype=torch.float32)


def _wcumsum_backward_impl(grad: torch.Tensor, retention: torch.Tensor | None, out: torch.Tensor, reverse: bool,
                           need_retention: bool) -> list[torch.Tensor]:
    gx = fused.wcumsum(grad, retention, not reverse)
    if retention is None or not need_retention:
        return [gx, gx.new_empty(0)]
    # z_t = a_t z_{t-1} + x_t  =>  dL/dlog a_t = gx_t * a_t z_{t-1}
    z_prev = torch.zeros_like(out)
    if reverse:
        z_prev[:, :, :-1] = out[:, :, 1:]
    else:
        z_prev[:, :, 1:] = out[:, :, :-1]
    if retention.ndim == 4:
        a = retention.to(torch.float32).exp()
        if reverse:
            a_shift = torch.zeros_like(a)
            a_shift[:, :, :-1] = a[:, :, 1:]
            a = a_shift
        gl = (gx * z_prev).sum(-1, keepdim=True) * a
        if reverse:
            shifted = torch.zeros_like(gl)
            shifted[:, :, 1:] = gl[:, :, :-1]
            gl = shifted
        return [gx, gl.to(retention.dtype)]
    a = retention.to(torch.float32).exp().view(1, -1, 1, 1)
    gret = ((gx * z_prev).sum(dim=(0, 2, 3)) * a.view(-1)).to(retention.dtype).view_as(retention)
    return [gx, gret]


def _wcumsum_backward_fake(grad, retention, out, reverse, need_retention):
    if retention is None or not need_retention:
        return [torch.empty_like(grad, dtype=torch.float32), grad.new_empty(0)]
    return [torch.empty_like(grad, dtype=torch.float32), torch.empty_like(retention)]


def _wcumsum_setup(ctx, inputs, output):
    x, retention, reverse = inputs
    ctx.reverse = reverse
    ctx.x_dtype = x.dtype
    ctx.need_retention = retention is not None and retention.requires_grad
    ctx.save_for_backward(retention, output)


def _wcumsum_backward(ctx, grad, bwd):
    retention, out = ctx.saved_tensors
    gx, gret = bwd(grad.float(), retention, out, ctx.reverse, ctx.need_retention)
    return gx.to(ctx.x_dtype), (gret if ctx.need_retention else None), None


_wcumsum_op = HipOp("wcumsum", forward=_wcumsum_forward, forward_fake=_wcumsum_fake,
                    backward_impl=_wcumsum_backward_impl, backward_fake=_wcumsum_backward_fake,
                    setup=_wcumsum_setup, backward=_wcumsum_backward)


def _retention_stream(retention, like: torch.Tensor):
    """[H] -> [B,H,T,1] (interface.py:110-117)."""
    if retention is None or retention.ndim == 4:
        return retention
    heads = like.shape[1]
    return retention.to(dtype=like.dtype, device=like.device).view(1, heads, 1, 1).expand(
        like.shape[0], heads, like.shape[2], 1
    )


def _dedupe(views, key_kind):
    terms = [view.scan_terms(key_kind) for view in views]
    retentions: list = []
    slots = []
    for view_terms in terms:
        row = []
        for _, retention in view_terms:
            slot = next((i for i, r in enumerate(retentions) if r is retention), None)
            if slot is None:
                slot = len(retentions)
                retentions.append(retention)
            row.append(slot)
        slots.append(tuple(row))
    return terms, retentions, slots


def _combine(terms, slots, scanned, zeros):
    outputs = []
    for view_terms, view_slots in zip(terms, slots):
        if not view_terms:
            outputs.append(zeros())
            continue
        total = None
        for (coefficient, _), slot in zip(view_terms, view_slots):
            piece = scanned[slot]
            piece = piece if coefficient == 1.0 else coefficient * piece
            total = piece if total is None else total + piece
        outputs.append(total)
    return tuple(outputs)


def _subtracts(terms) -> bool:
    """Whether some view is a difference of scans (a stale view)."""
    return any(c < 0 for view_terms in terms for c, _ in view_terms)


def scan_views(views, q, k, v, key_kind: str) -> tuple:
    """Scan one stream set through several temporal views (interface.py:120-195).

    Each distinct retention is scanned once by the hip backend and every view
    is assembled as its signed combination of those scans.  A difference of
    scans (a stale view: plain - fast, nearly equal over recent tokens) is
    formed from fp32 scan outputs and rounded once.
    """
    terms, retentions, slots = _dedupe(views, key_kind)

    def zeros():
        return v.new_zeros(*q.shape[:3], v.shape[-1])

    if not retentions:
        return tuple(zeros() for _ in views)
    contributing = next(view for view, view_terms in zip(views, terms) if view_terms)
    chunk = getattr(contributing, "chunk", scan_hip.DEFAULT_CHUNK)
    f32 = _subtracts(terms)
    scanned = scan_hip.linattn_views(q, k, v, tuple(retentions), chunk, out_f32=f32)
    out = _combine(terms, slots, scanned, zeros)
    return tuple(o.to(q.dtype) for o in out) if f32 else out


def scan_views_mass(views, q, k, v, key_kind: str) -> tuple:
    """Like :func:`scan_views` against ``cat([v, 1])``, returning ``(num, mass)``
    per view without materialising the unit column (engine.py:430-442).  A
    difference of scans keeps its numerator in fp32 (masses are fp32)."""
    terms, retentions, slots = _dedupe(views, key_kind)

    def zeros():
        return v.new_zeros(*q.shape[:3], v.shape[-1])

    def zmass():
        return torch.zeros(*q.shape[:3], dtype=torch.float32, device=q.device)

    if not retentions:
        return tuple((zeros(), zmass()) for _ in views)
    contributing = next(view for view, view_terms in zip(views, terms) if view_terms)
    chunk = getattr(contributing, "chunk", scan_hip.DEFAULT_CHUNK)
    pairs = scan_hip.linattn_views_mass(q, k, v, tuple(retentions), chunk, out_f32=_subtracts(terms))
    nums = _combine(terms, slots, [p[0] for p in pairs], zeros)
    masses = _combine(terms, slots, [p[1] for p in pairs], zmass)
    return tuple(zip(nums, masses))


class Accumulator:
    """Plain / EMA / static-bank accumulation context (interface.py:198-248)."""

    def __init__(self, backend: str, decay_d=None, decay_m=None, eps: float = 1e-6,
                 chunk: int = scan_hip.DEFAULT_CHUNK, static_log_alpha=None):
        self.backend = backend
        self.decay = {"d": decay_d, "m": decay_m}
        self.eps = eps
        self.chunk = chunk
        self.static_log_alpha = static_log_alpha

    def mass_cum(self, keys: torch.Tensor) -> torch.Tensor:
        decay = self.decay["m"]
        if decay is None:
            return causal_prefix_sum(keys)
        if self.static_log_alpha is not None:
            return ema_cumsum(keys, self.static_log_alpha, self.chunk)
        return decayed_prefix(keys, decay)

    def retention_m(self):
        """The retention of this view's key prefix: None, static [H] or per-token [B,H,T,1]."""
        if self.decay["m"] is None:
            return None
        return self.static_log_alpha if self.static_log_alpha is not None else self.decay["m"]

    def abs_mass(self, query: torch.Tensor, keys: torch.Tensor):
        """sum_j |query_j| (this view's decayed prefix of |keys|)_j in fp32 on
        one HIP launch per direction, or None where that op does not apply
        (continuation, a retention that takes a gradient, other widths)."""
        ret = self.retention_m()
        if stream.active() is not None or not fused.abs_mass_eligible(query, keys, ret):
            return None
        return fused.abs_mass(query, keys, ret)

    def scan_terms(self, key_kind: str):
        decay = self.decay[key_kind]
        if decay is None:
            return ((1.0, None),)
        if self.static_log_alpha is not None:
            return ((1.0, self.static_log_alpha),)
        return ((1.0, decay),)

    def __call__(self, q, k, v, key_kind: str):
        return scan_views((self,), q, k, v, key_kind)[0]


class FadeStale:
    """Stale view S_slow - S_fast (interface.py:251-279)."""

    def __init__(self, slow: Accumulator, fast: Accumulator, log_alpha: torch.Tensor, chunk: int = 64):
        self.slow, self.fast = slow, fast
        self.log_alpha = log_alpha
        self.chunk = chunk

    @property
    def backend(self) -> str:
        return self.slow.backend

    def scan_terms(self, key_kind: str):
        return self.slow.scan_terms(key_kind) + tuple(
            (-coefficient, retention) for coefficient, retention in self.fast.scan_terms(key_kind)
        )

    def __call__(self, q, k, v, key_kind: str):
        return scan_views((self,), q, k, v, key_kind)[0]

    def mass_cum(self, keys: torch.Tensor) -> torch.Tensor:
        # the difference of two nearly equal prefixes is formed in fp32
        k32 = keys.float()
        return (causal_prefix_sum(k32) - ema_cumsum(k32, self.log_alpha, self.chunk)).to(keys.dtype)

    def abs_mass(self, query: torch.Tensor, keys: torch.Tensor):
        if (stream.active() is not None or not fused.abs_mass_eligible(query, keys, None)
                or not fused.abs_mass_eligible(query, keys, self.log_alpha)):
            return None
        return fused.abs_mass(query, keys, None) - fused.abs_mass(query, keys, self.log_alpha)


class FadeFast:
    """Recency view (interface.py:282-307)."""

    def __init__(self, fast: Accumulator, log_alpha: torch.Tensor, chunk: int = 64):
        self.fast = fast
        self.log_alpha = log_alpha
        self.chunk = chunk

    @property
    def backend(self) -> str:
        return self.fast.backend

    def scan_terms(self, key_kind: str):
        return self.fast.scan_terms(key_kind)

    def __call__(self, q, k, v, key_kind: str):
        return scan_views((self,), q, k, v, key_kind)[0]

    def mass_cum(self, keys: torch.Tensor) -> torch.Tensor:
        return ema_cumsum(keys, self.log_alpha, self.chunk)

    def abs_mass(self, query: torch.Tensor, keys: torch.Tensor):
        if stream.active() is not None or not fused.abs_mass_eligible(query, keys, self.log_alpha):
            return None
        return fused.abs_mass(query, keys, self.log_alpha)


class NullAccumulator:
    """Zero-memory view (interface.py:310-327)."""

    backend = "hip"
    chunk = scan_hip.DEFAULT_CHUNK

    def scan_terms(self, key_kind: str):
        return ()

    def __call__(self, q, k, v, key_kind: str):
        return v.new_zeros(*q.shape[:3], v.shape[-1])

    def mass_cum(self, keys: torch.Tensor) -> torch.Tensor:
        return torch.zeros_like(keys)
