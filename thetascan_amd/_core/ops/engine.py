"""Write streams and dual-form read of the ThetaScan memory on the hip backend.

Host-side mirror of src/thetascan/_core/ops/engine.py:117-553 for every
configuration the public API accepts (both families, any depth, one or two
Jacobian steps, all read normalizations, value anchors).  Every scan goes
through ``interface.scan_views`` / ``scan_views_mass`` (the HIP chunked scan),
and key masses through the HIP decayed prefix sum.  Depth-1 ReLU^2 GN writes
and reads run in the HIP GN kernels (``gn.write``, ``gn.read_stage``,
``gn.normalized_read``); the depth-1 kernel-memory hot path bypasses this
module entirely (see ``fused.kernel_mixer``).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from . import gn, interface, kernel_features
from .linear import head_matmul
from ..modules.norms import rmsnorm


def _ein_w(W, x, pat):
    """Per-head GEMV of a [B,H,T,*] stream; the GPU forms run as batched GEMMs
    (linear.head_matmul)."""
    if x.is_cuda and x.ndim == 4 and W.ndim == 3 and W.shape[0] in (1, x.shape[1]):
        if pat in ("hmd,bhtd->bhtm", "hdm,bhtm->bhtd"):
            return head_matmul(x, W, True)
        if pat == "hdm,bhtd->bhtm":
            return head_matmul(x, W, False)
    if W.shape[0] == 1 and x.shape[1] != 1:
        W = W.expand(x.shape[1], -1, -1)
    return torch.einsum(pat, W, x)


def _gain_for(softmax_gain, cfg, reference):
    gain = cfg.softmax_gain if softmax_gain is None else softmax_gain
    if not torch.is_tensor(gain) or gain.ndim == 0:
        return gain
    return kernel_features.head_parameter(gain, reference)


def relu2(pre):
    r = F.relu(pre)
    return r * r


def drelu2(pre, h):
    return 2.0 * F.relu(pre)


def dsilu(pre, h=None):
    s = torch.sigmoid(pre)
    return s * (1 + pre * (1 - s))


def dtanh(pre, h):
    return 1.0 - h * h


# sigma and sigma'(pre, h) of the GN hidden layer (nonlin.py:28-31; tanh has no
# counterpart in the reference)
ELEMENTWISE = {"relu2": (relu2, drelu2), "silu": (F.silu, dsilu), "tanh": (torch.tanh, dtanh)}


def damping(cfg) -> float:
    """The Jacobi diagonal's damping: the reference's is eps (engine.py:255)."""
    return cfg.eps if cfg.gn_damping is None else float(cfg.gn_damping)


def key_mass(cfg, view, qf, keys, mass):
    """The mass a normalized read divides by, num / (mass + eps)
    (engine.py:440-442, 503-506): the scan's unit column ``mass`` for the
    reference's nonnegative features.  tanh features are signed, so their
    products cancel and that column can cross zero; the mass is then the one
    of the absolute features, sum_i w_i |qf| . |k_i| = |qf| . (the view's
    decayed prefix of |k|) in fp32 [B,H,T], equal to the unit column for
    nonnegative features, and |num| / mass <= max |value|."""
    if cfg.nonlin != "tanh":
        return mass
    return (qf.abs().float() * view.mass_cum(keys.abs().float())).sum(-1)


def hrot_stream(h, hrot):
    """Feature-space RoPE of an LA2 stream (engine.py:74-86)."""
    if hrot is None:
        return h
    cos, sin, rot = hrot
    h1, h2 = h[..., :rot:2], h[..., 1:rot:2]
    out = torch.stack((h1 * cos - h2 * sin, h1 * sin + h2 * cos), dim=-1).flatten(-2)
    return torch.cat([out, h[..., rot:]], dim=-1)


@dataclass
class BlockCtx:
    x: torch.Tensor
    pre: torch.Tensor
    h: torch.Tensor
    inv_a: torch.Tensor
    preb: torch.Tensor | None = None
    inv_b: torch.Tensor | None = None


@dataclass
class Streams:
    la1: list = field(default_factory=list)
    la2: list = field(default_factory=list)


def _features(pre, cfg, softmax_gain, controls):
    if cfg.write_rule == "kernel":
        controls = controls or {}
        return kernel_features.feature_map(
            pre, cfg, softmax_gain=softmax_gain, spline_scale=controls.get("spline_scale"),
            score_bias=controls.get("score_bias"), relu2_threshold=controls.get("relu2_threshold"),
            relative_threshold=controls.get("relative_threshold"),
            sparse_blend_alpha=controls.get("sparse_blend_alpha"),
        )
    if cfg.nonlin == "softmax_hidden":
        return torch.softmax(pre * _gain_for(softmax_gain, cfg, pre), dim=-1)
    return ELEMENTWISE[cfg.nonlin][0](pre)


def _threshold(pre, Wg, cfg):
    if cfg.learn_thresh:
        return pre - Wg[..., 0].unsqueeze(0).unsqueeze(2).to(pre.dtype)
    return pre


def _block_forward(W1, W2, Wg, cfg, x, delta=None, softmax_gain=None, kernel_controls=None):
    """engine.py:117-158"""
    a = _ein_w(W1, x, "hmd,bhtd->bhtm")
    if delta is not None:
        a = a + delta["g_a"] * (delta["x0"] * x).sum(-1, keepdim=True)
    if cfg.nonlin == "swiglu":
        b = _ein_w(Wg, x, "hmd,bhtd->bhtm")
        if delta is not None:
            b = b + delta["g_b"] * (delta["x0"] * x).sum(-1, keepdim=True)
        pre, inv_a = rmsnorm(a, cfg.eps)
        preb, inv_b = rmsnorm(b, cfg.eps)
        ctx = BlockCtx(x=x, pre=pre, h=F.silu(preb) * pre, inv_a=inv_a, preb=preb, inv_b=inv_b)
    else:
        pre, inv_a = rmsnorm(a, cfg.eps)
        pre = _threshold(pre, Wg, cfg)
        ctx = BlockCtx(x=x, pre=pre, h=_features(pre, cfg, softmax_gain, kernel_controls), inv_a=inv_a)
    u = _ein_w(W2, ctx.h, "hdm,bhtm->bhtd")
    if delta is not None:
        u = u + delta["lam_hat"] * (delta["h0"] * ctx.h).sum(-1, keepdim=True)
    return u, ctx


def _forward_theta0(weights, cfg, k, deltas=None, softmax_gain=None, kernel_controls=None):
    s = 1.0 / math.sqrt(cfg.depth)
    x, ctxs = k, []
    for l, (W1, W2, Wg) in enumerate(weights):
        u, ctx = _block_forward(W1, W2, Wg, cfg, x, None if deltas is None else deltas[l],
                                softmax_gain=softmax_gain, kernel_controls=kernel_controls)
        ctxs.append(ctx)
        x = x + s * u
    return x, ctxs


def _g_from_lambda(W2, cfg, ctx, lam):
    """S^T (W2^T lam) (engine.py:180-195)."""
    u2 = _ein_w(W2, lam, "hdm,bhtd->bhtm")
    if cfg.nonlin == "softmax_hidden":
        hu = ctx.h * u2
        return (hu - ctx.h * hu.sum(-1, keepdim=True)) * (ctx.inv_a * cfg.softmax_gain)
    if cfg.nonlin == "swiglu":
        return torch.cat([F.silu(ctx.preb) * u2 * ctx.inv_a,
                          ctx.pre * dsilu(ctx.preb) * u2 * ctx.inv_b], dim=-1)
    return ELEMENTWISE[cfg.nonlin][1](ctx.pre, ctx.h) * u2 * ctx.inv_a


def _lambda_solve(weights, cfg, ctxs, r):
    """Jacobi-preconditioned residual (engine.py:215-255)."""
    diag = None
    for (W1, W2, Wg), c in zip(weights, ctxs):
        hh = (c.h * c.h).sum(-1, keepdim=True)
        xx = (c.x * c.x).sum(-1, keepdim=True)
        if cfg.nonlin == "softmax_hidden":
            s2 = c.h * c.h
            A = _ein_w(W2 * W2, s2, "hdm,bhtm->bhtd")
            Bv = _ein_w(W2, s2, "hdm,bhtm->bhtd")
            cv = _ein_w(W2, c.h, "hdm,bhtm->bhtd")
            rowsq = (c.inv_a * cfg.softmax_gain) ** 2 * (A - 2.0 * cv * Bv + cv * cv * s2.sum(-1, keepdim=True))
        else:
            if cfg.nonlin == "swiglu":
                sa = F.silu(c.preb) * c.inv_a
                sb = c.pre * dsilu(c.preb) * c.inv_b
                s2 = sa * sa + sb * sb
            else:
                sv = ELEMENTWISE[cfg.nonlin][1](c.pre, c.h) * c.inv_a
                s2 = sv * sv
            rowsq = _ein_w(W2 * W2, s2, "hdm,bhtm->bhtd")
        term = hh + xx * rowsq
        diag = term if diag is None else diag + term
    return r / (diag / cfg.depth + damping(cfg))


def write_streams(weights, cfg, k, v, hrot=None, softmax_gain=None, kernel_controls=None):
    """Per-token write streams (engine.py:260-340) -> (Streams, ctxs, o).

    Depth-1 ReLU^2 GN memories run the whole write in the HIP GN kernel
    (``gn.write``); ``ctxs`` and ``o`` are then ``None`` (no caller reads them).
    """
    s = 1.0 / math.sqrt(cfg.depth)
    if gn.eligible(cfg, weights, k, v):
        W1, W2, Wg = weights[0]
        tau = Wg[..., 0] if cfg.learn_thresh else None
        h, lam_hat, g = gn.write(k, v, W1, W2, tau, s=s, inv_depth=1.0 / cfg.depth, eps=cfg.eps,
                                 nonlin=cfg.nonlin, damping=damping(cfg))
        streams = Streams()
        streams.la1.append((k, g) if cfg.fast_w1 else None)
        streams.la2.append((hrot_stream(h, hrot), lam_hat))
        return streams, None, None
    m = weights[0][1].shape[-1]
    o, ctxs = _forward_theta0(weights, cfg, k, softmax_gain=softmax_gain, kernel_controls=kernel_controls)
    hks = [hrot_stream(c.h, hrot) for c in ctxs] if hrot is not None else None
    if cfg.write_rule == "kernel":
        if cfg.value_centers:
            Cv = weights[0][2]
            Cve = Cv if Cv.shape[0] == v.shape[1] else Cv.expand(v.shape[1], -1, -1)
            vn = v / v.norm(dim=-1, keepdim=True).clamp_min(cfg.eps)
            lam = torch.softmax(cfg.softmax_gain * torch.einsum("hvd,bhtd->bhtv", Cve, vn), -1).to(v.dtype)
        else:
            lam = v
    else:
        lam = _lambda_solve(weights, cfg, ctxs, v - o)
    streams = Streams()
    deltas = []
    for l, (W1, W2, Wg) in enumerate(weights):
        lam_hat = s * lam
        if cfg.fast_w1:
            g = s * _g_from_lambda(W2, cfg, ctxs[l], lam)
            streams.la1.append((ctxs[l].x, g))
            deltas.append({"x0": ctxs[l].x, "h0": ctxs[l].h, "lam_hat": lam_hat, "g_a": g[..., :m],
                           "g_b": g[..., m:] if g.shape[-1] > m else None})
        else:
            streams.la1.append(None)
        key_h = ctxs[l].h if hks is None else hks[l]
        if cfg.write_rule == "kernel":
            key_h = key_h.to(lam_hat.dtype)
        streams.la2.append((key_h, lam_hat))
    if cfg.write_iters == 2:
        o2, ctxs2 = _forward_theta0(weights, cfg, k, deltas=deltas, softmax_gain=softmax_gain,
                                    kernel_controls=kernel_controls)
        lam2 = _lambda_solve(weights, cfg, ctxs2, v - o2)
        hks2 = [hrot_stream(c.h, hrot) for c in ctxs2] if hrot is not None else None
        for l, (W1, W2, Wg) in enumerate(weights):
            streams.la1.append((ctxs2[l].x, s * _g_from_lambda(W2, cfg, ctxs2[l], lam2)))
            streams.la2.append((ctxs2[l].h if hks2 is None else hks2[l], s * lam2))
    return streams, ctxs, o


def _normalized(num, mass, eps, dtype):
    """num / (mass + eps) in fp32 (mass is an fp32 scan column), in ``dtype``."""
    return (num.float() / (mass.unsqueeze(-1).float() + eps)).to(dtype)


def dual_read_views(weights, cfg, q, streams, views, hrot=None, softmax_gain=None, kernel_controls=None):
    """f_{theta_t}(q_t) for several temporal views (engine.py:345-544)."""
    s = 1.0 / math.sqrt(cfg.depth)
    L, m = cfg.depth, weights[0][1].shape[-1]
    n_iter = cfg.write_iters

    def features(a, b, Wg):
        if cfg.nonlin == "swiglu":
            h = F.silu(rmsnorm(b, cfg.eps)[0]) * rmsnorm(a, cfg.eps)[0]
        else:
            h = _features(_threshold(rmsnorm(a, cfg.eps)[0], Wg, cfg), cfg, softmax_gain, kernel_controls)
        return h, hrot_stream(h, hrot)

    def memory(group, l, Wg, hq):
        shared = not isinstance(hq, list)
        queries = [hq] * len(group) if shared else hq
        if not cfg.read_norm:
            terms = []
            for it in range(n_iter):
                keys, vals = streams.la2[it * L + l]
                if shared:
                    scanned = interface.scan_views(group, hq, keys, vals, "m")
                else:
                    scanned = [interface.scan_views((view,), one, keys, vals, "m")[0]
                               for view, one in zip(group, queries)]
                terms = list(scanned) if not terms else [a + b for a, b in zip(terms, scanned)]
            mems = terms
        else:
            keys, vals = streams.la2[l]
            if cfg.read_norm_mode == "key_mass":
                if shared:
                    pairs = interface.scan_views_mass(group, hq.to(keys.dtype), keys, vals, "m")
                else:
                    pairs = [interface.scan_views_mass((view,), one.to(keys.dtype), keys, vals, "m")[0]
                             for view, one in zip(group, queries)]
                mems = [_normalized(num, key_mass(cfg, view, one, keys, mass), cfg.eps, vals.dtype)
                        for view, one, (num, mass) in zip(group, queries, pairs)]
            else:
                mems = []
                for view, one in zip(group, queries):
                    kcum = view.mass_cum(keys.to(one.dtype))
                    mems.append(interface.scan_views((view,), (one / (kcum + cfg.eps)).to(keys.dtype),
                                                     keys, vals, "m")[0])
        if cfg.value_centers:
            Cve = Wg if Wg.shape[0] == q.shape[1] else Wg.expand(q.shape[1], -1, -1)
            mems = [torch.einsum("hvd,bhtv->bhtd", Cve.to(mem.dtype), mem) for mem in mems]
        return mems

    gn_read = gn.read_eligible(cfg, weights, q)

    def gn_layer(group, l, x):
        """Depth-1 ReLU^2 GN read on the HIP read stages (engine.py:467-544)."""
        W1, W2, Wg = weights[l]
        tau = Wg[..., 0] if cfg.learn_thresh else None
        entry = streams.la1[l]
        keys, vals = streams.la2[l]
        if cfg.read_norm_w1:
            if entry is None:
                raise RuntimeError("read_norm_w1 requires an LA1 GN stream")
            h0, _ = gn.read_stage(x, W1, tau=tau, eps=cfg.eps)
            h0q = hrot_stream(h0, hrot).to(keys.dtype)
            pairs = interface.scan_views_mass(group, h0q, keys, entry[1], "m")
            stage = [(num, key_mass(cfg, view, h0q, keys, mass), gn.READ_NORMALIZED)
                     for view, (num, mass) in zip(group, pairs)]
        elif entry is not None:
            corrs = interface.scan_views(group, x, entry[0], entry[1], "d")
            stage = [(corr[..., :m], None, gn.READ_PLAIN) for corr in corrs]
        else:
            stage = [(None, None, gn.READ_NONE)] * len(group)
        outputs = []
        for view, (num1, mass1, corr) in zip(group, stage):
            h, resid = gn.read_stage(x, W1, W2, tau, num1, mass1, corr=corr, want_resid=True, s=s, eps=cfg.eps,
                                     nonlin=cfg.nonlin)
            hq = hrot_stream(h, hrot).to(keys.dtype)
            if cfg.read_norm:
                (num2, mass2), = interface.scan_views_mass((view,), hq, keys, vals, "m")
                mass2 = key_mass(cfg, view, hq, keys, mass2)
            else:
                num2, mass2 = interface.scan_views((view,), hq, keys, vals, "m")[0], None
            outputs.append(gn.normalized_read(num2, mass2, resid, s=s, eps=cfg.eps))
        return outputs

    def layer(group, l, x):
        if gn_read:
            return gn_layer(group, l, x)
        W1, W2, Wg = weights[l]
        a = _ein_w(W1, x, "hmd,bhtd->bhtm")
        b = _ein_w(Wg, x, "hmd,bhtd->bhtm") if cfg.nonlin == "swiglu" else None
        preacts = bs = None
        if cfg.read_norm_w1:
            pre0 = _threshold(rmsnorm(a, cfg.eps)[0], Wg, cfg)
            h0q = hrot_stream(relu2(pre0), hrot)
            feature_keys = streams.la2[l][0]
            entry = streams.la1[l]
            if entry is None:
                raise RuntimeError("read_norm_w1 requires an LA1 GN stream")
            h0q = h0q.to(feature_keys.dtype)
            pairs = interface.scan_views_mass(group, h0q, feature_keys, entry[1], "m")
            preacts = [a + _normalized(num, key_mass(cfg, view, h0q, feature_keys, mass), cfg.eps, a.dtype)[..., :m]
                       for view, (num, mass) in zip(group, pairs)]
            bs = [b] * len(group)
        else:
            for it in range(n_iter):
                entry = streams.la1[it * L + l]
                if entry is None:
                    continue
                corrs = interface.scan_views(group, x, entry[0], entry[1], "d")
                if preacts is None:
                    preacts, bs = [a] * len(group), [b] * len(group)
                preacts = [pre + corr[..., :m] for pre, corr in zip(preacts, corrs)]
                if b is not None:
                    bs = [one + corr[..., m:] for one, corr in zip(bs, corrs)]
        if preacts is None:
            h, hq = features(a, b, Wg)
            base = _ein_w(W2, h, "hdm,bhtm->bhtd")
            if (n_iter == 1 and not cfg.value_centers and x.is_cuda and x.dtype in (torch.bfloat16, torch.float32)
                    and (not cfg.read_norm or cfg.read_norm_mode == "key_mass")):
                # x + s (W2 h + num / (mass + eps)) per view on the HIP read
                # kernel, the residual x + s W2 h formed once for every view
                resid = torch.add(x, base, alpha=s)
                keys, vals = streams.la2[l]
                if cfg.read_norm:
                    hq = hq.to(keys.dtype)
                    pairs = [(num, key_mass(cfg, view, hq, keys, mass))
                             for view, (num, mass) in zip(group, interface.scan_views_mass(group, hq, keys, vals, "m"))]
                else:
                    pairs = [(num, None) for num in interface.scan_views(group, hq, keys, vals, "m")]
                return [gn.normalized_read(num, mass, resid, s=s, eps=cfg.eps) for num, mass in pairs]
            return [x + s * (base + mem) for mem in memory(group, l, Wg, hq)]
        outputs = []
        for view, pre, one_b in zip(group, preacts, bs):
            h, hq = features(pre, one_b, Wg)
            base = _ein_w(W2, h, "hdm,bhtm->bhtd")
            outputs.append(x + s * (base + memory([view], l, Wg, hq)[0]))
        return outputs

    xs = [q] * len(views)
    for l in range(L):
        if all(one is xs[0] for one in xs):
            xs = layer(list(views), l, xs[0])
        else:
            xs = [layer([view], l, one)[0] for view, one in zip(views, xs)]
    return tuple(xs)


def dual_read(weights, cfg, q, streams, acc, hrot=None, softmax_gain=None, kernel_controls=None):
    """Single-view :func:`dual_read_views` (engine.py:547-553)."""
    return dual_read_views(weights, cfg, q, streams, (acc,), hrot=hrot, softmax_gain=softmax_gain,
                           kernel_controls=kernel_controls)[0]
