"""The composed path of the ThetaScan memory on the hip backend.

This serves every configuration the public API accepts that the one-call and
multi-view feature-kernel paths do not: both memory families, any depth, one
or two Jacobian steps, all read normalizations and value anchors.  The
semantics are those of src/thetascan/_core/ops/engine.py:117-553; the
organisation is this module's own:

* ``FastNet`` is the fast network at its slow weights.  It evaluates one
  block's activation (``Act``) at a stream of block inputs, the block's output
  W2 h, the Jacobian-transpose payload S^T W2^T lam of a write, and the
  block's share of the Gauss-Newton diagonal.
* ``FastNet.deposits`` turns keys and values into the payload channels of the
  write: one ``Deposit`` per (Jacobian step, layer), holding the LA2 channel
  (rotated hidden features -> s lam) and, when W1 is fast, the LA1 channel
  (block input -> s S^T W2^T lam).
* ``FastNet.recall`` reads every temporal view through those channels, layer
  by layer; views share every tensor until a view-dependent correction enters
  a query, and the scans of shared queries form each score tile once.

What runs where: every scan in ``interface.scan_views`` / ``scan_views_mass``
(HIP chunked scans), every decayed key mass in the HIP prefix sum, the
value-anchor deposit (``maps.anchor_code``), the kernel feature maps
(``kernel_features.kmap``, ``maps.bspline_norm_features``), the
depth-1 GN writes and reads of the HIP GN kernels (``gn.write``,
``gn.read_stage``), every other GN block's RMSNorm, nonlinearity and Jacobian
scales (``gn.act_rows``: any depth, both Gauss-Newton steps, SwiGLU), the
normalized read epilogue in ``gn.normalized_read`` (HIP; with one view it
also applies the output gate, see ``GateRequest``) and the per-head GEMMs in
``linear.head_matmul``.  The remaining elementwise work (the
products of the scales with the GEMM outputs, the Jacobi division) is torch
on the GPU.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import gn, interface, kernel_features, maps
from .linear import head_matmul
from ..modules.norms import rmsnorm


# ------------------------------------------------------------------ output gate

class GateRequest:
    """An output gate silu(x W_g^T + b) (block.py:721-722) that the read
    epilogue of a single view may apply.  ``pre`` is the [B,H,T,d] view of
    the pre-activation x W_g^T without the bias, formed on first use (so a
    read that does not take the gate costs no GEMM).  A read that applies
    silu(pre + bias) inside its HIP epilogue writes its output token-major
    (``gn.normalized_read``) and sets ``applied``; otherwise the caller
    applies the gate itself."""

    def __init__(self, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None, heads: int, width: int):
        self.x, self.weight, self.bias = x, weight, bias
        self.heads, self.width = heads, width
        self.applied = False
        self._pre = None

    @property
    def pre(self) -> torch.Tensor:
        if self._pre is None:
            from .linear import linear

            B, T, _ = self.x.shape
            self._pre = linear(self.x, self.weight).view(B, T, self.heads, self.width).transpose(1, 2)
        return self._pre

    def fits(self, num: torch.Tensor, resid: torch.Tensor) -> bool:
        """Whether the HIP read epilogue can apply the gate to this read."""
        B, T, _ = self.x.shape
        return (num.is_cuda and num.dtype in (torch.bfloat16, torch.float32) and resid.dtype == num.dtype
                and self.x.dtype == num.dtype and self.weight.dtype == num.dtype
                and tuple(num.shape) == (B, self.heads, T, self.width) and resid.shape == num.shape)

    def read(self, num, mass, resid, s: float, eps: float) -> torch.Tensor:
        """The gated read epilogue (marks the gate applied)."""
        self.applied = True
        return gn.normalized_read(num, mass, resid, s=s, eps=eps, gate=self.pre, gate_bias=self.bias)


# ------------------------------------------------------------------ per-head products

def _per_head(x: torch.Tensor, W: torch.Tensor, transpose: bool) -> torch.Tensor:
    """x [B,H,T,K] times W^T (``transpose``: W [H|1,N,K]) or W (W [H|1,K,N])
    for every head, as one batched GEMM on the GPU."""
    if x.is_cuda and x.ndim == 4 and W.ndim == 3 and W.shape[0] in (1, x.shape[1]):
        return head_matmul(x, W, transpose)
    Wh = W.expand(x.shape[1], -1, -1) if W.shape[0] == 1 else W
    return torch.matmul(x, (Wh.transpose(-1, -2) if transpose else Wh).unsqueeze(0))


# ------------------------------------------------------------------ nonlinearities

def _relu_sq(z):
    r = F.relu(z)
    return r * r


def _silu_slope(z):
    sg = torch.sigmoid(z)
    return sg * (1 + z * (1 - sg))


# value and slope (as a function of the pre-activation z and the value h) of
# the GN hidden nonlinearities (nonlin.py:28-31; tanh is this build's extension)
_NONLIN = {
    "relu2": (_relu_sq, lambda z, h: 2.0 * F.relu(z)),
    "silu": (F.silu, lambda z, h: _silu_slope(z)),
    "tanh": (torch.tanh, lambda z, h: 1.0 - h * h),
}


def damping(cfg) -> float:
    """The diagonal damping of the Jacobi solve: the reference uses eps
    (engine.py:255); ``gn_damping`` sets its own value."""
    return cfg.eps if cfg.gn_damping is None else float(cfg.gn_damping)


def key_mass(cfg, view, query, keys, unit_mass):
    """The mass a normalized read divides by, num / (mass + eps)
    (engine.py:440-442, 503-506).  For the reference's nonnegative features it
    is the scan's unit column ``unit_mass``.  Signed (tanh) features cancel in
    that column, which can then cross zero; their mass is the one of the
    absolute features, |query| . (the view's decayed prefix of |keys|), in
    fp32 -- equal to the unit column for nonnegative features -- so that
    |num| / mass <= max |value| (one ts_abs_mass launch per direction where
    the view allows it, else torch around the HIP prefix sum)."""
    if cfg.nonlin != "tanh":
        return unit_mass
    mass = view.abs_mass(query, keys) if hasattr(view, "abs_mass") else None
    if mass is not None:
        return mass
    return (query.abs().float() * view.mass_cum(keys.abs().float())).sum(-1)


def _divide(num, mass, eps, dtype):
    """num / (mass + eps) in fp32 (mass is an fp32 scan column), as ``dtype``."""
    return (num.float() / (mass.unsqueeze(-1).float() + eps)).to(dtype)


# ------------------------------------------------------------------ records

@dataclass(frozen=True)
class Act:
    """One block evaluated on a stream of block inputs ``inp``: ``z`` the
    RMS-normed (and thresholded) main pre-activation with ``rz`` = 1/rms,
    ``h`` the hidden features, and for SwiGLU the gate branch ``zg``, ``rzg``.
    A GN block whose activation ran in ts_gn_act carries its Jacobian scales
    instead: ``sa`` = sigma'(z) rz (SwiGLU: silu(zg) rz) and, for SwiGLU,
    ``sb`` = z silu'(zg) rzg."""
    inp: torch.Tensor
    z: torch.Tensor | None
    rz: torch.Tensor | None
    h: torch.Tensor
    zg: torch.Tensor | None = None
    rzg: torch.Tensor | None = None
    sa: torch.Tensor | None = None
    sb: torch.Tensor | None = None


@dataclass(frozen=True)
class Deposit:
    """What one write step leaves for one layer: the LA2 channel (keys
    ``feat``, the rotated hidden features; values ``pay`` = s lam) and, when W1
    is fast, the LA1 channel (keys ``inp``, the block input; values ``jac`` =
    s S^T W2^T lam, [.., m] or [.., 2m] for SwiGLU)."""
    feat: torch.Tensor
    pay: torch.Tensor
    inp: torch.Tensor | None = None
    jac: torch.Tensor | None = None


# ------------------------------------------------------------------ the fast network

class FastNet:
    """The fast network of one mixer forward at its slow weights.

    ``layers``: per depth level (W1 [H|1,m,d], W2 [H|1,d,m], Wg) with Wg the
    SwiGLU gate weights, the learned threshold [H,m,1] or the value codebook
    [1,V,d]; ``hrot``: (cos, sin, rot) of the feature-space RoPE or None;
    ``gain``: the learned softmax sharpness or None; ``controls``: the kernel
    feature map's learned controls."""

    def __init__(self, layers, cfg, hrot=None, gain=None, controls=None, out_gate=None):
        self.layers = layers
        self.cfg = cfg
        self.hrot = hrot
        self.gain = gain
        self.controls = controls or {}
        self.out_gate = out_gate
        self.s = 1.0 / math.sqrt(cfg.depth)
        self.width = layers[0][1].shape[-1]
        self.gated = cfg.nonlin == "swiglu"

    def _scaled(self, t: torch.Tensor) -> torch.Tensor:
        """s * t for the depth scale s = 1 / sqrt(depth): t itself at depth 1
        (the product by 1.0 is the identity, bit for bit)."""
        return t if self.s == 1.0 else self.s * t

    # ---- pieces of one block

    def rotate(self, h):
        """Feature-space RoPE of hidden features (engine.py:74-86): interleaved
        pairs of the first ``rot`` features turn by the token's angles."""
        if self.hrot is None:
            return h
        cos, sin, rot = self.hrot
        even, odd = h[..., :rot:2], h[..., 1:rot:2]
        turned = torch.stack((even * cos - odd * sin, even * sin + odd * cos), dim=-1).flatten(-2)
        return torch.cat([turned, h[..., rot:]], dim=-1)

    def _shift(self, z, l):
        """Subtract the learned per-head threshold tau [H,m] (a constant of x)."""
        if not self.cfg.learn_thresh:
            return z
        tau = self.layers[l][2][..., 0]
        return z - tau.unsqueeze(0).unsqueeze(2).to(z.dtype)

    def hidden(self, z):
        """Hidden features of a normed (thresholded) pre-activation."""
        cfg = self.cfg
        if cfg.write_rule == "kernel":
            c = self.controls
            return kernel_features.feature_map(
                z, cfg, softmax_gain=self.gain, spline_scale=c.get("spline_scale"), score_bias=c.get("score_bias"),
                relu2_threshold=c.get("relu2_threshold"), relative_threshold=c.get("relative_threshold"),
                sparse_blend_alpha=c.get("sparse_blend_alpha"))
        if cfg.nonlin == "softmax_hidden":
            g = cfg.softmax_gain if self.gain is None else self.gain
            if torch.is_tensor(g) and g.ndim > 0:
                g = kernel_features.head_parameter(g, z)
            return torch.softmax(z * g, dim=-1)
        return _NONLIN[cfg.nonlin][0](z)

    def _fused_map(self, a) -> bool:
        """Whether the kernel family's RMSNorm, threshold and feature map (with
        every learned control) run as one HIP launch on ``a`` = W1 x: ts_kmap
        for the softmax partition and the ReLU^2 ridge, ts_bspline_norm for
        the projected B-spline map."""
        if self.cfg.write_rule != "kernel":
            return False
        if self.cfg.kernel_kind == "projected_bspline":
            return maps.bspline_norm_supported(a)
        return kernel_features.kmap_eligible(a, self.cfg)

    def _kmap(self, l, a):
        c = self.controls
        tau = self.layers[l][2][..., 0] if self.cfg.learn_thresh else None
        if self.cfg.kernel_kind == "projected_bspline":
            cfg = self.cfg
            scale = c.get("spline_scale")
            H, P = a.shape[1], a.shape[-1]
            shift = None if tau is None else -tau.float().reshape(-1, P).expand(H, P)
            return maps.bspline_norm_features(a, shift=shift, eps=cfg.eps, n_basis=cfg.bspline_basis_count,
                                              degree=cfg.bspline_degree, bound=cfg.bspline_bound,
                                              scale=cfg.bspline_scale if scale is None else scale)
        return kernel_features.kmap(
            a, self.cfg, rms=True, tau=tau, softmax_gain=self.gain, score_bias=c.get("score_bias"),
            relu2_threshold=c.get("relu2_threshold"), relative_threshold=c.get("relative_threshold"),
            sparse_blend_alpha=c.get("sparse_blend_alpha"))

    def _gn_rows(self, a) -> bool:
        """Whether a GN block's RMSNorm, nonlinearity and Jacobian scales run
        as one ts_gn_act launch on ``a`` = W1 x (relu2, silu, tanh, SwiGLU)."""
        return self.cfg.write_rule == "gn" and gn.act_rows_eligible(a, self.cfg.nonlin)

    def _tau(self, l):
        return self.layers[l][2][..., 0] if self.cfg.learn_thresh and not self.gated else None

    def act(self, l, x, main_shift=None, gate_shift=None):
        """Block ``l`` at inputs ``x``; ``main_shift`` / ``gate_shift`` add to
        the raw pre-activations W1 x / Wg x before the RMSNorm.  A kernel
        memory's features come from one ts_kmap launch (its pre-activation is
        then not kept: only the GN family's Jacobian payloads read it); a GN
        block's features and Jacobian scales from one ts_gn_act launch."""
        W1, _, Wg = self.layers[l]
        a = _per_head(x, W1, True)
        if main_shift is not None:
            a = a + main_shift
        if not self.gated and self._fused_map(a):
            return Act(x, None, None, self._kmap(l, a))
        b = None
        if self.gated:
            b = _per_head(x, Wg, True)
            if gate_shift is not None:
                b = b + gate_shift
        if self._gn_rows(a):
            h, sa, sb = gn.act_rows(a, b, self._tau(l), nonlin=self.cfg.nonlin, eps=self.cfg.eps)
            return Act(x, None, None, h, sa=sa, sb=sb)
        z, rz = rmsnorm(a, self.cfg.eps)
        if self.gated:
            zg, rzg = rmsnorm(b, self.cfg.eps)
            return Act(x, z, rz, F.silu(zg) * z, zg, rzg)
        z = self._shift(z, l)
        return Act(x, z, rz, self.hidden(z))

    def out(self, l, h):
        """The block's output W2 h."""
        return _per_head(h, self.layers[l][1], True)

    def _slope(self, act):
        """dh/da as a per-feature scale for the elementwise nets (1/rms
        included: RMSNorm enters through its scalar factor only)."""
        if act.sa is not None:
            return act.sa
        return _NONLIN[self.cfg.nonlin][1](act.z, act.h) * act.rz

    def _gate_scales(self, act):
        """SwiGLU's two per-feature scales (main branch, gate branch)."""
        if act.sa is not None:
            return act.sa, act.sb
        return F.silu(act.zg) * act.rz, act.z * _silu_slope(act.zg) * act.rzg

    def jac_payload(self, l, act, lam):
        """S^T (W2^T lam): the LA1 values of block ``l`` (engine.py:180-195)."""
        u = _per_head(lam, self.layers[l][1], False)
        cfg = self.cfg
        if cfg.nonlin == "softmax_hidden":
            hu = act.h * u
            return (hu - act.h * hu.sum(-1, keepdim=True)) * (act.rz * cfg.softmax_gain)
        if self.gated:
            sa, sb = self._gate_scales(act)
            return torch.cat([sa * u, sb * u], dim=-1)
        return self._slope(act) * u

    def gram_share(self, l, act):
        """Block ``l``'s term of the Gauss-Newton diagonal, ||h||^2 + ||x||^2
        rowsq(W2 S) (engine.py:215-255)."""
        cfg = self.cfg
        W2 = self.layers[l][1]
        hh = act.h.square().sum(-1, keepdim=True)
        xx = act.inp.square().sum(-1, keepdim=True)
        if cfg.nonlin == "softmax_hidden":
            # softmax Jacobian g (diag h - h h^T): rowsq = g^2 r^2 (A - 2 c B + c^2 S)
            p2 = act.h.square()
            A = _per_head(p2, W2 * W2, True)
            Bv = _per_head(p2, W2, True)
            c = _per_head(act.h, W2, True)
            rowsq = (act.rz * cfg.softmax_gain).square() * (A - 2.0 * c * Bv + c * c * p2.sum(-1, keepdim=True))
        else:
            if self.gated:
                sa, sb = self._gate_scales(act)
                sq = sa * sa + sb * sb
            else:
                sq = self._slope(act).square()
            rowsq = _per_head(sq, W2 * W2, True)
        return hh + xx * rowsq

    # ---- the network at the slow weights

    def run(self, k, own=None):
        """The blocks in sequence on keys ``k`` -> (acts, output).  ``own``:
        the previous step's deposits; each block then adds this token's own
        write of that step (a rank-one correction per token: the second
        Gauss-Newton step linearizes at theta0 + the token's own delta)."""
        acts, x = [], k
        for l in range(len(self.layers)):
            main_shift = gate_shift = out_shift = None
            if own is not None:
                dep = own[l]
                dot = (dep.inp * x).sum(-1, keepdim=True)
                main_shift = dep.jac[..., :self.width] * dot
                if self.gated:
                    gate_shift = dep.jac[..., self.width:] * dot
            act = self.act(l, x, main_shift, gate_shift)
            u = self.out(l, act.h)
            if own is not None:
                u = u + own[l].pay * (own[l].h0 * act.h).sum(-1, keepdim=True)
            acts.append(act)
            x = x + self._scaled(u)
        return acts, x

    def solve(self, acts, residual):
        """Jacobi-preconditioned residual: r / (diag / depth + damping)."""
        diag = sum(self.gram_share(l, act) for l, act in enumerate(acts))
        return residual / (diag / self.cfg.depth + damping(self.cfg))

    # ---- write

    def _anchor_code(self, v):
        """The value-anchor deposit softmax(gain C_v v / max(||v||, eps)) over
        the value codebook (engine.py:284-296): ts_anchor_fwd / ts_anchor_bwd."""
        cfg = self.cfg
        return maps.anchor_code(v, self.layers[0][2], gain=cfg.softmax_gain, eps=cfg.eps)

    def deposits(self, k, v):
        """Per-token payload channels of the write -> ``steps[step][layer]``
        (engine.py:260-340)."""
        cfg = self.cfg
        if gn.eligible(cfg, self.layers, k, v):
            W1, W2, Wg = self.layers[0]
            h, pay, jac = gn.write(k, v, W1, W2, Wg[..., 0] if cfg.learn_thresh else None, s=self.s,
                                   inv_depth=1.0 / cfg.depth, eps=cfg.eps, nonlin=cfg.nonlin, damping=damping(cfg))
            return [[Deposit(self.rotate(h), pay, k if cfg.fast_w1 else None, jac if cfg.fast_w1 else None)]]
        acts, out = self.run(k)
        if cfg.write_rule == "kernel":
            lam = self._anchor_code(v) if cfg.value_centers else v
        else:
            lam = self.solve(acts, v - out)
        steps = [self._step(acts, lam, cast=cfg.write_rule == "kernel")]
        if cfg.write_iters == 2:
            acts2, out2 = self.run(k, own=steps[0])
            steps.append(self._step(acts2, self.solve(acts2, v - out2), cast=False))
        return [[Deposit(d.feat, d.pay, d.inp, d.jac) for d in step] for step in steps]

    def _step(self, acts, lam, cast):
        step = []
        for l, act in enumerate(acts):
            feat = self.rotate(act.h)
            pay = self._scaled(lam)
            if cast:
                feat = feat.to(pay.dtype)
            dep = _Written(feat, pay)
            if self.cfg.fast_w1:
                dep = _Written(feat, pay, act.inp, self._scaled(self.jac_payload(l, act, lam)), act.h)
            step.append(dep)
        return step

    # ---- read

    def recall(self, q, steps, views):
        """f_theta_t(q_t) for every temporal view (engine.py:345-544)."""
        outs = [q] * len(views)
        gate = self.out_gate if len(views) == 1 else None
        for l in range(len(self.layers)):
            last = gate if l == len(self.layers) - 1 else None
            if all(x is outs[0] for x in outs):
                outs = self._read_layer(list(views), l, outs[0], steps, last)
            else:
                outs = [self._read_layer([view], l, x, steps, last)[0] for view, x in zip(views, outs)]
        return tuple(outs)

    def _features_at(self, l, main, gate):
        """Hidden features of raw pre-activations -> (h, rotated h)."""
        eps = self.cfg.eps
        if self._gn_rows(main):
            h = gn.act_rows(main, gate, self._tau(l), nonlin=self.cfg.nonlin, eps=eps, want_scales=False)[0]
        elif self.gated:
            h = F.silu(rmsnorm(gate, eps)[0]) * rmsnorm(main, eps)[0]
        elif self._fused_map(main):
            h = self._kmap(l, main)
        else:
            h = self.hidden(self._shift(rmsnorm(main, eps)[0], l))
        return h, self.rotate(h)

    def _memory(self, group, l, queries, steps):
        """The LA2 read of every view of ``group``: ``queries`` is one rotated
        feature tensor shared by the group, or one per view."""
        cfg = self.cfg
        shared = torch.is_tensor(queries)
        per_view = [queries] * len(group) if shared else queries
        first = steps[0][l]
        if not cfg.read_norm:
            total = None
            for step in steps:
                dep = step[l]
                if shared:
                    got = list(interface.scan_views(group, queries, dep.feat, dep.pay, "m"))
                else:
                    got = [interface.scan_views((view,), one, dep.feat, dep.pay, "m")[0]
                           for view, one in zip(group, per_view)]
                total = got if total is None else [a + b for a, b in zip(total, got)]
            mems = total
        elif cfg.read_norm_mode == "key_mass":
            if shared:
                pairs = interface.scan_views_mass(group, queries.to(first.feat.dtype), first.feat, first.pay, "m")
            else:
                pairs = [interface.scan_views_mass((view,), one.to(first.feat.dtype), first.feat, first.pay, "m")[0]
                         for view, one in zip(group, per_view)]
            mems = [_divide(num, key_mass(cfg, view, one, first.feat, mass), cfg.eps, first.pay.dtype)
                    for view, one, (num, mass) in zip(group, per_view, pairs)]
        else:
            # per-feature normalization: the query is divided by its own view's
            # decayed key mass before the scan
            mems = []
            for view, one in zip(group, per_view):
                kcum = view.mass_cum(first.feat.to(one.dtype))
                mems.append(interface.scan_views((view,), (one / (kcum + cfg.eps)).to(first.feat.dtype),
                                                 first.feat, first.pay, "m")[0])
        if cfg.value_centers:
            book = self.layers[l][2]
            mems = [_per_head(mem, book.to(mem.dtype), False) for mem in mems]
        return mems

    def _read_layer(self, group, l, x, steps, out_gate=None):
        """One depth level for the views of ``group``, which share the input
        ``x``; ``out_gate`` is a ``GateRequest`` the last level may apply."""
        cfg = self.cfg
        if gn.read_eligible(cfg, self.layers, x):
            return self._read_layer_gn(group, l, x, steps, out_gate)
        W1, W2, Wg = self.layers[l]
        m = self.width
        main = _per_head(x, W1, True)
        gate = _per_head(x, Wg, True) if self.gated else None
        mains = gates = None
        if cfg.read_norm_w1:
            # two-stage read: the LA1 payloads addressed by the positive
            # slow-weight features of x against the LA2 keys, normalized by the
            # matched mass, correct the pre-activation
            first = steps[0][l]
            if first.jac is None:
                raise RuntimeError("read_norm_w1 requires an LA1 GN stream")
            if gn.act_rows_eligible(main, "relu2"):
                h0 = gn.act_rows(main, None, self._tau(l), nonlin="relu2", eps=cfg.eps, want_scales=False)[0]
            else:
                h0 = _relu_sq(self._shift(rmsnorm(main, cfg.eps)[0], l))
            probe = self.rotate(h0).to(first.feat.dtype)
            pairs = interface.scan_views_mass(group, probe, first.feat, first.jac, "m")
            mains = [main + _divide(num, key_mass(cfg, view, probe, first.feat, mass), cfg.eps, main.dtype)[..., :m]
                     for view, (num, mass) in zip(group, pairs)]
            gates = [gate] * len(group)
        else:
            for step in steps:
                dep = step[l]
                if dep.jac is None:
                    continue
                corr = interface.scan_views(group, x, dep.inp, dep.jac, "d")
                if mains is None:
                    mains, gates = [main] * len(group), [gate] * len(group)
                mains = [a + c[..., :m] for a, c in zip(mains, corr)]
                if gate is not None:
                    gates = [b + c[..., m:] for b, c in zip(gates, corr)]
        if mains is None:
            h, hq = self._features_at(l, main, gate)
            base = self.out(l, h)
            if (len(steps) == 1 and not cfg.value_centers and x.is_cuda and x.dtype in (torch.bfloat16, torch.float32)
                    and (not cfg.read_norm or cfg.read_norm_mode == "key_mass")):
                # x + s (W2 h + num / (mass + eps)) per view in the HIP read
                # epilogue, the residual x + s W2 h formed once for all views
                return self._normalized_reads(group, l, hq, torch.add(x, base, alpha=self.s), steps, out_gate)
            return [x + self._scaled(base + mem) for mem in self._memory(group, l, hq, steps)]
        outs = []
        for view, a, b in zip(group, mains, gates):
            h, hq = self._features_at(l, a, b)
            outs.append(x + self._scaled(self.out(l, h) + self._memory([view], l, hq, steps)[0]))
        return outs

    def _normalized_reads(self, group, l, hq, resid, steps, out_gate=None):
        cfg = self.cfg
        dep = steps[0][l]
        if cfg.read_norm:
            hq = hq.to(dep.feat.dtype)
            pairs = [(num, key_mass(cfg, view, hq, dep.feat, mass))
                     for view, (num, mass) in zip(group, interface.scan_views_mass(group, hq, dep.feat, dep.pay, "m"))]
        else:
            pairs = [(num, None) for num in interface.scan_views(group, hq, dep.feat, dep.pay, "m")]
        if out_gate is not None and len(pairs) == 1 and out_gate.fits(pairs[0][0], resid):
            return [out_gate.read(pairs[0][0], pairs[0][1], resid, self.s, cfg.eps)]
        return [gn.normalized_read(num, mass, resid, s=self.s, eps=cfg.eps) for num, mass in pairs]

    def _read_layer_gn(self, group, l, x, steps, out_gate=None):
        """A depth-1 GN read on the HIP read stages (engine.py:467-544): stage
        one corrects the pre-activation, stage two reads LA2 with the
        corrected features; the epilogue of a single view applies
        ``out_gate`` where it fits."""
        cfg = self.cfg
        W1, W2, Wg = self.layers[l]
        tau = Wg[..., 0] if cfg.learn_thresh else None
        dep = steps[0][l]
        if cfg.read_norm_w1:
            if dep.jac is None:
                raise RuntimeError("read_norm_w1 requires an LA1 GN stream")
            h0, _ = gn.read_stage(x, W1, tau=tau, eps=cfg.eps)
            probe = self.rotate(h0).to(dep.feat.dtype)
            pairs = interface.scan_views_mass(group, probe, dep.feat, dep.jac, "m")
            stage = [(num, key_mass(cfg, view, probe, dep.feat, mass), gn.READ_NORMALIZED)
                     for view, (num, mass) in zip(group, pairs)]
        elif dep.jac is not None:
            stage = [(corr[..., :self.width], None, gn.READ_PLAIN)
                     for corr in interface.scan_views(group, x, dep.inp, dep.jac, "d")]
        else:
            stage = [(None, None, gn.READ_NONE)] * len(group)
        outs = []
        for view, (num1, mass1, kind) in zip(group, stage):
            h, resid = gn.read_stage(x, W1, W2, tau, num1, mass1, corr=kind, want_resid=True, s=self.s, eps=cfg.eps,
                                     nonlin=cfg.nonlin)
            hq = self.rotate(h).to(dep.feat.dtype)
            if cfg.read_norm:
                (num2, mass2), = interface.scan_views_mass((view,), hq, dep.feat, dep.pay, "m")
                mass2 = key_mass(cfg, view, hq, dep.feat, mass2)
            else:
                num2, mass2 = interface.scan_views((view,), hq, dep.feat, dep.pay, "m")[0], None
            if out_gate is not None and len(group) == 1 and out_gate.fits(num2, resid):
                outs.append(out_gate.read(num2, mass2, resid, self.s, cfg.eps))
            else:
                outs.append(gn.normalized_read(num2, mass2, resid, s=self.s, eps=cfg.eps))
        return outs


@dataclass(frozen=True)
class _Written(Deposit):
    """A deposit as written, with the hidden features ``h0`` the second
    Gauss-Newton step's own-write correction needs (not a scan channel)."""
    h0: torch.Tensor | None = None


def memory_forward(layers, cfg, k, v, q, views, hrot=None, gain=None, controls=None, out_gate=None):
    """The memory read f_theta_t(q_t) of every temporal view after writing
    keys ``k`` and values ``v`` (engine.py:260-553).  ``out_gate`` is an
    optional ``GateRequest`` (its ``applied`` tells whether the read took it)."""
    net = FastNet(layers, cfg, hrot=hrot, gain=gain, controls=controls, out_gate=out_gate)
    return net.recall(q, net.deposits(k, v), views)
