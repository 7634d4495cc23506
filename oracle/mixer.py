"""CPU restatement of the ThetaScan mixer forward (test infrastructure only).

Functional form of the reference module: ``forward(core, params, x)`` takes a
flat core-config dict (see :func:`core_config`), a parameter dict keyed by the
reference's state-dict names, and ``x [B,T,D]``.  Everything is plain torch
on the CPU (float64 for parity), differentiable, and computed view by view
without the reference's tile sharing (which changes nothing mathematically).

Followed files: src/thetascan/config.py:703-796 (config translation),
src/thetascan/_core/modules/block.py:546-724 (mixer),
src/thetascan/_core/ops/engine.py:117-544 (write streams and dual read),
src/thetascan/_core/ops/kernel_features.py (feature maps),
src/thetascan/_core/ops/interface.py:58-327 (temporal views),
src/thetascan/_core/modules/{rope,norms,gates}.py.

Pinned by the fifteen reference mixer cases in tests/golden (outputs and every
parameter gradient, float64, rel 1e-9) and by the feature-map, RoPE and scan
vectors there; see tests/test_oracle_golden.py.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import expansion
from . import scans

EPS = 1e-6


# ---------------------------------------------------------------- config

def core_config(pub: dict) -> dict:
    """Public manifest (ThetaScanConfig.to_dict()) -> flat core settings.

    Follows src/thetascan/config.py:703-796; unspecified core fields take the
    core defaults of src/thetascan/_core/config.py:24-199.
    """
    H = pub["n_heads"]
    d = pub["head_dim"] or pub["d_model"] // H
    c = {
        "d_model": pub["d_model"], "n_heads": H, "head_dim": d,
        "mem_hidden": pub["memory_multiplier"] * d,
        "feature_expansion": pub["feature_expansion"], "expansion_key": pub["expansion_key"],
        "depth": pub["depth"], "backend": pub["runtime"]["backend"],
        "scan_chunk": pub["runtime"]["scan_chunk"],
        "rope": pub["rope"]["mode"], "rope_frac": pub["rope"]["fraction"],
        "rope_base": pub["rope"]["base"], "rope_placement": pub["rope"]["placement"],
        "out_gate": pub["output_gate"], "share_kq": pub["share_key_query"],
        "key_value_heads": pub["key_value_heads"], "eps": EPS,
    }
    t = pub["temporal"]
    c["accumulation"] = "ema_gate" if t["mode"] == "ema" else "sum"
    c["read_fade"] = t["mode"] == "bank"
    c["read_fade_mode"] = t["bank_mode"]
    c["fade_blend_mode"] = t["blend_mode"]
    c["fade_branches"] = t["recency_branches"]
    if pub["family"] == "gn":
        g = pub["gn"]
        c.update(
            write_rule="gn",
            nonlin="relu2" if g["nonlinearity"] == "relu2_threshold" else g["nonlinearity"],
            learn_thresh=g["nonlinearity"] == "relu2_threshold",
            write_iters=g["jacobian_steps"], fast_w1=True,
            read_norm=g["read_normalization"] != "none",
            read_norm_w1=g["read_normalization"] == "both_feature_mass",
            read_norm_mode="key_mass", kernel_kind="softmax_partition", value_centers=0,
            value_mlp_mult=0.0, softmax_gain=1.0, softmax_gain_mode="fixed",
            kernel_sparsity="none",
        )
    else:
        k = pub["kernel"]
        c.update(
            write_rule="kernel",
            nonlin="softmax_hidden" if k["feature_map"] == "softmax_partition" else "relu2",
            learn_thresh=False, write_iters=1, fast_w1=False, read_norm_w1=False,
            kernel_kind=k["feature_map"], kernel_sparsity=k["sparsity"],
            kernel_threshold_temperature=k["threshold_temperature"],
            bspline_basis_count=k["bspline_basis_count"], bspline_degree=k["bspline_degree"],
            bspline_bound=k["bspline_bound"], bspline_scale=k["bspline_scale"],
            softmax_gain=k["kernel_sharpness"], softmax_gain_mode=k["kernel_sharpness_mode"],
            read_norm=k["read_normalization"] != "none",
            read_norm_mode=k["read_normalization"] if k["read_normalization"] != "none" else "key_mass",
            value_centers=k["value_anchors"] if k["value_representation"] == "value_anchors" else 0,
            value_mlp_mult=k["value_mlp_multiplier"] if k["value_representation"] == "value_mlp" else 0.0,
        )
    return c


# ---------------------------------------------------------------- small ops

def rmsnorm(a, eps=EPS):
    """norms.py:5-9 -- returns (normed, 1/rms)."""
    inv = torch.rsqrt(a.pow(2).mean(-1, keepdim=True) + eps)
    return a * inv, inv


def l2norm(x, eps=EPS):
    """norms.py:12"""
    return x / x.norm(dim=-1, keepdim=True).clamp_min(eps)


def rope_rot(width: int, mode: str, frac: float) -> int:
    """Rotated channel count (rope.py:64-67, block.py:606-609)."""
    max_rot = width // 2 * 2
    if mode == "full":
        return max_rot
    return min(max_rot, max(2, int(width * frac) // 2 * 2))


def rope_table(T: int, rot: int, base: float, dtype):
    """fp32 (fp64 for fp64 streams) phases, cast once (rope.py:7-38)."""
    pd = torch.float64 if dtype == torch.float64 else torch.float32
    inv = 1.0 / (base ** (torch.arange(0, rot, 2, dtype=pd) / rot))
    f = torch.outer(torch.arange(T, dtype=pd), inv)
    return f.cos().to(dtype), f.sin().to(dtype)


def rotate_pairs(x, cos, sin, rot):
    """Interleaved pair rotation of the first ``rot`` channels (rope.py:57-72)."""
    x1, x2 = x[..., :rot:2], x[..., 1:rot:2]
    o1 = x1 * cos - x2 * sin
    o2 = x1 * sin + x2 * cos
    return torch.cat([torch.stack((o1, o2), dim=-1).flatten(-2), x[..., rot:]], dim=-1)


def apply_rope(x, mode, frac, base):
    if mode == "none":
        return x
    rot = rope_rot(x.shape[-1], mode, frac)
    if rot == 0:
        return x
    cos, sin = rope_table(x.shape[2], rot, base, x.dtype)
    return rotate_pairs(x, cos, sin, rot)


def head_param(value, ref):
    """[H] or [H,M] control broadcast over [B,H,T,M] (kernel_features.py:12-31)."""
    value = value.to(ref.dtype)
    if value.ndim == 1:
        return value.view(1, -1, 1, 1)
    return value.view(1, value.shape[0], 1, value.shape[1])


# ---------------------------------------------------------------- feature maps

def relu2_ridge(pre, score_bias=None, tau=None, eps=EPS):
    """kernel_features.py:116-135"""
    if score_bias is not None:
        pre = pre + head_param(score_bias, pre)
    if tau is not None:
        pre = pre - head_param(tau, pre)
    f = torch.relu(pre).square()
    mass = f.sum(-1, keepdim=True)
    return torch.where(mass > eps, f / mass.clamp_min(eps), torch.full_like(f, 1.0 / f.shape[-1]))


def relative_threshold(logits, rho, temperature, straight_through, eps=EPS):
    """kernel_features.py:43-70"""
    shifted = logits - logits.amax(-1, keepdim=True)
    margin = shifted - head_param(rho, logits).clamp(min=eps, max=1.0 - eps).log()
    soft = torch.sigmoid(margin / temperature)
    gate = ((margin >= 0.0).to(soft.dtype) + soft - soft.detach()) if straight_through else soft
    w = shifted.exp() * gate
    return w / w.sum(-1, keepdim=True).clamp_min(eps)


def softmax_partition(pre, gain, score_bias=None, sparsity="none", rho=None, blend=None,
                      temperature=0.25, eps=EPS):
    """kernel_features.py:73-113"""
    scores = pre if score_bias is None else pre + head_param(score_bias, pre)
    g = gain if not torch.is_tensor(gain) else head_param(gain, scores)
    logits = scores * g
    dense = torch.softmax(logits, -1)
    if sparsity == "none":
        return dense
    sparse = relative_threshold(logits, rho, temperature, sparsity != "relative_soft", eps)
    if sparsity != "relative_st_blend":
        return sparse
    return dense + head_param(blend, logits) * (sparse - dense)


def bspline_basis(x, n_basis=8, degree=3, bound=3.0):
    """Clamped open-uniform Cox-de Boor basis (kernel_features.py:138-205)."""
    dtype = x.dtype
    lo = torch.tensor(-bound, dtype=dtype)
    hi = torch.tensor(bound, dtype=dtype)
    n_inner = n_basis - degree - 1
    interior = torch.linspace(-bound, bound, n_inner + 2, dtype=dtype)[1:-1] if n_inner else x.new_empty(0)
    knots = torch.cat([lo.repeat(degree + 1), interior, hi.repeat(degree + 1)])
    x = torch.minimum(x.clamp(min=-bound, max=bound), torch.nextafter(hi, lo)).unsqueeze(-1)
    basis = ((x >= knots[:-1]) & (x < knots[1:])).to(dtype)
    tiny = torch.finfo(dtype).tiny
    for order in range(1, degree + 1):
        n = knots.numel() - order - 1
        ld = knots[order:order + n] - knots[:n]
        rd = knots[order + 1:order + 1 + n] - knots[1:1 + n]
        lc = torch.where(ld > 0, (x - knots[:n]) / ld.clamp_min(tiny), torch.zeros_like(ld))
        rc = torch.where(rd > 0, (knots[order + 1:order + 1 + n] - x) / rd.clamp_min(tiny), torch.zeros_like(rd))
        basis = lc * basis[..., :n] + rc * basis[..., 1:n + 1]
    basis = basis.clamp_min(0.0)
    return basis / basis.sum(-1, keepdim=True).clamp_min(tiny)


def bspline_features(pre, scale, c):
    """kernel_features.py:208-230"""
    s = scale if not torch.is_tensor(scale) else head_param(scale, pre)
    basis = bspline_basis(pre * s, c["bspline_basis_count"], c["bspline_degree"], c["bspline_bound"])
    return basis.flatten(-2) / float(pre.shape[-1])


def feature_map(pre, c, ctl):
    """kernel_features.py:233-273"""
    kind = c["kernel_kind"]
    if kind == "softmax_partition":
        gain = ctl["gain"] if ctl["gain"] is not None else c["softmax_gain"]
        return softmax_partition(pre, gain, ctl["score_bias"], c["kernel_sparsity"], ctl["rho"],
                                 ctl["blend"], c.get("kernel_threshold_temperature", 0.25))
    if kind == "relu2_ridge":
        return relu2_ridge(pre, ctl["score_bias"], ctl["tau"])
    scale = ctl["spline_scale"] if ctl["spline_scale"] is not None else c["bspline_scale"]
    return bspline_features(pre, scale, c)


def relu2(pre):
    return torch.relu(pre).square()


def drelu2(pre):
    return 2.0 * torch.relu(pre)


def dsilu(pre):
    s = torch.sigmoid(pre)
    return s * (1 + pre * (1 - s))


def dtanh(pre):
    return 1.0 - torch.tanh(pre).square()


# tanh (sigma' = 1 - tanh^2) is this build's extension of the reference's
# relu2 / silu table (nonlin.py:28-31); the write and read formulas around it
# are the reference's, with the damping of the Jacobi diagonal and the key
# mass of signed features below.
ACT = {"relu2": (relu2, drelu2), "silu": (F.silu, dsilu), "tanh": (torch.tanh, dtanh)}


def damping(c) -> float:
    """The Jacobi diagonal's damping; the reference's is eps (engine.py:255)."""
    return EPS if c.get("gn_damping") is None else float(c["gn_damping"])


def key_mass(view, qf, keys, unit_mass, c):
    """The mass a normalized read divides by, num / (mass + eps)
    (engine.py:440-442, 503-506).  For the reference's nonnegative features it
    is the scan's unit column, sum_i w_i qf . k_i.  tanh features are signed,
    so those products cancel and the mass can cross zero; the mass is then
    that of the absolute features, sum_i w_i |qf| . |k_i| = |qf| . (the view's
    decayed prefix of |k|), which equals the unit column for nonnegative
    features and bounds the read: |num| / mass <= max |value|."""
    if c["nonlin"] == "tanh":
        return (qf.abs() * view.mass_cum(keys.abs())).sum(-1, keepdim=True)
    return unit_mass


def ein(W, x, pat):
    """einsum with a head-shared [1,...] weight (engine.py:36-40)."""
    if W.shape[0] == 1 and x.shape[1] != 1:
        W = W.expand(x.shape[1], -1, -1)
    return torch.einsum(pat, W, x)


# ---------------------------------------------------------------- temporal views

class View:
    """A temporal view: signed scan terms + a key-mass accumulator.

    kinds: "plain" (sum or the ema stream), "fast" (static bank branch),
    "stale" (plain - fast), "null" (zero memory).  interface.py:198-327.
    """

    def __init__(self, kind, decay=None, log_alpha=None, scan=scans.linattn_naive):
        self.kind, self.decay, self.log_alpha = kind, decay, log_alpha
        self.linattn = scan

    def terms(self):
        if self.kind == "null":
            return ()
        if self.kind == "fast":
            return ((1.0, self.log_alpha),)
        plain = ((1.0, self.decay),)
        if self.kind == "stale":
            return plain + ((-1.0, self.log_alpha),)
        return plain

    def scan(self, q, k, v):
        out = q.new_zeros(*q.shape[:3], v.shape[-1])
        for coef, ret in self.terms():
            if ret is not None and ret.ndim == 1:
                ret = scans.as_stream(ret, q)
            out = out + coef * self.linattn(q, k, v, ret)
        return out

    def mass_cum(self, keys):
        if self.kind == "null":
            return torch.zeros_like(keys)
        if self.kind == "fast":
            return scans.ema_cumsum(keys, self.log_alpha)
        if self.kind == "stale":
            return keys.cumsum(2) - scans.ema_cumsum(keys, self.log_alpha)
        if self.decay is None:
            return keys.cumsum(2)
        ones = keys.new_ones(*keys.shape[:3], 1)
        return self.linattn(ones, ones, keys, self.decay)


# ---------------------------------------------------------------- engine

def block_forward(W1, W2, Wg, c, x, ctl, delta=None):
    """engine.py:117-158 -> (u, ctx)"""
    a = ein(W1, x, "hmd,bhtd->bhtm")
    if delta is not None:
        a = a + delta["g_a"] * (delta["x0"] * x).sum(-1, keepdim=True)
    ctx = {"x": x}
    if c["nonlin"] == "swiglu":
        b = ein(Wg, x, "hmd,bhtd->bhtm")
        if delta is not None:
            b = b + delta["g_b"] * (delta["x0"] * x).sum(-1, keepdim=True)
        pre, inv_a = rmsnorm(a)
        preb, inv_b = rmsnorm(b)
        h = F.silu(preb) * pre
        ctx.update(pre=pre, preb=preb, inv_a=inv_a, inv_b=inv_b, h=h)
    else:
        pre, inv_a = rmsnorm(a)
        if c["learn_thresh"]:
            pre = pre - Wg[..., 0].unsqueeze(0).unsqueeze(2)
        if c["write_rule"] == "kernel":
            h = feature_map(pre, c, ctl)
        elif c["nonlin"] == "softmax_hidden":
            h = torch.softmax(pre * c["softmax_gain"], -1)
        else:
            h = ACT[c["nonlin"]][0](pre)
        ctx.update(pre=pre, inv_a=inv_a, h=h)
    u = ein(W2, ctx["h"], "hdm,bhtm->bhtd")
    if delta is not None:
        u = u + delta["lam_hat"] * (delta["h0"] * ctx["h"]).sum(-1, keepdim=True)
    return u, ctx


def forward_theta0(weights, c, k, ctl, deltas=None):
    """engine.py:161-175"""
    s = 1.0 / math.sqrt(c["depth"])
    x, ctxs = k, []
    for l, (W1, W2, Wg) in enumerate(weights):
        u, ctx = block_forward(W1, W2, Wg, c, x, ctl, None if deltas is None else deltas[l])
        ctxs.append(ctx)
        x = x + s * u
    return x, ctxs


def g_from_lambda(W2, c, ctx, lam):
    """engine.py:180-195"""
    u2 = ein(W2, lam, "hdm,bhtd->bhtm")
    if c["nonlin"] == "swiglu":
        return torch.cat([F.silu(ctx["preb"]) * u2 * ctx["inv_a"],
                          ctx["pre"] * dsilu(ctx["preb"]) * u2 * ctx["inv_b"]], dim=-1)
    return ACT[c["nonlin"]][1](ctx["pre"]) * u2 * ctx["inv_a"]


def lambda_solve(weights, c, ctxs, r):
    """Jacobi-preconditioned residual (engine.py:215-255)."""
    diag = 0.0
    for (W1, W2, Wg), ctx in zip(weights, ctxs):
        hh = (ctx["h"] * ctx["h"]).sum(-1, keepdim=True)
        xx = (ctx["x"] * ctx["x"]).sum(-1, keepdim=True)
        if c["nonlin"] == "swiglu":
            sa = F.silu(ctx["preb"]) * ctx["inv_a"]
            sb = ctx["pre"] * dsilu(ctx["preb"]) * ctx["inv_b"]
            s2 = sa * sa + sb * sb
        else:
            s = ACT[c["nonlin"]][1](ctx["pre"]) * ctx["inv_a"]
            s2 = s * s
        diag = diag + hh + xx * ein(W2 * W2, s2, "hdm,bhtm->bhtd")
    return r / (diag / c["depth"] + damping(c))


def write_streams(weights, c, k, v, hrot, ctl):
    """engine.py:260-340 -> dict(la1=[...], la2=[...])"""
    s = 1.0 / math.sqrt(c["depth"])
    m = weights[0][1].shape[-1]
    o, ctxs = forward_theta0(weights, c, k, ctl)

    def rot(h):
        return h if hrot is None else rotate_pairs(h, *hrot)

    if c["write_rule"] == "kernel":
        if c["value_centers"]:
            Cv = weights[0][2]
            Cv = Cv if Cv.shape[0] == v.shape[1] else Cv.expand(v.shape[1], -1, -1)
            vn = v / v.norm(dim=-1, keepdim=True).clamp_min(EPS)
            lam = torch.softmax(c["softmax_gain"] * torch.einsum("hvd,bhtd->bhtv", Cv, vn), -1)
        else:
            lam = v
    else:
        lam = lambda_solve(weights, c, ctxs, v - o)
    la1, la2, deltas = [], [], []
    for l, (W1, W2, Wg) in enumerate(weights):
        lam_hat = s * lam
        if c["fast_w1"]:
            g = s * g_from_lambda(W2, c, ctxs[l], lam)
            la1.append((ctxs[l]["x"], g))
            deltas.append({"x0": ctxs[l]["x"], "h0": ctxs[l]["h"], "lam_hat": lam_hat,
                           "g_a": g[..., :m], "g_b": g[..., m:] if g.shape[-1] > m else None})
        else:
            la1.append(None)
        la2.append((rot(ctxs[l]["h"]), lam_hat))
    if c["write_iters"] == 2:
        o2, ctxs2 = forward_theta0(weights, c, k, ctl, deltas=deltas)
        lam2 = lambda_solve(weights, c, ctxs2, v - o2)
        for l, (W1, W2, Wg) in enumerate(weights):
            la1.append((ctxs2[l]["x"], s * g_from_lambda(W2, c, ctxs2[l], lam2)))
            la2.append((rot(ctxs2[l]["h"]), s * lam2))
    return {"la1": la1, "la2": la2}


def read_view(weights, c, q, streams, view, hrot, ctl):
    """One view of engine.dual_read_views (engine.py:345-544)."""
    s = 1.0 / math.sqrt(c["depth"])
    L = c["depth"]
    m = weights[0][1].shape[-1]

    def rot(h):
        return h if hrot is None else rotate_pairs(h, *hrot)

    def features(a, b, Wg):
        if c["nonlin"] == "swiglu":
            h = F.silu(rmsnorm(b)[0]) * rmsnorm(a)[0]
        else:
            pre = rmsnorm(a)[0]
            if c["learn_thresh"]:
                pre = pre - Wg[..., 0].unsqueeze(0).unsqueeze(2)
            if c["write_rule"] == "kernel":
                h = feature_map(pre, c, ctl)
            elif c["nonlin"] == "softmax_hidden":
                h = torch.softmax(pre * c["softmax_gain"], -1)
            else:
                h = ACT[c["nonlin"]][0](pre)
        return h, rot(h)

    x = q
    for l, (W1, W2, Wg) in enumerate(weights):
        a = ein(W1, x, "hmd,bhtd->bhtm")
        b = ein(Wg, x, "hmd,bhtd->bhtm") if c["nonlin"] == "swiglu" else None
        if c["read_norm_w1"]:
            pre0 = rmsnorm(a)[0]
            if c["learn_thresh"]:
                pre0 = pre0 - Wg[..., 0].unsqueeze(0).unsqueeze(2)
            h0q = rot(relu2(pre0))
            fkeys = streams["la2"][l][0]
            gvals = streams["la1"][l][1]
            corr1 = view.scan(h0q, fkeys, torch.cat([gvals, gvals.new_ones(*gvals.shape[:3], 1)], -1))
            a = a + corr1[..., :m] / (key_mass(view, h0q, fkeys, corr1[..., -1:], c) + EPS)
        else:
            for it in range(c["write_iters"]):
                entry = streams["la1"][it * L + l]
                if entry is None:
                    continue
                corr = view.scan(x, entry[0], entry[1])
                a = a + corr[..., :m]
                if b is not None:
                    b = b + corr[..., m:]
        h, hq = features(a, b, Wg)
        base = ein(W2, h, "hdm,bhtm->bhtd")
        if not c["read_norm"]:
            mem = 0.0
            for it in range(c["write_iters"]):
                keys, vals = streams["la2"][it * L + l]
                mem = mem + view.scan(hq, keys, vals)
        else:
            keys, vals = streams["la2"][l]
            if c["read_norm_mode"] == "key_mass":
                corr = view.scan(hq, keys, torch.cat([vals, vals.new_ones(*vals.shape[:3], 1)], -1))
                mem = corr[..., :-1] / (key_mass(view, hq, keys, corr[..., -1:], c) + EPS)
            else:
                kcum = view.mass_cum(keys)
                mem = view.scan(hq / (kcum + EPS), keys, vals)
        if c["value_centers"]:
            Cv = Wg if Wg.shape[0] == q.shape[1] else Wg.expand(q.shape[1], -1, -1)
            mem = torch.einsum("hvd,bhtv->bhtd", Cv, mem)
        x = x + s * (base + mem)
    return x


# ---------------------------------------------------------------- mixer

def effective_weights(c, params):
    """block.py:546-567 (expansion maps rebuilt from the key, float32)."""
    out = []
    for l in range(c["depth"]):
        W1, W2 = params[f"W1.{l}"], params[f"W2.{l}"]
        Wg = params.get(f"Wg.{l}")
        if c["feature_expansion"] > 1:
            m = c["mem_hidden"]
            b = m // c["feature_expansion"]
            # W1's rows are features, or the projections of a B-spline map
            # (hidden / basis count, block.py:214-222); expanding the latter is
            # an extension of this build
            nb = c["bspline_basis_count"] if c["kernel_kind"] == "projected_bspline" else 1
            E1 = expansion.row_map((1, m // nb, b // nb), c["expansion_key"], f"w1-expand-layer-{l}").to(W1.dtype)
            E2 = expansion.row_map((1, b, m), c["expansion_key"], f"w2-expand-layer-{l}").to(W2.dtype)
            W1 = torch.matmul(E1, W1)
            W2 = torch.matmul(W2, E2)
        out.append((W1, W2, Wg))
    return out


def kernel_controls(c, params):
    """block.py:408-456 (forward values)."""
    tiny = lambda t: t.clamp_min(torch.finfo(t.dtype).tiny)  # noqa: E731
    raw = params.get("kernel_sharpness_raw")
    sraw = params.get("bspline_scale_raw")
    rraw = params.get("kernel_relative_threshold_raw")
    braw = params.get("kernel_sparse_blend_raw")
    blend = None
    if braw is not None:
        sur = torch.sigmoid(braw)
        blend = braw.clamp(0.0, 1.0).detach() + sur - sur.detach()
    return {
        "gain": None if raw is None else tiny(F.softplus(raw)),
        "spline_scale": None if sraw is None else tiny(F.softplus(sraw)),
        "score_bias": params.get("kernel_score_bias"),
        "tau": params.get("kernel_relu2_threshold"),
        "rho": None if rraw is None else torch.sigmoid(rraw),
        "blend": blend,
    }


def project(c, params, x):
    """q, k, v [B,H,T,d] for the three projection layouts (block.py:577-594)."""
    B, T, _ = x.shape
    H, d = c["n_heads"], c["head_dim"]
    if c["key_value_heads"] is not None:
        G = c["key_value_heads"]
        q = F.linear(x, params["proj_q.weight"]).view(B, T, H, d).transpose(1, 2)
        k = F.linear(x, params["proj_k.weight"]).view(B, T, G, d).transpose(1, 2)
        v = F.linear(x, params["proj_v.weight"]).view(B, T, G, d).transpose(1, 2)
        return q, k.repeat_interleave(H // G, dim=1), v.repeat_interleave(H // G, dim=1)
    if c["share_kq"]:
        kqb = params["kq_bias"].to(x.dtype)
        q = F.linear(x, params["proj_q1.weight"]).unsqueeze(1) + kqb[0][None, :, None, :]
        k = F.linear(x, params["proj_k1.weight"]).unsqueeze(1) + kqb[1][None, :, None, :]
        v = F.linear(x, params["proj_v.weight"]).view(B, T, H, d).transpose(1, 2)
        return q, k, v
    qkv = F.linear(x, params["proj_qkv.weight"])
    q, k, v = qkv.view(B, T, 3, H, d).permute(2, 0, 3, 1, 4)
    return q, k, v


SCANS = {"naive": scans.linattn_naive, "quad": scans.linattn_quad, "cumsum": scans.linattn_cumsum,
         "chunk": scans.linattn_chunk}


def _write_side(c, params, x):
    """Projections, RoPE, L2 norm, value MLP, decay gate and the write
    streams (block.py:573-665)."""
    B, T, _ = x.shape
    H = c["n_heads"]
    q, k, v = project(c, params, x)
    if c["rope_placement"] == "input":
        q = apply_rope(q, c["rope"], c["rope_frac"], c["rope_base"])
        k = apply_rope(k, c["rope"], c["rope_frac"], c["rope_base"])
    q, k = l2norm(q), l2norm(k)
    if c["value_mlp_mult"] > 0:
        hid = F.silu(F.linear(v, params["vmlp_in.weight"], params["vmlp_in.bias"]))
        v = v + F.linear(hid, params["vmlp_out.weight"], params["vmlp_out.bias"])
    hrot = None
    if c["rope_placement"] == "feature" and c["rope"] != "none":
        rot = rope_rot(c["mem_hidden"], c["rope"], c["rope_frac"])
        if rot:
            cos, sin = rope_table(T, rot, c["rope_base"], x.dtype)
            hrot = (cos, sin, rot)
    decay = None
    if c["accumulation"] == "ema_gate":
        g = F.linear(x, params["decay.g.lin.weight"], params["decay.g.lin.bias"])
        decay = -F.softplus(g.view(B, T, H, 1).transpose(1, 2))
    weights = effective_weights(c, params)
    ctl = kernel_controls(c, params)
    streams = write_streams(weights, c, k, v, hrot, ctl)
    return q, streams, hrot, ctl, weights, decay


def kernel_final_states(c, params, x):
    """Memory of a depth-1 kernel mixer after the last token, per view, by the
    closed form N_T = sum_i w_i phi(k_i) v_i^T and D_T = sum_i w_i phi(k_i)
    (the brute-force DW2 / Smass of engine.py:669-703 at t = T-1): the plain
    sum (w_i = 1, or the ema stream's prod_{i<j<T} a_j) first, then every
    recency branch (w_i = alpha^(T-1-i)).  Returns [(N [B,H,m,d], D [B,H,m])]."""
    _, streams, _, _, _, decay = _write_side(c, params, x)
    keys, vals = streams["la2"][0]
    T = keys.shape[2]
    weights = []
    if decay is None:
        weights.append(keys.new_ones(1, 1, T))
    else:
        tail = decay[..., 0].flip(-1).cumsum(-1).flip(-1)  # sum_{j>=i} log a_j
        weights.append(torch.cat([tail[..., 1:], tail.new_zeros(*tail.shape[:2], 1)], -1).exp())
    if c["read_fade"]:
        raw = params["fade_alpha"]
        raw = raw.unsqueeze(0) if raw.ndim == 1 else raw
        lags = torch.arange(T - 1, -1, -1, dtype=keys.dtype)
        for j in range(c["fade_branches"]):
            la = -F.softplus(-raw[j])
            weights.append((la.view(1, -1, 1) * lags.view(1, 1, T)).exp())
    out = []
    for w in weights:
        wk = keys * w.unsqueeze(-1)
        out.append((torch.einsum("bhtm,bhtd->bhmd", wk, vals), wk.sum(2)))
    return out


def forward(c, params, x, backend: str = "naive"):
    """ThetaScan forward x[B,T,D] -> y[B,T,D] (block.py:573-724).

    ``backend`` picks the oracle scan: the naive loop (parity target), the
    quadratic form, the prefix-sum form (the CPU baseline algorithm), or the
    tiled form (64-token tiles; equal to the naive loop at 1e-12, linear in T,
    for long sequences).
    """
    scan = SCANS[backend]
    B, T, _ = x.shape
    H, d = c["n_heads"], c["head_dim"]
    q, streams, hrot, ctl, weights, decay = _write_side(c, params, x)

    def read(view):
        return read_view(weights, c, q, streams, view, hrot, ctl)

    y = read(View("plain", decay=decay, scan=scan))
    if c["read_fade"]:
        raw = params["fade_alpha"]
        eta = params["fade_eta"]
        if c["fade_blend_mode"] == "tanh":
            eta = torch.tanh(eta)
        if raw.ndim == 1:
            raw, eta = raw.unsqueeze(0), eta.unsqueeze(0)
        base = y
        if c["read_fade_mode"] == "fast":
            out = base
            for j in range(c["fade_branches"]):
                la = -F.softplus(-raw[j])
                out = out + eta[j].view(1, -1, 1, 1) * (read(View("fast", log_alpha=la, scan=scan)) - base)
            y = out
        else:
            null = read(View("null", scan=scan))
            out = base
            for j in range(c["fade_branches"]):
                la = -F.softplus(-raw[j])
                stale = read(View("stale", decay=None, log_alpha=la, scan=scan))
                out = out - eta[j].view(1, -1, 1, 1) * (stale - null)
            y = out
    if c["out_gate"]:
        gate = F.linear(x, params["ogate.g.lin.weight"], params["ogate.g.lin.bias"])
        y = y * F.silu(gate.view(B, T, H, d).transpose(1, 2))
    y = y.transpose(1, 2).reshape(B, T, H * d)
    return F.linear(y, params["proj_out.weight"])
