"""HIP GN write payloads (ts_gn_write_fwd/bwd) against the oracle (fp64, CPU).

The oracle's write_streams (a restatement of engine.py:117-340, pinned by the
reference's GN mixer vectors in tests/golden) gives h, s*lam and g for a
depth-1 ReLU^2 memory; its autograd gives every gradient the HIP backward
must reproduce: dx (through h, lam and g), dv, dW1, dW2 and the per-feature
threshold.  Both hidden nonlinearities of the reference are covered: ReLU^2
and SiLU (nonlin.py:18-31; the SiLU slope needs the pre-activation and its
backward silu'').
"""
from __future__ import annotations

import pytest
import torch

from oracle import mixer
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu


def _cfg(learn_thresh, nonlin="relu2"):
    return {"write_rule": "gn", "nonlin": nonlin, "depth": 1, "fast_w1": True, "write_iters": 1,
            "learn_thresh": learn_thresh, "value_centers": 0}


def _case(B, H, T, d, m, learn_thresh, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(B, H, T, d, generator=g, dtype=torch.float64)
    k = k / k.norm(dim=-1, keepdim=True)
    v = torch.randn(B, H, T, d, generator=g, dtype=torch.float64)
    w1 = torch.randn(H, m, d, generator=g, dtype=torch.float64) / d ** 0.5
    w2 = torch.randn(H, d, m, generator=g, dtype=torch.float64) * 0.3
    wg = (torch.randn(H, m, 1, generator=g, dtype=torch.float64) * 0.3) if learn_thresh else None
    rnd = lambda t: None if t is None else t.to(dtype).to(torch.float64)  # noqa: E731
    return rnd(k), rnd(v), rnd(w1), rnd(w2), rnd(wg)


BF = torch.bfloat16
# hidden widths 192 and 384 in bf16 at head widths 32 and 64 run the chunked kernels
WIDE = [pytest.param(BF, 64, 192, True, 90, id="bf16-wide-d64-m192"),
        pytest.param(BF, 32, 384, True, 70, id="bf16-wide-d32-m384"),
        pytest.param(BF, 64, 384, False, 100, id="bf16-wide-d64-m384")]


@pytest.mark.parametrize("nonlin", ["relu2", "silu"])
@pytest.mark.parametrize("dtype,d,m,learn_thresh,T", [
    (dt, *case) for dt in (torch.float32, BF)
    for case in [(16, 48, False, 70), (64, 128, False, 150), (32, 96, True, 64), (16, 16, True, 33),
                 (128, 64, False, 40)]] + [(torch.float32, 64, 192, True, 90)] + WIDE)
def test_gn_write_matches_oracle(cuda, dtype, d, m, learn_thresh, T, nonlin):
    from thetascan_amd._core.ops import gn

    B, H = 2, 3
    k, v, w1, w2, wg = _case(B, H, T, d, m, learn_thresh, 100 * d + m + T, dtype)
    c = _cfg(learn_thresh, nonlin)
    # oracle forward + backward (fp64)
    rk, rv, rw1, rw2 = (t.clone().requires_grad_(True) for t in (k, v, w1, w2))
    rwg = wg.clone().requires_grad_(True) if learn_thresh else None
    st = mixer.write_streams([(rw1, rw2, rwg)], c, rk, rv, None, {})
    (xk, g_ref), = st["la1"]
    (h_ref, lam_ref), = st["la2"]
    gen = torch.Generator().manual_seed(7)
    dh = torch.randn(h_ref.shape, generator=gen, dtype=torch.float64)
    dl = torch.randn(lam_ref.shape, generator=gen, dtype=torch.float64)
    dg = torch.randn(g_ref.shape, generator=gen, dtype=torch.float64) * 0.1
    torch.autograd.backward([h_ref, lam_ref, g_ref], [dh, dl, dg])

    dev = lambda t: None if t is None else t.to(cuda, dtype).requires_grad_(True)  # noqa: E731
    x_, v_, w1_, w2_ = dev(k), dev(v), dev(w1), dev(w2)
    tau_ = dev(wg[..., 0].contiguous()) if learn_thresh else None
    h, lam, g = gn.write(x_, v_, w1_, w2_, tau_, nonlin=nonlin)
    torch.autograd.backward([h, lam, g], [dh.to(cuda, dtype), dl.to(cuda, dtype), dg.to(cuda, dtype)])

    tol = 1e-3 if dtype == torch.float32 else 2e-2
    for name, a, e in (("h", h, h_ref), ("lam", lam, lam_ref), ("g", g, g_ref)):
        assert rel_err(a, e) < tol, (name, d, m, learn_thresh, rel_err(a, e))
    gtol = tol
    grads = [("dx", x_.grad, rk.grad), ("dv", v_.grad, rv.grad), ("dW1", w1_.grad, rw1.grad),
             ("dW2", w2_.grad, rw2.grad)]
    if learn_thresh:
        grads.append(("dtau", tau_.grad, rwg.grad[..., 0]))
    errs = {name: rel_err(a, e) for name, a, e in grads}
    print(f"errors gn write {nonlin} {dtype} d{d} m{m}: " + " ".join(f"{k} {v:.2e}" for k, v in errs.items()),
          flush=True)
    for name, a, e in grads:
        assert rel_err(a, e) < gtol, (name, d, m, learn_thresh, rel_err(a, e))


def test_gn_write_rejects_unsupported_widths(cuda):
    from thetascan_amd._core.ops import gn

    x = torch.zeros(1, 1, 8, 24, device=cuda)
    w1 = torch.zeros(1, 32, 24, device=cuda)
    w2 = torch.zeros(1, 24, 32, device=cuda)
    with pytest.raises(NotImplementedError):
        gn.write(x, x, w1, w2)


@pytest.mark.parametrize("nonlin", ["relu2", "silu"])
@pytest.mark.parametrize("dtype,d,m,learn_thresh,T", [
    (dt, *case) for dt in (torch.float32, BF)
    for case in [(16, 48, True, 70), (64, 128, False, 130), (32, 96, False, 64)]] +
    [(torch.float32, 64, 192, True, 90)] + WIDE)
def test_gn_read_stage_matches_block_forward(cuda, dtype, d, m, learn_thresh, T, nonlin):
    """Stage without a correction: h and q + s W2 h are the oracle's
    block_forward (engine.py:117-158) of the query, gradients included."""
    from thetascan_amd._core.ops import gn

    B, H = 2, 3
    q, _, w1, w2, wg = _case(B, H, T, d, m, learn_thresh, 7 * d + m + T, dtype)
    c = _cfg(learn_thresh, nonlin)
    rq, rw1, rw2 = (t.clone().requires_grad_(True) for t in (q, w1, w2))
    rwg = wg.clone().requires_grad_(True) if learn_thresh else None
    u, ctx = mixer.block_forward(rw1, rw2, rwg, c, rq, {})
    h_ref, resid_ref = ctx["h"], rq + u
    gen = torch.Generator().manual_seed(3)
    dh = torch.randn(h_ref.shape, generator=gen, dtype=torch.float64)
    dr = torch.randn(resid_ref.shape, generator=gen, dtype=torch.float64)
    torch.autograd.backward([h_ref, resid_ref], [dh, dr])

    dev = lambda t: t.to(cuda, dtype).requires_grad_(True)  # noqa: E731
    q_, w1_, w2_ = dev(q), dev(w1), dev(w2)
    tau_ = dev(wg[..., 0].contiguous()) if learn_thresh else None
    h, resid = gn.read_stage(q_, w1_, w2_, tau_, want_resid=True, nonlin=nonlin)
    torch.autograd.backward([h, resid], [dh.to(cuda, dtype), dr.to(cuda, dtype)])
    tol = 1e-3 if dtype == torch.float32 else 2e-2
    pairs = [("dq", q_.grad, rq.grad), ("dW1", w1_.grad, rw1.grad), ("dW2", w2_.grad, rw2.grad)]
    print(f"errors gn read {nonlin} {dtype} d{d} m{m}: h {rel_err(h, h_ref):.2e} resid {rel_err(resid, resid_ref):.2e} "
          + " ".join(f"{n} {rel_err(a, e):.2e}" for n, a, e in pairs), flush=True)
    assert rel_err(h, h_ref) < tol and rel_err(resid, resid_ref) < tol
    gtol = tol
    if learn_thresh:
        pairs.append(("dtau", tau_.grad, rwg.grad[..., 0]))
    for name, a, e in pairs:
        assert rel_err(a, e) < gtol, (name, rel_err(a, e))


@pytest.mark.parametrize("corr", [1, 2])
@pytest.mark.parametrize("dtype,d,m", [(torch.float32, 32, 64), (BF, 64, 384), (BF, 32, 192)])
def test_gn_read_stage_correction_gradients(cuda, corr, dtype, d, m):
    """Stage with the LA1 correction (plain, or divided by its mass): the HIP
    backward agrees with fp64 autograd of rmsnorm(W1 q + c) composed from the
    oracle's rmsnorm, for q, num, mass, W1, W2 and tau (fp32 at rel 1e-3, bf16
    at 2e-2; measured at most 3.1e-6 and 5.1e-3)."""
    from thetascan_amd._core.ops import gn

    B, H, T = 2, 2, 75
    q, _, w1, w2, wg = _case(B, H, T, d, m, True, 11 + corr, dtype)
    gen = torch.Generator().manual_seed(5)
    num = torch.randn(B, H, T, m, generator=gen, dtype=torch.float64).to(dtype).double()
    mass = torch.rand(B, H, T, generator=gen, dtype=torch.float64) + 0.5
    leaves = [t.clone().requires_grad_(True) for t in (q, w1, w2, wg, num, mass)]
    rq, rw1, rw2, rwg, rnum, rmass = leaves
    cc = rnum / (rmass.unsqueeze(-1) + 1e-6) if corr == 2 else rnum
    a = torch.einsum("hmd,bhtd->bhtm", rw1, rq) + cc
    pre = mixer.rmsnorm(a)[0] - rwg[..., 0].unsqueeze(0).unsqueeze(2)
    h_ref = torch.relu(pre) ** 2
    resid_ref = rq + torch.einsum("hdm,bhtm->bhtd", rw2, h_ref)
    dh = torch.randn(h_ref.shape, generator=gen, dtype=torch.float64)
    dr = torch.randn(resid_ref.shape, generator=gen, dtype=torch.float64)
    torch.autograd.backward([h_ref, resid_ref], [dh, dr])

    dts = (dtype, dtype, dtype, torch.float32, dtype, torch.float32)
    dev = [t.to(cuda, dt).requires_grad_(True)
           for t, dt in zip((q, w1, w2, wg[..., 0].contiguous(), num, mass), dts)]
    q_, w1_, w2_, tau_, num_, mass_ = dev
    h, resid = gn.read_stage(q_, w1_, w2_, tau_, num_, mass_ if corr == 2 else None, corr=corr, want_resid=True)
    torch.autograd.backward([h, resid], [dh.to(cuda, dtype), dr.to(cuda, dtype)])
    tol = gtol = 1e-3 if dtype == torch.float32 else 2e-2
    pairs = [("dq", q_.grad, rq.grad), ("dW1", w1_.grad, rw1.grad), ("dW2", w2_.grad, rw2.grad),
             ("dtau", tau_.grad, rwg.grad[..., 0]), ("dnum", num_.grad, rnum.grad)]
    if corr == 2:
        pairs.append(("dmass", mass_.grad, rmass.grad))
    print(f"errors gn read corr {corr} {dtype} d{d} m{m}: h {rel_err(h, h_ref):.2e} resid "
          f"{rel_err(resid, resid_ref):.2e} " + " ".join(f"{n} {rel_err(a, e):.2e}" for n, a, e in pairs), flush=True)
    assert rel_err(h, h_ref) < tol and rel_err(resid, resid_ref) < tol
    for name, a, e in pairs:
        assert rel_err(a, e) < gtol, (name, rel_err(a, e))


def test_normalized_read_matches_formula(cuda):
    """The read epilogue y = resid + s num / (mass + eps) with its gradients."""
    from thetascan_amd._core.ops import gn

    g = torch.Generator().manual_seed(9)
    num, resid = (torch.randn(2, 3, 40, 32, generator=g, dtype=torch.float64) for _ in range(2))
    mass = torch.rand(2, 3, 40, generator=g, dtype=torch.float64) + 0.3
    leaves = [t.clone().requires_grad_(True) for t in (num, mass, resid)]
    y_ref = leaves[2] + 0.5 * leaves[0] / (leaves[1].unsqueeze(-1) + 1e-6)
    dy = torch.randn(y_ref.shape, generator=g, dtype=torch.float64)
    y_ref.backward(dy)
    dev = [t.to(cuda, torch.float32).requires_grad_(True) for t in (num, mass, resid)]
    y = gn.normalized_read(dev[0], dev[1], dev[2], s=0.5)
    y.backward(dy.to(cuda, torch.float32))
    assert rel_err(y, y_ref) < 1e-5
    for a, e in zip(dev, leaves):
        assert rel_err(a.grad, e.grad) < 1e-5


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (BF, 2e-2)])
def test_gated_read_matches_formula(cuda, dtype, tol):
    """The read epilogue with the output gate, y = (resid + s num / (mass +
    eps)) * silu(gate + bias), written token-major, against float64 autograd:
    y, dnum, dmass, dresid, dgate and the bias gradient (fp32 at 1e-5, bf16
    within one rounding)."""
    from thetascan_amd._core.ops import gn

    g = torch.Generator().manual_seed(11)
    B, H, T, d = 2, 3, 70, 32
    num, resid, gate = (torch.randn(B, H, T, d, generator=g, dtype=torch.float64) for _ in range(3))
    mass = torch.rand(B, H, T, generator=g, dtype=torch.float64) + 0.3
    bias = torch.randn(H * d, generator=g, dtype=torch.float64)
    num, resid, gate = (t.to(dtype).double() for t in (num, resid, gate))
    leaves = [t.clone().requires_grad_(True) for t in (num, mass, resid, gate, bias)]
    n, m, r, gt, b = leaves
    y_ref = (r + 0.5 * n / (m.unsqueeze(-1) + 1e-6)) * torch.nn.functional.silu(gt + b.view(H, 1, d))
    dy = torch.randn(B, T, H, d, generator=g, dtype=torch.float64).transpose(1, 2)
    y_ref.backward(dy)

    dev = [t.detach().to(cuda, dtype if i != 1 else torch.float32).requires_grad_(True)
           for i, t in enumerate((num, mass, resid, gate, bias))]
    # the gate as the projection gives it: a [B,H,T,d] view of [B,T,H*d]
    gate_tok = dev[3].detach().transpose(1, 2).contiguous().transpose(1, 2).requires_grad_(True)
    y = gn.normalized_read(dev[0], dev[1], dev[2], s=0.5, gate=gate_tok, gate_bias=dev[4])
    assert y.shape == (B, H, T, d) and y.transpose(1, 2).is_contiguous()
    y.backward(dy.to(cuda, dtype))
    torch.cuda.synchronize()
    errs = {"y": rel_err(y.float(), y_ref), "dnum": rel_err(dev[0].grad.float(), n.grad),
            "dmass": rel_err(dev[1].grad, m.grad), "dresid": rel_err(dev[2].grad.float(), r.grad),
            "dgate": rel_err(gate_tok.grad.float(), gt.grad), "dbias": rel_err(dev[4].grad.float(), b.grad)}
    print(f"gated read {dtype}: {errs}", flush=True)
    for k, e in errs.items():
        assert e < tol, (k, e)


def _gated_config(kind):
    import dataclasses

    import thetascan_amd as ts

    if kind == "gn_tanh":
        public = ts.ThetaScanConfig(
            d_model=128, n_heads=2, memory_multiplier=2, family="gn",
            gn=ts.GNConfig(nonlinearity="relu2", jacobian_steps=1, read_normalization="both_feature_mass"),
            temporal=ts.TemporalConfig(mode="sum"), runtime=ts.RuntimeConfig(backend="hip", scan_chunk=64))
        return dataclasses.replace(public._to_core_config(), nonlin="tanh", gn_damping=1e-2)
    public = ts.ThetaScanConfig(
        d_model=128, n_heads=2, memory_multiplier=2, family="kernel",
        kernel=ts.KernelConfig(feature_map="projected_bspline", read_normalization="key_mass"),
        temporal=ts.TemporalConfig(mode="ema"), runtime=ts.RuntimeConfig(backend="hip", scan_chunk=64))
    return public._to_core_config()


@pytest.mark.parametrize("kind", ["gn_tanh", "kernel_bspline_ema"])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (BF, 2e-2)])
def test_mixer_gate_in_the_read_epilogue(cuda, dtype, tol, kind, monkeypatch):
    """A single-view mixer on the composed path with the output gate (the
    tanh GN workload's layout, and a B-spline kernel memory with an EMA view,
    at small shapes) applies the gate inside the HIP read epilogue; its
    output and every gradient agree with the same mixer whose gate is a
    separate product after the read (bf16: one rounding step apart)."""
    from thetascan_amd import _lib
    from thetascan_amd._core.modules import block as block_mod

    cfg = _gated_config(kind)
    torch.manual_seed(0)
    module = block_mod.ThetaScan(cfg)
    g = torch.Generator().manual_seed(2)
    with torch.no_grad():
        for _, p in sorted(module.named_parameters()):
            p.add_(torch.randn(p.shape, generator=g) * 0.05)
    module = module.to(cuda, dtype)
    x = torch.randn(2, 150, 128, generator=g).to(cuda, dtype)
    dy = torch.randn(2, 150, 128, generator=g).to(cuda, dtype)

    def run():
        module.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        with _lib.record_launches() as recs:
            y = module(xx)
            y.backward(dy)
            torch.cuda.synchronize()
        grads = {n: p.grad.float().clone() for n, p in module.named_parameters() if p.grad is not None}
        return y.float(), xx.grad.float(), grads, recs

    requests = []
    plain_gate = block_mod.ThetaScan._read_gate

    def spy(self, *args):
        requests.append(plain_gate(self, *args))
        return requests[-1]

    monkeypatch.setattr(block_mod.ThetaScan, "_read_gate", spy)
    y1, dx1, g1, recs = run()
    assert requests and requests[0] is not None and requests[0].applied, "the read epilogue did not take the gate"
    assert any(r[0] == "ts_read_fwd" for r in recs)
    monkeypatch.setattr(block_mod.ThetaScan, "_read_gate", lambda self, *a: None)
    y0, dx0, g0, _ = run()
    assert set(g1) == set(g0)
    errs = {"y": rel_err(y1, y0), "dx": rel_err(dx1, dx0)}
    errs.update({n: rel_err(g1[n], g0[n]) for n in g0})
    worst = max(errs, key=errs.get)
    print(f"gate in read {kind} {dtype}: worst {worst} {errs[worst]:.3g}", flush=True)
    for k, e in errs.items():
        assert e < tol, (k, e)
