"""Parity at the secondary workloads' own shapes (GPU tests).

* ThetaScan-GN: fast net 64 -> 128 -> 64 with tanh, damping 1e-2, two-stage
  read normalization, d_model 512, H8, T2048, bf16.  B=1 against the float64
  oracle on the output, dx and every parameter gradient, then B=8 made of
  eight copies of that sequence against the same oracle rows (and eight times
  its parameter gradients).
* The long-context bank: the five retentions of a four-rate bank (the plain
  sum and 0.9, 0.99, 0.999, 0.9999) scanned with the key-mass column at
  dk 128, dv 64, T=32768 against the float64 tiled oracle; and the B-spline
  four-rate bank mixer forward on one T=32768 sequence against the float64
  oracle mixer.
* The hybrid language model at B64 T1024: fwd+bwd with finite gradients, both
  ThetaScan layers on the HIP feature-kernel path, Adam steps that lower the
  loss, and the per-row int8 round trip of its weights within 1e-3 relative
  of the bf16 eval loss (the host model is this build's own definition, so
  this has no reference number: parity unpinned).

Bars: rel 2e-2 in bf16 (max |a - e| / max |e|, the reference's metric,
tests/test_scan_chunk.py:125-138).
"""
from __future__ import annotations

import dataclasses

import pytest
import torch

from oracle import mixer as oracle_mixer
from oracle import scans as oracle
from tests.conftest import rel_err

pytestmark = pytest.mark.gpu

DAMP = 1e-2
RATES = (0.9, 0.99, 0.999, 0.9999)


# ------------------------------------------------------------------ ThetaScan-GN, d512 H8 T2048

def gn_workload(cuda, seed):
    """The GN workload's mixer: tanh fast net 64 -> 128 -> 64, damping 1e-2,
    both-feature-mass read, plain sum, chunk 64; slow reference weights W1, W2
    ~ N(0, 0.02).  Returns the bf16 module and the oracle's flat config."""
    import thetascan_amd as ts
    from thetascan_amd._core.modules.block import ThetaScan as CoreMixer

    public = ts.ThetaScanConfig(
        d_model=512, n_heads=8, memory_multiplier=2, family="gn",
        gn=ts.GNConfig(nonlinearity="relu2", jacobian_steps=1, read_normalization="both_feature_mass"),
        temporal=ts.TemporalConfig(mode="sum"), runtime=ts.RuntimeConfig(backend="hip", scan_chunk=64),
    )
    cfg = dataclasses.replace(public._to_core_config(), nonlin="tanh", gn_damping=DAMP)
    torch.manual_seed(seed)
    module = CoreMixer(cfg)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.startswith(("W1.", "W2.")):
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    core = dict(oracle_mixer.core_config(public.to_dict()), nonlin="tanh", gn_damping=DAMP)
    return module.to(cuda, torch.bfloat16), core


def _oracle_fwd_bwd(core, module, x, dy):
    params = {k: v.detach().double().cpu().clone().requires_grad_(True) for k, v in module.named_parameters()}
    x64 = x.clone().requires_grad_(True)
    y = oracle_mixer.forward(core, params, x64, backend="chunk")
    (y * dy).sum().backward()
    return y.detach(), x64.grad, {k: p.grad for k, p in params.items() if p.grad is not None}


def test_gn_workload_at_T2048_matches_float64_oracle(cuda):
    """The output, dx and every parameter gradient at rel 2e-2."""
    module, core = gn_workload(cuda, 40)
    g = torch.Generator().manual_seed(41)
    B, T, D = 1, 2048, 512
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64).to(torch.bfloat16).double()
    dy = torch.randn(B, T, D, generator=g, dtype=torch.float64) * 0.1
    y64, dx64, grads64 = _oracle_fwd_bwd(core, module, x, dy)
    for reps in (1, 8):
        module.zero_grad(set_to_none=True)
        xb = x.repeat(reps, 1, 1).to(cuda, torch.bfloat16).requires_grad_(True)
        yb = module(xb)
        (yb.float() * dy.repeat(reps, 1, 1).to(cuda, torch.float32)).sum().backward()
        torch.cuda.synchronize()
        errs = {"y": max(rel_err(yb[r:r + 1], y64) for r in range(reps)),
                "dx": max(rel_err(xb.grad[r:r + 1], dx64) for r in range(reps))}
        for name, p in module.named_parameters():
            if name in grads64 and grads64[name].abs().max() > 0:
                errs[name] = rel_err(p.grad, reps * grads64[name])
        print(f"gn workload B={reps} T={T} path={module.last_path} "
              + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
        for name, err in errs.items():
            assert err < 2e-2, (reps, name, err)


# ------------------------------------------------------------------ the long-context bank, T=32768

@pytest.mark.parametrize("mass", [False, True])
def test_bank_views_scan_at_T32768_matches_float64_oracle(cuda, mass):
    """Five retentions over dk 128 and dv 64 (plus the key-mass column) at
    T=32768 (512 tiles of 64): each view's output and mass against the float64
    tiled oracle, which equals the sequential recurrence at 1e-12."""
    from thetascan_amd._core.ops import scan_hip

    B, H, T, dk, dv = 1, 2, 32768, 128, 64
    g = torch.Generator().manual_seed(32768)
    # nonnegative feature-like keys and queries, as the B-spline map produces
    q = (torch.rand(B, H, T, dk, generator=g, dtype=torch.float64) / dk).to(torch.bfloat16)
    k = (torch.rand(B, H, T, dk, generator=g, dtype=torch.float64) / dk).to(torch.bfloat16)
    v = torch.randn(B, H, T, dv, generator=g, dtype=torch.float64).to(torch.bfloat16)
    rets = (None,) + tuple(torch.full((H,), r, dtype=torch.float64).log() for r in RATES)
    dev = [t.to(cuda) for t in (q, k, v)]
    dev_rets = tuple(None if r is None else r.to(cuda, torch.float32) for r in rets)
    if mass:
        got = scan_hip.linattn_views_mass(*dev, dev_rets)
    else:
        got = [(out, None) for out in scan_hip.linattn_views(*dev, dev_rets)]
    torch.cuda.synchronize()
    v_ext = torch.cat([v.double(), torch.ones(B, H, T, 1, dtype=torch.float64)], -1) if mass else v.double()
    for r, (out, m) in zip(rets, got):
        decay = None if r is None else oracle.as_stream(r, q)
        ref = oracle.linattn_chunk(q.double(), k.double(), v_ext, decay)
        e_out = rel_err(out, ref[..., :dv])
        e_mass = rel_err(m, ref[..., dv]) if mass else 0.0
        print(f"views T32768 rate={None if r is None else float(r[0].exp()):} out={e_out:.2e} mass={e_mass:.2e}",
              flush=True)
        assert e_out < 2e-2 and e_mass < 2e-2


def bank4_workload(cuda, seed):
    """The long-context workload's mixer (core config: B-spline map with 8
    basis functions, 2x expansion to m = 128, key-mass read, fast bank of the
    four rates, chunk 128) in bf16, and the oracle's flat config."""
    import thetascan_amd as ts
    from thetascan_amd._core.modules.block import ThetaScan as CoreMixer

    public = ts.ThetaScanConfig(
        d_model=512, n_heads=8, memory_multiplier=2, family="kernel",
        kernel=ts.KernelConfig(feature_map="projected_bspline", read_normalization="key_mass"),
        temporal=ts.TemporalConfig(mode="bank", bank_mode="fast", recency_branches=2, retention_inits=(0.9, 0.999)),
        runtime=ts.RuntimeConfig(backend="hip", scan_chunk=128),
    )
    cfg = dataclasses.replace(public._to_core_config(), feature_expansion=2, fade_branches=4, fade_alpha_inits=RATES)
    torch.manual_seed(seed)
    module = CoreMixer(cfg)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.startswith("W2.") or name == "fade_eta":
                p.copy_(torch.randn(p.shape, generator=g) * (0.3 if name == "fade_eta" else 0.02))
    core = dict(oracle_mixer.core_config(public.to_dict()), feature_expansion=2, fade_branches=4)
    return module.to(cuda, torch.bfloat16), core


def test_bank4_mixer_forward_at_T32768_matches_float64_oracle(cuda):
    module, core = bank4_workload(cuda, 50)
    g = torch.Generator().manual_seed(51)
    x = torch.randn(1, 32768, 512, generator=g, dtype=torch.float64).to(torch.bfloat16).double()
    with torch.no_grad():
        y = module(x.to(cuda, torch.bfloat16))
        torch.cuda.synchronize()
        params = {k: v.detach().double().cpu() for k, v in module.named_parameters()}
        y64 = oracle_mixer.forward(core, params, x, backend="chunk")
    errs = [rel_err(y[:, a:a + 4096], y64[:, a:a + 4096]) for a in range(0, 32768, 4096)]
    print(f"bank4 mixer T32768 path={module.last_path} rel err per 4096-token block "
          + " ".join(f"{e:.2e}" for e in errs), flush=True)
    assert rel_err(y, y64) < 2e-2


# ------------------------------------------------------------------ the hybrid LM, B64 T1024

def _affine_batches(g, dev, B, T):
    """A learnable stream: token_{t+1} = (5 token_t + 3) mod 1024."""
    from thetascan_amd import hybrid_lm as lm

    start = torch.randint(0, lm.VOCAB, (B, 1), generator=g)
    seq = [start]
    for _ in range(T):
        seq.append((seq[-1] * 5 + 3) % lm.VOCAB)
    s = torch.cat(seq, 1).to(dev)
    return s[:, :-1], s[:, 1:]


def test_hybrid_lm_at_B64_T1024(cuda):
    from thetascan_amd import hybrid_lm as lm

    torch.manual_seed(0)
    model = lm.HybridLM().to(cuda, torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    opt = torch.optim.Adam(model.parameters(), lr=2e-3)
    losses = []
    for step in range(6):
        x, y = _affine_batches(g, cuda, 64, 1024)
        loss = model(x, y)
        opt.zero_grad(set_to_none=True)
        loss.backward()
        for name, p in model.named_parameters():
            assert p.grad is not None and torch.isfinite(p.grad.float()).all(), name
        opt.step()
        losses.append(float(loss.detach()))
        print(f"hybrid LM B64 T1024 step {step} loss {losses[-1]:.4f}", flush=True)
    for layer in lm.THETA_LAYERS:
        assert model.blocks[layer].attn._core.last_path == "fused", layer
    assert losses[-1] < 0.8 * losses[0]
    model.eval()
    with torch.no_grad():
        x, y = _affine_batches(g, cuda, 64, 1024)
        base = float(model(x, y))
        model.load_state_dict(lm.int8_round_trip(model))
        quant = float(model(x, y))
    print(f"B64 T1024 eval loss bf16 {base:.6f} int8 round trip {quant:.6f}", flush=True)
    assert abs(quant - base) / base < 1e-3
