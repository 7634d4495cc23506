"""Parity at the benchmarked shapes (GPU tests).

* The one-view scan at B2 H8 T4096 d64 with the automatic segmentation (eight
  segments of eight 64-token tiles per (b, h)) against the float64 tiled
  oracle, forward and every gradient.
* Both headline mixer variants -- feature RoPE with the unnormalized read, and
  input RoPE with the key-mass read -- at d_model 512, H8, d64, m64, T4096 in
  bf16: forward, dx and every parameter gradient of B=2 against the float64
  oracle, then B=8 made of four copies of those two sequences against the same
  oracle rows (and four times its parameter gradients).
* The ThetaScan-Kernel CPU-reference workload: B2 T1024 d512 H8, softmax
  partition, a fast recency bank with per-head retentions drawn from
  U[0.9, 0.999] (``fade_alpha = logit(alpha)``) and non-zero blends, fp32 at
  rel 1e-3, and its memory after the last token (the streaming state) against
  the closed form N_T = sum_i w_i phi(k_i) v_i^T, D_T = sum_i w_i phi(k_i)
  per view.
* A temporal-bank mixer and a GN mixer in bf16 against the oracle (rel 2e-2).

The oracle is ``oracle.mixer.forward`` with the tiled scan (``linattn_chunk``,
equal to the sequential recurrence at 1e-12, linear in T).
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import torch

from oracle import mixer as oracle_mixer
from oracle import scans as oracle
from tests.conftest import rel_err
from tests.test_mixer_gpu import _headline_config, _seeded, build_module

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = json.loads((GOLDEN / "mixer_cases.json").read_text())


# ------------------------------------------------------------------ scan

def _retention(kind, B, H, T, g):
    if kind == "none":
        return None
    if kind == "static":
        return torch.log(torch.rand(H, generator=g, dtype=torch.float64) * 0.099 + 0.9)
    return -torch.rand(B, H, T, 1, generator=g, dtype=torch.float64) * 0.05


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("kind", ["none", "static", "stream"])
def test_scan_at_T4096_matches_float64_oracle(cuda, dtype, kind):
    from thetascan_amd._core.ops import scan_hip

    B, H, T, D = 2, 8, 4096, 64
    g = torch.Generator().manual_seed(4096)
    q, k, v = (torch.randn(B, H, T, D, generator=g, dtype=torch.float64).to(dtype).to(torch.float64)
               for _ in range(3))
    q, k = q / 8.0, k / 8.0
    ret = _retention(kind, B, H, T, g)
    dy = torch.randn(B, H, T, D, generator=g, dtype=torch.float64).to(dtype).to(torch.float64)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v)]
    r64 = None if ret is None else ret.clone().requires_grad_(True)
    decay = None if r64 is None else (oracle.as_stream(r64, q) if r64.ndim == 1 else r64)
    ref = oracle.linattn_chunk(*leaves, decay)
    (ref * dy).sum().backward()

    dev = [x.detach().to(cuda, dtype).requires_grad_(True) for x in (q, k, v)]
    r_dev = None if ret is None else ret.to(cuda, torch.float32).requires_grad_(True)
    out = scan_hip.linattn_views(*dev, (r_dev,), 64)[0]
    (out.float() * dy.to(cuda, torch.float32)).sum().backward()
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-3
    print(f"scan T4096 {kind} {dtype}", flush=True)
    assert rel_err(out, ref) < tol
    for a, b in zip(dev, leaves):
        assert rel_err(a.grad, b.grad) < tol
    if r_dev is not None:
        assert rel_err(r_dev.grad, r64.grad) < tol


# ------------------------------------------------------------------ headline mixer

def _oracle_run(pub, module, x, dy):
    core = oracle_mixer.core_config(pub)
    params = {k: v.detach().double().cpu().clone().requires_grad_(True) for k, v in module._core.named_parameters()}
    x64 = x.clone().requires_grad_(True)
    y = oracle_mixer.forward(core, params, x64, backend="chunk")
    (y * dy).sum().backward()
    return y.detach(), x64.grad, {k: p.grad for k, p in params.items() if p.grad is not None}


@pytest.mark.parametrize("variant", [("feature", "none"), ("input", "key_mass")])
def test_headline_mixer_at_T4096_matches_float64_oracle(cuda, variant):
    """The benchmarked mixer at its own sequence length, bf16 (rel 2e-2)."""
    placement, normalization = variant
    pub = _headline_config(placement, normalization)
    module = build_module(pub, cuda, torch.float32)
    _seeded(module, 7)
    module = module.to(torch.bfloat16)
    g = torch.Generator().manual_seed(8)
    B, T, D = 2, 4096, 512
    # identical inputs on both sides: the bf16 values of x and the weights
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64).to(torch.bfloat16).double()
    dy = torch.randn(B, T, D, generator=g, dtype=torch.float64) * 0.1
    y64, dx64, grads64 = _oracle_run(pub, module, x, dy)

    for reps in (1, 4):
        module.zero_grad(set_to_none=True)
        xb = x.repeat(reps, 1, 1).to(cuda, torch.bfloat16).requires_grad_(True)
        yb = module(xb)
        assert module._core.last_path == "fused"
        (yb.float() * dy.repeat(reps, 1, 1).to(cuda, torch.float32)).sum().backward()
        torch.cuda.synchronize()
        print(f"headline {variant} B={B * reps}", flush=True)
        for r in range(reps):
            rows = slice(r * B, (r + 1) * B)
            assert rel_err(yb[rows], y64) < 2e-2, (variant, reps, r)
            assert rel_err(xb.grad[rows], dx64) < 2e-2, (variant, reps, r)
        for name, p in module._core.named_parameters():
            if name in grads64 and grads64[name].abs().max() > 0:
                assert rel_err(p.grad, reps * grads64[name]) < 2e-2, (variant, reps, name)


# ------------------------------------------------------------------ CPU-reference workload (bank)

def _bank_config(d_model, heads, feature_map="softmax_partition", normalization="key_mass", branches=1,
                 bank_mode="fast"):
    pub = _headline_config("input", normalization, feature_map, d_model=d_model, heads=heads)
    pub["temporal"].update(mode="bank", bank_mode=bank_mode, recency_branches=branches,
                           retention_inits=[0.9, 0.99][:branches] if branches > 1 else None)
    pub["output_gate"] = False
    return pub


def _per_head_retentions(module, H, g, branches=1):
    """fade_alpha = logit(alpha_h), alpha_h ~ U[0.9, 0.999]; eta ~ U[-0.5, 0.5] (non-zero)."""
    core = module._core
    with torch.no_grad():
        alpha = torch.rand(core.fade_alpha.shape, generator=g, dtype=torch.float64) * 0.099 + 0.9
        core.fade_alpha.copy_(torch.log(alpha / (1 - alpha)))
        core.fade_eta.copy_(torch.rand(core.fade_eta.shape, generator=g, dtype=torch.float64) - 0.5)


def test_cpu_reference_workload_matches_oracle_fp32(cuda):
    """B2 T1024 d512 H8 m64 softmax partition, fast bank with per-head
    retentions from U[0.9, 0.999], fp32: forward, dx and every parameter
    gradient against the float64 oracle."""
    pub = _bank_config(512, 8)
    module = build_module(pub, cuda, torch.float32)
    _seeded(module, 11)
    g = torch.Generator().manual_seed(12)
    _per_head_retentions(module, 8, g)
    B, T = 2, 1024
    x = torch.randn(B, T, 512, generator=g, dtype=torch.float64)
    dy = torch.randn(B, T, 512, generator=g, dtype=torch.float64) * 0.1
    y64, dx64, grads64 = _oracle_run(pub, module, x, dy)
    xf = x.to(cuda, torch.float32).requires_grad_(True)
    y = module(xf)
    (y * dy.to(cuda, torch.float32)).sum().backward()
    print(f"cpu-reference workload path={module._core.last_path}", flush=True)
    worst = max((rel_err(p.grad, grads64[n]), n) for n, p in module._core.named_parameters()
                if n in grads64 and grads64[n].abs().max() > 0)
    print(f"errors config 1 fp32: y {rel_err(y, y64):.2e} dx {rel_err(xf.grad, dx64):.2e} "
          f"worst parameter gradient {worst[0]:.2e} ({worst[1]})", flush=True)
    assert rel_err(y, y64) < 1e-3
    assert rel_err(xf.grad, dx64) < 1e-3
    for name, p in module._core.named_parameters():
        if name in grads64 and grads64[name].abs().max() > 0:
            assert rel_err(p.grad, grads64[name]) < 1e-3, name
    # the memory after the last token, per view: N_T = sum_i w_i phi(k_i) v_i^T
    # and D_T = sum_i w_i phi(k_i) (plain sum, then the recency branch)
    with torch.no_grad():
        _, state = module(xf.detach(), state=module.initial_state())
    params = {k: v.detach().double().cpu() for k, v in module._core.named_parameters()}
    finals = oracle_mixer.kernel_final_states(oracle_mixer.core_config(pub), params, x)
    assert len(state.carries) == len(finals) == 2
    m = d = 64
    for (blocks), (N, D) in zip(state.carries, finals):
        fin = blocks[0]
        assert rel_err(fin[:, :, :m, :d], N) < 1e-3
        assert rel_err(fin[:, :, :m, d], D) < 1e-3


# ------------------------------------------------------------------ bf16 bank and GN mixers

def _dx_of_reference_in_bf16(pub, module, x, dy, dx64, monkeypatch):
    """rel error of dx when the reference algorithm itself runs in bf16: the
    oracle executed with bf16 tensors (every operation rounds its result to
    bf16, as eager bf16 torch does) and its scans accumulating in fp32 from
    the bf16 operands, as the reference's chunk backend does."""
    real = oracle_mixer.SCANS["chunk"]

    def chunk_fp32_state(q, k, v, decay=None, chunk=64):
        return real(q.float(), k.float(), v.float(), None if decay is None else decay.float()).to(q.dtype)

    monkeypatch.setitem(oracle_mixer.SCANS, "chunk", chunk_fp32_state)
    try:
        core = oracle_mixer.core_config(pub)
        params = {k: v.detach().to("cpu", torch.bfloat16).clone().requires_grad_(True)
                  for k, v in module._core.named_parameters()}
        xb = x.to(torch.bfloat16).clone().requires_grad_(True)
        y = oracle_mixer.forward(core, params, xb, backend="chunk")
        (y * dy.to(torch.bfloat16)).sum().backward()
    finally:
        monkeypatch.setitem(oracle_mixer.SCANS, "chunk", real)
    return rel_err(xb.grad, dx64)


def _bf16_against_oracle(cuda, pub, module, B, T, seed, tol=2e-2, monkeypatch=None):
    """bf16 module against the float64 oracle on identical inputs (the bf16
    values of x and of every parameter).  With ``monkeypatch`` the bar of dx is
    the larger of ``tol`` and 1.25 times the error of the reference algorithm
    itself run in bf16 (an ill-conditioned input gradient: the key's L2-norm
    backward removes a large radial component, so bf16 storage of the key
    gradient is amplified)."""
    g = torch.Generator().manual_seed(seed)
    D = pub["d_model"]
    module = module.to(torch.bfloat16)
    x = torch.randn(B, T, D, generator=g, dtype=torch.float64).to(torch.bfloat16).double()
    dy = torch.randn(B, T, D, generator=g, dtype=torch.float64) * 0.1
    y64, dx64, grads64 = _oracle_run(pub, module, x, dy)
    dx_tol = tol
    if monkeypatch is not None:
        # for reference: the reference algorithm run in bf16 has an input-gradient
        # error of its own (printed); the HIP path is held to the bf16 bar regardless
        floor = _dx_of_reference_in_bf16(pub, module, x, dy, dx64, monkeypatch)
        print(f"dx of the reference algorithm in bf16: {floor:.4f}", flush=True)
    xb = x.to(cuda, torch.bfloat16).requires_grad_(True)
    yb = module(xb)
    (yb.float() * dy.to(cuda, torch.float32)).sum().backward()
    worst = max((rel_err(p.grad, grads64[n]), n) for n, p in module._core.named_parameters()
                if n in grads64 and grads64[n].abs().max() > 0)
    print(f"errors bf16: y {rel_err(yb, y64):.2e} dx {rel_err(xb.grad, dx64):.2e} (bar {dx_tol:.2e}) "
          f"worst parameter gradient {worst[0]:.2e} ({worst[1]})", flush=True)
    assert rel_err(yb, y64) < tol
    assert rel_err(xb.grad, dx64) < dx_tol
    for name, p in module._core.named_parameters():
        if name in grads64 and grads64[name].abs().max() > 0:
            assert rel_err(p.grad, grads64[name]) < tol, name


@pytest.mark.parametrize("bank_mode,branches", [("fast", 2), ("stale", 1)])
def test_bank_mixer_bf16_matches_oracle(cuda, bank_mode, branches):
    pub = _bank_config(256, 4, "relu2_ridge", "key_mass", branches, bank_mode)
    module = build_module(pub, cuda, torch.float32)
    _seeded(module, 21)
    _per_head_retentions(module, 4, torch.Generator().manual_seed(22), branches)
    print(f"bank bf16 {bank_mode} {branches}", flush=True)
    _bf16_against_oracle(cuda, pub, module, 2, 700, 23)


def test_gn_mixer_bf16_matches_oracle(cuda, monkeypatch):
    pub = json.loads(json.dumps(CASES["gn_relu2_plain_sum"]["config"]))
    pub.update(d_model=256, n_heads=4)
    pub["runtime"]["scan_chunk"] = 64
    module = build_module(pub, cuda, torch.float32)
    g = torch.Generator().manual_seed(31)
    with torch.no_grad():
        for name, p in sorted(module._core.named_parameters()):
            if name.startswith("W2."):
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    print("gn bf16", flush=True)
    _bf16_against_oracle(cuda, pub, module, 2, 600, 32, monkeypatch=monkeypatch)
