"""Pins of the oracle's GN extensions (CPU tests): the tanh hidden layer, a
Jacobi damping separate from eps and the key mass of signed features.

The reference has none of them (its GN nonlinearities are relu2, silu and
swiglu, nonlin.py:28-31; its damping is eps, engine.py:255), so they are
pinned by mathematics the oracle's code does not restate:
* tanh' against a central difference;
* the write payloads of one token against a Gauss-Newton construction by
  autograd Jacobians: lam = r / (diag(J J^T) + damping), J the Jacobian of the
  fast network's output in its weights (RMSNorm's scale held fixed, the
  reference's scalar-derivative approximation), and g = (du/da)^T lam;
* the key mass of signed (tanh) features against the double sum over tokens
  and features of |q| |k| with each view's weights written out, the bound
  |read| <= max |value| it gives, and its equality with the unit-column mass
  for nonnegative features;
* with relu2 and damping = eps the golden reference mixer is reproduced, and
  a larger damping changes it.
"""
from __future__ import annotations

import pytest
import torch

from oracle import mixer
from tests.test_oracle_golden import close, load_case


def test_tanh_slope_is_the_derivative():
    pre = torch.linspace(-4, 4, 101, dtype=torch.float64)
    h = 1e-6
    numeric = (torch.tanh(pre + h) - torch.tanh(pre - h)) / (2 * h)
    assert torch.allclose(mixer.ACT["tanh"][1](pre), numeric, atol=1e-9)


@pytest.mark.parametrize("nonlin,damping", [("tanh", 1e-2), ("tanh", None), ("relu2", 1e-2)])
def test_write_of_one_token_is_the_damped_gauss_newton_step(nonlin, damping):
    g = torch.Generator().manual_seed(41)
    d, m = 5, 7
    x = torch.randn(1, 1, 1, d, generator=g, dtype=torch.float64)
    v = torch.randn(1, 1, 1, d, generator=g, dtype=torch.float64)
    W1 = torch.randn(1, m, d, generator=g, dtype=torch.float64) / d ** 0.5
    W2 = torch.randn(1, d, m, generator=g, dtype=torch.float64) * 0.4
    c = {"write_rule": "gn", "nonlin": nonlin, "depth": 1, "fast_w1": True, "write_iters": 1,
         "learn_thresh": False, "value_centers": 0, "gn_damping": damping}
    st = mixer.write_streams([(W1, W2, None)], c, x, v, None, {})
    (_, g_or), = st["la1"]
    (_, lam_or), = st["la2"]

    sigma = {"tanh": torch.tanh, "relu2": lambda p: torch.relu(p) ** 2}[nonlin]
    xv, vv = x[0, 0, 0], v[0, 0, 0]
    a0 = W1[0] @ xv
    rinv = torch.rsqrt(a0.square().mean() + 1e-6)  # held fixed

    def fast_net(w1, w2):
        return xv + w2 @ sigma((w1 @ xv) * rinv)

    J1, J2 = torch.autograd.functional.jacobian(fast_net, (W1[0], W2[0]))
    diag = J1.reshape(d, -1).square().sum(1) + J2.reshape(d, -1).square().sum(1)
    r = vv - fast_net(W1[0], W2[0])
    lam = r / (diag + (1e-6 if damping is None else damping))
    assert torch.allclose(lam_or[0, 0, 0], lam, rtol=1e-10, atol=1e-12)

    a = a0.clone().requires_grad_(True)
    u = W2[0] @ sigma(a * rinv)
    (g_auto,) = torch.autograd.grad(u, a, lam)
    assert torch.allclose(g_or[0, 0, 0], g_auto, rtol=1e-10, atol=1e-12)


def _weights(kind, T, H, log_alpha, decay):
    """w[h, t, i] of a view by its definition, i <= t (interface.py:198-327):
    plain 1 or prod_{s=i+1..t} a_s, fast alpha^(t-i), stale 1 - alpha^(t-i)."""
    w = torch.zeros(H, T, T, dtype=torch.float64)
    for h in range(H):
        for t in range(T):
            for i in range(t + 1):
                fast = float(torch.exp(log_alpha[h] * (t - i)))
                if kind == "plain":
                    w[h, t, i] = float(torch.exp(decay[0, h, i + 1:t + 1, 0].sum())) if decay is not None else 1.0
                elif kind == "fast":
                    w[h, t, i] = fast
                else:
                    w[h, t, i] = 1.0 - fast
    return w


@pytest.mark.parametrize("kind,stream", [("plain", False), ("plain", True), ("fast", False), ("stale", False)])
def test_signed_feature_mass_is_the_absolute_feature_mass(kind, stream):
    g = torch.Generator().manual_seed(5)
    B, H, T, m, dv = 1, 2, 9, 4, 3
    qf = torch.tanh(torch.randn(B, H, T, m, generator=g, dtype=torch.float64) * 2)
    kf = torch.tanh(torch.randn(B, H, T, m, generator=g, dtype=torch.float64) * 2)
    vals = torch.randn(B, H, T, dv, generator=g, dtype=torch.float64)
    log_alpha = torch.log(torch.tensor([0.8, 0.95], dtype=torch.float64))
    decay = -torch.rand(B, H, T, 1, generator=g, dtype=torch.float64) * 0.3 if stream else None
    view = mixer.View(kind, decay=decay, log_alpha=None if kind == "plain" else log_alpha)
    unit = torch.full((B, H, T, 1), float("nan"), dtype=torch.float64)
    w = _weights(kind, T, H, log_alpha, decay)
    brute = torch.einsum("hti,htj,hij->ht", w, qf[0].abs(), kf[0].abs()).view(B, H, T, 1)
    tanh_mass = mixer.key_mass(view, qf, kf, unit, {"nonlin": "tanh"})
    assert torch.allclose(tanh_mass, brute, rtol=1e-12, atol=1e-12)
    # the normalized read is a signed average of the values: |read| <= max |v|
    num = view.scan(qf, kf, vals)
    assert torch.allclose(num, torch.einsum("hti,htj,hij,hid->htd", w, qf[0], kf[0], vals[0]).unsqueeze(0),
                          rtol=1e-12, atol=1e-12)
    assert (num.abs() <= tanh_mass * vals.abs().amax() * (1 + 1e-12)).all()
    # nonnegative features: it is the scan's unit column, the reference's mass
    pos_q, pos_k = qf.abs(), kf.abs()
    col = view.scan(pos_q, pos_k, torch.ones(B, H, T, 1, dtype=torch.float64))
    assert torch.allclose(mixer.key_mass(view, pos_q, pos_k, unit, {"nonlin": "tanh"}), col, rtol=1e-12, atol=1e-12)
    assert mixer.key_mass(view, pos_q, pos_k, col, {"nonlin": "relu2"}) is col


def test_relu2_with_damping_eps_reproduces_the_reference_and_damping_acts():
    pub, params, _, arrays = load_case("gn_relu2_plain_sum")
    core = mixer.core_config(pub)
    same = dict(core, gn_damping=1e-6)
    y = mixer.forward(same, params, arrays["x"])
    assert close(y, arrays["y"])
    other = dict(core, gn_damping=1e-2)
    y2 = mixer.forward(other, params, arrays["x"])
    assert not close(y2, arrays["y"], 1e-6)
