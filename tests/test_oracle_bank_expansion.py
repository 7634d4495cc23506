"""Pins of the oracle's bank and expansion extensions (CPU tests).

The long-context workload blends four recency rates {0.9, 0.99, 0.999,
0.9999} and expands a cubic B-spline memory 2x on its projection rows.  The
reference caps a bank at two branches (config.py:351-352) and expands only
the ReLU^2 ridge map (config.py:569-573), so both are pinned here by
identities the oracle's code does not restate:
* a J-rate bank is the sum of J one-rate banks minus (J - 1) bankless
  mixers, since the blend R_0 + sum_j eta_j (R_j - R_0) (fast) and
  R_0 - sum_j eta_j (S_j - N) (stale) is linear in the reads
  (tests/test_temporal_bank.py:66-112 pins the J = 2 case in the reference);
* the expanded B-spline mixer is the dense B-spline mixer whose trainable
  weights are E1 W1 and W2 E2, with E1 [16 x 8] and E2 [64 x 128] fixed
  +-1 rows of unit norm derived from the expansion key.
"""
from __future__ import annotations

import dataclasses
import json
from pathlib import Path

import pytest
import torch

from oracle import expansion
from oracle import mixer

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = json.loads((GOLDEN / "mixer_cases.json").read_text())
RATES = (0.9, 0.99, 0.999, 0.9999)


def _bspline_pub(mode="fast"):
    pub = json.loads(json.dumps(CASES["kernel_bspline_bank2"]["config"]))
    pub["temporal"]["bank_mode"] = mode
    return pub


def _params(c, seed, branches, expansion_factor=1):
    """Parameters of the core module for the oracle's flat config ``c``
    (float64), with seeded nonzero W2 and blends."""
    import thetascan_amd as ts
    from thetascan_amd._core.modules.block import ThetaScan as CoreMixer

    pub = _bspline_pub(c["read_fade_mode"])
    cfg = dataclasses.replace(ts.ThetaScanConfig.from_dict(pub)._to_core_config(), fade_branches=branches,
                              fade_alpha_inits=RATES[:branches], feature_expansion=expansion_factor)
    torch.manual_seed(seed)
    module = CoreMixer(cfg)
    g = torch.Generator().manual_seed(seed + 1)
    params = {}
    for name, p in module.named_parameters():
        t = p.detach().double().clone()
        if name.startswith("W2.") or name == "fade_eta":
            t = torch.randn(t.shape, generator=g, dtype=torch.float64) * (0.5 if name == "fade_eta" else 0.2)
        params[name] = t
    return params


@pytest.mark.parametrize("mode", ["fast", "stale"])
def test_four_rate_bank_is_the_sum_of_one_rate_banks(mode):
    c4 = dict(mixer.core_config(_bspline_pub(mode)), fade_branches=4)
    p4 = _params(c4, 3, 4)
    x = torch.randn(1, 40, 32, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    y4 = mixer.forward(c4, p4, x)
    ys = []
    for j in range(4):
        pj = dict(p4, fade_alpha=p4["fade_alpha"][j].clone(), fade_eta=p4["fade_eta"][j].clone())
        ys.append(mixer.forward(dict(c4, fade_branches=1), pj, x))
    plain = {k: v for k, v in p4.items() if not k.startswith("fade_")}
    y0 = mixer.forward(dict(c4, read_fade=False), plain, x)
    assert torch.allclose(y4, sum(ys) - 3 * y0, rtol=1e-10, atol=1e-12)
    # the rates matter: dropping one branch changes the output
    p3 = dict(p4, fade_alpha=p4["fade_alpha"][:3].clone(), fade_eta=p4["fade_eta"][:3].clone())
    assert not torch.allclose(mixer.forward(dict(c4, fade_branches=3), p3, x), y4, rtol=1e-6)


def test_expanded_bspline_is_the_dense_bspline_with_mapped_weights():
    c = dict(mixer.core_config(_bspline_pub()), feature_expansion=2, fade_branches=2)
    p = _params(c, 5, 2, expansion_factor=2)
    m, nb = c["mem_hidden"], c["bspline_basis_count"]
    assert p["W1.0"].shape == (2, m // 2 // nb, 16) and p["W2.0"].shape == (2, 16, m // 2)
    E1 = expansion.row_map((1, m // nb, m // 2 // nb), "thetascan", "w1-expand-layer-0").double()
    E2 = expansion.row_map((1, m // 2, m), "thetascan", "w2-expand-layer-0").double()
    for E in (E1, E2):  # +-1 rows of unit norm
        assert torch.allclose(E.abs(), torch.full_like(E, E.shape[-1] ** -0.5), rtol=1e-7, atol=0)
    x = torch.randn(1, 30, 32, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    dense = dict(p, **{"W1.0": torch.matmul(E1, p["W1.0"]), "W2.0": torch.matmul(p["W2.0"], E2)})
    y = mixer.forward(c, p, x)
    y_dense = mixer.forward(dict(c, feature_expansion=1), dense, x)
    assert torch.allclose(y, y_dense, rtol=1e-12, atol=1e-13)
