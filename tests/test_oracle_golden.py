"""Pin the CPU oracle to the reference's golden vectors (CPU tests).

The vectors in tests/golden were written by tests/golden/make_golden.py from
the reference implementation (float64, naive backend).  Each oracle function
must reproduce them to float64 round-off; closed-form checks cover what the
vectors leave open (tests/test_oracle_closed_forms.py).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import expansion, mixer, scans

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = json.loads((GOLDEN / "mixer_cases.json").read_text())


def load_case(name):
    data = np.load(GOLDEN / f"mixer_{name}.npz", allow_pickle=False)
    params = {k[len("param:_core."):]: torch.from_numpy(data[k]) for k in data.files if k.startswith("param:")}
    grads = {k[len("grad:_core."):]: torch.from_numpy(data[k]) for k in data.files if k.startswith("grad:_core.")}
    arrays = {k: torch.from_numpy(data[k]) for k in ("x", "dy", "y", "grad:x")}
    return CASES[name]["config"], params, grads, arrays


def close(a, b, rel=1e-9):
    scale = b.abs().max().clamp_min(1e-300)
    return float((a - b).abs().max() / scale) < rel


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_mixer_matches_reference(name):
    pub, params, grads, arrays = load_case(name)
    core = mixer.core_config(pub)
    leaves = {k: v.clone().requires_grad_(True) for k, v in params.items()}
    x = arrays["x"].clone().requires_grad_(True)
    y = mixer.forward(core, leaves, x)
    assert close(y.detach(), arrays["y"]), name
    (y * arrays["dy"]).sum().backward()
    assert close(x.grad, arrays["grad:x"], 1e-8), name
    for pname, g in grads.items():
        assert leaves[pname].grad is not None, (name, pname)
        assert close(leaves[pname].grad, g, 1e-8), (name, pname)


def test_oracle_scans_match_reference_vectors():
    d = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "scan_streams.npz").items()}
    q, k, v, la, decay = d["q"], d["k"], d["v"], d["log_alpha"], d["decay"]
    static = scans.as_stream(la, q)
    assert close(scans.linattn_naive(q, k, v), d["naive_sum"], 1e-12)
    assert close(scans.linattn_naive(q, k, v, static), d["naive_static"], 1e-12)
    assert close(scans.linattn_naive(q, k, v, decay), d["naive_stream"], 1e-12)
    assert close(scans.linattn_quad(q, k, v, decay), d["quad_stream"], 1e-12)
    assert close(scans.linattn_cumsum(q, k, v), d["cumsum_sum"], 1e-12)
    assert close(scans.linattn_cumsum(q, k, v, decay), d["cumsum_stream"], 1e-9)
    assert close(scans.linattn_naive(q, k, v, static), d["chunk8_static"], 1e-12)
    assert close(scans.ema_cumsum(k, la), d["ema_cumsum_k"], 1e-12)
    assert close(scans.causal_prefix_sum(k), d["prefix_k"], 1e-12)
    # gradients of <dO, scan> (reference chunk backend, fp64) through the oracle
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    lar = la.clone().requires_grad_(True)
    out = scans.linattn_naive(*leaves, scans.as_stream(lar, q))
    (out * d["dO"]).sum().backward()
    for leaf, key in zip(leaves + [lar], ("grad_q", "grad_k", "grad_v", "grad_log_alpha")):
        assert close(leaf.grad, d[key], 1e-10), key


def test_oracle_feature_maps_match_reference_vectors():
    d = {k: torch.from_numpy(v) for k, v in np.load(GOLDEN / "features.npz").items()}
    pre, tau, rho, blend = d["pre"], d["tau"], d["rho"], d["blend"]
    assert close(mixer.relu2_ridge(pre, None, tau), d["relu2"], 1e-12)
    assert close(mixer.softmax_partition(pre, 8.0), d["softmax"], 1e-12)
    for mode in ("relative_soft", "relative_st", "relative_st_blend"):
        got = mixer.softmax_partition(pre, 8.0, None, mode, rho, blend, 0.25)
        assert close(got, d[f"softmax_{mode}"], 1e-12), mode
    assert close(mixer.bspline_basis(d["bspline_coords"], 8, 3, 3.0), d["bspline_basis"], 1e-12)
    c = {"bspline_basis_count": 8, "bspline_degree": 3, "bspline_bound": 3.0}
    assert close(mixer.bspline_features(pre[..., :4], 1.0, c), d["bspline_features"], 1e-12)
    assert close(mixer.apply_rope(d["rope_x"], "partial", 0.5, 10000.0), d["rope_partial"], 1e-12)
    assert close(mixer.apply_rope(d["rope_x"], "full", 0.5, 1337.0), d["rope_full"], 1e-12)
    for shape, role in (((1, 16, 8), "w1-expand-layer-0"), ((1, 8, 16), "w2-expand-layer-0")):
        got = expansion.row_map(shape, "thetascan", role).double()
        assert torch.equal(got, d[f"rowmap_{role}"]), role
    fp = expansion.fingerprint("thetascan", 192, 2, 1)
    assert bytes(d["fingerprint"].tolist()) == fp
