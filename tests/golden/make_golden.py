"""Write golden vectors from the reference implementation (run in the build
container only; the reference never travels with the repository).

    python tests/golden/make_golden.py [--reference /root/reference/src]

The reference is pure Python over torch.  It is imported here for exactly the
functions no closed form or brute-force check pins on its own: the end-to-end
mixer forward/backward for each configuration family, the feature maps with
their numerical safeguards, RoPE, and the SHAKE256 expansion maps.  Scan
vectors for the reference's own ``_streams`` fixture are included too, so the
oracle's scans are checked against the reference's numbers and not only
against closed forms.

Every case is a small float64 computation with the ``naive`` backend (the
parity target).  Inputs, parameters, outputs and gradients are stored as
``.npz`` arrays (no pickles) next to a JSON manifest of the configurations.
"""
from __future__ import annotations

import argparse
import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().to(torch.float64).numpy()


def perturb_parameters(module: torch.nn.Module, seed: int, scale: float = 0.05) -> None:
    """Move every parameter off its (often zero) initialisation, deterministically."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sorted(module.named_parameters()):
            p.add_(torch.randn(p.shape, generator=g, dtype=p.dtype) * scale)


def mixer_cases(api):
    C = api
    H = 2
    D = 32
    small = dict(d_model=D, n_heads=H)
    cases = {
        # configuration 1 family: softmax partition, m = d, per-head bank retention
        "kernel_softmax_bank_fast": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="kernel",
            kernel=C.KernelConfig(feature_map="softmax_partition", read_normalization="key_mass"),
            temporal=C.TemporalConfig(mode="bank", bank_mode="fast", retention_init=0.95),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        # configuration 2a: ReLU^2 ridge, feature RoPE, no normalization
        "kernel_relu2_feature_rope": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="kernel",
            kernel=C.KernelConfig(feature_map="relu2_ridge", read_normalization="none"),
            rope=C.RoPEConfig(mode="partial", fraction=0.5, placement="feature"),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        # configuration 2b: ReLU^2 ridge, input RoPE, key-mass normalization
        "kernel_relu2_key_mass": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="kernel",
            kernel=C.KernelConfig(feature_map="relu2_ridge", read_normalization="key_mass"),
            rope=C.RoPEConfig(mode="partial", fraction=0.5, placement="input"),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        "kernel_relu2_threshold_feature_mass_ema": C.ThetaScanConfig(
            **small, memory_multiplier=2, family="kernel",
            kernel=C.KernelConfig(feature_map="relu2_ridge", relu2_threshold_mode="learned_per_head",
                                  read_normalization="feature_mass"),
            temporal=C.TemporalConfig(mode="ema"),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        "kernel_softmax_sparse_st_blend_stale": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="kernel",
            kernel=C.KernelConfig(feature_map="softmax_partition", sparsity="relative_st_blend",
                                  sparse_blend_init=0.5, kernel_sharpness_mode="learned_per_head"),
            temporal=C.TemporalConfig(mode="bank", bank_mode="stale", recency_branches=2),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        "kernel_bspline_bank2": C.ThetaScanConfig(
            **small, memory_multiplier=2, family="kernel",
            kernel=C.KernelConfig(feature_map="projected_bspline", bspline_scale_mode="learned_per_head"),
            rope=C.RoPEConfig(mode="partial", fraction=0.5),
            temporal=C.TemporalConfig(mode="bank", recency_branches=2, retention_inits=(0.9, 0.999)),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        "kernel_value_anchors_gqa": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="kernel", key_value_heads=1,
            kernel=C.KernelConfig(feature_map="softmax_partition", value_representation="value_anchors",
                                  value_anchors=5, score_bias=True),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        "kernel_value_mlp_share_kq": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="kernel", share_key_query=True, output_gate=False,
            kernel=C.KernelConfig(feature_map="relu2_ridge", value_representation="value_mlp",
                                  kernel_sharpness_mode="fixed"),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        "kernel_expanded_reference_v0_1": C.ThetaScanConfig.from_dict(
            {"preset": "kernel_expanded_reference_v0_1", "d_model": D, "n_heads": H,
             "runtime": {"backend": "naive"}}
        ),
        "gn_reference_v0_1": C.ThetaScanConfig.from_dict(
            {"preset": "gn_reference_v0_1", "d_model": D, "n_heads": H, "runtime": {"backend": "naive"}}
        ),
        "gn_expanded_reference_v0_1": C.ThetaScanConfig.from_dict(
            {"preset": "gn_expanded_reference_v0_1", "d_model": D, "n_heads": H,
             "runtime": {"backend": "naive"}}
        ),
        "gn_relu2_plain_sum": C.ThetaScanConfig(
            **small, memory_multiplier=2, family="gn", runtime=C.RuntimeConfig(backend="naive"),
        ),
        "gn_silu_two_steps_ema": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="gn",
            gn=C.GNConfig(nonlinearity="silu", jacobian_steps=2),
            temporal=C.TemporalConfig(mode="ema"),
            rope=C.RoPEConfig(mode="full"),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        "gn_relu2_w2_mass_stale_tanh": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="gn",
            gn=C.GNConfig(nonlinearity="relu2", read_normalization="w2_feature_mass"),
            temporal=C.TemporalConfig(mode="bank", bank_mode="stale", blend_mode="tanh"),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
        "gn_swiglu_depth2": C.ThetaScanConfig(
            **small, memory_multiplier=1, family="gn", depth=2,
            gn=C.GNConfig(nonlinearity="swiglu"),
            runtime=C.RuntimeConfig(backend="naive"),
        ),
    }
    return cases


def write_mixer_cases(api, out_dir: Path) -> dict:
    manifest = {}
    B, T = 2, 80
    for index, (name, config) in enumerate(mixer_cases(api).items()):
        torch.manual_seed(1000 + index)
        mixer = api.ThetaScan(config).double()
        perturb_parameters(mixer, 2000 + index)
        g = torch.Generator().manual_seed(3000 + index)
        x = torch.randn(B, T, config.d_model, generator=g, dtype=torch.float64)
        dy = torch.randn(B, T, config.d_model, generator=g, dtype=torch.float64)
        x.requires_grad_(True)
        y = mixer(x)
        (y * dy).sum().backward()
        arrays = {"x": _np(x), "dy": _np(dy), "y": _np(y), "grad:x": _np(x.grad)}
        for pname, p in mixer.named_parameters():
            arrays[f"param:{pname}"] = _np(p)
            if p.grad is not None:
                arrays[f"grad:{pname}"] = _np(p.grad)
        for bname, buf in mixer.named_buffers():
            if buf is not None and buf.dtype == torch.uint8:
                arrays[f"buffer:{bname}"] = buf.cpu().numpy()
        np.savez_compressed(out_dir / f"mixer_{name}.npz", **arrays)
        manifest[name] = {"config": json.loads(json.dumps(config.to_dict())), "B": B, "T": T}
        print(f"mixer {name}: y {tuple(y.shape)} |y|max {float(y.detach().abs().max()):.3e}", flush=True)
    return manifest


def write_scan_vectors(out_dir: Path) -> None:
    from thetascan._core.ops import scan_chunk, scan_cumsum, scan_naive, scan_quad
    from thetascan._core.ops.interface import causal_prefix_sum, ema_cumsum

    # The reference's _streams fixture (tests/test_scan_chunk.py:18-24).
    torch.manual_seed(20260725)
    B, H, T, Dk, Dv = 2, 3, 37, 5, 4
    q = torch.randn(B, H, T, Dk, dtype=torch.float64)
    k = torch.randn(B, H, T, Dk, dtype=torch.float64)
    v = torch.randn(B, H, T, Dv, dtype=torch.float64)
    log_alpha = torch.tensor([-0.05, -0.4, -2.0], dtype=torch.float64)
    torch.manual_seed(11)
    decay = -torch.rand(B, H, T, 1, dtype=torch.float64)
    static_stream = log_alpha.view(1, H, 1, 1).expand(B, H, T, 1)
    arrays = {"q": q, "k": k, "v": v, "log_alpha": log_alpha, "decay": decay}
    arrays["naive_sum"] = scan_naive.linattn(q, k, v)
    arrays["naive_static"] = scan_naive.linattn(q, k, v, static_stream)
    arrays["naive_stream"] = scan_naive.linattn(q, k, v, decay)
    arrays["quad_stream"] = scan_quad.linattn(q, k, v, decay)
    arrays["cumsum_sum"] = scan_cumsum.linattn(q, k, v)
    arrays["cumsum_stream"] = scan_cumsum.linattn(q, k, v, decay)
    arrays["chunk8_static"] = scan_chunk.linattn(q, k, v, chunk=8, log_alpha=log_alpha)
    # gradients of a fixed linear functional through quad (fp64)
    g = torch.Generator().manual_seed(7)
    dO = torch.randn(B, H, T, Dv, generator=g, dtype=torch.float64)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)]
    la = log_alpha.clone().requires_grad_(True)
    out = scan_chunk.linattn(*leaves, chunk=8, log_alpha=la)
    (out * dO).sum().backward()
    arrays.update({"dO": dO, "grad_q": leaves[0].grad, "grad_k": leaves[1].grad,
                   "grad_v": leaves[2].grad, "grad_log_alpha": la.grad})
    arrays["ema_cumsum_k"] = ema_cumsum(k, log_alpha, 8)
    arrays["prefix_k"] = causal_prefix_sum(k)
    np.savez_compressed(out_dir / "scan_streams.npz", **{key: _np(val) for key, val in arrays.items()})
    print("scan vectors written", flush=True)


def write_feature_vectors(out_dir: Path) -> None:
    from thetascan._core.modules import rope as rope_mod
    from thetascan._core.modules.block import _expansion_fingerprint, _fixed_row_map
    from thetascan._core.ops import kernel_features as kf

    g = torch.Generator().manual_seed(99)
    pre = torch.randn(2, 3, 11, 16, generator=g, dtype=torch.float64) * 1.5
    pre[0, 0, 0] = -1.0  # an all-negative row exercises the uniform fallback
    tau = torch.randn(3, generator=g, dtype=torch.float64) * 0.3
    rho = torch.tensor([0.01, 0.2, 0.5], dtype=torch.float64)
    blend = torch.tensor([0.0, 0.3, 1.0], dtype=torch.float64)
    arrays = {"pre": pre, "tau": tau, "rho": rho, "blend": blend}
    arrays["relu2"] = kf.relu2_ridge_features(pre, score_bias=None, relu2_threshold=tau, eps=1e-6)
    arrays["softmax"] = kf.softmax_partition_features(
        pre, gain=None, fallback_gain=8.0, score_bias=None, sparsity="none", relative_threshold=None,
        threshold_temperature=0.25, eps=1e-6)
    for mode in ("relative_soft", "relative_st", "relative_st_blend"):
        arrays[f"softmax_{mode}"] = kf.softmax_partition_features(
            pre, gain=None, fallback_gain=8.0, score_bias=None, sparsity=mode, relative_threshold=rho,
            sparse_blend_alpha=blend, threshold_temperature=0.25, eps=1e-6)
    coords = torch.linspace(-4.0, 4.0, 97, dtype=torch.float64).view(1, 1, 97, 1)
    arrays["bspline_coords"] = coords
    arrays["bspline_basis"] = kf.open_uniform_bspline_basis(coords, n_basis=8, degree=3, bound=3.0)
    arrays["bspline_features"] = kf.projected_bspline_features(
        pre[..., :4], n_basis=8, degree=3, bound=3.0, scale=None, fallback_scale=1.0)
    x = torch.randn(2, 3, 11, 12, generator=g, dtype=torch.float64)
    arrays["rope_x"] = x
    arrays["rope_partial"] = rope_mod.apply_rope(x, "partial", 0.5, 10000.0)
    arrays["rope_full"] = rope_mod.apply_rope(x, "full", 0.5, 1337.0)
    for shape, role in (((1, 16, 8), "w1-expand-layer-0"), ((1, 8, 16), "w2-expand-layer-0")):
        arrays[f"rowmap_{role}"] = _fixed_row_map(shape, key="thetascan", role=role, center_rows=False)
    fp = _expansion_fingerprint(key="thetascan", effective_hidden=192, feature_expansion=2, depth=1)
    out = {key: _np(val) for key, val in arrays.items()}
    out["fingerprint"] = fp.numpy()
    np.savez_compressed(out_dir / "features.npz", **out)
    print("feature vectors written", flush=True)


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--reference", default="/root/reference/src")
    args = parser.parse_args()
    sys.path.insert(0, args.reference)
    import thetascan as api  # the reference package

    torch.set_num_threads(4)
    write_scan_vectors(HERE)
    write_feature_vectors(HERE)
    manifest = write_mixer_cases(api, HERE)
    (HERE / "mixer_cases.json").write_text(json.dumps(manifest, indent=1, sort_keys=True))


if __name__ == "__main__":
    main()
