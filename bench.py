#!/usr/bin/env python3
"""ThetaScan-Kernel mixer fwd+bwd throughput on one MI355X.

Workload (the headline configuration): kernel memory, ReLU^2-ridge features,
m = head_dim = 64, H = 8, d_model = 512, 64-token scan tiles, B = 8, T = 4096,
bf16 activations and weights with fp32 scan state.  The literal variant
(RoPE on features, unnormalized read) is the headline ``value``; the
key-mass-normalized variant (input RoPE) is timed beside it.  Inputs are
synthetic: x ~ N(0,1), upstream gradient ~ N(0, (1e-2)^2), weights seeded
(Xavier-uniform projections, W1 ~ N(0,1/d), W2 and the output gate ~ N(0,0.02)).

One step = forward + backward of the whole mixer (projections included).
The timed region brackets exactly ``--steps`` steps with a device
synchronisation on both sides, inputs already resident in HBM.

Extra objects on the JSON line:
  roofline      -- the dominant kernel (the forward scan) against HBM peak:
                   algorithmic bytes per launch / mean launch time (HIP events)
  cpu_baseline  -- the CPU oracle's prefix-sum (``cumsum``) mixer, fp32,
                   fwd+bwd on a bounded sample, on this host's cores
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

METRIC = "mixer tokens/s fwd+bwd (B8 T4096 H8 d64 bf16); % of MFMA/HBM roofline"
HBM_PEAK_GBS = 8000.0
B, T, H, D_HEAD, D_MODEL = 8, 4096, 8, 64, 512


def headline_config(variant: str):
    import thetascan_amd as ts

    if variant == "feature_rope":
        rope = ts.RoPEConfig(mode="partial", fraction=0.5, placement="feature")
        norm = "none"
    else:
        rope = ts.RoPEConfig(mode="partial", fraction=0.5, placement="input")
        norm = "key_mass"
    return ts.ThetaScanConfig(
        d_model=D_MODEL, n_heads=H, memory_multiplier=1, family="kernel",
        kernel=ts.KernelConfig(feature_map="relu2_ridge", read_normalization=norm),
        rope=rope, temporal=ts.TemporalConfig(mode="sum"),
        runtime=ts.RuntimeConfig(backend="hip", scan_chunk=64),
    )


def seeded_module(config, seed: int):
    import torch
    import thetascan_amd as ts

    torch.manual_seed(seed)
    module = ts.ThetaScan(config)
    core = module._core
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for lin in (core.proj_qkv, core.proj_out):
            bound = (6.0 / (lin.weight.shape[0] + lin.weight.shape[1])) ** 0.5
            lin.weight.copy_((torch.rand(lin.weight.shape, generator=g) * 2 - 1) * bound)
        core.W1[0].copy_(torch.randn(core.W1[0].shape, generator=g) / D_HEAD ** 0.5)
        core.W2[0].copy_(torch.randn(core.W2[0].shape, generator=g) * 0.02)
        core.ogate.g.lin.weight.copy_(torch.randn(core.ogate.g.lin.weight.shape, generator=g) * 0.02)
    return module


def time_steps(module, x, dy, steps: int, warmup: int):
    import torch

    def step():
        module.zero_grad(set_to_none=True)
        y = module(x)
        y.backward(dy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def scan_roofline(module, x, reps: int = 20):
    """Mean duration of the forward scan kernel chain on the step's real inputs."""
    import torch
    from thetascan_amd._core.ops import fused, scan_hip

    core = module._core
    cfg = core.cfg
    with torch.no_grad():
        qkv = torch.nn.functional.linear(x, core.proj_qkv.weight).view(B, T, 3, H, D_HEAD)
        (W1, W2, _), = core._weights()
        feat_rot = 32 if cfg.rope_placement == "feature" else 0
        in_rot = 32 if cfg.rope_placement == "input" else 0
        spec = fused.FeatureSpec(fused._lib.FEAT_RELU2, 64, 1.0, in_rot, feat_rot, 10000.0, 1.0)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        phi_k, _ = fused.feature_fwd(spec, k, W1.contiguous(), None, None, False)
        phi_q, _ = fused.feature_fwd(spec, q, W1.contiguous(), W2.contiguous(), None, True)
        mass = cfg.read_norm

        def run():
            scan_hip.scan_launch(phi_q, phi_k, v, v_ext="ones" if mass else None, want_ext_out=mass)

        for _ in range(3):
            run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    n = B * H * T
    # algorithmic bytes: read phi_q, phi_k (m = 64), v (d = 64) in bf16; write num (bf16) [+ fp32 mass]
    per_token = 3 * 64 * 2 + 64 * 2 + (4 if mass else 0)
    algo = n * per_token
    achieved = algo / (ms * 1e-3) / 1e9
    return {
        "kernel": "forward scan (ts_scan_fwd: summary + prefix + main kernels)",
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
        "ms_per_launch": round(ms, 4), "algorithmic_bytes": algo, "bytes_per_token_head": per_token,
    }


def cpu_baseline(budget_s: float = 20.0):
    """fp32 fwd+bwd of the oracle mixer with the reference's prefix-sum scan on the host CPU."""
    import torch
    from oracle import mixer as oracle_mixer

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    config = headline_config("feature_rope")
    module = seeded_module(config, 0)
    core = oracle_mixer.core_config(config.to_dict())
    params = {k: v.detach().float().clone().requires_grad_(True) for k, v in module._core.named_parameters()}
    Bs, Ts = 1, T
    g = torch.Generator().manual_seed(7)
    x = torch.randn(Bs, Ts, D_MODEL, generator=g)
    dy = torch.randn(Bs, Ts, D_MODEL, generator=g) * 1e-2

    def run():
        for p in params.values():
            p.grad = None
        t0 = time.perf_counter()
        y = oracle_mixer.forward(core, params, x, backend="cumsum")
        y.backward(dy)
        return time.perf_counter() - t0

    first = run()
    reps = max(1, min(5, int(budget_s / max(first, 1e-3))))
    times = [run() for _ in range(reps)]
    t = statistics.median(times)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((line.split(":", 1)[1].strip() for line in f if line.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": round(Bs * Ts / t, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
        "sample": f"B={Bs} T={Ts} (one of the {B} sequences of the workload), fp32, oracle mixer with the cumsum scan, "
                  f"median of {reps} after 1 warmup",
        "cpu": model, "ms_per_step": round(t * 1e3, 1),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-variant", action="store_true", help="skip the key-mass variant")
    ap.add_argument("--steps-only", action="store_true", help="time the steps only (for profilers)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one MI355X only; --gpus {args.gpus} (WORLD_SIZE={world}) is not supported "
              "in this build: every box here has one GPU", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(B, T, D_MODEL, generator=g).to(dev, torch.bfloat16)
    dy = (torch.randn(B, T, D_MODEL, generator=g) * 1e-2).to(dev, torch.bfloat16)

    module = seeded_module(headline_config("feature_rope"), 0).to(dev, torch.bfloat16)
    ms = time_steps(module, x, dy, args.steps, args.warmup)
    assert module._core.last_path == "fused"
    if args.steps_only:
        print(json.dumps({"ms_per_step": ms}), flush=True)
        return 0
    tokens = B * T
    out = {
        "metric": METRIC, "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (x ~ N(0,1), dy ~ N(0,1e-4), seeded weights)",
        "config": {"workload": "ThetaScan-Kernel mixer fwd+bwd, ReLU^2 ridge, m=64, chunk 64, feature RoPE, "
                               "unnormalized read",
                   "batch": B, "seq_len": T, "heads": H, "head_dim": D_HEAD, "d_model": D_MODEL,
                   "parallelism": "single GPU"},
    }
    out["roofline"] = scan_roofline(module, x)
    if not args.no_variant:
        module_b = seeded_module(headline_config("key_mass"), 0).to(dev, torch.bfloat16)
        ms_b = time_steps(module_b, x, dy, args.steps, args.warmup)
        out["variants"] = {
            "input_rope_key_mass": {"value": round(tokens / (ms_b * 1e-3), 1), "ms_per_step": round(ms_b, 4),
                                    "roofline": scan_roofline(module_b, x)},
        }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
