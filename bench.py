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
synchronisation on both sides, inputs already resident in HBM; Python's
cyclic garbage collector is paused over the warmup and the timed steps
(after a full collection before the warmup), so a collection of the
interpreter's heap -- tens of milliseconds of host time -- cannot land in a
timed step.  The
projection GEMMs run the library solutions measured for these shapes
(thetascan_amd.gemm_solutions; ``--library-gemm-heuristics`` times the
libraries' own choice instead); ``gemm_solutions`` on the line says which.

Extra objects on the JSON line:
  roofline      -- the HIP entry point with the most time per step against
                   HBM peak: algorithmic bytes per launch / mean launch time,
                   from events bracketing each launch on its own stream during
                   real fwd+bwd steps (an instrumented replay after the
                   clean timed region); ``traffic`` is the HBM bytes per launch
                   measured with rocprofv3 PMC counters when recorded
  passes        -- the same figures for every HIP entry point of the step
  scan_mfma     -- the scan's tile contractions against the dense bf16 MFMA peak
  cpu_baseline  -- the CPU oracle's prefix-sum (``cumsum``) mixer, fp32,
                   fwd+bwd on a bounded sample, on this host's cores
  decode        -- one-token decode latency of the headline mixer after its
                   4096-token prompt (B8), eager and as HIP-graph replays
"""
from __future__ import annotations

import argparse
import contextlib
import gc
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
MFMA_PEAK_TFLOPS = 2500.0  # dense bf16
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


@contextlib.contextmanager
def paused_gc():
    """Python's cyclic garbage collector paused over a warmup and the timed
    steps after it, after one full collection whose survivors are frozen out
    of later ones.  A full collection walks the interpreter's whole heap
    (about 65 ms of host time in these processes); left running it lands in a
    random timed step and adds its length to that step (the GPU idles behind
    the host meanwhile), which is host noise, not the workload.  The
    collection runs before the warmup: steps right after one ran 2-4 %
    slower in measurement, a transient the warmup absorbs."""
    was = gc.isenabled()
    gc.collect()
    gc.freeze()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()
        gc.unfreeze()


def time_steps(module, x, dy, steps: int, warmup: int, graphed=None, train: bool = True):
    """Mean ms per fwd+bwd step over exactly ``steps`` steps after ``warmup``.

    With ``graphed`` (a ``torch.cuda.make_graphed_callables`` wrapper of the
    module) each step replays the captured forward and backward graphs: the
    same kernels on the same data, without the host launch overhead."""
    import torch

    fwd = module if graphed is None else graphed

    def step():
        if not train:
            with torch.no_grad():
                fwd(x)
            return
        module.zero_grad(set_to_none=True)
        y = fwd(x)
        y.backward(dy)

    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with paused_gc():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        start.record()
        for _ in range(steps):
            step()
        stop.record()
        torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def scan_flops(B_, H_, T_, dk, dv, tile=64):
    """Algorithmic MFMA work of one forward scan over full 64-token tiles:
    per token and head C*dk (scores) + C*dv (P.V) + dk*dv (carried-state read)
    + dk*dv (state update) multiply-adds."""
    return 2 * B_ * H_ * T_ * (tile * dk + tile * dv + 2 * dk * dv)


def graphed_step_ms(module, x, dy, steps: int, warmup: int):
    """Step time of graph replays of a copy of ``module`` (capture replaces the
    copy's forward; the original stays eager for the per-kernel timing)."""
    import copy

    import torch

    twin = copy.deepcopy(module)
    graphed = torch.cuda.make_graphed_callables(twin, (x,), num_warmup_iters=3)
    return time_steps(twin, x, dy, steps, warmup, graphed)


def pass_profile(module, x, dy, steps: int = 5, train: bool = True):
    """Per-entry-point timing inside real fwd+bwd steps.

    Every HIP entry point called during ``steps`` steps is bracketed by events
    on the stream it launches on (``_lib.record_launches``), with the GPU kept
    behind the host so that no event pair includes host submission time.  Returns, per entry
    point, launches per step, mean duration per launch and achieved GB/s of its
    algorithmic bytes (inputs read once, outputs written once).
    """
    import torch

    def step():
        if train:
            module.zero_grad(set_to_none=True)
            module(x).backward(dy)
        else:
            with torch.no_grad():
                module(x)

    with paused_gc():
        return _pass_profile(module, x, dy, steps, step)


def _pass_profile(module, x, dy, steps, step):
    import torch
    from thetascan_amd import _lib

    step()
    torch.cuda.synchronize()
    # The recorded step submits one entry point at a time from Python, slower
    # than the GPU runs them; a start event would then also time the host's
    # submission of its launch.  A device-side sleep queued ahead of each step
    # (longer than the host takes to submit the whole step) keeps the GPU
    # behind the host, so every event pair brackets GPU work only.
    with _lib.record_launches():
        t0 = time.perf_counter()
        step()
        host_s = time.perf_counter() - t0
        torch.cuda.synchronize()
    probe_cycles = 1 << 20
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    torch.cuda._sleep(probe_cycles)
    b.record()
    torch.cuda.synchronize()
    cycles_per_s = probe_cycles / max(a.elapsed_time(b) * 1e-3, 1e-6)
    sleep_cycles = int(cycles_per_s * (2.0 * host_s + 1e-3))
    with _lib.record_launches() as recs:
        for _ in range(steps):
            torch.cuda._sleep(sleep_cycles)
            step()
        torch.cuda.synchronize()
        rows = [(name, a.elapsed_time(b), nb) for name, a, b, nb in recs]
    table = {}
    for name, ms, nb in rows:
        t = table.setdefault(name, {"launches": 0, "ms": 0.0, "bytes": 0})
        t["launches"] += 1
        t["ms"] += ms
        t["bytes"] += nb
    out = {}
    for name, t in sorted(table.items(), key=lambda kv: -kv[1]["ms"]):
        gbs = t["bytes"] / (t["ms"] * 1e-3) / 1e9
        out[name] = {
            "launches_per_step": t["launches"] / steps,
            "ms_per_step": round(t["ms"] / steps, 4),
            "ms_per_launch": round(t["ms"] / t["launches"], 4),
            "bytes_per_launch": t["bytes"] // t["launches"],
            "achieved_GBs": round(gbs, 1),
            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        }
    return out


def roofline_of(passes: dict, traffic: dict) -> dict:
    """The dominant entry point (most time per step) against the HBM roofline."""
    name, p = next(iter(passes.items()))
    entry = {
        "kernel": name, "bound": "hbm", "achieved": p["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": p["hbm_frac"], "traffic": traffic.get(name), "ms_per_launch": p["ms_per_launch"],
        "bytes_per_launch": p["bytes_per_launch"], "launches_per_step": p["launches_per_step"],
    }
    return entry


def load_traffic() -> dict:
    """HBM bytes per launch measured with rocprofv3 PMC counters (FETCH_SIZE +
    WRITE_SIZE, scaled by the same counters on a plain copy), keyed by entry
    point; empty when no measurement is recorded."""
    path = os.path.join(REPO, "profiles", "traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return {}
    return {k: v["bytes_per_launch"] for k, v in data.get("entry_points", {}).items() if "bytes_per_launch" in v}


def copy_calibration(n_mib: int = 256, reps: int = 3):
    """A plain device copy of a known size (for scaling PMC byte counters)."""
    import torch

    src = torch.ones(n_mib * (1 << 20) // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"copy_bytes_each_way": src.numel() * 4, "reps": reps}


def scan_mfma(passes: dict) -> dict | None:
    """Intra-chunk MFMA work of the forward scan against the dense bf16 peak."""
    p = passes.get("ts_scan_fwd")
    if p is None:
        return None
    flops = scan_flops(B, H, T, 64, 64)
    achieved = flops / (p["ms_per_launch"] * 1e-3) / 1e12
    return {"kernel": "ts_scan_fwd", "bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / MFMA_PEAK_TFLOPS, 4), "flops_per_launch": flops}


def cpu_baseline(budget_s: float = 12.0):
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

    # two untimed warmups, then the median of at least 5 timed steps (as many
    # as fit the budget, at most 25)
    first = min(run(), run())
    reps = max(5, min(25, int(budget_s / max(first, 1e-3))))
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
                  f"median of {reps} after 2 warmups",
        "cpu": model, "ms_per_step": round(t * 1e3, 1),
    }


# The other workloads the path serves, measured with ``--workload``:
#   bank          the headline mixer with the key-mass read and input RoPE
#                 and a fast bank of two recency rates {0.9, 0.99} (views
#                 path: multi-view scan, retention gradients pair by pair),
#                 B8 T4096 H8 d64, bf16, fwd+bwd;
#   preset_kernel, preset_gn, preset_gn_expanded
#                 the reference's three published presets
#                 (kernel_expanded_reference_v0_1: m = 384, shared key/query,
#                 learned ReLU^2 threshold, fast bank of two half-lives;
#                 gn_reference_v0_1: GN m = 192; gn_expanded_reference_v0_1:
#                 GN m = 384) at d_model 512, B8 T4096, bf16, fwd+bwd; these
#                 lines also report the step's peak memory above the resident
#                 parameters and inputs;
#   gn            damped Gauss-Newton memory, fast net 64 -> 128 -> 64 with tanh
#                 and damping 1e-2 (this build's extension of the core config:
#                 the public config, like the reference's, offers relu2/silu),
#                 two-stage read normalization (tanh features: the mass of the
#                 absolute features), B8 T2048 H8 d64, slow reference weights
#                 W1, W2 ~ N(0, 0.02), bf16, fwd+bwd;
#   bspline_bank  kernel memory with the cubic B-spline map (8 basis functions)
#                 expanded 2x on its projection rows by fixed key-derived sign
#                 maps (8 trainable projections -> 16 -> m = 128 features),
#                 key-mass read, a bank of four recency rates {0.9, 0.99,
#                 0.999, 0.9999} (fast blend), B2 T32768 H8 d64, bf16, forward
#                 only (both extensions of the core config: the public config,
#                 like the reference's, stops at two rates and expands only
#                 the ReLU^2 map);
#   lm            the 17.06M-parameter hybrid language model (9 layers,
#                 d_model 512, vocabulary 1024, attention in all layers but 4
#                 and 5, which are ThetaScan-Kernel memories at m = 128 by 2x
#                 expansion), B64 T1024 uniform random tokens, bf16, fwd+bwd;
#                 the line also reports the eval loss change of the per-row
#                 int8 round trip of its weights.
OTHER = {
    "gn": dict(B=8, T=2048, train=True,
               metric="GN mixer tokens/s fwd+bwd (B8 T2048 H8 d64 m128 tanh, damping 1e-2, bf16)"),
    "bank": dict(B=8, T=4096, train=True,
                 metric="bank mixer tokens/s fwd+bwd (B8 T4096 H8 d64 m64 ReLU^2, fast bank {0.9, 0.99}, "
                        "key-mass read, bf16)"),
    "preset_kernel": dict(B=8, T=4096, train=True, preset="kernel_expanded_reference_v0_1",
                          metric="kernel_expanded_reference_v0_1 tokens/s fwd+bwd (B8 T4096 d_model 512, m=384, bf16)"),
    "preset_gn": dict(B=8, T=4096, train=True, preset="gn_reference_v0_1",
                      metric="gn_reference_v0_1 tokens/s fwd+bwd (B8 T4096 d_model 512, m=192, bf16)"),
    "preset_gn_expanded": dict(B=8, T=4096, train=True, preset="gn_expanded_reference_v0_1",
                               metric="gn_expanded_reference_v0_1 tokens/s fwd+bwd (B8 T4096 d_model 512, m=384, bf16)"),
    "lm": dict(B=64, T=1024, train=True,
               metric="hybrid LM tokens/s fwd+bwd (17.06M params, 2 ThetaScan layers, B64 T1024, bf16)"),
    "bspline_bank": dict(B=2, T=32768, train=False,
                         metric="B-spline 4-rate bank mixer tokens/s fwd (B2 T32768 H8 d64 m128 2x expanded, bf16)"),
}


def other_config(name: str):
    """The core (flat) configuration of a secondary workload."""
    import dataclasses

    import thetascan_amd as ts

    if "preset" in OTHER[name]:
        public = getattr(ts.ThetaScanConfig, OTHER[name]["preset"])(d_model=D_MODEL, n_heads=H)
        public.runtime.backend = "hip"
        return public._to_core_config()
    if name == "bank":
        public = ts.ThetaScanConfig(
            d_model=D_MODEL, n_heads=H, memory_multiplier=1, family="kernel",
            kernel=ts.KernelConfig(feature_map="relu2_ridge", read_normalization="key_mass"),
            rope=ts.RoPEConfig(mode="partial", fraction=0.5, placement="input"),
            temporal=ts.TemporalConfig(mode="bank", bank_mode="fast", recency_branches=2, retention_inits=(0.9, 0.99)),
            runtime=ts.RuntimeConfig(backend="hip", scan_chunk=64),
        )
        return public._to_core_config()
    if name == "gn":
        public = ts.ThetaScanConfig(
            d_model=D_MODEL, n_heads=H, memory_multiplier=2, family="gn",
            gn=ts.GNConfig(nonlinearity="relu2", jacobian_steps=1, read_normalization="both_feature_mass"),
            temporal=ts.TemporalConfig(mode="sum"), runtime=ts.RuntimeConfig(backend="hip", scan_chunk=64),
        )
        return dataclasses.replace(public._to_core_config(), nonlin="tanh", gn_damping=1e-2)
    public = ts.ThetaScanConfig(
        d_model=D_MODEL, n_heads=H, memory_multiplier=2, family="kernel",
        kernel=ts.KernelConfig(feature_map="projected_bspline", read_normalization="key_mass"),
        temporal=ts.TemporalConfig(mode="bank", bank_mode="fast", recency_branches=2, retention_inits=(0.9, 0.999)),
        runtime=ts.RuntimeConfig(backend="hip", scan_chunk=128),
    )
    return dataclasses.replace(public._to_core_config(), feature_expansion=2, fade_branches=4,
                               fade_alpha_inits=(0.9, 0.99, 0.999, 0.9999))


def run_lm(args) -> dict:
    """The hybrid language model's training step on uniform random tokens."""
    import torch

    from thetascan_amd import hybrid_lm as lm

    spec = OTHER["lm"]
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    model = lm.HybridLM().to(dev, torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    x = torch.randint(0, lm.VOCAB, (spec["B"], spec["T"]), generator=g).to(dev)
    y = torch.randint(0, lm.VOCAB, (spec["B"], spec["T"]), generator=g).to(dev)

    def step():
        model.zero_grad(set_to_none=True)
        model(x, y).backward()

    with paused_gc():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / args.steps * 1e3
    model.eval()
    with torch.no_grad():
        base = float(model(x[:8], y[:8]))
        model.load_state_dict(lm.int8_round_trip(model))
        quant = float(model(x[:8], y[:8]))
    tokens = spec["B"] * spec["T"]
    return {
        "metric": spec["metric"], "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (uniform random tokens, seeded init)", "execution": "eager",
        "path": model.blocks[lm.THETA_LAYERS[0]].attn._core.last_path,
        "config": {"workload": "lm", "batch": spec["B"], "seq_len": spec["T"], "params": lm.parameter_count(model),
                   "layers": lm.LAYERS, "theta_layers": list(lm.THETA_LAYERS), "parallelism": "single GPU"},
        "int8_round_trip": {"eval_loss": round(base, 6), "eval_loss_int8": round(quant, 6),
                            "rel": round(abs(quant - base) / base, 8), "parity": "unpinned"},
    }


def run_other(name: str, args) -> dict:
    """One JSON line for a non-headline workload (no CPU baseline)."""
    import torch

    if name == "lm":
        return run_lm(args)

    from thetascan_amd._core.modules.block import ThetaScan as CoreMixer

    spec = OTHER[name]
    dev = torch.device("cuda", 0)
    torch.manual_seed(0)
    module = CoreMixer(other_config(name))
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for pname, p in sorted(module.named_parameters()):
            if name == "gn" and pname.startswith(("W1.", "W2.")):
                p.copy_(torch.randn(p.shape, generator=g) * 0.02)
            elif "fade_eta" in pname or (p.ndim >= 2 and float(p.abs().max()) == 0.0):
                p.copy_(torch.randn(p.shape, generator=g) * (0.3 if "fade_eta" in pname else 0.02))
    module = module.to(dev, torch.bfloat16)
    x = torch.randn(spec["B"], spec["T"], D_MODEL, generator=g).to(dev, torch.bfloat16)
    dy = (torch.randn(spec["B"], spec["T"], D_MODEL, generator=g) * 1e-2).to(dev, torch.bfloat16)
    torch.cuda.synchronize()
    resident = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    ms = time_steps(module, x, dy, args.steps, args.warmup, train=spec["train"])
    peak = torch.cuda.max_memory_allocated() - resident
    passes = pass_profile(module, x, dy, train=spec["train"])
    return {
        "metric": spec["metric"], "value": round(spec["B"] * spec["T"] / (ms * 1e-3), 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (x ~ N(0,1), seeded weights)", "execution": "eager",
        "path": module.last_path,
        "config": {"workload": name, "batch": spec["B"], "seq_len": spec["T"], "heads": H, "head_dim": D_HEAD,
                   "d_model": D_MODEL, "mem_hidden": module.cfg.mem_hidden, "parallelism": "single GPU"},
        "peak_memory_bytes": peak,
        "roofline": roofline_of(passes, {}), "passes": passes,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=("headline", *OTHER), default="headline",
                    help="headline (default) or one of the other workloads of the path")
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mode", choices=("eager", "graph"), default="eager",
                    help="time eager execution (default) or graph replays of the captured step")
    ap.add_argument("--no-variant", action="store_true", help="skip the key-mass variant")
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the configurations 3, 4 and 5 lines of the default run")
    ap.add_argument("--no-decode", action="store_true", help="skip the one-token decode latency")
    ap.add_argument("--steps-only", action="store_true", help="time the steps only (for profilers)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a 256 MiB device copy (reference for PMC byte counters)")
    ap.add_argument("--library-gemm-heuristics", action="store_true",
                    help="time the headline with the libraries' own GEMM solution choice instead of the "
                         "measured table (thetascan_amd.gemm_solutions)")
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
    if args.workload != "headline":
        print(json.dumps(run_other(args.workload, args)), flush=True)
        return 0
    from thetascan_amd import gemm_solutions

    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(B, T, D_MODEL, generator=g).to(dev, torch.bfloat16)
    dy = (torch.randn(B, T, D_MODEL, generator=g) * 1e-2).to(dev, torch.bfloat16)

    # the projection GEMMs replay the solutions measured for these shapes
    measured = gemm_solutions.use_measured_gemms(not args.library_gemm_heuristics)
    module = seeded_module(headline_config("feature_rope"), 0).to(dev, torch.bfloat16)
    ms_eager = time_steps(module, x, dy, args.steps, args.warmup)
    assert module._core.last_path == "fused"
    execution = "eager"
    ms = ms_eager
    if args.mode == "graph":
        try:
            ms = graphed_step_ms(module, x, dy, args.steps, args.warmup)
            execution = "graph"
        except Exception as exc:  # capture unsupported here: report eager, say why
            print(f"graph capture failed ({exc!r}); reporting eager execution", file=sys.stderr)
    if args.calibrate_copy:
        copy_calibration()
    if args.steps_only:
        print(json.dumps({"ms_per_step": ms}), flush=True)
        return 0
    tokens = B * T
    out = {
        "metric": METRIC, "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (x ~ N(0,1), dy ~ N(0,1e-4), seeded weights)",
        "execution": ("hip-graph replay of the captured fwd+bwd step (torch.cuda.make_graphed_callables)"
                      if execution == "graph" else "eager"),
        "eager": {"value": round(tokens / (ms_eager * 1e-3), 1), "ms_per_step": round(ms_eager, 4)}
        if execution == "graph" else None,
        "config": {"workload": "ThetaScan-Kernel mixer fwd+bwd, ReLU^2 ridge, m=64, chunk 64, feature RoPE, "
                               "unnormalized read",
                   "batch": B, "seq_len": T, "heads": H, "head_dim": D_HEAD, "d_model": D_MODEL,
                   "parallelism": "single GPU"},
        "gemm_solutions": ("measured table (" + gemm_solutions.TABLE.name + ", "
                           + str(len(gemm_solutions.read_table()[1])) + " shapes)") if measured
        else "library heuristics",
    }
    traffic = load_traffic()
    passes = pass_profile(module, x, dy)
    out["roofline"] = roofline_of(passes, traffic)
    out["passes"] = passes
    out["scan_mfma"] = scan_mfma(passes)
    if not args.no_variant:
        module_b = seeded_module(headline_config("key_mass"), 0).to(dev, torch.bfloat16)
        ms_b_eager = time_steps(module_b, x, dy, args.steps, args.warmup)
        ms_b = ms_b_eager
        if execution == "graph":
            ms_b = graphed_step_ms(module_b, x, dy, args.steps, args.warmup)
        passes_b = pass_profile(module_b, x, dy)
        out["variants"] = {
            "input_rope_key_mass": {"value": round(tokens / (ms_b * 1e-3), 1), "ms_per_step": round(ms_b, 4),
                                    "eager": {"value": round(tokens / (ms_b_eager * 1e-3), 1),
                                              "ms_per_step": round(ms_b_eager, 4)} if execution == "graph" else None,
                                    "roofline": roofline_of(passes_b, {}), "passes": passes_b},
        }
    # the other workloads keep the libraries' own choice (their shapes are not in the table)
    gemm_solutions.use_measured_gemms(False)
    if not args.no_workloads:
        out["workloads"] = other_workloads(args)
    if not args.no_decode:
        out["decode"] = decode_latency(x)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)
    return 0


def decode_latency(x, steps: int = 200, warmup: int = 20) -> dict:
    """One-token decode of the headline mixer (feature RoPE, bf16) for the B
    sequences of ``x`` after their T-token prompt: the prompt is run into the
    streaming state once (``prefill_ms``), then each step feeds one token per
    sequence -- eagerly (``mixer(x_t, state=s)``) and as replays of the
    captured step (thetascan_amd.DecodeGraph).  Latency is the wall time per
    step over ``steps`` steps after ``warmup``, with a device synchronisation
    on both sides; ``tokens_per_s`` counts B tokens per graph step."""
    import torch
    from thetascan_amd import DecodeGraph

    module = seeded_module(headline_config("feature_rope"), 0).to(x.device, torch.bfloat16)
    tok = x[:, -1:].contiguous()
    with torch.no_grad():
        module(x, state=module.initial_state())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _, state = module(x, state=module.initial_state())
        torch.cuda.synchronize()
        prefill_ms = (time.perf_counter() - t0) * 1e3
        s = state
        with paused_gc():
            for _ in range(warmup):
                _, s = module(tok, state=s)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                _, s = module(tok, state=s)
            torch.cuda.synchronize()
            eager_us = (time.perf_counter() - t0) / steps * 1e6
        dec = DecodeGraph(module, state)
        with paused_gc():
            for _ in range(warmup):
                dec.step(tok)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                dec.step(tok)
            torch.cuda.synchronize()
            graph_us = (time.perf_counter() - t0) / steps * 1e6
    return {"batch": x.shape[0], "prompt_tokens": x.shape[1], "prefill_ms": round(prefill_ms, 3),
            "steps": steps, "eager_us_per_step": round(eager_us, 1), "graph_us_per_step": round(graph_us, 1),
            "tokens_per_s": round(x.shape[0] / (graph_us * 1e-6), 1),
            "state_bytes": state.nbytes}


def other_workloads(args) -> dict:
    """Configurations 3 (GN), 4 (B-spline bank) and 5 (hybrid LM) in the
    default run, each with its own steps (at most 20 timed after 5 warmups):
    the figures ``--workload`` reports in full, minus the per-pass table."""
    sub = argparse.Namespace(**vars(args))
    sub.steps, sub.warmup = min(args.steps, 20), min(args.warmup, 5)
    res = {}
    for name in ("gn", "bspline_bank", "lm"):
        line = run_other(name, sub)
        keep = {k: line[k] for k in ("metric", "value", "unit", "ms_per_step", "steps", "warmup", "path")
                if k in line}
        keep["config"] = line["config"]
        if "roofline" in line:
            keep["roofline"] = line["roofline"]
        for k in ("peak_memory_bytes", "int8_round_trip"):
            if k in line:
                keep[k] = line[k]
        res[name] = keep
    return res


if __name__ == "__main__":
    sys.exit(main())
