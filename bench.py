"""Benchmark of one Polar Express step (``polar_step``) on one MI355X.

Metric: polar_step µs and TFLOP/s (% of dense bf16 MFMA peak) at
[8,512,2048] and 4096×14336.  ``value`` is the TFLOP/s of the headline workload, a
single ``polar_step`` on a bf16 [4096,14336] matrix with inputs resident in HBM,
counting the credited FLOPs M²N + 2M³ + 2M²N per matrix.  The [8,512,2048] case is
reported in ``secondary``.

Timing follows the driver contract (W untimed warm-up calls, then exactly K calls
between two device synchronisations) — the reference's own method is the same loop
(README.md:179-191).  Per-kernel durations come from HIP events recorded on the
launch stream between the stages of a step sequence launched through the C ABI (so each
stage sees the caches as inside a step); ``roofline`` uses the dominant kernel (stage 3,
P·X + a·X).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "polar_step µs & TFLOP/s (% bf16 MFMA peak) at [8,512,2048] and 4096×14336"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (published)
PEAK_HBM_GBS = 8000.0
COEFFS = (8.156554524902461, -22.48329292557795, 15.878769915207462)  # tests/test_polar_step.py:14
HEADLINE = (1, 4096, 14336)
SECONDARY = (8, 512, 2048)
# Every BASELINE.json configuration on the GPU: (config, shape, steps per call).  Config 0 is
# the reference's CPU plumbing case, timed here on the GPU as well; five-step calls chain the
# five coefficient triples (polar_express without normalisation = five polar_step calls).
CONFIGS = (
    ("cfg0", (129, 130), 1),
    ("cfg1", (2, 150, 2050), 1),
    ("cfg2", (8, 512, 2048), 1),
    ("cfg3", (8, 512, 2048), 5),
    ("cfg4", (4096, 14336), 1),
    ("cfg4", (4096, 14336), 5),
    ("cfg4", (14336, 4096), 1),
    ("cfg4", (14336, 4096), 5),
    ("cfg4", (4, 4096, 4096), 1),
    ("cfg4", (4, 4096, 4096), 5),
)
TRAFFIC_SUMMARY = ROOT / "profiles" / "apply_4096x14336_hbm_traffic.txt"


def config_call(shape, steps: int):
    """The GPU call of one configuration: one polar_step, or the five-step chain."""
    import torch
    import muon_fusion_ascend950_amd as mf

    x = make_input(shape, seed=0).cuda()
    if steps == 1:
        a, b, c = COEFFS
        return (lambda: mf.polar_step(x, a, b, c)), x
    coeffs = mf.COEFFICIENTS[:steps]
    return (lambda: mf.polar_express(x, coeffs, normalize=False)), x


def all_configs(calls_budget_s: float = 0.25):
    """µs per call and credited TFLOP/s (% of the dense bf16 peak) of every configuration."""
    rows = []
    for name, shape, steps in CONFIGS:
        fn, x = config_call(shape, steps)
        batch = shape[0] if len(shape) == 3 else 1
        m, n = shape[-2], shape[-1]
        once = time_calls(fn, 3, 2)
        calls = max(5, min(200, int(calls_budget_s / max(once, 1e-6))))
        sec = time_calls(fn, calls, 3)
        flops = steps * credited_flops(batch, m, n)
        rows.append({"config": name, "shape": list(shape), "steps_per_call": steps,
                     "us_per_call": round(sec * 1e6, 2),
                     "tflops": round(flops / sec / 1e12, 2),
                     "pct_bf16_peak": round(100 * flops / sec / 1e12 / PEAK_BF16_TFLOPS, 2)})
        del x
    return rows


def credited_flops(batch: int, m: int, n: int) -> int:
    m, n = min(m, n), max(m, n)
    return batch * (m * m * n + 2 * m**3 + 2 * m * m * n)


def make_input(shape, seed: int = 0):
    """Seeded bf16 N(0,1) on the CPU, normalised per matrix (tests/test_polar_step.py:38-39)."""
    import torch

    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, dtype=torch.bfloat16, generator=gen)
    return x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)


def time_calls(fn, steps: int, warmup: int) -> float:
    """Seconds per call: warm-up, then exactly `steps` calls between synchronisations."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def kernel_us(fn, launches: int, warmup: int = 3) -> float:
    """Average device duration (µs) of one launch, from HIP events on the current stream."""
    import torch

    for _ in range(warmup):
        fn()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(launches):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) * 1e3 / launches


def stage_times(batch: int, m: int, n: int, launches: int, warmup: int = 3):
    """µs per launch of each stage as it runs inside a step: gram, poly and apply are
    launched in step order through the C ABI with polar_step's workspace (A and P in
    it, the same stream-K split as in the step), `launches` times, with HIP events on
    torch's current stream (the launch stream) between the stages; each stage's time is
    the sum of its event intervals / launches."""
    import torch
    from muon_fusion_ascend950_amd import capi

    x = make_input((batch, m, n), seed=0).cuda()
    ws, info = capi.alloc_workspace(batch, m, n)
    mp = info.padded_rows
    p_off = -(-info.gram_bytes // 256) * 256
    gram = ws[:info.gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    poly = ws[p_off:p_off + info.gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    y = torch.empty_like(x)
    a, b, c = COEFFS
    stages = (("gram", lambda: capi.gram(x, gram, workspace=ws)),
              ("poly", lambda: capi.poly(gram, poly, batch, m, n, b, c, workspace=ws)),
              ("apply", lambda: capi.apply(poly, x, y, a, workspace=ws)))
    for _ in range(warmup):
        for _, fn in stages:
            fn()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)]
              for _ in range(launches)]
    for ev in events:
        ev[0].record()
        for i, (_, fn) in enumerate(stages):
            fn()
            ev[i + 1].record()
    torch.cuda.synchronize()
    return {name: sum(ev[i].elapsed_time(ev[i + 1]) for ev in events) * 1e3 / launches
            for i, (name, _) in enumerate(stages)}


def torch_eager(x):
    """The README's comparison point (README.md:172-174), plain PyTorch on the GPU.
    The transposed operand is materialised first (batched bf16 products with a
    transposed right operand are avoided on ROCm)."""
    import torch

    a, b, c = COEFFS
    gram = torch.matmul(x, x.mT.contiguous())
    return a * x + torch.matmul(b * gram + c * torch.matmul(gram, gram), x)


MUON_LR, MUON_MOMENTUM, MUON_WD = 0.02, 0.95, 0.01


def muon_tensors(m: int, n: int):
    """fp32 parameter, gradient and momentum buffer of one [m, n] matrix on the GPU."""
    import torch

    gen = torch.Generator().manual_seed(2)
    p = (torch.randn(m, n, generator=gen) * 0.02).cuda()
    g = (torch.randn(m, n, generator=gen) * 1e-3).cuda()
    buf = (torch.randn(m, n, generator=gen) * 1e-3).cuda()
    return p, g, buf


def muon_eager_step(p, g, buf, coefficients):
    """nanochat's Muon step in plain PyTorch on the GPU (momentum lerps, bf16 Polar
    Express with the reference recipe's normalisation, decoupled decay, shape-scaled
    add): the comparison point of the native update."""
    import torch

    buf.lerp_(g, 1 - MUON_MOMENTUM)
    u = g.lerp(buf, MUON_MOMENTUM)
    x = u.bfloat16()
    x = x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)
    for a, b, c in coefficients:
        gram = torch.matmul(x, x.mT.contiguous())
        x = a * x + torch.matmul(b * gram + c * torch.matmul(gram, gram), x)
    p.mul_(1 - MUON_LR * MUON_WD)
    p.add_(x, alpha=-MUON_LR * max(1.0, p.size(-2) / p.size(-1)) ** 0.5)


def read_traffic():
    """HBM bytes per stage-3 launch from the committed rocprofv3 --pmc summary, if any."""
    if not TRAFFIC_SUMMARY.is_file():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", TRAFFIC_SUMMARY.read_text(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(budget_s: float = 12.0):
    """The oracle's restatement of the reference formula, bf16 torch on the host CPU."""
    import torch
    from oracle import polar_oracle as O

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    batch, m, n = HEADLINE
    x = make_input((m, n), seed=0)
    samples = []
    with torch.no_grad():
        O.reference_formula_torch(x, [COEFFS])  # warm-up
        t_end = time.perf_counter() + budget_s
        while len(samples) < 3 or (time.perf_counter() < t_end and len(samples) < 15):
            t0 = time.perf_counter()
            O.reference_formula_torch(x, [COEFFS])
            samples.append(time.perf_counter() - t0)
    med = statistics.median(samples)
    flops = credited_flops(batch, m, n)
    return {
        "value": round(flops / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"reference formula (tests/test_polar_step.py:22-28) in bf16 torch on the host CPU, "
                   f"[4096,14336] one step, median of {len(samples)} runs after 1 warm-up "
                   f"({med * 1e3:.0f} ms/step)"),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile", action="store_true",
                    help="only the headline step loop and three 1 GiB device copies (the "
                         "calibration kernel of known size), for rocprofv3 runs")
    ap.add_argument("--profile-secondary", action="store_true",
                    help="only the [8,512,2048] step loop, for rocprofv3 runs")
    ap.add_argument("--profile-configs", action="store_true",
                    help="only a few calls of every BASELINE configuration in turn, for rocprofv3 "
                         "counter runs")
    ap.add_argument("--profile-muon", action="store_true",
                    help="only a loop of Muon updates of one fp32 [4096,14336] parameter, "
                         "for rocprofv3 runs")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: polar_step is a single-GPU operator; this build measures one GPU only "
              "(batch/parameter sharding across GPUs is a design note, not run). Use --gpus 1.",
              file=sys.stderr)
        return 2

    import torch
    import muon_fusion_ascend950_amd as mf

    torch.cuda.set_device(0)
    a, b, c = COEFFS
    out = {}

    # ---- headline: [4096,14336], one step
    batch, m, n = HEADLINE
    if args.profile_muon:
        p, g, buf = muon_tensors(m, n)
        sec = time_calls(lambda: mf.muon_update(p, g, buf, lr=MUON_LR, momentum=MUON_MOMENTUM,
                                                weight_decay=MUON_WD), args.steps, args.warmup)
        print(json.dumps({"profile": "muon_update fp32 [4096,14336]", "steps": args.steps,
                          "us_per_update": round(sec * 1e6, 2)}), flush=True)
        return 0
    if args.profile_configs:
        for name, shape, steps in CONFIGS:
            fn, x = config_call(shape, steps)
            sec = time_calls(fn, args.steps, args.warmup)
            print(json.dumps({"profile": name, "shape": list(shape), "steps_per_call": steps,
                              "us_per_call": round(sec * 1e6, 2)}), flush=True)
            del x
        return 0
    if args.profile_secondary:
        x2 = make_input(SECONDARY, seed=0).cuda()
        sec = time_calls(lambda: mf.polar_step(x2, a, b, c), args.steps, args.warmup)
        print(json.dumps({"profile": "polar_step [8,512,2048]", "steps": args.steps,
                          "us_per_step": round(sec * 1e6, 2)}), flush=True)
        return 0
    x = make_input((m, n), seed=0).cuda()
    if args.profile:
        sec = time_calls(lambda: mf.polar_step(x, a, b, c), args.steps, args.warmup)
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)  # reads and writes exactly 1 GiB
        torch.cuda.synchronize()
        print(json.dumps({"profile": "polar_step [4096,14336]", "steps": args.steps,
                          "us_per_step": round(sec * 1e6, 2), "copy_bytes": 1 << 30}), flush=True)
        return 0
    sec = time_calls(lambda: mf.polar_step(x, a, b, c), args.steps, args.warmup)
    flops = credited_flops(batch, m, n)
    tflops = flops / sec / 1e12
    st = stage_times(batch, m, n, launches=max(10, args.steps // 2))
    apply_flops = 2 * batch * m * m * n
    achieved = apply_flops / (st["apply"] * 1e-6) / 1e12
    traffic = read_traffic()

    # ---- secondary: [8,512,2048], one step
    b2, m2, n2 = SECONDARY
    x2 = make_input(SECONDARY, seed=0).cuda()
    sec2 = time_calls(lambda: mf.polar_step(x2, a, b, c), max(args.steps, 100), args.warmup)
    fl2 = credited_flops(b2, m2, n2)
    st2 = stage_times(b2, m2, n2, launches=max(20, args.steps))
    # bytes that must move at least: X in, Y out; with A and P stored: + 4·B·M²·2 + X re-read
    hbm2 = 2 * b2 * m2 * n2 * 2 + 4 * b2 * m2 * m2 * 2 + b2 * m2 * n2 * 2

    # five steps after the normalisation (the reference's examples/five_steps.py loop):
    # one polar_express call vs normalisation in torch + five polar_step calls
    raw = make_input((m, n), seed=1) * 3.0
    def reference_loop():
        y = raw / (raw.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)
        for a_, b_, c_ in mf.COEFFICIENTS:
            y = mf.polar_step(y, a_, b_, c_)
        return y
    raw = raw.cuda()
    sec_express = time_calls(lambda: mf.polar_express(raw), 10, 3)
    sec_loop = time_calls(reference_loop, 10, 3)

    # Muon update of one fp32 [4096,14336] parameter: the native update (momentum pass,
    # normalisation, 5 steps, parameter update) vs nanochat's step in PyTorch eager
    p, g, buf = muon_tensors(m, n)
    sec_muon = time_calls(lambda: mf.muon_update(p, g, buf, lr=MUON_LR, momentum=MUON_MOMENTUM,
                                                 weight_decay=MUON_WD), 10, 3)
    sec_muon_eager = time_calls(lambda: muon_eager_step(p, g, buf, mf.COEFFICIENTS), 5, 2)
    del p, g, buf

    # PyTorch eager on the same GPU (the reference's comparison point, README.md:172-208)
    eager = time_calls(lambda: torch_eager(x), 10, 3)
    eager2 = time_calls(lambda: torch_eager(x2), 50, 5)

    result = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16, normalised per matrix as tests/test_polar_step.py:38-39)",
        "config": {
            "workload": "polar_step on bf16 [4096,14336], one step, coefficients (8.1566,-22.4833,15.8788)",
            "shape": [m, n],
            "steps_per_call": 1,
            "credited_gflop": round(flops / 1e9, 3),
            "parallelism": "single GPU",
        },
        "us_per_step": round(sec * 1e6, 2),
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "kernel_us": {k: round(v, 2) for k, v in st.items()},
        "torch_eager_us": round(eager * 1e6, 2),
        "speedup_vs_torch_eager": round(eager / sec, 3),
        "roofline": {
            "bound": "mfma",
            "kernel": "stage 3 apply (Y = a·X + P·X)",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
        },
        "five_step": {
            "workload": "normalise + 5 steps on bf16 [4096,14336] (examples/five_steps.py loop)",
            "polar_express_us": round(sec_express * 1e6, 2),
            "torch_norm_plus_5_polar_step_us": round(sec_loop * 1e6, 2),
            "tflops": round(5 * flops / sec_express / 1e12, 2),
        },
        "muon_update": {
            "workload": ("Muon update of one fp32 [4096,14336] parameter: Nesterov momentum, "
                         "normalise + 5 steps (bf16), decoupled weight decay, shape-scaled step"),
            "native_us": round(sec_muon * 1e6, 2),
            "torch_eager_us": round(sec_muon_eager * 1e6, 2),
            "speedup_vs_torch_eager": round(sec_muon_eager / sec_muon, 3),
            "elementwise_us": round((sec_muon - sec_express) * 1e6, 2),
        },
        "secondary": {
            "workload": "polar_step on bf16 [8,512,2048], one step",
            "us_per_step": round(sec2 * 1e6, 2),
            "tflops": round(fl2 / sec2 / 1e12, 2),
            "pct_bf16_peak": round(100 * fl2 / sec2 / 1e12 / PEAK_BF16_TFLOPS, 2),
            "pct_hbm_peak": round(100 * hbm2 / sec2 / 1e9 / PEAK_HBM_GBS, 2),
            "kernel_us": {k: round(v, 2) for k, v in st2.items()},
            "torch_eager_us": round(eager2 * 1e6, 2),
            "speedup_vs_torch_eager": round(eager2 / sec2, 3),
        },
    }
    result["all_configs"] = all_configs()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
