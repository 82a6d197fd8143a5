"""Benchmark of one Polar Express step (``polar_step``) on one MI355X.

Metric: polar_step µs and TFLOP/s (% of dense bf16 MFMA peak) at
[8,512,2048] and 4096×14336.  ``value`` is the TFLOP/s of the headline workload, a
single ``polar_step`` on a bf16 [4096,14336] matrix with inputs resident in HBM,
counting the credited FLOPs M²N + 2M³ + 2M²N per matrix.  The [8,512,2048] case is
reported in ``secondary``.

Order of a run (rank 0, one GPU):

1. accuracy gate of the headline input (the reference's method runs its
   ``assert_close(…, 6e-2)`` before timing, README.md:179-203), then ``--settle-s``
   seconds of headline calls: from idle the GPU's power management needs about 50
   steps (≈35 ms of load) to reach its steady clock — the first 2 steps run fast, steps
   3-5 at ~1.4x their steady time, then the clock recovers — so a short W/K window
   would otherwise time that transient;
2. the driver contract: W untimed warm-up calls, then exactly K timed calls between two
   device synchronisations → ``value``, ``ms_per_step``;
3. per-stage device times inside a step (``kernel_us``): R repetitions of the step
   (gram, poly, apply), of its tail (poly, apply) and of apply alone, launched through the
   C ABI with the step's workspace and stream-K split, each captured in a HIP graph and
   replayed between two HIP events on the launch stream (no host gaps); stage times are
   the differences, so they sum to the replayed step (``graph_step_us``); ``roofline``
   uses stage 3 (P·X + a·X), the dominant kernel;
4. every BASELINE.json configuration with the reference's timing method (20 warm-ups,
   then the median of 5 repeats of 100 calls, README.md:179-191) after its accuracy gate
   (6e-2 against the fp32 formula, and relF = ‖Y − Y_fp32‖_F / ‖Y_fp32‖_F);
5. comparison points (PyTorch eager on the GPU, five steps, the Muon update) and the
   CPU baseline (the oracle's restatement of the reference formula on the host cores).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
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
GATE_TOL = 6e-2  # tests/test_polar_step.py:42,53
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
# CPU baseline shapes (every BASELINE.json configuration's shape): shape and runs after
# one warm-up
CPU_SHAPES = (((129, 130), 50), ((2, 150, 2050), 50), ((8, 512, 2048), 50), ((4096, 14336), 40),
              ((4, 4096, 4096), 20))
TRAFFIC_SUMMARY = ROOT / "profiles" / "apply_4096x14336_hbm_traffic.txt"
STAGES = ("gram", "poly", "apply")


# ----------------------------------------------------------------------------- workloads
def credited_flops(batch: int, m: int, n: int) -> int:
    m, n = min(m, n), max(m, n)
    return batch * (m * m * n + 2 * m**3 + 2 * m * m * n)


def make_input(shape, seed: int = 0):
    """Seeded bf16 N(0,1) on the CPU, normalised per matrix (tests/test_polar_step.py:38-39)."""
    import torch

    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, dtype=torch.bfloat16, generator=gen)
    return x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)


def torch_formula(x, coefficients):
    """The reference's formula (tests/test_polar_step.py:22-28, README.md:172-174) in
    plain PyTorch at x's dtype: gram = x @ x.mT; x = a*x + (b*gram + c*gram@gram) @ x.
    The transposed operand is materialised first (batched bf16 products with a transposed
    right operand are avoided on ROCm)."""
    import torch

    out = x
    for a, b, c in coefficients:
        gram = torch.matmul(out, out.mT.contiguous())
        out = a * out + torch.matmul(b * gram + c * torch.matmul(gram, gram), out)
    return out


def config_call(shape, steps: int):
    """The GPU call of one configuration: one polar_step, or the five-step chain."""
    import muon_fusion_ascend950_amd as mf

    x = make_input(shape, seed=0).cuda()
    if steps == 1:
        a, b, c = COEFFS
        return (lambda: mf.polar_step(x, a, b, c)), x
    coeffs = mf.COEFFICIENTS[:steps]
    return (lambda: mf.polar_express(x, coeffs, normalize=False)), x


def accuracy(y, x, coefficients) -> dict:
    """The reference's gate (assert_close rtol = atol = 6e-2 against the formula, here in
    fp32 on the GPU) and the normwise error relF, which the gate alone cannot replace (an
    all-zero output passes it at these magnitudes)."""
    import torch

    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        ref = torch_formula(x.float(), coefficients)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = prev
    yf = y.float()
    ok = bool(torch.isclose(yf, ref, rtol=GATE_TOL, atol=GATE_TOL).all().item())
    rel = ((yf - ref).norm() / ref.norm()).item()
    del ref, yf
    return {"gate_6e-2": "pass" if ok else "FAIL", "relF_vs_fp32_formula": float(f"{rel:.3e}")}


# ----------------------------------------------------------------------------- timing
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


def reference_method(fn, warmup: int = 20, calls: int = 100, repeats: int = 5) -> float:
    """README.md:179-191: warm-up, then the median over `repeats` of `calls` back-to-back
    calls bracketed by device synchronisations (seconds per call)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    samples = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        torch.cuda.synchronize()
        samples.append((time.perf_counter() - t0) / calls)
    return statistics.median(samples)


def interleaved(fns, calls: int, warmup: int, rounds: int = 5) -> list:
    """Seconds per call of each function, timed in alternation (`rounds` rounds of
    `calls` calls each after `warmup` calls): the median per function, so that a drift
    of the GPU clock affects the variants alike."""
    samples = [[] for _ in fns]
    for _ in range(rounds):
        for i, fn in enumerate(fns):
            samples[i].append(time_calls(fn, calls, warmup))
    return [statistics.median(s) for s in samples]


def settle(fn, seconds: float) -> int:
    """Run `fn` back to back for `seconds` (the GPU's clock settles under sustained load)."""
    import torch

    calls = 0
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(10):
            fn()
        calls += 10
        torch.cuda.synchronize()
    return calls


def stage_times(batch: int, m: int, n: int, launches: int, repeats: int = 3) -> dict:
    """µs per launch of each stage inside a step, from HIP-graph replays without host
    gaps: `launches` repetitions of a stage sequence through the C ABI (polar_step's
    workspace, A and P in it, the same stream-K split as inside the step) are captured
    in one graph and replayed between two HIP events on the capturing stream (the
    median of `repeats` replays).  Three sequences: the step (gram, poly, apply),
    its tail (poly, apply) and apply alone.  apply = apply alone, poly = tail - apply,
    gram = step - tail: each stage runs where it runs in a step (gram after an apply,
    before a poly), and the three sum to the replayed step ("step")."""
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
    calls = {"gram": lambda: capi.gram(x, gram, workspace=ws),
             "poly": lambda: capi.poly(gram, poly, batch, m, n, b, c, workspace=ws),
             "apply": lambda: capi.apply(poly, x, y, a, workspace=ws)}
    for name in STAGES:  # A and P in place before any stage is timed
        calls[name]()
    torch.cuda.synchronize()
    sequences = {"step": STAGES, "tail": STAGES[1:], "apply": STAGES[2:]}
    per = {}
    stream = torch.cuda.Stream()
    for key, seq in sequences.items():
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for _ in range(launches):
                    for name in seq:
                        calls[name]()
        graph.replay()  # warm-up replay
        torch.cuda.synchronize()
        samples = []
        for _ in range(repeats):
            start = torch.cuda.Event(enable_timing=True)
            stop = torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                start.record()
                graph.replay()
                stop.record()
            stop.synchronize()
            samples.append(start.elapsed_time(stop) * 1e3 / launches)
        per[key] = statistics.median(samples)
        del graph
    torch.cuda.synchronize()
    return {"gram": per["step"] - per["tail"], "poly": per["tail"] - per["apply"],
            "apply": per["apply"], "step": per["step"]}


def instep_kernel_times(batch: int, m: int, n: int, steps: int) -> dict:
    """µs of each stage kernel inside eager steps: `steps` steps run as their three stage
    calls through the C ABI (polar_step's workspace, the step's own plan and split, so
    each call is the kernel the step launches, in its place), with a HIP event recorded
    on the launch stream before gram and after each stage; the median over the steps of
    each interval.  Unlike stage_times (differences of graph replays) every kernel is
    timed directly where it runs, its dispatch from the stream's queue included; each
    timed event also adds a release between two kernels, so the intervals over-state
    the kernels by that much ("step" against an untimed step shows it)."""
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
    calls = (lambda: capi.gram(x, gram, workspace=ws),
             lambda: capi.poly(gram, poly, batch, m, n, b, c, workspace=ws),
             lambda: capi.apply(poly, x, y, a, workspace=ws))
    for call in calls:
        call()
    torch.cuda.synchronize()
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for ev in events:
        ev[0].record()
        for i, call in enumerate(calls):
            call()
            ev[i + 1].record()
    torch.cuda.synchronize()
    per = {name: statistics.median(ev[i].elapsed_time(ev[i + 1]) * 1e3 for ev in events)
           for i, name in enumerate(STAGES)}
    per["step"] = statistics.median(ev[0].elapsed_time(ev[3]) * 1e3 for ev in events)
    return per


def sustained(fn, seconds: float) -> tuple:
    """µs per call over `seconds` of back-to-back calls (synchronised once a second)."""
    import torch

    calls = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            fn()
        calls += 50
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) / calls, calls


# ----------------------------------------------------------------------------- comparison points
MUON_LR, MUON_MOMENTUM, MUON_WD = 0.02, 0.95, 0.01


# One Muon optimizer step over two transformer layers' matrices at d = 768 (attention
# q, k, v, o [768,768]; MLP [3072,768] and [768,3072]): small matrices, each of whose
# steps leaves most CUs idle
OPT_SHAPES = [(768, 768)] * 8 + [(3072, 768)] * 2 + [(768, 3072)] * 2


def optimizer_step_us(grouped: bool) -> float:
    """µs per Muon.step over OPT_SHAPES: one native update per parameter
    (grouped=False) or same-shape parameters batched into one (Muon's default)."""
    import torch
    import muon_fusion_ascend950_amd as mf

    gen = torch.Generator().manual_seed(3)
    params = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).cuda()) for s in OPT_SHAPES]
    for prm in params:
        prm.grad = (torch.randn(prm.shape, generator=gen) * 1e-3).cuda()
    opt = mf.Muon(params, lr=MUON_LR, momentum=MUON_MOMENTUM, weight_decay=MUON_WD,
                  group_shapes=grouped)
    return time_calls(opt.step, 10, 3) * 1e6


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
    buf.lerp_(g, 1 - MUON_MOMENTUM)
    u = g.lerp(buf, MUON_MOMENTUM)
    x = u.bfloat16()
    x = x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)
    x = torch_formula(x, coefficients)
    p.mul_(1 - MUON_LR * MUON_WD)
    p.add_(x, alpha=-MUON_LR * max(1.0, p.size(-2) / p.size(-1)) ** 0.5)


def read_traffic():
    """HBM bytes per stage-3 launch from the committed rocprofv3 --pmc summary, if any."""
    if not TRAFFIC_SUMMARY.is_file():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", TRAFFIC_SUMMARY.read_text(), re.M)
    return float(m.group(1)) if m else None


def run_metadata() -> dict:
    """What the reference asks results to be published with (README.md:208): device,
    framework versions, tuning variables and the timing method."""
    import torch

    props = torch.cuda.get_device_properties(0)
    tuning = {k: v for k, v in sorted(os.environ.items()) if k.startswith("MUON_POLAR_")}
    return {
        "device": props.name,
        "arch": getattr(props, "gcnArchName", ""),
        "compute_units": props.multi_processor_count,
        "torch": torch.__version__,
        "hip": torch.version.hip,
        "python": platform.python_version(),
        "tuning_variables": tuning or "defaults",
        "timing": ("value: settle, W warm-up calls, K calls between device synchronisations; "
                   "all_configs: 20 warm-ups, median of 5 x 100 calls (README.md:179-191); "
                   "kernel_us: HIP-graph replays of R steps, R (poly, apply) and R apply "
                   "between HIP events on the launch stream; stage times are their "
                   "differences (roofline.achieved uses apply); event_kernel_us: R eager "
                   "steps as their three stage launches with a HIP event recorded after "
                   "each, median interval per stage: every stage timed where it runs, but "
                   "each timed event adds a release between kernels (event_step_us against "
                   "graph_step_us shows its cost), so these over-state each kernel; "
                   "sustained: back-to-back headline calls for sustained.seconds after "
                   "the K timed calls"),
    }


def cpu_info() -> dict:
    model, flags = "", set()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name") and not model:
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    isa = [f for f in ("amx_bf16", "amx_tile", "avx512_bf16", "avx512f", "avx2") if f in flags]
    return {"cpu_model": model, "isa_flags": isa}


def cpu_baseline() -> dict:
    """The oracle's restatement of the reference formula, bf16 torch on the host CPU.

    Threads: the host cores this process may use (its affinity), capped at the box's CPU
    share of 16 threads per GPU (the GPU boxes give each GPU 16 host threads and set
    OMP_NUM_THREADS to that)."""
    import torch
    from oracle import polar_oracle as O

    affinity = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "16") or 16)
    cores = max(1, min(affinity, share))
    torch.set_num_threads(cores)
    rows = []
    headline = None
    with torch.no_grad():
        for shape, runs in CPU_SHAPES:
            x = make_input(shape, seed=0)
            O.reference_formula_torch(x, [COEFFS])  # warm-up
            samples = []
            for _ in range(runs):
                t0 = time.perf_counter()
                O.reference_formula_torch(x, [COEFFS])
                samples.append(time.perf_counter() - t0)
            med = statistics.median(samples)
            batch = shape[0] if len(shape) == 3 else 1
            tf = credited_flops(batch, shape[-2], shape[-1]) / med / 1e12
            rows.append({"shape": list(shape), "runs": runs, "us_per_step": round(med * 1e6, 1),
                         "tflops": round(tf, 4)})
            if tuple(shape) == HEADLINE[1:]:
                headline = (tf, med, runs)
    tf, med, runs = headline
    return {
        "value": round(tf, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"reference formula (tests/test_polar_step.py:22-28) in bf16 torch on the host "
                   f"CPU, [4096,14336] one step, median of {runs} runs after 1 warm-up "
                   f"({med * 1e3:.0f} ms/step); other BASELINE shapes in 'shapes'"),
        "torch_threads": torch.get_num_threads(),
        "affinity_cores": affinity,
        "thread_policy": (f"min(affinity cores {affinity}, OMP_NUM_THREADS {share}): the GPU box's "
                          f"host share is 16 threads per GPU; the baseline plan asks for every "
                          f"affinity core"
                          + (", which this equals" if cores == affinity else
                             f", {affinity - cores} of which are left out by the cap")),
        **cpu_info(),
        "shapes": rows,
    }


# ----------------------------------------------------------------------------- phases
def all_configs():
    """µs per call (reference method), credited TFLOP/s, % of the dense bf16 peak and the
    accuracy gate of every BASELINE.json configuration."""
    rows = []
    for name, shape, steps in CONFIGS:
        import muon_fusion_ascend950_amd as mf

        fn, x = config_call(shape, steps)
        gate = accuracy(fn(), x, mf.COEFFICIENTS[:steps] if steps > 1 else [COEFFS])
        batch = shape[0] if len(shape) == 3 else 1
        m, n = shape[-2], shape[-1]
        sec = reference_method(fn)
        flops = steps * credited_flops(batch, m, n)
        rows.append({"config": name, "shape": list(shape), "steps_per_call": steps,
                     "us_per_call": round(sec * 1e6, 2),
                     "tflops": round(flops / sec / 1e12, 2),
                     "pct_bf16_peak": round(100 * flops / sec / 1e12 / PEAK_BF16_TFLOPS, 2),
                     **gate})
        print(json.dumps({"config": name, "shape": list(shape), "steps": steps,
                          "us_per_call": round(sec * 1e6, 2), **gate}), file=sys.stderr, flush=True)
        del x
    return rows


def headline_phase(args, x):
    """Gate, settle, then the contract's W + K calls; per-stage times after it."""
    import torch
    import muon_fusion_ascend950_amd as mf

    a, b, c = COEFFS
    gate = accuracy(mf.polar_step(x, a, b, c), x, [COEFFS])
    step = lambda: mf.polar_step(x, a, b, c)  # noqa: E731
    settled = settle(step, args.settle_s)
    sec = time_calls(step, args.steps, args.warmup)
    torch.cuda.synchronize()
    return gate, settled, sec, step


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-s", type=float, default=1.0,
                    help="seconds of headline calls before the warm-up (GPU clock settling)")
    ap.add_argument("--stage-launches", type=int, default=50,
                    help="repetitions of each stage sequence (step, tail, apply) in the "
                         "graph-replayed stage timing")
    ap.add_argument("--sustain-s", type=float, default=2.0,
                    help="seconds of back-to-back headline calls after the timed K (the "
                         "'sustained' figure; 0 skips it)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile", action="store_true",
                    help="only the headline phase (gate, settle, W + K steps), the stage "
                         "timing of [4096,14336] and [8,512,2048], and three 1 GiB device copies "
                         "(the calibration kernel of known size), for rocprofv3 runs")
    ap.add_argument("--profile-secondary", action="store_true",
                    help="only the [8,512,2048] step loop, for rocprofv3 runs")
    ap.add_argument("--profile-configs", action="store_true",
                    help="only a few calls of every BASELINE configuration in turn, then three "
                         "1 GiB device copies (the calibration kernel), for rocprofv3 counter runs")
    ap.add_argument("--profile-muon", action="store_true",
                    help="only a loop of Muon updates of one fp32 [4096,14336] parameter, "
                         "for rocprofv3 runs")
    ap.add_argument("--profile-shape", default=None, metavar="BxMxN",
                    help="only --settle-s seconds, then W + K polar_step calls on one bf16 "
                         "[B,M,N] input (e.g. 4x4096x4096), for rocprofv3 runs")
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
    batch, m, n = HEADLINE

    if args.profile_muon:
        p, g, buf = muon_tensors(m, n)
        sec = time_calls(lambda: mf.muon_update(p, g, buf, lr=MUON_LR, momentum=MUON_MOMENTUM,
                                                weight_decay=MUON_WD), args.steps, args.warmup)
        print(json.dumps({"profile": "muon_update fp32 [4096,14336]", "steps": args.steps,
                          "us_per_update": round(sec * 1e6, 2)}), flush=True)
        return 0
    if args.profile_shape:
        shape = tuple(int(v) for v in args.profile_shape.split("x"))
        xs = make_input(shape, seed=0).cuda()
        fn = lambda: mf.polar_step(xs, a, b, c)  # noqa: E731
        t_end = time.perf_counter() + args.settle_s
        while time.perf_counter() < t_end:
            fn()
            torch.cuda.synchronize()
        sec = time_calls(fn, args.steps, args.warmup)
        print(json.dumps({"profile": "polar_step", "shape": list(shape), "steps": args.steps,
                          "us_per_step": round(sec * 1e6, 2)}), flush=True)
        return 0
    if args.profile_configs:
        for name, shape, steps in CONFIGS:
            fn, x = config_call(shape, steps)
            sec = time_calls(fn, args.steps, args.warmup)
            print(json.dumps({"profile": name, "shape": list(shape), "steps_per_call": steps,
                              "us_per_call": round(sec * 1e6, 2)}), flush=True)
            del x
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)  # reads and writes exactly 1 GiB: the counters' calibration
        torch.cuda.synchronize()
        return 0
    if args.profile_secondary:
        x2 = make_input(SECONDARY, seed=0).cuda()
        sec = time_calls(lambda: mf.polar_step(x2, a, b, c), args.steps, args.warmup)
        print(json.dumps({"profile": "polar_step [8,512,2048]", "steps": args.steps,
                          "us_per_step": round(sec * 1e6, 2)}), flush=True)
        return 0

    # ---- headline: [4096,14336], one step (the driver contract)
    x = make_input((m, n), seed=0).cuda()
    gate, settled, sec, step_fn = headline_phase(args, x)
    flops = credited_flops(batch, m, n)
    tflops = flops / sec / 1e12
    print(json.dumps({"phase": "headline", "us_per_step": round(sec * 1e6, 2),
                      "settle_calls": settled, **gate}), file=sys.stderr, flush=True)
    # 2 s of back-to-back headline calls: the rate a long optimizer run sustains
    sec_sus, calls_sus = sustained(step_fn, args.sustain_s) if args.sustain_s > 0 else (None, 0)
    st = stage_times(batch, m, n, launches=args.stage_launches)
    ist = instep_kernel_times(batch, m, n, steps=args.stage_launches)
    apply_flops = 2 * batch * m * m * n
    # the roofline's duration: apply launches back to back in a replayed graph (no host
    # gaps, no event between kernels; its rocprof trace agrees with the in-step one)
    achieved = apply_flops / (st["apply"] * 1e-6) / 1e12
    b2, m2, n2 = SECONDARY
    st2 = stage_times(b2, m2, n2, launches=max(args.stage_launches, 100))
    ist2 = instep_kernel_times(b2, m2, n2, steps=max(args.stage_launches, 100))
    if args.profile:
        src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)  # reads and writes exactly 1 GiB
        torch.cuda.synchronize()
        print(json.dumps({"profile": "polar_step [4096,14336] + stage loops", "steps": args.steps,
                          "warmup": args.warmup, "settle_calls": settled,
                          "us_per_step": round(sec * 1e6, 2),
                          "kernel_us": {k: round(st[k], 2) for k in STAGES},
                          "event_kernel_us": {k: round(ist[k], 2) for k in STAGES},
                          "graph_step_us": round(st["step"], 2),
                          "secondary_kernel_us": {k: round(st2[k], 2) for k in STAGES},
                          "secondary_graph_step_us": round(st2["step"], 2),
                          "stage_launches": [args.stage_launches, max(args.stage_launches, 100)],
                          "copy_bytes": 1 << 30}), flush=True)
        return 0
    traffic = read_traffic()

    # ---- secondary: [8,512,2048], one step (reference method)
    x2 = make_input(SECONDARY, seed=0).cuda()
    gate2 = accuracy(mf.polar_step(x2, a, b, c), x2, [COEFFS])
    sec2 = reference_method(lambda: mf.polar_step(x2, a, b, c))
    fl2 = credited_flops(b2, m2, n2)
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
    sec_express, sec_loop = interleaved([lambda: mf.polar_express(raw), reference_loop], 10, 2)

    # Muon update of one fp32 [4096,14336] parameter: the native update (momentum pass,
    # normalisation, 5 steps, parameter update) vs nanochat's step in PyTorch eager
    p, g, buf = muon_tensors(m, n)
    sec_muon = time_calls(lambda: mf.muon_update(p, g, buf, lr=MUON_LR, momentum=MUON_MOMENTUM,
                                                 weight_decay=MUON_WD), 10, 3)
    sec_muon_eager = time_calls(lambda: muon_eager_step(p, g, buf, mf.COEFFICIENTS), 5, 2)
    del p, g, buf
    opt_single_us, opt_grouped_us = optimizer_step_us(False), optimizer_step_us(True)

    # PyTorch eager on the same GPU (the reference's comparison point, README.md:172-208)
    eager = time_calls(lambda: torch_formula(x, [COEFFS]), 10, 3)
    eager2 = time_calls(lambda: torch_formula(x2, [COEFFS]), 50, 5)

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
        "accuracy": gate,
        "settle": {"seconds": args.settle_s, "calls": settled},
        "sustained": ({"seconds": args.sustain_s, "calls": calls_sus,
                       "us_per_step": round(sec_sus * 1e6, 2),
                       "pct_bf16_peak": round(100 * flops / sec_sus / 1e12 / PEAK_BF16_TFLOPS, 2)}
                      if sec_sus else None),
        "kernel_us": {k: round(st[k], 2) for k in STAGES},
        "kernel_us_sum": round(sum(st[k] for k in STAGES), 2),
        "graph_step_us": round(st["step"], 2),
        "event_kernel_us": {k: round(ist[k], 2) for k in STAGES},
        "event_step_us": round(ist["step"], 2),
        "torch_eager_us": round(eager * 1e6, 2),
        "speedup_vs_torch_eager": round(eager / sec, 3),
        "roofline": {
            "bound": "mfma",
            "kernel": ("stage 3 apply (Y = a·X + P·X), 481.0 GFLOP per launch, over kernel_us.apply "
                       "(graph-replayed apply launches between HIP events on the launch stream)"),
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
        },
        "five_step": {
            "workload": "normalise + 5 steps on bf16 [4096,14336] (the loop of the reference's "
                        "examples/five_steps.py:17-20)",
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
        "muon_optimizer": {
            "workload": ("one Muon.step over 12 fp32 matrices (two layers at d = 768: 8 x "
                         "[768,768], 2 x [3072,768], 2 x [768,3072]), 5 steps each"),
            "one_call_per_parameter_us": round(opt_single_us, 2),
            "same_shape_batched_us": round(opt_grouped_us, 2),
            "speedup": round(opt_single_us / opt_grouped_us, 3),
        },
        "secondary": {
            "workload": "polar_step on bf16 [8,512,2048], one step",
            "us_per_step": round(sec2 * 1e6, 2),
            "tflops": round(fl2 / sec2 / 1e12, 2),
            "pct_bf16_peak": round(100 * fl2 / sec2 / 1e12 / PEAK_BF16_TFLOPS, 2),
            "pct_hbm_peak": round(100 * hbm2 / sec2 / 1e9 / PEAK_HBM_GBS, 2),
            "accuracy": gate2,
            "kernel_us": {k: round(st2[k], 2) for k in STAGES},
            "kernel_us_sum": round(sum(st2[k] for k in STAGES), 2),
            "event_kernel_us": {k: round(ist2[k], 2) for k in STAGES},
            "graph_step_us": round(st2["step"], 2),
            "torch_eager_us": round(eager2 * 1e6, 2),
            "speedup_vs_torch_eager": round(eager2 / sec2, 3),
        },
        "run": run_metadata(),
    }
    result["all_configs"] = all_configs()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
