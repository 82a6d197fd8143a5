"""Orthogonalise a batch of matrices with the five Polar Express steps on one MI355X.

Runs the same computation two ways and compares them:

* ``polar_express(x)`` — one call: the Frobenius normalisation and the five steps of
  ``COEFFICIENTS`` run as native kernels that reuse one plan and one workspace;
* the per-step loop a caller of the reference writes around ``polar_step``
  (normalise in PyTorch, then one ``polar_step`` per coefficient triple).

Then it reports how far the singular values of the result sit from 1 (the iteration maps
each singular value of the normalised input towards 1) and the time per call of each form.

    python examples/five_steps.py [--shape 8 512 2048] [--seed 0]
"""

from __future__ import annotations

import argparse
import time

import torch

from muon_fusion_ascend950_amd import COEFFICIENTS, polar_express, polar_step


def per_step_loop(x: torch.Tensor) -> torch.Tensor:
    y = x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)
    for a, b, c in COEFFICIENTS:
        y = polar_step(y, a, b, c)
    return y


def us_per_call(fn, calls: int = 50) -> float:
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / calls * 1e6


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--shape", type=int, nargs="+", default=[8, 512, 2048])
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args()

    gen = torch.Generator().manual_seed(args.seed)  # seeded on the host: same input every run
    x = torch.randn(*args.shape, generator=gen).to(torch.bfloat16).cuda()

    fused = polar_express(x)
    looped = per_step_loop(x)
    diff = (fused.float() - looped.float()).norm() / looped.float().norm()
    print(f"shape {list(x.shape)}: polar_express vs per-step loop, relative difference {diff:.2e}")

    sv = torch.linalg.svdvals(fused.float())
    print(f"singular values after {len(COEFFICIENTS)} steps: min {sv.min():.3f}, "
          f"median {sv.median():.3f}, max {sv.max():.3f}")

    print(f"polar_express {us_per_call(lambda: polar_express(x)):.1f} us per call, "
          f"per-step loop {us_per_call(lambda: per_step_loop(x)):.1f} us per call")


if __name__ == "__main__":
    main()
