"""Writes tests/golden/polar_golden.npz — small input/output vectors of the oracle.

The reference ships no golden vectors (its tests draw unseeded device RNG,
tests/test_polar_step.py:38,47), so these fixtures are produced by this build's
CPU oracle (oracle/polar_oracle.py, itself pinned by tests/test_oracle.py) from
seeded inputs that follow the reference's input recipe (tests/test_polar_step.py:38-39).
They freeze the oracle's outputs so that a GPU run, which has no reference tree,
checks against the same numbers.  Run from the repository root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import polar_oracle as O  # noqa: E402

# (name, shape, steps, seed): shapes of the reference's own tests
# (tests/test_polar_step.py:36,47) plus tiny and batched unaligned cases.
CASES = [
    ("x129x130_1step", (129, 130), 1, 11),
    ("x1x130x129_1step", (1, 130, 129), 1, 12),
    ("x2x150x170_1step", (2, 150, 170), 1, 13),
    ("x1x129x130_5step", (1, 129, 130), 5, 14),
    ("x3x5_1step", (3, 5), 1, 15),
    ("x1x1_1step", (1, 1), 1, 16),
    ("x1x17_1step", (1, 17), 1, 17),
    ("x64x64_1step", (64, 64), 1, 18),
]


def bf16_bits(t) -> np.ndarray:
    import torch

    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def compute(shape, steps, seed):
    x = O.make_input(shape, seed=seed)
    x64 = O.to_numpy_f64(x)
    coeffs = O.COEFFICIENTS[:steps]
    fused = x64
    exact = x64
    for a, b, c in coeffs:
        fused = O.wrapper_step(fused, a, b, c, step=O.polar_step_fused)
        exact = O.wrapper_step(exact, a, b, c, step=O.polar_step_f64)
    return bf16_bits(x), O.f32_to_bf16_bits(fused.astype(np.float32)), exact


def main() -> None:
    out = {}
    for name, shape, steps, seed in CASES:
        xb, fb, ex = compute(shape, steps, seed)
        out[f"{name}.x_bits"] = xb
        out[f"{name}.fused_bits"] = fb
        out[f"{name}.exact_f32"] = ex.astype(np.float32)
        out[f"{name}.meta"] = np.array([steps, seed], dtype=np.int64)
    path = Path(__file__).resolve().parent / "polar_golden.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
