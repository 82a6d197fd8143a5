"""Seeded random shapes through polar_step against the oracle (marked ``gpu``).

The hand-picked shapes of the other tests cover each plan decision on purpose; these
draw 24 shapes at random (batch 1-3, each side 1-760 or 1-2100, wide and tall, every
residue of n mod 64), so the plans they land on (tile sizes, ring depths, stream-K
splits, K masks, padded copies, the right-Gram form, the wrapper's transpose) are
whatever the shape gives.  Each result must pass the reference's normwise gate
against the exact float64 step and match the oracle's rounding-point emulation
element by element (at most 0.1% of elements more than one bf16 ulp apart), as in
the hand-picked tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
from tests.test_polar_step_gpu import assert_matches_oracle, run_steps

pytestmark = pytest.mark.gpu

C0 = O.COEFFICIENTS[0]


def random_shapes(count: int, seed: int):
    rng = np.random.default_rng(seed)
    shapes = []
    for _ in range(count):
        b = int(rng.integers(1, 4))
        short = int(rng.integers(1, 761))
        long = int(rng.integers(short, 2101))
        m, n = (short, long) if rng.random() < 0.6 else (long, short)
        shapes.append((b, m, n))
    return shapes


SHAPES = random_shapes(24, seed=2026)


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    yield


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_random_shape_matches_oracle(shape):
    print(f"random shape {shape}", flush=True)
    x = O.make_input(shape, seed=sum(shape))
    y = run_steps(x, [C0])
    assert y.shape == x.shape
    assert torch.isfinite(y.float()).all()
    assert_matches_oracle(y, x, [C0], rel_exact=1e-2)
