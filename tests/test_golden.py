"""The committed golden vectors (tests/golden/polar_golden.npz) still match the oracle.

They are the fixtures the GPU tests compare against; this CPU test shows that the
pinned oracle and the input recipe reproduce them bit for bit.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from tests.golden.make_golden import CASES, compute

GOLDEN = Path(__file__).resolve().parent / "golden" / "polar_golden.npz"


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


@pytest.mark.parametrize("name,shape,steps,seed", CASES, ids=[c[0] for c in CASES])
def test_golden_vectors_reproduce(golden, name, shape, steps, seed):
    xb, fb, ex = compute(shape, steps, seed)
    assert np.array_equal(golden[f"{name}.x_bits"], xb)
    assert np.array_equal(golden[f"{name}.fused_bits"], fb)
    assert np.allclose(golden[f"{name}.exact_f32"], ex, rtol=1e-6, atol=1e-9)
    assert golden[f"{name}.x_bits"].shape == tuple(shape)
