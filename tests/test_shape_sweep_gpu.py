"""Seeded sweep of polar_step over random shapes on the GPU (marked ``gpu``).

The fixed-shape tests pick their cases by hand; this sweep draws 32 shapes from a
seeded generator so that the width classes that choose different code paths all
meet a spread of heights, batches and orientations:

* n odd (zero-padded copy of X), n even but not a multiple of 8 (rows read in place
  from 4-byte boundaries, the straddling chunk zeroed in LDS), n a multiple of 8 but
  not of 64 (in place, the last K-step's chunks past n masked), n a multiple of 64;
* M <= N (the direct form; 64, 128, 192 or 256 tiles by size, diagonal pairs and
  stream-K splits where the plan takes them) and M > N (right-Gram form when
  N % 8 == 0, else the reference's transpose around the op, ops.py:26-32);
* batch 1 to 3.

Each shape runs through the public ``polar_step`` twice:

* an exact-sum input (sparse ±1 X, integer coefficients): every sum a kernel forms is
  an integer below 2^24, so Y must equal the oracle's rounding-point emulation bit
  for bit (for M > N the oracle runs on Xᵀ and its result is transposed back, which
  is the same sums);
* the reference's own input recipe (tests/test_polar_step.py:38-39) against the
  float64 formula: relF <= 1e-2 and the 6e-2 gate of tests/test_polar_step.py:42.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
import functools

from tests.sweep_shapes import SWEEP_CONFIGS, sweep_config_shapes, sweep_shapes
from tests.test_polar_step_gpu import bits

pytestmark = pytest.mark.gpu

DEV = "cuda"
C0 = O.COEFFICIENTS[0]
EXACT_COEFFS = (2.0, -1.0, 1.0)


SHAPES = sweep_shapes()


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    yield


def polar_step(x, a, b, c):
    from muon_fusion_ascend950_amd import polar_step as ps

    return ps(x, a, b, c)


def test_sweep_covers_every_width_class_and_orientation():
    """The generator reaches every path the sweep is meant to cover."""
    classes = set()
    for batch, m, n in SHAPES:
        cls = "odd" if n % 2 else "even" if n % 8 else "mult8" if n % 64 else "mult64"
        classes.add((cls, "tall" if m > n else "wide"))
    for cls in ("odd", "even", "mult8", "mult64"):
        assert (cls, "wide") in classes
    assert any(c[1] == "tall" and c[0] in ("mult8", "mult64") for c in classes)  # right-Gram form
    assert any(c[1] == "tall" and c[0] in ("odd", "even") for c in classes)  # transposed route
    assert any(b > 1 for b, _, _ in SHAPES)


@functools.lru_cache(maxsize=None)
def _exact_input(batch, m, n):
    """Sparse ±1 batch whose sums stay exact in fp32, and the oracle's Y for it."""
    wide_shape = (batch, min(m, n), max(m, n))
    for nnz in (16, 8, 4, 2, 1):
        nnz = min(nnz, wide_shape[2])
        mats = O.sparse_sign_input(wide_shape, nnz, seed=31)
        refs = [O.polar_step_fused_sparse(xm, *EXACT_COEFFS) for xm in mats]
        if max(r[1] for r in refs) < 2**24:
            break
    else:  # pragma: no cover - one nonzero per row always stays exact here
        raise AssertionError("no exact-sum input for this shape")
    x = np.stack([xm.toarray() for xm in mats])
    y = np.stack([r[0] for r in refs])
    if m > n:
        x, y = x.transpose(0, 2, 1), y.transpose(0, 2, 1)
    return np.ascontiguousarray(x), np.ascontiguousarray(y)


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{b}x{m}x{n}" for b, m, n in SHAPES])
def test_sweep_exact_sums_are_bitwise(shape):
    _assert_exact_bitwise(shape)


CONFIG_SHAPES = sweep_config_shapes()


@pytest.mark.parametrize("config", sorted(SWEEP_CONFIGS))
@pytest.mark.parametrize("shape", CONFIG_SHAPES, ids=[f"{b}x{m}x{n}" for b, m, n in CONFIG_SHAPES])
def test_sweep_configurations_exact_sums_are_bitwise(monkeypatch, shape, config):
    """The same exact-sum check with a tuned configuration (tile size, waves, ring
    depths, stream-K off, register-staged kernels): every kernel family the knobs reach
    forms the same exact sums."""
    for k, v in SWEEP_CONFIGS[config].items():
        monkeypatch.setenv(k, v)
    _assert_exact_bitwise(shape, config)


def _assert_exact_bitwise(shape, config="default"):
    batch, m, n = shape
    x_np, y_ref = _exact_input(batch, m, n)
    print(f"sweep exact {shape} {config}", flush=True)
    x = torch.from_numpy(x_np.astype(np.float32)).to(torch.bfloat16).to(DEV)
    y = polar_step(x if batch > 1 else x[0], *EXACT_COEFFS)
    torch.cuda.synchronize()
    got = bits(y).reshape(batch, m, n)
    want = O.f32_to_bf16_bits(y_ref.astype(np.float32))
    bad = np.flatnonzero(got.ravel() != want.ravel())
    assert bad.size == 0, (f"{shape}: {bad.size} of {got.size} elements differ, first at "
                           f"{np.unravel_index(bad[0], got.shape)}")


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{b}x{m}x{n}" for b, m, n in SHAPES])
def test_sweep_matches_float64_formula(shape):
    batch, m, n = shape
    x_cpu = O.make_input(shape if batch > 1 else (m, n), seed=32)
    print(f"sweep random {shape}", flush=True)
    y = polar_step(x_cpu.to(DEV), *C0)
    torch.cuda.synchronize()
    exact = O.wrapper_step(O.to_numpy_f64(x_cpu), *C0, step=O.polar_step_f64)
    yn = y.float().cpu().numpy().astype(np.float64)
    assert O.rel_frobenius(yn, exact) <= 1e-2
    torch.testing.assert_close(y.float().cpu(), torch.from_numpy(exact).float(), rtol=6e-2,
                               atol=6e-2)
