"""Seeded random cases — shape x configuration x output offset — bit for bit on
exact-sum inputs (marked ``gpu``).

The other sweeps fix the configuration per shape list; here each of 160 cases draws its
shape (batch 1-4, up to 6M elements, every width class, wide and tall), one of nine
configurations (the tuned ones, the defaults, and the defaults without the two-round
stream-K split, diagonal pairs or apply's column halves) and where Y starts (0, 1 or 2
elements past a 16-byte boundary: the 16-byte, 4-byte-aligned and 2-byte store paths).
Every case's plan was checked on the CPU first
(``tests/test_plan_extents.py::test_random_case_plans_store_inside_their_buffers``).
With sparse ±1 X and integer coefficients every sum is exact in fp32, so Y must equal
the oracle's rounding-point emulation bit for bit, and nothing may be written outside Y.
The first 40 cases also run polar_express (1-5 steps, one workspace reused across the
steps) against as many chained polar_step calls, bit for bit, and 30 wide cases run the
stage entry points (gram, poly, apply) against the step and the oracle.
"""

from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
from tests.sweep_shapes import FUZZ_CONFIGS, fuzz_cases

pytestmark = pytest.mark.gpu

DEV = "cuda"
EXACT = (2.0, -1.0, 1.0)
CASES = fuzz_cases()
KNOBS = sorted({k for v in FUZZ_CONFIGS.values() for k in v})


@functools.lru_cache(maxsize=8)
def _exact_input(batch, m, n, seed):
    wide = (batch, min(m, n), max(m, n))
    for nnz in (16, 8, 4, 2, 1):
        mats = O.sparse_sign_input(wide, min(nnz, wide[2]), seed=seed)
        refs = [O.polar_step_fused_sparse(xm, *EXACT) for xm in mats]
        if max(r[1] for r in refs) < 2**24:
            break
    else:  # pragma: no cover - one nonzero per row always stays exact
        raise AssertionError("no exact-sum input")
    x = np.stack([xm.toarray() for xm in mats])
    y = np.stack([r[0] for r in refs])
    if m > n:
        x, y = x.transpose(0, 2, 1), y.transpose(0, 2, 1)
    return np.ascontiguousarray(x), np.ascontiguousarray(y)


@pytest.mark.parametrize("case", range(len(CASES)),
                         ids=[f"{b}x{m}x{n}-{c}-off{o}" for (b, m, n), c, o in CASES])
def test_random_case_is_bitwise(monkeypatch, case):
    import muon_fusion_ascend950_amd as mf
    from muon_fusion_ascend950_amd import capi

    (batch, m, n), config, offset = CASES[case]
    for k in KNOBS:
        monkeypatch.delenv(k, raising=False)
    for k, v in FUZZ_CONFIGS[config].items():
        monkeypatch.setenv(k, v)
    print(f"random case {case}: {(batch, m, n)} {config} offset {offset}", flush=True)
    x_np, y_ref = _exact_input(batch, m, n, seed=1000 + case)
    x = torch.from_numpy(x_np.astype(np.float32)).to(torch.bfloat16).to(DEV)
    if m > n and n % 8 != 0:
        y = mf.polar_step(x, *EXACT)  # the reference wrapper's transposed route
        flat = None
    else:
        ws, _ = capi.alloc_workspace(batch, m, n)
        flat = torch.full((x.numel() + offset + 8,), float("nan"), dtype=torch.bfloat16,
                          device=DEV)
        y = flat[offset:offset + x.numel()].view(x.shape)
        capi.step(x, y, ws, *EXACT)
    torch.cuda.synchronize()
    got = y.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(y_ref.shape)
    want = O.f32_to_bf16_bits(y_ref.astype(np.float32))
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, (f"{bad.size} of {got.size} elements differ, first at "
                           f"{np.unravel_index(bad[0], got.shape)}")
    if flat is not None:
        assert torch.isnan(flat[:offset]).all() and torch.isnan(flat[offset + x.numel():]).all()


EXPRESS_CASES = CASES[:40]


@pytest.mark.parametrize("case", range(len(EXPRESS_CASES)),
                         ids=[f"{b}x{m}x{n}-{c}" for (b, m, n), c, _ in EXPRESS_CASES])
def test_random_case_express_equals_chained_steps(monkeypatch, case):
    """polar_express without normalisation (one plan and one workspace reused across the
    steps, the iterate alternating between two buffers) equals chained polar_step calls
    (a fresh workspace each) bit for bit, for 1 to 5 steps, under the case's configuration."""
    import muon_fusion_ascend950_amd as mf

    (batch, m, n), config, _offset = EXPRESS_CASES[case]
    for k in KNOBS:
        monkeypatch.delenv(k, raising=False)
    for k, v in FUZZ_CONFIGS[config].items():
        monkeypatch.setenv(k, v)
    steps = 1 + case % 5
    print(f"random express case {case}: {(batch, m, n)} {config} steps {steps}", flush=True)
    x = O.make_input((batch, m, n), seed=2000 + case).to(DEV)
    got = mf.polar_express(x, O.COEFFICIENTS[:steps], normalize=False)
    want = x
    for a, b, c in O.COEFFICIENTS[:steps]:
        want = mf.polar_step(want, a, b, c)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, want)


STAGE_CASES = [c for c in CASES if c[0][1] <= c[0][2]][:30]


@pytest.mark.parametrize("case", range(len(STAGE_CASES)),
                         ids=[f"{b}x{m}x{n}-{c}" for (b, m, n), c, _ in STAGE_CASES])
def test_random_case_stage_calls(monkeypatch, case):
    """The stage entry points (gram, poly, apply) on random cases (M <= N), each under its
    configuration: given the step's workspace they reproduce the step's A, P and Y bit for
    bit on a random input; without a workspace (one tile per workgroup, no split) their Y
    equals the oracle's bit for bit on the exact-sum input."""
    from muon_fusion_ascend950_amd import capi

    (batch, m, n), config, _offset = STAGE_CASES[case]
    for k in KNOBS:
        monkeypatch.delenv(k, raising=False)
    for k, v in FUZZ_CONFIGS[config].items():
        monkeypatch.setenv(k, v)
    print(f"random stage case {case}: {(batch, m, n)} {config}", flush=True)
    a, b, c = O.COEFFICIENTS[case % 5]
    x = O.make_input((batch, m, n), seed=4000 + case).to(DEV)
    ws, info = capi.alloc_workspace(batch, m, n)
    y_step = torch.empty_like(x)
    capi.step(x, y_step, ws, a, b, c)
    mp, gram_bytes = info.padded_rows, info.gram_bytes
    p_off = -(-gram_bytes // 256) * 256
    a_step = ws[:gram_bytes].clone()
    p_step = ws[p_off:p_off + gram_bytes].clone()
    gram = torch.empty(batch, mp, mp, dtype=torch.bfloat16, device=DEV)
    poly = torch.empty_like(gram)
    y = torch.empty_like(x)
    capi.gram(x, gram, workspace=ws)
    capi.poly(gram, poly, batch, m, n, b, c, workspace=ws)
    capi.apply(poly, x, y, a, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(gram.view(torch.uint8).reshape(-1), a_step)
    assert torch.equal(poly.view(torch.uint8).reshape(-1), p_step)
    assert torch.equal(y, y_step)

    x_np, y_ref = _exact_input(batch, m, n, seed=1000 + CASES.index(STAGE_CASES[case]))
    xe = torch.from_numpy(x_np.astype(np.float32)).to(torch.bfloat16).to(DEV)
    ye = torch.empty_like(xe)
    capi.gram(xe, gram)
    capi.poly(gram, poly, batch, m, n, *EXACT[1:])
    capi.apply(poly, xe, ye, EXACT[0])
    torch.cuda.synchronize()
    got = ye.view(torch.int16).cpu().numpy().view(np.uint16)
    want = O.f32_to_bf16_bits(y_ref.astype(np.float32))
    assert np.array_equal(got, want)
