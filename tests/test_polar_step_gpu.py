"""GPU parity of the HIP path against the oracle (MI355X only; marked ``gpu``).

Mirrors the reference's own tests (tests/test_polar_step.py:36-53: three one-step
shapes incl. the M > N wrapper and a five-step loop, gate rtol = atol = 6e-2 against
the PyTorch formula) and adds what that gate cannot see (it accepts an all-zero output
at these magnitudes):

* normwise error relF = ‖Y − Y_exact‖_F / ‖Y_exact‖_F against the float64 formula,
  ≤ 1e-2 for one step and ≤ 3e-2 for five steps;
* agreement with the oracle's rounding-point emulation (oracle.polar_step_fused):
  relF ≤ 2e-3 and at most 0.1% of elements more than one bf16 ulp apart;
* the committed golden vectors;
* per-stage checks through the C ABI (A and P bitwise symmetric, zero padding,
  each stage against the oracle applied to the previous GPU stage);
* exact (bitwise) properties at full size: masking == zero padding, the M > N
  wrapper == transposed call, batch == per-matrix calls, run-to-run determinism,
  tile configuration does not change results;
* the large BASELINE shapes against a float32 torch formula on the GPU.
"""

from __future__ import annotations

import os
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O

pytestmark = pytest.mark.gpu

C0 = O.COEFFICIENTS[0]
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden" / "polar_golden.npz"


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    torch.backends.cuda.matmul.allow_tf32 = False
    yield


def polar_step(x, a, b, c):
    from muon_fusion_ascend950_amd import polar_step as ps

    return ps(x, a, b, c)


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu").contiguous().view(torch.int16).numpy().view(np.uint16)


def run_steps(x_cpu, coefficients):
    out = x_cpu.to(DEV)
    for a, b, c in coefficients:
        out = polar_step(out, a, b, c)
    torch.cuda.synchronize()
    return out


def assert_matches_oracle(y: torch.Tensor, x_cpu: torch.Tensor, coefficients, rel_exact: float):
    x64 = O.to_numpy_f64(x_cpu)
    exact, fused = x64, x64
    for a, b, c in coefficients:
        exact = O.wrapper_step(exact, a, b, c, step=O.polar_step_f64)
        fused = O.wrapper_step(fused, a, b, c, step=O.polar_step_fused)
    yn = y.float().cpu().numpy().astype(np.float64)
    assert O.rel_frobenius(yn, exact) <= rel_exact
    assert O.rel_frobenius(yn, fused) <= 2e-3 * len(coefficients)
    if len(coefficients) == 1:
        # element-wise agreement with the rounding-point emulation; after several steps
        # the iteration amplifies rounding differences, so only normwise checks apply
        ulp = O.bf16_ulp_distance(bits(y), O.f32_to_bf16_bits(fused.astype(np.float32)))
        assert (ulp > 1).mean() <= 1e-3


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (8 significant bits)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0**-126)))
    return 2.0 ** (e - 7)


def assert_within_dot_bound(got: np.ndarray, exact: np.ndarray, magnitude: np.ndarray):
    """|got − exact| ≤ ulp_bf16(exact) + 2⁻¹⁶·magnitude, where magnitude is the sum of
    |terms| of each output (fp32 accumulation error is proportional to it; one bf16 ulp
    covers the final rounding, including a flip caused by the accumulation error)."""
    err = np.abs(got - exact)
    bound = bf16_ulp(exact) + 2.0**-16 * magnitude
    worst = np.max(err / bound)
    assert worst <= 1.0, f"error reaches {worst:.2f}x the bound"


# ----------------------------------------------------------------------------- reference tests
@pytest.mark.parametrize("shape", [(129, 130), (2, 150, 2050), (1, 130, 129)])
def test_one_step_matches_reference(shape):
    x = O.make_input(shape, seed=1)
    xd = x.to(DEV)
    expected = O.reference_formula_torch(xd, [C0])  # bf16 on the device, as the reference test
    actual = polar_step(xd, *C0)
    torch.testing.assert_close(actual.float(), expected.float(), rtol=6e-2, atol=6e-2)
    assert actual.shape == x.shape and actual.dtype == torch.bfloat16
    assert_matches_oracle(actual, x, [C0], rel_exact=1e-2)


def test_external_five_step_loop():
    x = O.make_input((1, 129, 130), seed=2)
    xd = x.to(DEV)
    expected = O.reference_formula_torch(xd, O.COEFFICIENTS)
    actual = run_steps(x, O.COEFFICIENTS)
    torch.testing.assert_close(actual.float(), expected.float(), rtol=6e-2, atol=6e-2)
    assert_matches_oracle(actual, x, O.COEFFICIENTS, rel_exact=3e-2)


def test_zero_output_would_fail_the_normwise_gate():
    x = O.make_input((2, 150, 2050), seed=3)
    exact = O.polar_step_f64(O.to_numpy_f64(x), *C0)
    assert O.rel_frobenius(np.zeros_like(exact), exact) > 0.5


# ----------------------------------------------------------------------------- golden vectors
def _golden_cases():
    from tests.golden.make_golden import CASES

    return CASES


@pytest.mark.parametrize("case", _golden_cases(), ids=lambda c: c[0])
def test_golden_vectors(case):
    name, shape, steps, _seed = case
    with np.load(GOLDEN, allow_pickle=False) as data:
        xb = data[f"{name}.x_bits"]
        fused = data[f"{name}.fused_bits"]
        exact = data[f"{name}.exact_f32"].astype(np.float64)
    x = torch.from_numpy(xb.view(np.int16).copy()).view(torch.bfloat16)
    y = run_steps(x, O.COEFFICIENTS[:steps])
    assert y.shape == tuple(shape)
    yn = y.float().cpu().numpy().astype(np.float64)
    assert O.rel_frobenius(yn, exact) <= (1e-2 if steps == 1 else 3e-2)
    fused_f = O.bf16_bits_to_f32(fused).astype(np.float64)
    assert O.rel_frobenius(yn, fused_f) <= 2e-3 * steps
    if steps == 1:
        ulp = O.bf16_ulp_distance(bits(y), fused)
        assert (ulp > 1).mean() <= 1e-3


# ----------------------------------------------------------------------------- edge shapes
@pytest.mark.parametrize("shape", [(1, 1), (1, 17), (3, 5), (5, 3), (64, 64), (257, 257),
                                   (2, 65, 200), (300, 701), (3, 200, 136), (1, 513, 520),
                                   (2, 1, 4096)])
def test_edge_shapes(shape):
    x = O.make_input(shape, seed=4)
    y = run_steps(x, [C0])
    assert y.shape == x.shape
    assert torch.isfinite(y.float()).all()
    assert_matches_oracle(y, x, [C0], rel_exact=1e-2)


@pytest.mark.parametrize("shape", [(512, 16, 64), (64, 128, 128), (1, 8, 131072), (2, 3, 40000),
                                   (1, 65536, 8), (3, 20000, 24)])
def test_extreme_aspect_and_batch(shape):
    """Many tiny matrices (a grid of thousands of workgroups), and very wide or very tall
    skinny matrices: one tile per side with a K loop of hundreds or thousands of steps,
    which the stream-K split cuts over many workgroups (the right-Gram form for the tall
    ones)."""
    print(f"extreme {shape}", flush=True)
    x = O.make_input(shape, seed=5)
    y = run_steps(x, [C0])
    assert y.shape == x.shape
    assert torch.isfinite(y.float()).all()
    assert_matches_oracle(y, x, [C0], rel_exact=1e-2)


# ----------------------------------------------------------------------------- stages via the C ABI
def _stages(x3: torch.Tensor, b: float, c: float):
    from muon_fusion_ascend950_amd import capi

    batch, m, n = x3.shape
    info = capi.query(batch, m, n)
    mp = info.padded_rows
    gram = torch.empty(batch, mp, mp, dtype=torch.bfloat16, device=DEV)
    poly = torch.empty_like(gram)
    capi.gram(x3, gram)
    capi.poly(gram, poly, batch, m, n, b, c)
    torch.cuda.synchronize()
    return gram, poly, mp


@pytest.mark.parametrize("shape", [(2, 150, 2050), (1, 129, 130), (8, 512, 2048), (1, 300, 701),
                                   (2, 300, 1000)])
def test_stages_against_oracle(shape):
    from muon_fusion_ascend950_amd import capi

    a, b, c = C0
    x = O.make_input(shape, seed=5)
    xd = x.to(DEV)
    gram, poly, mp = _stages(xd, b, c)
    batch, m, n = shape
    gb, pb = bits(gram), bits(poly)
    # bitwise symmetric, exact zero padding
    assert np.array_equal(gb, np.swapaxes(gb, -1, -2))
    assert np.array_equal(pb, np.swapaxes(pb, -1, -2))
    g = gram.float().cpu().numpy().astype(np.float64)
    p = poly.float().cpu().numpy().astype(np.float64)
    assert not g[:, m:, :].any() and not g[:, :, m:].any()
    assert not p[:, m:, :].any() and not p[:, :, m:].any()
    x64 = O.to_numpy_f64(x)
    ax = np.abs(x64)
    # stage 1 vs exact X·Xᵀ
    g_exact = O.gram_f64(x64)
    assert_within_dot_bound(g[:, :m, :m], g_exact, ax @ np.swapaxes(ax, -1, -2))
    ug = O.bf16_ulp_distance(gb[:, :m, :m], O.f32_to_bf16_bits(g_exact.astype(np.float32)))
    assert (ug > 1).mean() < 5e-3
    # stage 2 vs exact b·A + c·A·A on the GPU's A (b, c as fp32)
    b32, c32 = float(np.float32(b)), float(np.float32(c))
    g32 = g[:, :m, :m]
    p_exact = b32 * g32 + c32 * (g32 @ g32)
    ag = np.abs(g32)
    assert_within_dot_bound(p[:, :m, :m], p_exact, abs(b32) * ag + abs(c32) * (ag @ ag))
    # stage 3 vs exact a·X + P·X on the GPU's P
    y = torch.empty_like(xd)
    capi.apply(poly, xd, y, a)
    torch.cuda.synchronize()
    a32 = float(np.float32(a))
    y_exact = a32 * x64 + p[:, :m, :m] @ x64
    yn = y.float().cpu().numpy().astype(np.float64)
    assert_within_dot_bound(yn, y_exact, abs(a32) * ax + np.abs(p[:, :m, :m]) @ ax)
    uy = O.bf16_ulp_distance(bits(y), O.f32_to_bf16_bits(y_exact.astype(np.float32)))
    assert (uy > 1).mean() < 5e-3
    # whole step through the C ABI equals the torch op, bit for bit, and the three
    # stage calls given the same workspace (same stream-K split, if any); without
    # a workspace the stages run unsplit, equal to fp32 rounding
    ws, _info = capi.alloc_workspace(batch, m, n)
    y2 = torch.empty_like(xd)
    capi.step(xd, y2, ws, a, b, c)
    y3 = polar_step(xd, a, b, c)
    g_ws = torch.empty_like(gram)
    p_ws = torch.empty_like(poly)
    y4 = torch.empty_like(xd)
    capi.gram(xd, g_ws, workspace=ws)
    capi.poly(g_ws, p_ws, batch, m, n, b, c, workspace=ws)
    capi.apply(p_ws, xd, y4, a, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y2, y3) and torch.equal(y2, y4)
    assert_close_kernels(y, y2)


def test_gram_special_cases():
    # orthonormal rows -> A = I (up to bf16 rounding of the input); [D 0] -> D²
    q, _ = torch.linalg.qr(torch.randn(512, 128, dtype=torch.float64, generator=torch.Generator().manual_seed(0)))
    x = q.T.contiguous().to(torch.bfloat16).unsqueeze(0).to(DEV)  # [1, 128, 512]
    gram, _poly, _mp = _stages(x, 0.0, 0.0)
    eye = torch.eye(128, dtype=torch.float32)
    assert (gram[0, :128, :128].float().cpu() - eye).abs().max() < 2e-2
    d = torch.tensor([0.5, -2.0, 3.0, 0.25], dtype=torch.bfloat16)
    x = torch.zeros(1, 4, 40, dtype=torch.bfloat16)
    x[0, :, :4] = torch.diag(d)
    gram, poly, _ = _stages(x.to(DEV), 1.5, -0.5)
    want = torch.diag(d.float() ** 2)
    assert torch.equal(gram[0, :4, :4].float().cpu(), want)
    dd = d.float() ** 2
    assert torch.allclose(poly[0, :4, :4].float().cpu(), torch.diag(1.5 * dd - 0.5 * dd * dd), rtol=1e-2)


def test_apply_special_cases():
    from muon_fusion_ascend950_amd import capi

    a = C0[0]
    x = O.make_input((1, 100, 300), seed=6).to(DEV)
    info = capi.query(1, 100, 300)
    mp = info.padded_rows
    y = torch.empty_like(x)
    zero = torch.zeros(1, mp, mp, dtype=torch.bfloat16, device=DEV)
    capi.apply(zero, x, y, a)
    torch.cuda.synchronize()
    # with P = 0 the kernel's sums are a·X alone: one fp32 product (an fma into a
    # zero accumulator inside the K loop) rounded once, as torch rounds the fp32
    # product (distance 0 treats a signed zero as equal to zero)
    want = (x.float() * np.float32(a)).to(torch.bfloat16)
    assert O.bf16_ulp_distance(bits(y), bits(want)).max() == 0
    eye = torch.zeros_like(zero)
    eye[0, :100, :100] = torch.eye(100, dtype=torch.bfloat16, device=DEV)
    capi.apply(eye, x, y, 1.0)
    torch.cuda.synchronize()
    assert torch.equal(y, (2.0 * x.float()).to(torch.bfloat16))


# ----------------------------------------------------------------------------- exact properties
def assert_close_kernels(a: torch.Tensor, b: torch.Tensor):
    """Two kernel paths with different (equally valid) rounding points: normwise
    agreement to bf16 precision and almost all elements within one bf16 ulp."""
    an, bn = a.float().cpu().numpy().astype(np.float64), b.float().cpu().numpy().astype(np.float64)
    assert O.rel_frobenius(an, bn) <= 2e-3
    assert (O.bf16_ulp_distance(bits(a), bits(b)) > 1).mean() <= 2e-3


@pytest.mark.parametrize("shape", [(2, 150, 2050), (1, 129, 130), (3, 300, 701), (2, 100, 512)])
def test_masking_equals_zero_padding(monkeypatch, shape):
    """Reference binding pads to 128/16 and crops (binding.cpp:630-672); masking must
    give the same numbers, bit for bit: rows of n % 8 != 0 elements reach the same
    DMA-fed kernels through a zero-padded copy, and the register-staged family
    (MUON_POLAR_STREAM=0) masks element-wise.  (Unsplit kernels: a stream-K split
    depends on the tile count, which padding changes.)"""
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    x = O.make_input(shape, seed=7).to(DEV)
    batch, m, n = shape
    rows = -(-m // 128) * 128
    cols = max(-(-n // 16) * 16, rows)
    padded = torch.zeros(batch, rows, cols, dtype=torch.bfloat16, device=DEV)
    padded[:, :m, :n] = x
    y = polar_step(x, *C0)
    yp = polar_step(padded, *C0)[:, :m, :n]
    torch.cuda.synchronize()
    assert torch.equal(y, yp)
    monkeypatch.setenv("MUON_POLAR_STREAM", "0")
    ys = polar_step(x, *C0)
    yps = polar_step(padded, *C0)[:, :m, :n]
    torch.cuda.synchronize()
    assert torch.equal(ys, yps)


@pytest.mark.parametrize("shape", [(2, 300, 1000), (2, 1500, 3000), (1, 700, 5000), (3, 200, 136),
                                   (2, 40, 56), (1, 8, 8), (1, 129, 130), (2, 150, 2050),
                                   (3, 100, 1002), (1, 1000, 3002), (2, 40, 58)])
@pytest.mark.parametrize("split", ["1", "0"])
def test_rows_read_in_place_equal_a_zero_padded_copy(monkeypatch, shape, split):
    """n % 8 == 0, n % 64 != 0: gram reads X in place and masks the chunks of its
    last K-step past n (no padded copy).  A zero-padded input of roundup(n, 64)
    columns has the same tiles and K-steps, so the same plan (split or not): Y must
    equal its first n columns bit for bit.  Shapes: unsplit, split 128x128 and 64x64
    gram (with stream-K segments that hold the last K-step alone), n < 64 (the only
    K-step masked); and rows of n % 8 != 0 elements (the odd-width BASELINE
    configurations among them), which go through the step's own padded copy and
    must give the same bits as the caller's; m <= n throughout."""
    monkeypatch.setenv("MUON_POLAR_STREAM_K", split)
    batch, m, n = shape
    xc = O.make_input(shape, seed=31)
    x = xc.to(DEV)
    np_ = -(-n // 64) * 64
    padded = torch.zeros(batch, m, np_, dtype=torch.bfloat16, device=DEV)
    padded[:, :, :n] = x
    y = polar_step(x, *C0)
    yp = polar_step(padded, *C0)[:, :, :n]
    torch.cuda.synchronize()
    print(f"in-place rows {shape} split={split}", flush=True)
    assert torch.equal(y, yp)
    assert_matches_oracle(y, xc, [C0], 1e-2)


@pytest.mark.parametrize("shape", [(3, 700, 200), (1, 4100, 1000), (2, 130, 72)])
def test_tall_rows_read_in_place_equal_a_zero_padded_copy(monkeypatch, shape):
    """m > n, n % 8 == 0, n % 64 != 0: apply-right reads X rows in place with the
    last K-step masked; against X padded with zero columns to roundup(n, 64)
    (unsplit: padding changes the Gram's tile count, and unsplit results do not
    depend on the tiling), Y's first n columns are equal bit for bit."""
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    batch, m, n = shape
    x = O.make_input(shape, seed=32).to(DEV)
    np_ = -(-n // 64) * 64
    padded = torch.zeros(batch, m, np_, dtype=torch.bfloat16, device=DEV)
    padded[:, :, :n] = x
    y = polar_step(x, *C0)
    yp = polar_step(padded, *C0)[:, :, :n]
    torch.cuda.synchronize()
    print(f"in-place tall rows {shape}", flush=True)
    assert torch.equal(y, yp)


@pytest.mark.parametrize("shape", [(130, 129), (2, 700, 300), (2050, 150)])
def test_wrapper_transpose_is_exact(shape):
    x = O.make_input(shape, seed=8).to(DEV)
    y = polar_step(x, *C0)
    yt = polar_step(x.mT.contiguous(), *C0).mT
    torch.cuda.synchronize()
    assert y.shape == x.shape and torch.equal(y, yt)


def test_batch_equals_per_matrix_and_is_deterministic():
    x = O.make_input((4, 200, 520), seed=9).to(DEV)
    y = polar_step(x, *C0)
    for i in range(4):
        assert torch.equal(y[i], polar_step(x[i], *C0))
    assert torch.equal(y, polar_step(x, *C0))


@pytest.mark.parametrize("shape", [(1, 512, 8192), (2, 256, 4096), (8, 512, 2048)])
def test_misaligned_contiguous_input_takes_the_aligned_route(shape):
    """A contiguous X at an odd address (buf[1:].view(...)): the op copies it to an
    aligned buffer, so it runs the DMA-fed kernels and their stream-K split like an
    aligned input, bit for bit (the register-staged kernels would sum the split
    shapes' K terms in another order)."""
    b, m, n = shape
    x = O.make_input(shape, seed=12).to(DEV)
    buf = torch.empty(b * m * n + 1, dtype=torch.bfloat16, device=DEV)
    buf[1:].copy_(x.reshape(-1))
    xm = buf[1:].view(b, m, n)
    assert xm.is_contiguous() and xm.data_ptr() % 16 != 0
    assert torch.equal(polar_step(xm, *C0), polar_step(x, *C0))
    from muon_fusion_ascend950_amd import polar_express

    assert torch.equal(polar_express(xm, O.COEFFICIENTS[:2]), polar_express(x, O.COEFFICIENTS[:2]))
    assert torch.equal(xm, x)  # the input is read only


def test_noncontiguous_input():
    base = O.make_input((2, 300, 200), seed=10).to(DEV)
    x = base.transpose(1, 2)  # [2, 200, 300] non-contiguous
    assert torch.equal(polar_step(x, *C0), polar_step(x.contiguous(), *C0))


@pytest.mark.parametrize("stream", ["1", "0"])
@pytest.mark.parametrize("env", [
    {"MUON_POLAR_GRAM_TILE": "64", "MUON_POLAR_POLY_TILE": "64", "MUON_POLAR_APPLY_TILE_M": "64"},
    {"MUON_POLAR_GRAM_TILE": "128", "MUON_POLAR_APPLY_TILE_M": "128"},
    {"MUON_POLAR_GRAM_TILE": "256", "MUON_POLAR_POLY_TILE": "128", "MUON_POLAR_APPLY_TILE_M": "256",
     "MUON_POLAR_APPLY_TILE_N": "128"},
    {"MUON_POLAR_APPLY_TILE_M": "128", "MUON_POLAR_APPLY_TILE_N": "256"},
    {"MUON_POLAR_GRAM_TILE": "192", "MUON_POLAR_POLY_TILE": "192", "MUON_POLAR_PAIR": "0"},
    {"MUON_POLAR_GRAM_TILE": "256", "MUON_POLAR_APPLY_TILE_M": "256", "MUON_POLAR_WAVES": "8"},
    {"MUON_POLAR_GRAM_TILE": "128", "MUON_POLAR_POLY_TILE": "128", "MUON_POLAR_APPLY_TILE_M": "128",
     "MUON_POLAR_WAVES": "4"},
    {"MUON_POLAR_GRAM_TILE": "128", "MUON_POLAR_POLY_TILE": "128", "MUON_POLAR_APPLY_TILE_M": "128",
     "MUON_POLAR_WAVES": "8", "MUON_POLAR_GRAM_DEPTH": "4", "MUON_POLAR_POLY_DEPTH": "4",
     "MUON_POLAR_APPLY_DEPTH": "4"},
    {"MUON_POLAR_GRAM_TILE": "192", "MUON_POLAR_POLY_TILE": "256", "MUON_POLAR_PAIR": "0"},
    {"MUON_POLAR_GRAM_TILE": "128", "MUON_POLAR_POLY_TILE": "192", "MUON_POLAR_APPLY_TILE_M": "256",
     "MUON_POLAR_APPLY_TILE_N": "128", "MUON_POLAR_PAIR": "0"},
])
def test_tile_configuration_does_not_change_results(monkeypatch, stream, env):
    """Every tile shape accumulates each output in the same K order, so results are
    bit-identical across tile configurations of one kernel family (unsplit: a
    stream-K split cuts K where the tile count puts it).  192x192 tiles with 8 waves
    (wave pairs, two interleaved K chains per output) round differently and are
    checked in test_pair_gpu.py; here they run with 4 waves (MUON_POLAR_PAIR=0)."""
    monkeypatch.setenv("MUON_POLAR_STREAM", stream)
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    x = O.make_input((2, 300, 1000), seed=11).to(DEV)
    base = polar_step(x, *C0)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    other = polar_step(x, *C0)
    torch.cuda.synchronize()
    assert torch.equal(base, other)


@pytest.mark.parametrize("tiles", [(256, 192), (192, 256), (64, 192), (128, 64)])
@pytest.mark.parametrize("stream", ["1", "0"])
@pytest.mark.parametrize("shape", [(2, 300, 1000), (1, 136, 200)])
def test_unequal_symmetric_tiles_pad_with_zeros(monkeypatch, tiles, stream, shape):
    """A and P are [mp, mp] with mp the larger of the gram and poly tile extents; the
    stage with the smaller tile writes zeros past its tile grid.  Buffers filled with
    NaN bits first: the padding must come back as exact zeros, and A, P and Y equal
    those of equal tiles bit for bit (unsplit, both kernel families)."""
    from muon_fusion_ascend950_amd import capi

    a, b, c = C0
    batch, m, n = shape
    monkeypatch.setenv("MUON_POLAR_STREAM", stream)
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    monkeypatch.setenv("MUON_POLAR_PAIR", "0")  # one K chain per output at every tile size
    x = O.make_input(shape, seed=26).to(DEV)

    def stages():
        mp = capi.query(batch, m, n).padded_rows
        gram = torch.full((batch, mp, mp), float("nan"), dtype=torch.bfloat16, device=DEV)
        poly = torch.full_like(gram, float("nan"))
        y = torch.full_like(x, float("nan"))
        capi.gram(x, gram)
        capi.poly(gram, poly, batch, m, n, b, c)
        capi.apply(poly, x, y, a)
        torch.cuda.synchronize()
        return gram, poly, y, mp

    g0, p0, y0, _ = stages()
    monkeypatch.setenv("MUON_POLAR_GRAM_TILE", str(tiles[0]))
    monkeypatch.setenv("MUON_POLAR_POLY_TILE", str(tiles[1]))
    g1, p1, y1, mp = stages()
    ext = [-(-m // t) * t for t in tiles]
    print(f"tiles {tiles} stream {stream} shape {shape}: mp {mp}, extents {ext}", flush=True)
    assert mp == max(ext)
    for t1, t0 in ((g1, g0), (p1, p0)):
        assert torch.equal(t1[:, :m, :m], t0[:, :m, :m])
        assert bits(t1[:, m:, :]).max(initial=0) == 0 and bits(t1[:, :, m:]).max(initial=0) == 0
    assert torch.equal(y1, y0)


@pytest.mark.parametrize("env", [
    {"MUON_POLAR_GRAM_TILE": "64", "MUON_POLAR_POLY_TILE": "64", "MUON_POLAR_APPLY_TILE_M": "64",
     "MUON_POLAR_GRAM_DEPTH": "4", "MUON_POLAR_POLY_DEPTH": "8", "MUON_POLAR_APPLY_DEPTH": "2"},
    {"MUON_POLAR_GRAM_TILE": "64", "MUON_POLAR_POLY_TILE": "64", "MUON_POLAR_APPLY_TILE_M": "64",
     "MUON_POLAR_GRAM_DEPTH": "8", "MUON_POLAR_POLY_DEPTH": "2", "MUON_POLAR_APPLY_DEPTH": "4"},
    {"MUON_POLAR_GRAM_TILE": "128", "MUON_POLAR_APPLY_TILE_M": "128",
     "MUON_POLAR_GRAM_DEPTH": "4", "MUON_POLAR_POLY_DEPTH": "4", "MUON_POLAR_APPLY_DEPTH": "4"},
    {"MUON_POLAR_APPLY_TILE_M": "256", "MUON_POLAR_APPLY_TILE_N": "128", "MUON_POLAR_APPLY_DEPTH": "3"},
    {"MUON_POLAR_APPLY_TILE_M": "128", "MUON_POLAR_APPLY_TILE_N": "256", "MUON_POLAR_APPLY_DEPTH": "3"},
])
@pytest.mark.parametrize("shape", [(2, 300, 1000), (3, 100, 333)])
def test_ring_depth_does_not_change_results(monkeypatch, env, shape):
    """The LDS ring depth changes how many panels are in flight, not what is summed or in
    which order: results are bit-identical to the default depth (unsplit), including the
    4-slot epilogue-tile prefetch of the poly stage and the padded route of odd widths."""
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    x = O.make_input(shape, seed=21).to(DEV)
    base = polar_step(x, *C0)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    other = polar_step(x, *C0)
    torch.cuda.synchronize()
    assert torch.equal(base, other)


@pytest.mark.parametrize("shape,tile", [((1, 2000, 2048), "128"), ((2, 1100, 1536), "64"),
                                        ((1, 1300, 1536), "256")])
def test_tile_walk_does_not_change_results(monkeypatch, shape, tile):
    """The triangular stages walk their upper tiles row by row or in super-blocks of
    MUON_POLAR_SYM_GROUP x MUON_POLAR_SYM_GROUP tiles (ragged at the grid's edge): which
    workgroup computes a tile changes, not the tile's sums, so unsplit results are
    bit-identical for every block side, and any tile skipped or computed twice would show.
    16 to 18 tiles per side, so that blocks of 3, 5 and 8 leave ragged edge blocks."""
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    monkeypatch.setenv("MUON_POLAR_GRAM_TILE", tile)
    x = O.make_input(shape, seed=24).to(DEV)
    monkeypatch.setenv("MUON_POLAR_SYM_GROUP", "1")
    base = polar_step(x, *C0)
    for side in ("2", "3", "5", "8", "64"):
        monkeypatch.setenv("MUON_POLAR_SYM_GROUP", side)
        other = polar_step(x, *C0)
        torch.cuda.synchronize()
        assert torch.equal(base, other), f"block side {side}"


def test_ring_depth_rejects_missing_kernel(monkeypatch):
    monkeypatch.setenv("MUON_POLAR_GRAM_TILE", "256")
    monkeypatch.setenv("MUON_POLAR_GRAM_DEPTH", "4")
    x = O.make_input((1, 300, 1000), seed=22).to(DEV)
    with pytest.raises(RuntimeError, match="DEPTH"):
        polar_step(x, *C0)


@pytest.mark.parametrize("offset", [1, 2])
@pytest.mark.parametrize("shape", [(1, 256, 1024), (2, 150, 2050), (1, 129, 130), (3, 129, 257),
                                   (2, 200, 1001)])
def test_unaligned_output_pointer(shape, offset):
    """Y at an address that is not 16-byte aligned (a view `offset` elements into a
    buffer): at 2 bytes past a 16-byte boundary the DMA-fed apply kernel stores 2 bytes
    at a time; at 4 bytes past it, rows of an even number of elements take 16-byte stores
    at 4-byte aligned addresses inside the row and element stores for the chunk that
    ends it, and rows of an odd number do so on the rows whose start is 4-byte aligned
    (every other row; with an odd row count the pattern flips from one matrix of the
    batch to the next).  Either way the same bits as an aligned Y, and nothing written
    outside it."""
    from muon_fusion_ascend950_amd import capi

    a, b, c = C0
    x = O.make_input(shape, seed=23).to(DEV)
    ws, _ = capi.alloc_workspace(*shape)
    y = torch.empty_like(x)
    capi.step(x, y, ws, a, b, c)
    flat = torch.full((x.numel() + offset + 8,), float("nan"), dtype=torch.bfloat16, device=DEV)
    y_off = flat[offset:offset + x.numel()].view(x.shape)
    assert y_off.data_ptr() % 16 == 2 * offset
    capi.step(x, y_off, ws, a, b, c)
    torch.cuda.synchronize()
    assert torch.equal(y, y_off)
    assert torch.isnan(flat[:offset]).all()  # nothing written before the view
    assert torch.isnan(flat[offset + x.numel():]).all()  # nor after it


@pytest.mark.parametrize("shape", [(8, 512, 2048), (1, 1000, 3000), (3, 200, 264), (2, 64, 4096),
                                   (2, 300, 1001), (1, 130, 4099)])
def test_streaming_and_staged_kernels_agree(monkeypatch, shape):
    """DMA-fed kernels (a·X fma'd into the accumulators inside the K loop, stream-K
    splits, wave pairs) and register-staged kernels (a·X in the epilogue, one
    summation chain) agree to bf16 precision, and each matches the oracle."""
    x_cpu = O.make_input(shape, seed=14)
    x = x_cpu.to(DEV)
    fast = polar_step(x, *C0)
    monkeypatch.setenv("MUON_POLAR_STREAM", "0")
    staged = polar_step(x, *C0)
    torch.cuda.synchronize()
    assert_close_kernels(fast, staged)
    assert_matches_oracle(fast, x_cpu, [C0], rel_exact=1e-2)
    assert_matches_oracle(staged, x_cpu, [C0], rel_exact=1e-2)


def test_debug_sync_mode(monkeypatch):
    monkeypatch.setenv("MUON_POLAR_DEBUG_SYNC", "0")  # presence enables it, as in the reference
    x = O.make_input((2, 150, 2050), seed=12).to(DEV)
    y = polar_step(x, *C0)
    monkeypatch.delenv("MUON_POLAR_DEBUG_SYNC")
    assert torch.equal(y, polar_step(x, *C0))


def test_op_rejects_m_greater_than_n():
    x = torch.zeros(1, 9, 8, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="M <= N"):
        torch.ops.muon_ascend950.polar_step(x, *C0)


def test_runs_on_current_stream():
    x = O.make_input((8, 512, 2048), seed=13).to(DEV)
    ref = polar_step(x, *C0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        y = polar_step(x, *C0)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(ref, y)


# ----------------------------------------------------------------------------- BASELINE shapes
def _fp32_formula(x: torch.Tensor, coefficients) -> torch.Tensor:
    return O.reference_formula_torch(x.float(), coefficients)


@pytest.mark.parametrize("shape,steps", [((8, 512, 2048), 1), ((8, 512, 2048), 5),
                                         ((4096, 14336), 1), ((14336, 4096), 1),
                                         ((4, 4096, 4096), 1), ((4096, 14336), 5),
                                         ((4, 4096, 4096), 5), ((14336, 4096), 5)])
def test_baseline_shapes(shape, steps):
    """Every BASELINE.json workload on its default route (stream-K split on: the large
    shapes cut their last round), against the fp32 formula with the reference's 6e-2
    gate (tests/test_polar_step.py:42,53) and the normwise bound."""
    print(f"baseline {shape} x{steps}", flush=True)
    x = O.make_input(shape, seed=0).to(DEV)
    coeffs = O.COEFFICIENTS[:steps]
    y = x
    for a, b, c in coeffs:
        y = polar_step(y, a, b, c)
    ref32 = _fp32_formula(x, coeffs)
    torch.testing.assert_close(y.float(), ref32, rtol=6e-2, atol=6e-2)
    rel = ((y.float() - ref32).norm() / ref32.norm()).item()
    assert rel <= (1e-2 if steps == 1 else 3e-2), rel
    if steps == 1 and tuple(shape) == (8, 512, 2048):
        # the reference's bf16 formula passes the same gate
        ref16 = O.reference_formula_torch(x, coeffs)
        torch.testing.assert_close(y.float(), ref16.float(), rtol=6e-2, atol=6e-2)


@pytest.mark.parametrize("shape", [(8192, 16384), (2, 6144, 8192)])
def test_beyond_baseline_shapes(shape):
    """Larger than any BASELINE shape: the triangular stages run several full rounds of
    256x256 tiles (528 and 2 x 300 upper tiles on 256 CUs) before a stream-K remainder,
    which the BASELINE shapes (a partial first round) never exercise.  Against the fp32
    formula, with the north star's 6e-2 gate and the 1e-2 normwise bound of one step."""
    print(f"beyond baseline {shape}", flush=True)
    x = O.make_input(shape, seed=6).to(DEV)
    y = polar_step(x, *C0)
    ref32 = _fp32_formula(x, [C0])
    torch.testing.assert_close(y.float(), ref32, rtol=6e-2, atol=6e-2)
    rel = ((y.float() - ref32).norm() / ref32.norm()).item()
    assert rel <= 1e-2, rel


@pytest.mark.parametrize("shape", [(4, 1344, 5200), (1, 1504, 10000), (1, 12352, 1536)])
def test_long_k_gram_tile_rules(shape):
    """Shapes whose gram takes the long-K tile rules (256x256 tiles from A side 1281
    with 80+ K-steps; 128x128 tiles where 64x64 units outnumber the CUs at 128+
    K-steps, wide and right-Gram forms), both cut by stream-K: against the oracle's
    float64 step and its rounding-point emulation, element by element."""
    print(f"long-K gram rule {shape}", flush=True)
    x = O.make_input(shape, seed=7)
    y = run_steps(x, [C0])
    assert_matches_oracle(y, x, [C0], rel_exact=1e-2)


def test_svd_property_at_size():
    """One step maps singular values σ -> aσ + bσ³ + cσ⁵ (size-independent check)."""
    gen = torch.Generator().manual_seed(1)
    m, n = 512, 2048
    u, _ = torch.linalg.qr(torch.randn(m, m, dtype=torch.float64, generator=gen))
    v, _ = torch.linalg.qr(torch.randn(n, m, dtype=torch.float64, generator=gen))
    sigma = torch.linspace(0.05, 1.0, m, dtype=torch.float64)
    x = ((u * sigma) @ v.T).to(torch.bfloat16)
    y = polar_step(x.to(DEV), *C0).double().cpu()
    s_in = torch.linalg.svdvals(x.double())
    s_out = torch.linalg.svdvals(y)
    want = torch.from_numpy(O.scalar_polynomial(s_in.numpy(), [C0]))
    want, _ = torch.sort(want.abs(), descending=True)
    assert (s_out - want).abs().max() < 3e-2
