"""The 8-wave 192x192 kernels of the symmetric stages (wave pairs; marked ``gpu``).

On a 192x192 tile the 8-wave kernels give each 96x96 wave tile two waves, which split
every K-step's four k16 slices between them and add their halves once after the K
loop.  Each output then sums its K terms in two interleaved chains, so its rounding
differs from the 4-wave kernel's single chain; the checks:

* exact-sum inputs (sparse ±1 X, integer coefficients): every sum is an integer below
  2^24, so A, P and Y equal the oracle's rounding-point emulation bit for bit, with and
  without a stream-K split, after another input went through the same workspace;
* random inputs: the pair kernels agree with the 4-wave kernels to bf16 precision,
  give the same bits on every run, and match the oracle;
* the stage entry points (no workspace, one tile per workgroup) equal the step's
  stages bit for bit when the step is unsplit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
from tests.test_polar_step_gpu import assert_close_kernels, assert_matches_oracle, bits
from tests.test_stream_k_gpu import EXACT_COEFFS, assert_bits_equal, split_in_use

pytestmark = pytest.mark.gpu

DEV = "cuda"
C0 = O.COEFFICIENTS[0]
PAIRS = {"MUON_POLAR_GRAM_TILE": "192", "MUON_POLAR_POLY_TILE": "192", "MUON_POLAR_WAVES": "8"}


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    yield


def _capi():
    from muon_fusion_ascend950_amd import capi

    return capi


def polar_step(x, a, b, c):
    from muon_fusion_ascend950_amd import polar_step as ps

    return ps(x, a, b, c)


def _set(monkeypatch, env):
    for k, v in env.items():
        monkeypatch.setenv(k, v)


def test_pair_kernels_are_selected(monkeypatch):
    """192x192 tiles with 8 waves resolve to the pair kernels (the plan check walks them)."""
    _set(monkeypatch, PAIRS)
    capi = _capi()
    ext = capi.check_plan(1, 4096, 14336, 256)
    for s in (0, 1):
        st = ext.stage[s]
        assert (st.tile_m, st.tile_n, st.waves) == (192, 192, 8)
        assert st.coverage_ok and st.extents_ok


@pytest.mark.parametrize("split", ["1", "0"])
@pytest.mark.parametrize("shape", [(1, 4096, 14336), (2, 768, 8192), (1, 2000, 4040),
                                   (3, 136, 200)])
def test_exact_sums_are_bitwise(monkeypatch, shape, split):
    _set(monkeypatch, PAIRS)
    monkeypatch.setenv("MUON_POLAR_STREAM_K", split)
    capi = _capi()
    batch, m, n = shape
    mats = O.sparse_sign_input(shape, 16, seed=31)
    x = torch.from_numpy(np.stack([xm.toarray() for xm in mats]).astype(np.float32))
    x = x.to(torch.bfloat16).to(DEV)
    y = torch.empty_like(x)
    ws, info = capi.alloc_workspace(batch, m, n)
    print(f"pair exact sums {shape} split={split} split_in_use={split_in_use(*shape)}",
          flush=True)
    capi.step(O.make_input(shape, seed=32).to(DEV), y, ws, *C0)
    capi.step(x, y, ws, *EXACT_COEFFS)
    torch.cuda.synchronize()
    mp, gram_bytes = info.padded_rows, info.gram_bytes
    a_gpu = ws[:gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    p_off = -(-gram_bytes // 256) * 256
    p_gpu = ws[p_off:p_off + gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    for i, xm in enumerate(mats):
        y_ref, max_sum, a_ref, p_ref = O.polar_step_fused_sparse(xm, *EXACT_COEFFS,
                                                                 return_stages=True)
        assert max_sum < 2**24
        a_pad = np.zeros((mp, mp)); a_pad[:m, :m] = a_ref
        p_pad = np.zeros((mp, mp)); p_pad[:m, :m] = p_ref
        assert_bits_equal(bits(a_gpu[i]), O.f32_to_bf16_bits(a_pad.astype(np.float32)), "A")
        assert_bits_equal(bits(p_gpu[i]), O.f32_to_bf16_bits(p_pad.astype(np.float32)), "P")
        assert_bits_equal(bits(y[i]), O.f32_to_bf16_bits(y_ref.astype(np.float32)), "Y")


def test_a_split_is_exercised():
    """(2, 768, 8192) with 192x192 tiles cuts its 20 triangular tiles stream-K style."""
    import os

    saved = {k: os.environ.get(k) for k in PAIRS}
    os.environ.update(PAIRS)
    try:
        assert split_in_use(2, 768, 8192)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (2, 768, 8192), (3, 300, 1000)])
def test_pairs_agree_with_four_waves_and_repeat(monkeypatch, shape):
    _set(monkeypatch, PAIRS)
    x = O.make_input(shape, seed=33).to(DEV)
    first = polar_step(x, *C0)
    again = [polar_step(x, *C0) for _ in range(2)]
    monkeypatch.setenv("MUON_POLAR_WAVES", "4")
    four = polar_step(x, *C0)
    torch.cuda.synchronize()
    for y in again:
        assert torch.equal(first, y)
    assert_close_kernels(first, four)


@pytest.mark.parametrize("shape", [(1, 2000, 4040), (2, 150, 2050)])
def test_pairs_match_oracle(monkeypatch, shape):
    _set(monkeypatch, PAIRS)
    x_cpu = O.make_input(shape, seed=34)
    y = polar_step(x_cpu.to(DEV), *C0)
    torch.cuda.synchronize()
    assert_matches_oracle(y, x_cpu, [C0], rel_exact=1e-2)


@pytest.mark.parametrize("shape", [(1, 1000, 3000), (2, 300, 1000)])
def test_stage_calls_equal_the_unsplit_step(monkeypatch, shape):
    _set(monkeypatch, PAIRS)
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    capi = _capi()
    batch, m, n = shape
    a, b, c = C0
    x = O.make_input(shape, seed=35).to(DEV)
    ws, info = capi.alloc_workspace(batch, m, n)
    y_step = torch.empty_like(x)
    capi.step(x, y_step, ws, a, b, c)
    mp, gram_bytes = info.padded_rows, info.gram_bytes
    p_off = -(-gram_bytes // 256) * 256
    gram = torch.empty(batch, mp, mp, dtype=torch.bfloat16, device=DEV)
    poly = torch.empty_like(gram)
    y = torch.empty_like(x)
    capi.gram(x, gram)
    capi.poly(gram, poly, batch, m, n, b, c)
    capi.apply(poly, x, y, a)
    torch.cuda.synchronize()
    assert torch.equal(gram.view(torch.uint8).reshape(-1), ws[:gram_bytes])
    assert torch.equal(poly.view(torch.uint8).reshape(-1), ws[p_off:p_off + gram_bytes])
    assert torch.equal(y, y_step)


@pytest.mark.parametrize("shape", [(1, 14336, 4096), (2, 1000, 600), (1, 700, 200)])
def test_right_gram_pairs_equal_transposed_path(monkeypatch, shape):
    """The right-Gram form's 192x192 pairs (X columns as the N-contiguous operand, read
    transposed) sum the same products in the same two chains as the left form's pairs
    on the transposed input: unsplit, bit for bit."""
    _set(monkeypatch, PAIRS)
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    x = O.make_input(shape, seed=36).to(DEV)
    print(f"right-Gram pairs {shape}", flush=True)
    y = torch.ops.muon_ascend950.polar_step_tall(x, *C0)
    yt = torch.ops.muon_ascend950.polar_step(x.mT.contiguous(), *C0).mT.contiguous()
    torch.cuda.synchronize()
    assert torch.equal(y, yt)
