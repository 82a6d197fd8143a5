"""Diagonal pairs of the triangular stages (marked ``gpu``).

Where pairing the diagonal 64x64 tiles takes fewer rounds of one workgroup per CU,
gram and poly run each matrix's off-diagonal tiles and then pairs of diagonal tiles,
one pair per workgroup: the pair reads the two panels an off-diagonal tile reads and
computes each diagonal tile from its own panel ([8,512,2048]: 288 tiles -> 256
units, one per CU).  The two waves of a diagonal tile split the K-slices of its
block (0,1), which then sums in two interleaved chains, so the checks are:

* the plans pick the pairs (left form, right-Gram form, an odd tile count that
  leaves a last diagonal tile alone, a padded extent);
* exact-sum inputs (sparse ±1 X, integer coefficients): A, P and Y equal the
  oracle's rounding-point emulation bit for bit, after a NaN-filled workspace (every
  element of A and P written);
* random inputs: A's off-diagonal tiles equal those of MUON_POLAR_DIAG_PAIRS=0 bit
  for bit (the same units), A, P and Y agree with them to bf16 precision, every run
  gives the same bits, the stage entry points (no workspace) equal the step's
  stages, and Y matches the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
from tests.test_polar_step_gpu import assert_close_kernels, assert_matches_oracle, bits
from tests.test_stream_k_gpu import EXACT_COEFFS, assert_bits_equal

pytestmark = pytest.mark.gpu

DEV = "cuda"
C0 = O.COEFFICIENTS[0]
SHAPES = [(8, 512, 2048), (8, 2048, 512), (10, 440, 1024), (10, 1024, 440)]


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    yield


def _capi():
    from muon_fusion_ascend950_amd import capi

    return capi


def _cus() -> int:
    return torch.cuda.get_device_properties(0).multi_processor_count


def _stages(ws, info, batch):
    """A and P as the step left them in its workspace."""
    mp, gram_bytes = info.padded_rows, info.gram_bytes
    p_off = -(-gram_bytes // 256) * 256
    a = ws[:gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    p = ws[p_off:p_off + gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    return a, p


@pytest.mark.parametrize("shape", SHAPES)
def test_plans_use_diagonal_pairs(shape):
    capi = _capi()
    # -1: the resident workgroups per CU this device reports for each kernel
    plan = capi.check_plan(*shape, cus=_cus(), blocks_per_cu=(-1, -1, -1))
    for s in (0, 1):
        e = plan.stage[s]
        print(f"{shape} stage {s}: units {e.total_tiles} diag_pairs {e.diag_pairs}", flush=True)
        assert e.diag_pairs == 1 and e.sk_units == 0
        assert e.coverage_ok == 1 and e.extents_ok == 1


@pytest.mark.parametrize("shape", SHAPES)
def test_exact_sums_are_bitwise(shape):
    capi = _capi()
    batch, m, n = shape
    tall = m > n
    mats = O.sparse_sign_input(shape, 16, seed=51)
    x = torch.from_numpy(np.stack([xm.toarray() for xm in mats]).astype(np.float32))
    x = x.to(torch.bfloat16).to(DEV)
    y = torch.empty_like(x)
    ws, info = capi.alloc_workspace(batch, m, n)
    ws.fill_(0xFF)  # NaN bf16s: an element of A or P left unwritten shows
    print(f"diag pairs exact sums {shape}", flush=True)
    capi.step(x, y, ws, *EXACT_COEFFS)
    torch.cuda.synchronize()
    a_gpu, p_gpu = _stages(ws, info, batch)
    s = min(m, n)
    mp = info.padded_rows
    for i, xm in enumerate(mats):
        # m > n: the oracle's left form on Xᵀ (its A is XᵀX, its Y is Yᵀ)
        y_ref, max_sum, a_ref, p_ref = O.polar_step_fused_sparse(
            xm.T.tocsr() if tall else xm, *EXACT_COEFFS, return_stages=True)
        assert max_sum < 2**24
        a_pad = np.zeros((mp, mp)); a_pad[:s, :s] = a_ref
        p_pad = np.zeros((mp, mp)); p_pad[:s, :s] = p_ref
        assert_bits_equal(bits(a_gpu[i]), O.f32_to_bf16_bits(a_pad.astype(np.float32)), "A")
        assert_bits_equal(bits(p_gpu[i]), O.f32_to_bf16_bits(p_pad.astype(np.float32)), "P")
        want = O.f32_to_bf16_bits((y_ref.T if tall else y_ref).astype(np.float32))
        assert_bits_equal(bits(y[i]), want, "Y")


@pytest.mark.parametrize("shape", SHAPES)
def test_pairs_agree_with_single_tiles(monkeypatch, shape):
    capi = _capi()
    batch, m, n = shape
    x = O.make_input(shape, seed=52).to(DEV)
    ws, info = capi.alloc_workspace(batch, m, n)
    y = torch.empty_like(x)
    print(f"diag pairs vs single tiles {shape}", flush=True)
    capi.step(x, y, ws, *C0)
    a, p = (t.clone() for t in _stages(ws, info, batch))
    y_again = torch.empty_like(x)
    capi.step(x, y_again, ws, *C0)
    monkeypatch.setenv("MUON_POLAR_DIAG_PAIRS", "0")
    plan = capi.check_plan(*shape, cus=_cus(), blocks_per_cu=(2, 2, 2))
    assert plan.stage[0].diag_pairs == 0
    ws2, info2 = capi.alloc_workspace(batch, m, n)
    assert info2.padded_rows == info.padded_rows
    y2 = torch.empty_like(x)
    capi.step(x, y2, ws2, *C0)
    a2, p2 = _stages(ws2, info2, batch)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_again.view(torch.int16))
    # off-diagonal 64x64 tiles of A: the same units, bit for bit
    mp = info.padded_rows
    tile = torch.arange(mp, device=DEV) // 64
    off = (tile[:, None] != tile[None, :]).expand(batch, mp, mp)
    assert torch.equal(a.view(torch.int16)[off], a2.view(torch.int16)[off])
    assert_close_kernels(a, a2)
    assert_close_kernels(p, p2)
    assert_close_kernels(y, y2)


@pytest.mark.parametrize("shape", [(8, 512, 2048), (10, 440, 1024)])
def test_stage_calls_equal_the_step(shape):
    """The stage entry points (no workspace) run the same units."""
    capi = _capi()
    batch, m, n = shape
    a, b, c = C0
    x = O.make_input(shape, seed=53).to(DEV)
    ws, info = capi.alloc_workspace(batch, m, n)
    y_step = torch.empty_like(x)
    capi.step(x, y_step, ws, a, b, c)
    mp = info.padded_rows
    gram = torch.full((batch, mp, mp), float("nan"), dtype=torch.bfloat16, device=DEV)
    poly = torch.full_like(gram, float("nan"))
    y = torch.empty_like(x)
    capi.gram(x, gram)
    capi.poly(gram, poly, batch, m, n, b, c)
    capi.apply(poly, x, y, a)
    torch.cuda.synchronize()
    a_ws, p_ws = _stages(ws, info, batch)
    assert torch.equal(gram.view(torch.int16), a_ws.view(torch.int16))
    assert torch.equal(poly.view(torch.int16), p_ws.view(torch.int16))
    assert torch.equal(y.view(torch.int16), y_step.view(torch.int16))


@pytest.mark.parametrize("shape", [(8, 512, 2048), (10, 1024, 440)])
def test_pairs_match_oracle(shape):
    from muon_fusion_ascend950_amd import polar_step

    x_cpu = O.make_input(shape, seed=54)
    y = polar_step(x_cpu.to(DEV), *C0)
    torch.cuda.synchronize()
    assert_matches_oracle(y, x_cpu, [C0], rel_exact=1e-2)
