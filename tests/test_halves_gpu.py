"""Apply's last round as 256x128 column halves (marked ``gpu``).

When apply's 256x256 tiles leave a last round of between a quarter and a half of the
resident workgroups, each of those tiles runs as two 256x128 column halves, one per
workgroup, each over the whole K range, with the wave-pair kernel (two interleaved K
chains per output): no fp32 partials, no arrival words, no fix-up.  At [4096,14336]
(and the right-Gram form at [14336,4096]) that is 768 whole tiles and 256 halves.
A short last round that stream-K leaves whole (its shares would be under 20 K-steps)
runs as halves too: [2,2048,4352] 256 whole tiles and 32 halves, [1,3000,6000] 256 and
64 (edge tiles: the last column tile's second half lies past n).  The checks:

* the plan uses the halves at the headline shapes and leaves the workspace without
  apply partials;
* exact-sum inputs (sparse ±1 X, integer coefficients): Y equals the oracle's
  rounding-point emulation bit for bit, after another input went through the same
  workspace;
* random inputs: the halves agree with the stream-K split (MUON_POLAR_APPLY_HALVES=0)
  and with the unsplit step to bf16 precision, give the same bits on every run and
  match the oracle; rows and columns outside the halves are untouched (NaN-filled Y).
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


def _cus() -> int:
    return torch.cuda.get_device_properties(0).multi_processor_count


SHORT_ROUNDS = [(2, 2048, 4352), (1, 3000, 6000), (2, 4352, 2048), (1, 6000, 3000)]


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (1, 14336, 4096)] + SHORT_ROUNDS)
def test_headline_runs_halves(shape):
    capi = _capi()
    plan = capi.check_plan(*shape, cus=_cus(), blocks_per_cu=(-1, -1, -1))
    apply = plan.stage[2]
    print(f"{shape}: apply dp {apply.dp_tiles} of {apply.total_tiles}, units {apply.sk_units}",
          flush=True)
    assert apply.coverage_ok and apply.extents_ok
    assert apply.sk_units == 2 * (apply.total_tiles - apply.dp_tiles) > 0
    assert apply.partial_hi == 0 and apply.counter_hi == 0


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (1, 14336, 4096)] + SHORT_ROUNDS)
def test_exact_sums_are_bitwise(shape):
    capi = _capi()
    batch, m, n = shape
    tall = m > n
    mats = O.sparse_sign_input(shape, 16, seed=41)
    x = torch.from_numpy(np.stack([xm.toarray() for xm in mats]).astype(np.float32))
    x = x.to(torch.bfloat16).to(DEV)
    y = torch.empty_like(x)
    ws, _ = capi.alloc_workspace(batch, m, n)
    print(f"halves exact sums {shape}", flush=True)
    capi.step(O.make_input(shape, seed=42).to(DEV), y, ws, *C0)
    capi.step(x, y, ws, *EXACT_COEFFS)
    torch.cuda.synchronize()
    for i, xm in enumerate(mats):
        # m > n: the oracle's left form on Xᵀ, whose Y is Yᵀ
        y_ref, max_sum = O.polar_step_fused_sparse(xm.T.tocsr() if tall else xm, *EXACT_COEFFS)
        assert max_sum < 2**24
        want = O.f32_to_bf16_bits((y_ref.T if tall else y_ref).astype(np.float32))
        assert_bits_equal(bits(y[i]), want, "Y")


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (1, 14336, 4096)] + SHORT_ROUNDS)
def test_halves_agree_with_split_and_unsplit(monkeypatch, shape):
    x = O.make_input(shape, seed=43).to(DEV)
    halves = polar_step(x, *C0)
    again = [polar_step(x, *C0) for _ in range(2)]
    monkeypatch.setenv("MUON_POLAR_APPLY_HALVES", "0")
    split = polar_step(x, *C0)
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    unsplit = polar_step(x, *C0)
    torch.cuda.synchronize()
    for y in again:
        assert torch.equal(halves, y)
    assert_close_kernels(halves, split)
    assert_close_kernels(halves, unsplit)


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (1, 3000, 6000), (1, 6000, 3000)])
def test_halves_match_oracle(shape):
    x_cpu = O.make_input(shape, seed=44)
    y = polar_step(x_cpu.to(DEV), *C0)
    torch.cuda.synchronize()
    assert_matches_oracle(y, x_cpu, [C0], rel_exact=1e-2)


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (1, 3000, 6000)])
def test_halves_store_only_their_outputs(shape):
    """Every element of Y is written (NaN fill replaced everywhere), and equal to the
    torch op's result."""
    capi = _capi()
    x = O.make_input(shape, seed=45).to(DEV)
    y = torch.full_like(x, float("nan"))
    ws, _ = capi.alloc_workspace(*shape)
    capi.step(x, y, ws, *C0)
    torch.cuda.synchronize()
    assert not torch.isnan(y.float()).any()
    assert torch.equal(y, polar_step(x, *C0))
