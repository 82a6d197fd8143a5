"""polar_express (normalise + several steps in one call) on the GPU (marked ``gpu``).

No reference counterpart: it replaces the caller loop of the reference's
``examples/five_steps.py:17-20``.  Checks:

* without normalisation, k steps equal k chained ``polar_step`` calls bit for bit (same
  kernels; the iterate alternates between the output and one workspace buffer), for odd
  and even k, split and unsplit stages, both kernel families;
* the normalisation against the oracle's restatement of the reference recipe and against
  that recipe run by torch in bf16 on the same GPU (at most one bf16 ulp, almost always
  equal), per matrix of a batch, and the zero matrix (zeros, no NaN);
* normalise + the five triples against the reference loop (torch normalisation, then
  ``polar_step`` five times) and against the float64 formula;
* the ``[M,N]`` / ``M > N`` wrapper, and the C ABI entry with a caller workspace.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
from tests.test_polar_step_gpu import bits

pytestmark = pytest.mark.gpu

DEV = "cuda"
COEFFS = O.COEFFICIENTS


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    yield


def mf():
    import muon_fusion_ascend950_amd

    return muon_fusion_ascend950_amd


def raw_input(shape, seed, scale=3.0):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, dtype=torch.bfloat16, generator=gen) * scale).to(DEV)


# widths: multiples of 64 and of 8, even, odd (padded copy of X in every step; Y rows of
# alternating alignment, [3,129,257]); tall: right-Gram form ([2,1000,136]) and the
# transposed route of an unaligned width ([1,515,130])
@pytest.mark.parametrize("shape", [(8, 512, 2048), (2, 150, 2050), (3, 1024, 8192), (1, 4096, 14336),
                                   (2, 300, 1000), (3, 129, 257), (2, 1000, 136), (1, 515, 130)])
@pytest.mark.parametrize("k", [1, 2, 5])
def test_steps_equal_chained_polar_step(shape, k):
    x = O.make_input(shape, seed=40).to(DEV)
    got = mf().polar_express(x, COEFFS[:k], normalize=False)
    want = x
    for a, b, c in COEFFS[:k]:
        want = mf().polar_step(want, a, b, c)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


# partial sums over chunks of 4096 elements (ragged: [5,1000,1001], odd m·n), 8192 with a
# 16-element last chunk ([4100,4100]) and 16384 ([4096,14336])
@pytest.mark.parametrize("shape", [(3, 40, 70), (2, 150, 2050), (8, 512, 2048), (5, 1000, 1001),
                                   (1, 4100, 4100), (1, 4096, 14336)])
def test_normalization(shape):
    x = raw_input(shape, seed=41)
    x[0] *= 8.0  # matrices of a batch get different scales
    got = mf().polar_express(x, [], normalize=True)
    torch.cuda.synchronize()
    gb = bits(got)
    want = O.f32_to_bf16_bits(O.normalize_reference_rounding(O.to_numpy_f64(x)).astype(np.float32))
    assert O.bf16_ulp_distance(gb, want).max() <= 1
    assert (gb != want).mean() < 1e-3
    recipe = x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)  # torch bf16, same GPU
    torch.cuda.synchronize()
    rb = bits(recipe)
    assert O.bf16_ulp_distance(gb, rb).max() <= 1
    assert (gb != rb).mean() < 1e-3


def test_zero_matrix_normalizes_to_zero():
    x = torch.zeros(2, 64, 256, dtype=torch.bfloat16, device=DEV)
    x[1] = raw_input((64, 256), seed=42)
    y = mf().polar_express(x, COEFFS, normalize=True)
    torch.cuda.synchronize()
    assert not torch.isnan(y).any()
    assert not y[0].any()


@pytest.mark.parametrize("shape", [(8, 512, 2048), (1, 4096, 14336)])
def test_five_steps_against_reference_loop_and_formula(shape):
    x = raw_input(shape, seed=43)
    got = mf().polar_express(x)  # normalise + the five triples
    # the reference's example loop, with this build's polar_step
    loop = x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)
    for a, b, c in COEFFS:
        loop = mf().polar_step(loop, a, b, c)
    torch.cuda.synchronize()
    gn = got.float().cpu().numpy().astype(np.float64)
    ln = loop.float().cpu().numpy().astype(np.float64)
    assert O.rel_frobenius(gn, ln) <= 1e-2  # equal unless a normalised element differs by an ulp
    exact = O.reference_formula_f64(O.normalize_reference_rounding(O.to_numpy_f64(x)), COEFFS)
    assert O.rel_frobenius(gn, exact) <= 3e-2


@pytest.mark.parametrize("shape", [(130, 129), (2, 700, 300), (300, 64)])
def test_wrapper_shapes(shape):
    x = raw_input(shape, seed=44)
    y = mf().polar_express(x, COEFFS[:2])
    yt = mf().polar_express(x.mT.contiguous(), COEFFS[:2]).mT
    torch.cuda.synchronize()
    assert y.shape == x.shape and torch.equal(y, yt)


def test_c_abi_entry_with_caller_workspace():
    from muon_fusion_ascend950_amd import capi

    x = raw_input((4, 256, 1024), seed=45)
    ws, _info = capi.alloc_express_workspace(4, 256, 1024)
    y = torch.empty_like(x)
    capi.express(x, y, ws, COEFFS[:3], normalize=True)
    want = mf().polar_express(x, COEFFS[:3], normalize=True)
    torch.cuda.synchronize()
    assert torch.equal(y, want)
