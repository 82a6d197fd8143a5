"""Stream-K split of polar_step's stages on the GPU (marked ``gpu``).

When the last round of a stage's tiles would leave most CUs idle, polar_step cuts
those tiles' K loops into equal shares, one per workgroup, and the last contributor
to arrive sums the fp32 partials in a fixed order.  The checks:

* the split is in use for the shapes below (the workspace then holds partial slots);
* exact-sum inputs (sparse ±1 X, integer coefficients): every sum is an integer below
  2^24, so A, P and Y must equal the oracle's rounding-point emulation bit for bit,
  split or not — a partial dropped, counted twice or summed from a stale slot changes
  bits;
* random inputs: split and unsplit agree to bf16 precision, the split result is the
  same on every run (the summation order does not depend on which workgroup arrives
  last), and it matches the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
from tests.test_polar_step_gpu import assert_close_kernels, assert_matches_oracle, bits

pytestmark = pytest.mark.gpu

DEV = "cuda"
C0 = O.COEFFICIENTS[0]
EXACT_COEFFS = (2.0, -1.0, 1.0)
# (batch, m, n): batch crossing inside the split range, ragged m and n (padded rows,
# partial last K-step, edge column tiles), 64- and 128-row tiles.  (The headline
# shape splits no stage by default: gram and poly run one round of 192x192 tiles and
# apply's last round runs as 256x128 halves, test_halves_gpu.py; it is split here
# with 256x256 triangular tiles, and with the halves off.  [2,4096,4096] takes the
# two-round split of gram and poly: 256 units of 68 K-steps over all 272 tiles;
# [4096,17408] that of apply: 768 whole tiles, then 256 units over the last 320.
# [1,64,100000] and [1,8,131072]: one 64x64 gram tile of 1563 / 2048 K-steps cut
# into 24 / 32 shares of about 64 K-steps, so the last contributor adds 23 / 31
# partials.)
SPLIT_SHAPES = [(2, 512, 4096), (2, 1536, 4096), (1, 700, 5000), (2, 1500, 3000)]
# 256x256 tiles for the triangular stages (256 KiB partials)
BIG_TILES = {"MUON_POLAR_GRAM_TILE": "256", "MUON_POLAR_POLY_TILE": "256"}
# every stage of the headline split: 256x256 triangular tiles, apply's halves off
HEADLINE_SPLIT = {**BIG_TILES, "MUON_POLAR_APPLY_HALVES": "0"}


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


def split_in_use(batch, m, n) -> bool:
    info = _capi().query(batch, m, n)
    a_and_p = 2 * (-(-info.gram_bytes // 256) * 256)
    return info.workspace_bytes > a_and_p + 4096


def assert_bits_equal(got: np.ndarray, want: np.ndarray, what: str):
    bad = np.flatnonzero(got.ravel() != want.ravel())
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} elements differ, first at "
                           f"{np.unravel_index(bad[0], got.shape)}")


@pytest.mark.parametrize("shape", SPLIT_SHAPES)
def test_split_is_in_use(shape):
    assert split_in_use(*shape)


@pytest.mark.parametrize("split", ["1", "0"])
@pytest.mark.parametrize("shape,env", [(s, {}) for s in SPLIT_SHAPES] +
                         [((1, 4096, 14336), HEADLINE_SPLIT), ((2, 2048, 4096), BIG_TILES),
                          ((1, 4096, 14336), BIG_TILES), ((2, 4096, 4096), {}),
                          ((1, 4096, 17408), {}), ((1, 64, 100000), {}), ((1, 8, 131072), {})])
def test_exact_sums_are_bitwise(monkeypatch, shape, env, split):
    monkeypatch.setenv("MUON_POLAR_STREAM_K", split)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    if split == "1":
        assert split_in_use(*shape)
    capi = _capi()
    batch, m, n = shape
    mats = O.sparse_sign_input(shape, 16, seed=21)
    x = torch.from_numpy(np.stack([xm.toarray() for xm in mats]).astype(np.float32))
    x = x.to(torch.bfloat16).to(DEV)
    y = torch.empty_like(x)
    ws, info = capi.alloc_workspace(batch, m, n)
    print(f"exact sums {shape} split={split}", flush=True)
    # the workspace first carries another input: a partial left over from an
    # earlier call, read instead of this call's, would change bits
    capi.step(O.make_input(shape, seed=25).to(DEV), y, ws, *C0)
    capi.step(x, y, ws, *EXACT_COEFFS)
    torch.cuda.synchronize()
    mp, gram_bytes = info.padded_rows, info.gram_bytes
    a_gpu = ws[:gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    p_off = -(-gram_bytes // 256) * 256
    p_gpu = ws[p_off:p_off + gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    for i, xm in enumerate(mats):
        y_ref, max_sum, a_ref, p_ref = O.polar_step_fused_sparse(xm, *EXACT_COEFFS,
                                                                 return_stages=True)
        assert max_sum < 2**24  # every fp32 sum is exact
        a_pad = np.zeros((mp, mp)); a_pad[:m, :m] = a_ref
        p_pad = np.zeros((mp, mp)); p_pad[:m, :m] = p_ref
        assert_bits_equal(bits(a_gpu[i]), O.f32_to_bf16_bits(a_pad.astype(np.float32)), "A")
        assert_bits_equal(bits(p_gpu[i]), O.f32_to_bf16_bits(p_pad.astype(np.float32)), "P")
        assert_bits_equal(bits(y[i]), O.f32_to_bf16_bits(y_ref.astype(np.float32)), "Y")


@pytest.mark.parametrize("shape", [(1, 4096, 14336), (2, 512, 4096), (1, 700, 5000),
                                   (2, 4096, 4096), (1, 4096, 17408)])
def test_split_agrees_with_unsplit_and_is_deterministic(monkeypatch, shape):
    x = O.make_input(shape, seed=22).to(DEV)
    first = polar_step(x, *C0)
    again = [polar_step(x, *C0) for _ in range(3)]
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    unsplit = polar_step(x, *C0)
    torch.cuda.synchronize()
    for y in again:
        assert torch.equal(first, y)
    assert_close_kernels(first, unsplit)


def test_split_matches_oracle():
    shape = (2, 1500, 3000)
    x_cpu = O.make_input(shape, seed=23)
    y = polar_step(x_cpu.to(DEV), *C0)
    torch.cuda.synchronize()
    assert_matches_oracle(y, x_cpu, [C0], rel_exact=1e-2)


@pytest.mark.parametrize("shape", [(3, 2048, 4096), (1, 4096, 14336)])
def test_stage_calls_with_workspace_equal_the_step(shape):
    """The stage entry points given polar_step's workspace run the same split kernels."""
    capi = _capi()
    batch, m, n = shape
    a, b, c = C0
    x = O.make_input(shape, seed=24).to(DEV)
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
