"""polar_step and polar_express on tall inputs (M > N) in the right-Gram form (marked ``gpu``).

The reference's wrapper transposes an [M, N] input with M > N, runs the op on the
[N, M] copy and transposes back (muon_ascend950/ops.py:26-32).  For N % 8 == 0 this
build runs the same step without the copies:

    G = Xᵀ·X,   P = b·G + c·G²,   Y = a·X + X·P

G is the Gram matrix of the transposed input, P is symmetric, and X·P = (P·Xᵀ)ᵀ, so
every output is the same sum of the same products as on the transposed path.  The
checks:

* unsplit (MUON_POLAR_STREAM_K=0): bit for bit equal to the transposed path;
* exact-sum inputs (sparse ±1 X, integer coefficients): G, P and Y equal the oracle's
  rounding-point emulation bit for bit, split or not;
* random inputs with the stream-K split: deterministic, equal to the transposed path
  to bf16 precision (a split tile's partial sums round differently, and which tiles
  are split follows the tile order, which differs between the two forms), and
  matching the oracle;
* the wrapper dispatch, misaligned and non-contiguous inputs, graph capture, the
  C ABI entry and polar_express on tall inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
from tests.test_polar_step_gpu import assert_close_kernels, assert_matches_oracle, bits
from tests.test_stream_k_gpu import EXACT_COEFFS, HEADLINE_SPLIT, assert_bits_equal, split_in_use

pytestmark = pytest.mark.gpu

DEV = "cuda"
C0 = O.COEFFICIENTS[0]
# (batch, M, N), M > N, N % 8 == 0: the headline shape transposed (192x192 wave
# pairs for G and P, apply's last round as column halves; split on every stage with
# HEADLINE_SPLIT), ragged M and N (edge tiles, padded Gram rows, partial last
# K-step), small N (64-row tiles), batch.
TALL_SHAPES = [(1, 14336, 4096), (2, 700, 256), (3, 523, 200), (1, 4100, 1000), (4, 2048, 64)]


@pytest.fixture(scope="module", autouse=True)
def _native():
    assert torch.cuda.is_available(), "GPU tests need a ROCm GPU"
    import muon_fusion_ascend950_amd  # noqa: F401  (fails loudly without the HIP library)

    yield


def _capi():
    from muon_fusion_ascend950_amd import capi

    return capi


def step_tall(x, a, b, c):
    return torch.ops.muon_ascend950.polar_step_tall(x, float(a), float(b), float(c))


def step_transposed(x, a, b, c):
    """The reference wrapper's route: the op on the transposed copy, transposed back."""
    return torch.ops.muon_ascend950.polar_step(x.mT.contiguous(), float(a), float(b),
                                               float(c)).mT.contiguous()


@pytest.mark.parametrize("shape", TALL_SHAPES)
def test_unsplit_equals_transposed_path_bitwise(monkeypatch, shape):
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    # the transposed path's 192x192 wave-pair gram (two K chains per output) has no
    # right-Gram counterpart: compare one-chain kernels on both routes
    monkeypatch.setenv("MUON_POLAR_PAIR", "0")
    print(f"unsplit tall {shape}", flush=True)
    x = O.make_input(shape, seed=31).to(DEV)
    y = step_tall(x, *C0)
    yt = step_transposed(x, *C0)
    torch.cuda.synchronize()
    assert y.shape == x.shape
    assert_bits_equal(bits(y), bits(yt), "Y")


@pytest.mark.parametrize("split", ["1", "0"])
@pytest.mark.parametrize("shape,env", [((1, 14336, 4096), {}), ((1, 14336, 4096), HEADLINE_SPLIT),
                                       ((3, 523, 200), {}), ((2, 4096, 512), {})])
def test_exact_sums_are_bitwise(monkeypatch, shape, env, split):
    monkeypatch.setenv("MUON_POLAR_STREAM_K", split)
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    batch, m, n = shape
    if split == "1" and (env or shape[0] == 2):
        assert split_in_use(*shape)
    capi = _capi()
    mats = O.sparse_sign_input(shape, 16, seed=32)
    x = torch.from_numpy(np.stack([xm.toarray() for xm in mats]).astype(np.float32))
    x = x.to(torch.bfloat16).to(DEV)
    y = torch.empty_like(x)
    ws, info = capi.alloc_workspace(batch, m, n)
    print(f"exact sums tall {shape} split={split}", flush=True)
    # a different input through the same workspace first: stale partials would show
    capi.step(O.make_input(shape, seed=33).to(DEV), y, ws, *C0)
    capi.step(x, y, ws, *EXACT_COEFFS)
    torch.cuda.synchronize()
    mp, gram_bytes = info.padded_rows, info.gram_bytes
    g_gpu = ws[:gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    p_off = -(-gram_bytes // 256) * 256
    p_gpu = ws[p_off:p_off + gram_bytes].view(torch.bfloat16).view(batch, mp, mp)
    for i, xm in enumerate(mats):
        # the oracle's left form on Xᵀ: its A is XᵀX and its Y is Yᵀ
        yt_ref, max_sum, g_ref, p_ref = O.polar_step_fused_sparse(xm.T.tocsr(), *EXACT_COEFFS,
                                                                  return_stages=True)
        assert max_sum < 2**24
        g_pad = np.zeros((mp, mp)); g_pad[:n, :n] = g_ref
        p_pad = np.zeros((mp, mp)); p_pad[:n, :n] = p_ref
        assert_bits_equal(bits(g_gpu[i]), O.f32_to_bf16_bits(g_pad.astype(np.float32)), "G")
        assert_bits_equal(bits(p_gpu[i]), O.f32_to_bf16_bits(p_pad.astype(np.float32)), "P")
        assert_bits_equal(bits(y[i]), O.f32_to_bf16_bits(yt_ref.T.astype(np.float32)), "Y")


@pytest.mark.parametrize("shape,env", [((1, 14336, 4096), HEADLINE_SPLIT),
                                       ((1, 14336, 4096), {}), ((2, 4096, 512), {})])
def test_split_is_deterministic_and_close_to_transposed(monkeypatch, shape, env):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    assert split_in_use(*shape) == (env != {} or shape[0] == 2)
    print(f"split tall {shape}", flush=True)
    x = O.make_input(shape, seed=34).to(DEV)
    first = step_tall(x, *C0)
    again = [step_tall(x, *C0) for _ in range(2)]
    yt = step_transposed(x, *C0)
    torch.cuda.synchronize()
    for y in again:
        assert torch.equal(first, y)
    assert_close_kernels(first, yt)


@pytest.mark.parametrize("shape", [(2, 700, 256), (1, 4100, 1000), (1, 2600, 2048)])
def test_matches_oracle(shape):
    x_cpu = O.make_input(shape, seed=35)
    y = step_tall(x_cpu.to(DEV), *C0)
    torch.cuda.synchronize()
    # the oracle follows the reference wrapper (transpose when M > N)
    assert_matches_oracle(y, x_cpu, [C0], rel_exact=1e-2)


def test_wrapper_dispatches_to_right_gram():
    from muon_fusion_ascend950_amd import polar_step

    x = O.make_input((2, 700, 256), seed=36).to(DEV)
    assert torch.equal(polar_step(x, *C0), step_tall(x, *C0))
    x2 = x[0]
    assert torch.equal(polar_step(x2, *C0), step_tall(x2[None], *C0)[0])


def test_misaligned_and_noncontiguous_inputs():
    shape = (2, 700, 256)
    x = O.make_input(shape, seed=37).to(DEV)
    ref = step_tall(x, *C0)
    # data 2 bytes past a 16-byte boundary: the op aligns its own copy
    buf = torch.empty(x.numel() + 1, dtype=torch.bfloat16, device=DEV)
    xm = buf[1:].view(shape)
    xm.copy_(x)
    assert xm.data_ptr() % 16 != 0
    assert torch.equal(step_tall(xm, *C0), ref)
    xn = x.mT.contiguous().mT  # same values, column-major storage
    assert not xn.is_contiguous()
    assert torch.equal(step_tall(xn, *C0), ref)


def test_c_abi_tall_step_and_alignment_error():
    capi = _capi()
    shape = (2, 700, 256)
    batch, m, n = shape
    x = O.make_input(shape, seed=38).to(DEV)
    y = torch.empty_like(x)
    ws, _ = capi.alloc_workspace(batch, m, n)
    capi.step(x, y, ws, *C0)
    torch.cuda.synchronize()
    assert torch.equal(y, step_tall(x, *C0))
    buf = torch.empty(x.numel() + 1, dtype=torch.bfloat16, device=DEV)
    ym = buf[1:].view(shape)
    with pytest.raises(capi.CapiError, match="16-byte aligned"):
        capi.step(x, ym, ws, *C0)


def test_graph_replays_equal_eager():
    shape = (2, 4096, 1024)
    x = O.make_input(shape, seed=39).to(DEV)
    eager = step_tall(x, *C0)
    static_x = x.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step_tall(static_x, *C0)  # warm the plan cache and the allocator outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step_tall(static_x, *C0)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        torch.mm(x[0, :256].float(), x[0, :256].float().T)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("normalize", [False, True])
@pytest.mark.parametrize("shape", [(1, 14336, 4096), (3, 523, 200)])
def test_express_tall(monkeypatch, shape, normalize):
    """polar_express on M > N: with the split off, bit for bit the per-step loop and,
    without normalisation, the transposed path.  The normalisation sums squares in
    memory order, which the transposed copy changes (the bf16 norm may then differ
    by an ulp), so with it the check is: normalise alone (no steps), then the steps
    without normalisation, gives the same bits."""
    monkeypatch.setenv("MUON_POLAR_STREAM_K", "0")
    monkeypatch.setenv("MUON_POLAR_PAIR", "0")  # one K chain per output on both routes
    from muon_fusion_ascend950_amd import COEFFICIENTS, polar_express

    print(f"express tall {shape} normalize={normalize}", flush=True)
    x = O.make_input(shape, seed=40).to(DEV)
    flat = [float(v) for t in COEFFICIENTS for v in t]
    y = polar_express(x, normalize=normalize)
    yt = torch.ops.muon_ascend950.polar_express(x.mT.contiguous(), flat, normalize).mT
    loop = x
    for a, b, c in COEFFICIENTS:
        loop = step_tall(loop, a, b, c)
    torch.cuda.synchronize()
    if normalize:
        xn = polar_express(x, coefficients=(), normalize=True)
        assert_bits_equal(bits(y), bits(polar_express(xn, normalize=False)), "Y")
        yn = y.float().cpu().numpy().astype(np.float64)
        assert O.rel_frobenius(yn, yt.float().cpu().numpy().astype(np.float64)) <= 2e-2
    else:
        assert_bits_equal(bits(y), bits(yt.contiguous()), "Y")
        assert_bits_equal(bits(y), bits(loop), "Y (per-step loop)")
