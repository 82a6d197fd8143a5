"""Pins the CPU oracle (oracle/polar_oracle.py) before anything is checked against it.

The reference ships no golden vectors (its tests use unseeded device RNG,
tests/test_polar_step.py:38,47), so each oracle function is pinned by what the
mathematics fixes: the SVD closed form of the step, textbook special cases of each
stage, brute-force loops on tiny inputs, and torch's own bf16 rounding.  Planted
mistakes in copies of the oracle must fail these checks, which shows they can
tell a right formula from a plausible wrong one.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O

C0 = O.COEFFICIENTS[0]
RNG = np.random.default_rng(1234)


# ----------------------------------------------------------------------------- helpers
def random_orthogonal(k: int, rng=RNG) -> np.ndarray:
    q, r = np.linalg.qr(rng.standard_normal((k, k)))
    return q * np.sign(np.diag(r))


def svd_input(m: int, n: int, rng=RNG, lo=0.05, hi=1.0):
    """X = U diag(σ) Vᵀ with chosen σ in [lo, hi] (m <= n or m > n)."""
    k = min(m, n)
    u = random_orthogonal(m, rng)[:, :k]
    v = random_orthogonal(n, rng)[:, :k]
    sigma = np.sort(rng.uniform(lo, hi, size=k))[::-1]
    return (u * sigma) @ v.T, u, sigma, v


def closed_form(u, sigma, v, coefficients):
    return (u * O.scalar_polynomial(sigma, coefficients)) @ v.T


def brute_step(x, a, b, c):
    """Pure-Python triple loops (tiny inputs only)."""
    m, n = len(x), len(x[0])
    g = [[sum(x[i][k] * x[j][k] for k in range(n)) for j in range(m)] for i in range(m)]
    g2 = [[sum(g[i][k] * g[k][j] for k in range(m)) for j in range(m)] for i in range(m)]
    p = [[b * g[i][j] + c * g2[i][j] for j in range(m)] for i in range(m)]
    return [[a * x[i][j] + sum(p[i][k] * x[k][j] for k in range(m)) for j in range(n)]
            for i in range(m)]


# ----------------------------------------------------------------------------- bf16 rounding
def torch_bf16_bits(f32: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(f32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_bf16_rne_matches_torch_random_and_ties():
    raw = RNG.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    ties = (raw & np.uint32(0xFFFF0000)) | np.uint32(0x8000)  # exactly halfway cases
    near = (raw & np.uint32(0xFFFF0000)) | np.uint32(0x7FFF)
    for bits in (raw, ties, near):
        f = bits.view(np.float32)
        finite = np.isfinite(f)
        got = O.f32_to_bf16_bits(f[finite])
        want = torch_bf16_bits(f[finite])
        assert np.array_equal(got, want)


def test_bf16_rne_special_values():
    vals = np.array([0.0, -0.0, np.inf, -np.inf, 1.0, -1.0, 3.0e38, -3.0e38, 1e-40, -1e-40,
                     np.finfo(np.float32).max, np.finfo(np.float32).tiny,
                     1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8, 1.0 + 2.0**-9], dtype=np.float32)
    assert np.array_equal(O.f32_to_bf16_bits(vals), torch_bf16_bits(vals))
    nan = O.f32_to_bf16_bits(np.array([np.nan, -np.nan], dtype=np.float32))
    assert np.all(np.isnan(O.bf16_bits_to_f32(nan)))
    # round trip of every bf16 pattern that is a finite number
    allbits = np.arange(2**16, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_bits_to_f32(allbits)
    ok = np.isfinite(f)
    assert np.array_equal(O.f32_to_bf16_bits(f[ok]), allbits[ok])


# ----------------------------------------------------------------------------- full step
@pytest.mark.parametrize("m,n", [(1, 1), (3, 5), (16, 40), (40, 16), (33, 33), (64, 200)])
def test_step_matches_svd_closed_form(m, n):
    x, u, sigma, v = svd_input(m, n)
    expected = closed_form(u, sigma, v, [C0])
    got = O.polar_step_f64(x, *C0) if m <= n else O.wrapper_step(x, *C0, step=O.polar_step_f64)
    assert np.allclose(got, expected, rtol=0, atol=1e-12 * max(1.0, np.abs(expected).max()))


def test_five_steps_compose_scalar_polynomial():
    x, u, sigma, v = svd_input(24, 70)
    got = O.reference_formula_f64(x, O.COEFFICIENTS)
    assert np.allclose(got, closed_form(u, sigma, v, O.COEFFICIENTS), atol=1e-10)
    # Polar Express drives every singular value toward ~1.
    s = np.linalg.svd(got, compute_uv=False)
    assert np.all(np.abs(s - 1.0) < 0.35)


def test_batched_step_is_per_matrix():
    x = np.stack([svd_input(10, 30)[0] for _ in range(3)])
    got = O.polar_step_f64(x, *C0)
    for i in range(3):
        assert np.allclose(got[i], O.polar_step_f64(x[i], *C0), atol=1e-14)


@pytest.mark.parametrize("m,n", [(1, 1), (1, 17), (3, 5), (4, 4), (5, 3)])
def test_step_matches_bruteforce_loops(m, n):
    x = RNG.standard_normal((m, n)) * 0.3
    want = np.array(brute_step(x.tolist(), *C0))
    got = O.polar_step_f64(x, *C0)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------------------------- per stage
def test_gram_special_cases():
    q = random_orthogonal(12)[:5]  # orthonormal rows
    assert np.allclose(O.gram_f64(q), np.eye(5), atol=1e-12)
    d = np.diag([0.5, -2.0, 3.0])
    x = np.concatenate([d, np.zeros((3, 4))], axis=1)
    assert np.allclose(O.gram_f64(x), d @ d, atol=0)
    x = RNG.standard_normal((7, 11))
    g = O.gram_f64(x)
    assert np.isclose(np.trace(g), np.sum(x * x))
    assert np.array_equal(g, g.T) or np.allclose(g, g.T, atol=1e-15)
    assert np.all(np.diag(g) >= 0)


def test_poly_special_cases():
    b, c = C0[1], C0[2]
    assert np.allclose(O.poly_f64(np.eye(6), b, c), (b + c) * np.eye(6))
    d = np.array([0.1, -0.3, 0.7, 1.5])
    assert np.allclose(O.poly_f64(np.diag(d), b, c), np.diag(b * d + c * d * d))


def test_apply_special_cases():
    a = C0[0]
    x = RNG.standard_normal((5, 9))
    assert np.allclose(O.apply_f64(np.zeros((5, 5)), x, a), a * x)
    assert np.allclose(O.apply_f64(np.eye(5), x, a), (a + 1.0) * x)


# ----------------------------------------------------------------------------- rounding-point emulation
def test_fused_emulation_close_to_exact():
    x = O.to_numpy_f64(O.make_input((2, 150, 2050), seed=3))
    exact = O.polar_step_f64(x, *C0)
    fused, gram, poly = O.polar_step_fused(x, *C0, return_stages=True)
    assert O.rel_frobenius(fused, exact) < 3e-3
    # stored A and P are bf16 values and bitwise symmetric
    assert np.array_equal(O.bf16_round(gram), gram.astype(np.float32))
    assert np.array_equal(gram, np.swapaxes(gram, -1, -2))
    assert np.array_equal(poly, np.swapaxes(poly, -1, -2))
    x5 = O.to_numpy_f64(O.make_input((1, 129, 130), seed=4))
    assert O.rel_frobenius(O.five_step_fused(x5), O.reference_formula_f64(x5, O.COEFFICIENTS)) < 2e-2


def test_torch_formula_restatement():
    x = O.make_input((2, 40, 90), seed=5)
    x64 = O.to_numpy_f64(x)
    got64 = O.reference_formula_torch(x.double(), O.COEFFICIENTS[:2]).numpy()
    assert np.allclose(got64, O.reference_formula_f64(x64, O.COEFFICIENTS[:2]), atol=1e-12)
    got_bf16 = O.reference_formula_torch(x, [C0]).float().numpy()
    assert O.rel_frobenius(got_bf16, O.polar_step_f64(x64, *C0)) < 1e-2


def test_make_input_recipe():
    x = O.make_input((3, 20, 50), seed=7)
    assert x.dtype == torch.bfloat16 and x.shape == (3, 20, 50)
    assert torch.equal(x, O.make_input((3, 20, 50), seed=7))
    norms = x.float().norm(dim=(-2, -1))
    assert torch.all((norms > 0.97) & (norms < 1.0))  # ‖x‖/(1.01‖x‖) in bf16


# ----------------------------------------------------------------------------- boundary semantics
@pytest.mark.parametrize("shape", [(129, 130), (2, 150, 211), (1, 5, 9)])
def test_pad_crop_equals_masked(shape):
    x = O.to_numpy_f64(O.make_input(shape, seed=8))
    x3 = x[None] if x.ndim == 2 else x
    direct = O.polar_step_fused(x3, *C0)
    padded = O.pad_crop_step(x3, *C0)
    assert np.array_equal(direct, padded)


def test_wrapper_transpose_identity():
    x = O.to_numpy_f64(O.make_input((130, 129), seed=9))
    via_wrapper = O.wrapper_step(x, *C0, step=O.polar_step_f64)
    assert via_wrapper.shape == x.shape
    # Y = aX + (bXXᵀ + c(XXᵀ)²)X equals the transposed computation
    assert np.allclose(via_wrapper, O.polar_step_f64(x, *C0), atol=1e-12)


# ----------------------------------------------------------------------------- planted mistakes
def _mistakes():
    def drop_c(x, a, b, c):
        g = O.gram_f64(x)
        return a * x + (b * g) @ x

    def flip_b(x, a, b, c):
        return O.polar_step_f64(x, a, -b, c)

    def transposed_gram(x, a, b, c):
        g = np.swapaxes(x, -1, -2) @ x  # XᵀX instead of XXᵀ (square inputs)
        return a * x + (b * g + c * g @ g) @ x

    def linear_instead_of_square(x, a, b, c):
        g = O.gram_f64(x)
        return a * x + (b * g + c * g) @ x

    def drop_ax(x, a, b, c):
        return O.polar_step_f64(x, 0.0, b, c)

    return [drop_c, flip_b, transposed_gram, linear_instead_of_square, drop_ax]


@pytest.mark.parametrize("mistake", _mistakes(), ids=lambda f: f.__name__)
def test_closed_form_catches_planted_mistakes(mistake):
    # square, non-symmetric X so a transposed operand changes the result
    x, u, sigma, v = svd_input(12, 12)
    expected = closed_form(u, sigma, v, [C0])
    assert not np.allclose(mistake(x, *C0), expected, atol=1e-6)
    assert np.allclose(O.polar_step_f64(x, *C0), expected, atol=1e-12)


def test_zero_output_fails_normwise_gate():
    x = O.to_numpy_f64(O.make_input((2, 150, 2050), seed=10))
    ref = O.polar_step_f64(x, *C0)
    assert O.rel_frobenius(np.zeros_like(ref), ref) == pytest.approx(1.0)
    # ... while the reference's elementwise 6e-2 gate alone accepts zeros here
    torch.testing.assert_close(torch.zeros(ref.shape, dtype=torch.float64),
                               torch.from_numpy(ref), rtol=6e-2, atol=6e-2)


# ----------------------------------------------------------------------------- exact-sum inputs
@pytest.mark.parametrize("shape,nnz", [((2, 96, 300), 5), ((1, 64, 640), 16), ((1, 33, 70), 3)])
def test_sparse_fused_equals_dense_fused(shape, nnz):
    """The sparse restatement gives the dense rounding-point emulation's bits, stages too."""
    for xm in O.sparse_sign_input(shape, nnz, seed=4):
        y, max_sum, a, p = O.polar_step_fused_sparse(xm, 2.0, -1.0, 1.0, return_stages=True)
        yd, ad, pd = O.polar_step_fused(xm.toarray(), 2.0, -1.0, 1.0, return_stages=True)
        assert np.array_equal(y, yd) and np.array_equal(a, ad) and np.array_equal(p, pd)
        assert max_sum < 2**24


def test_sparse_input_shape_and_values():
    mats = O.sparse_sign_input((3, 40, 500), 7, seed=5)
    assert len(mats) == 3
    for xm in mats:
        d = xm.toarray()
        assert d.shape == (40, 500)
        assert set(np.unique(d)) <= {-1.0, 0.0, 1.0}
        assert (np.count_nonzero(d, axis=1) == 7).all()


def test_exact_sums_are_order_independent():
    """The premise of the bitwise split-K test: with these inputs the fp32 sum of any
    K-split, in any order, is the exact sum (brute force over splits in float32)."""
    xm = O.sparse_sign_input((1, 48, 1000), 16, seed=6)[0].toarray()
    exact = xm @ xm.T
    rng = np.random.default_rng(0)
    for _ in range(5):
        cuts = np.sort(rng.choice(np.arange(1, 1000), size=4, replace=False))
        parts = [(xm[:, lo:hi] @ xm[:, lo:hi].T).astype(np.float32)
                 for lo, hi in zip([0, *cuts], [*cuts, 1000])]
        total = np.float32(0)
        for part in rng.permutation(len(parts)):
            total = total + parts[part]
        assert np.array_equal(total.astype(np.float64), exact)


def test_exact_sums_catch_a_dropped_or_doubled_k_range():
    """Planted split-K mistakes (a 64-wide K range dropped, or counted twice, in the
    gram stage) change Y's bits, so the bitwise GPU test would see them."""
    xm = O.sparse_sign_input((1, 256, 4096), 16, seed=7)[0]
    y_ok = O.polar_step_fused_sparse(xm, 2.0, -1.0, 1.0)[0]
    d = xm.toarray()
    for lo in (0, 1024, 4032):
        dropped = d.copy()
        dropped[:, lo:lo + 64] = 0.0
        gram = O.bf16_round(dropped @ dropped.T).astype(np.float64)
        poly = O.bf16_round(-gram + gram @ gram).astype(np.float64)
        y_bad = O.bf16_round(2.0 * d + poly @ d)
        assert not np.array_equal(y_bad, y_ok)
        doubled = d @ d.T + d[:, lo:lo + 64] @ d[:, lo:lo + 64].T
        gram = O.bf16_round(doubled).astype(np.float64)
        poly = O.bf16_round(-gram + gram @ gram).astype(np.float64)
        assert not np.array_equal(O.bf16_round(2.0 * d + poly @ d), y_ok)


# ----------------------------------------------------------------------------- normalisation
@pytest.mark.parametrize("shape", [(3, 40, 70), (1, 129, 130), (2, 8, 2048)])
def test_normalization_matches_torch_bf16_recipe(shape):
    """The restatement reproduces the reference recipe run by torch in bf16 (CPU)."""
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(shape, dtype=torch.bfloat16, generator=gen) * 3.0
    want = x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)
    got = O.normalize_reference_rounding(O.to_numpy_f64(x))
    wb = want.contiguous().view(torch.int16).numpy().view(np.uint16)
    gb = O.f32_to_bf16_bits(got.astype(np.float32))
    assert O.bf16_ulp_distance(gb, wb).max() <= 1
    assert (gb != wb).mean() < 1e-3


def test_normalization_closed_forms():
    # a single nonzero v: norm = |v|, d = bf16(bf16(|v|·1.01) + 1e-6)
    x = np.zeros((1, 3, 4))
    x[0, 1, 2] = -2.5
    got = O.normalize_reference_rounding(x)
    d = O.bf16_round(O.bf16_round(np.float32(2.5) * np.float32(1.01)) + np.float32(1e-6)).item()
    assert got[0, 1, 2] == O.bf16_round(np.float32(-2.5) / np.float32(d)).item()
    assert np.count_nonzero(got) == 1
    # zero matrix: d = bf16(1e-6) > 0, output exactly zero (no NaN)
    z = O.normalize_reference_rounding(np.zeros((2, 4, 5)))
    assert not np.isnan(z).any() and not z.any()
    # planted mistake: dropping the 1.01 factor changes the result
    x = O.to_numpy_f64(torch.randn(2, 16, 40, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16))
    norm = O.bf16_round(np.sqrt((x * x).sum(axis=(-2, -1), keepdims=True)))
    wrong = O.bf16_round(x.astype(np.float32) / O.bf16_round(norm + np.float32(1e-6)))
    assert not np.array_equal(wrong, O.normalize_reference_rounding(x))


# ----------------------------------------------------------------------------- ulp metric
def _bf16_rank_table():
    """Rank of every finite bf16 bit pattern among the distinct finite bf16 values
    (+0 and -0 share one rank): an independent definition of ulp distance, from
    torch's own bf16 -> fp32 conversion and a sort."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    finite = np.isfinite(vals)
    distinct = np.unique(vals[finite])  # -0.0 == 0.0 collapse into one entry
    rank = np.full(1 << 16, -1, dtype=np.int64)
    rank[finite] = np.searchsorted(distinct, vals[finite])
    return bits, finite, rank


def test_bf16_ulp_distance_is_the_rank_distance_between_finite_values():
    """The metric used by the GPU parity gates counts the bf16 values between two
    patterns: checked against the rank of each value among all finite bf16 values,
    on adjacent pairs over the whole range, on random pairs, across zero, and on
    signed zeros."""
    bits, finite, rank = _bf16_rank_table()
    fb = bits[finite]
    # adjacent patterns of the same sign: distance 1 (exponent boundaries included)
    pos = fb[fb < 0x7F80]
    pos = pos[pos > 0]
    assert np.all(O.bf16_ulp_distance(pos[1:], pos[:-1]) == 1)
    assert O.bf16_ulp_distance([0x3F7F], [0x3F80])[0] == 1  # 1 - 2^-8 .. 1.0
    neg = np.sort(fb[(fb > 0x8000) & (fb < 0xFF80)])
    assert np.all(O.bf16_ulp_distance(neg[1:], neg[:-1]) == 1)
    # signed zeros are one value
    assert O.bf16_ulp_distance([0x0000], [0x8000])[0] == 0
    # across zero: the two distances to zero add up
    assert O.bf16_ulp_distance([0x0001], [0x8001])[0] == 2
    assert O.bf16_ulp_distance([0x3F80], [0xBF80])[0] == 2 * rank[0x3F80] - 2 * rank[0x0000]
    # random pairs of finite patterns against the rank table
    rng = np.random.default_rng(99)
    a = rng.choice(fb, 20000)
    b = rng.choice(fb, 20000)
    np.testing.assert_array_equal(O.bf16_ulp_distance(a, b), np.abs(rank[a] - rank[b]))
    # and a few large pairs, where the counts must not wrap
    assert O.bf16_ulp_distance([0x7F7F], [0xFF7F])[0] == rank[0x7F7F] - rank[0xFF7F]


def test_bf16_ulp_distance_rejects_planted_mistakes():
    """Plausible wrong maps fail the checks above: no sign handling (raw bit
    difference), and a sign map off by one (signed zeros one ulp apart)."""
    bits, finite, rank = _bf16_rank_table()

    def no_sign(a_bits, b_bits):
        return np.abs(np.asarray(a_bits, dtype=np.int32) - np.asarray(b_bits, dtype=np.int32))

    def off_by_one(a_bits, b_bits):
        def ordered(v):
            v = np.asarray(v, dtype=np.uint16).astype(np.int32)
            return np.where(v & 0x8000, 0x7FFF - v, v)

        return np.abs(ordered(a_bits) - ordered(b_bits))

    assert no_sign([0x0001], [0x8001])[0] != 2
    assert off_by_one([0x0000], [0x8000])[0] != 0
    rng = np.random.default_rng(5)
    fb = bits[finite]
    a, b = rng.choice(fb, 1000), rng.choice(fb, 1000)
    want = np.abs(rank[a] - rank[b])
    assert not np.array_equal(no_sign(a, b), want)
    assert not np.array_equal(off_by_one(a, b), want)
