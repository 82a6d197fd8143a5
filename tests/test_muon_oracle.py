"""Pins the oracle's Muon update (oracle/polar_oracle.py, ``muon_*``) on the CPU.

The update around the iteration has no code in the reference (README.md:130 leaves
momentum, weight decay and the parameter update to the caller, nanochat's Muon), so
what pins the restatement is what the mathematics fixes:

* torch.lerp itself, to within one ulp of the operands (torch's CPU kernel fuses the
  multiply-add; the oracle and the kernels round every operation on their own);
* momentum under a constant gradient: buf_k = (1 − β^k)·g, and the Nesterov input
  (1 − β^(k+1))·g;
* zero gradient: the parameter only decays, p·(1 − lr·wd), bit for bit;
* momentum 0: the iteration's input is the gradient itself, and the update is
  −lr·scale·U·diag(q(σ/d))·Vᵀ for g = U·diag(σ)·Vᵀ, q the composed step polynomial and d
  the normalisation divisor.

Planted mistakes in copies of the update must fail these checks.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import polar_oracle as O
from tests.test_oracle import svd_input

RNG = np.random.default_rng(4321)


# ----------------------------------------------------------------------------- lerp
@pytest.mark.parametrize("w", [0.05, 1.0 - 0.95, 0.3, 0.5, 0.7, 0.95, 0.0, 1.0])
def test_lerp_matches_torch_to_one_rounding(w):
    a = RNG.standard_normal(4096).astype(np.float32)
    b = (RNG.standard_normal(4096) * 3).astype(np.float32)
    got = O.lerp_f32(a, b, w)
    want = torch.lerp(torch.from_numpy(a), torch.from_numpy(b), float(w)).numpy()
    # the fused and unfused forms differ by the product's rounding: within one ulp of
    # the operands' magnitude (more ulps of a result that cancels towards zero)
    bound = np.spacing(np.maximum(np.abs(a), np.abs(b)))
    assert np.all(np.abs(got.astype(np.float64) - want) <= bound)
    if w == 0.0:
        assert np.array_equal(got, a)
    if w == 1.0:
        assert np.array_equal(got, b)


# ----------------------------------------------------------------------------- momentum
@pytest.mark.parametrize("beta", [0.95, 0.9, 0.3])
def test_momentum_closed_form_under_constant_gradient(beta):
    g = RNG.standard_normal((8, 24)).astype(np.float32)
    buf = np.zeros_like(g)
    for k in range(1, 31):
        buf, u_nesterov = O.muon_momentum(g, buf, beta, nesterov=True)
        expect_buf = (1.0 - beta**k) * g.astype(np.float64)
        expect_u = (1.0 - beta ** (k + 1)) * g.astype(np.float64)
        tol = 1e-6 * k * np.abs(g).max()
        assert np.abs(buf - expect_buf).max() <= tol
        assert np.abs(u_nesterov - expect_u).max() <= tol


def test_plain_momentum_returns_the_buffer():
    g = RNG.standard_normal((5, 7)).astype(np.float32)
    buf = RNG.standard_normal((5, 7)).astype(np.float32)
    new_buf, u = O.muon_momentum(g, buf, 0.95, nesterov=False)
    assert np.array_equal(u, new_buf)
    assert np.array_equal(new_buf, O.lerp_f32(buf, g, np.float32(1 - 0.95)))


def test_momentum_zero_passes_the_gradient_through():
    g = RNG.standard_normal((5, 7)).astype(np.float32)
    buf = RNG.standard_normal((5, 7)).astype(np.float32)
    for nesterov in (True, False):
        new_buf, u = O.muon_momentum(g, buf, 0.0, nesterov)
        assert np.array_equal(new_buf, g) and np.array_equal(u, g)


# ----------------------------------------------------------------------------- parameter update
@pytest.mark.parametrize("lr,wd", [(0.02, 0.0), (0.1, 0.2), (0.5, 1.0)])
def test_zero_gradient_only_decays(lr, wd):
    p = RNG.standard_normal((2, 6, 10)).astype(np.float32)
    zero = np.zeros_like(p)
    new_p, new_buf, o = O.muon_update_fused(p, zero, zero, 0.95, True, O.COEFFICIENTS, lr, wd, 1.3)
    assert np.array_equal(new_buf, zero) and not o.any()
    assert np.array_equal(new_p, p * np.float32(1.0 - lr * wd))


@pytest.mark.parametrize("m,n", [(24, 70), (70, 24)])
def test_update_follows_the_svd_closed_form(m, n):
    """momentum 0, param 0, no decay: −p'/(lr·scale) = U·diag(q(σ'/d))·Vᵀ where σ', U, V
    are the SVD of bf16(g) and d = ‖bf16(g)‖_F·1.01 + 1e-6 (exact), within the bf16
    iteration's error after five steps."""
    g, *_ = svd_input(m, n, rng=RNG, lo=0.1, hi=1.0)
    g = g.astype(np.float32)
    lr, scale = 0.1, 1.7
    new_p, _, _ = O.muon_update_fused(np.zeros_like(g), g, np.zeros_like(g), 0.0, True,
                                      O.COEFFICIENTS, lr, 0.0, scale)
    xb = O.bf16_round(g).astype(np.float64)
    u, s, vt = np.linalg.svd(xb, full_matrices=False)
    d = np.sqrt((xb * xb).sum()) * 1.01 + 1e-6
    expected = (u * O.scalar_polynomial(s / d, O.COEFFICIENTS)) @ vt
    got = -new_p.astype(np.float64) / (lr * scale)
    # five bf16 steps and the bf16 normalisation: the reference's own 6e-2 gate
    # (tests/test_polar_step.py:42); the planted mistakes below land above 0.3
    assert O.rel_frobenius(got, expected) <= 6e-2


# ----------------------------------------------------------------------------- planted mistakes
def _blend_with_old_buffer(g, buf, beta, nesterov):
    new_buf = O.lerp_f32(buf, g, np.float32(1 - beta))
    return new_buf, O.lerp_f32(g, buf, np.float32(beta))


def _swapped_weight(g, buf, beta, nesterov):
    new_buf = O.lerp_f32(buf, g, np.float32(beta))
    return new_buf, O.lerp_f32(g, new_buf, np.float32(beta))


@pytest.mark.parametrize("mistake", [_blend_with_old_buffer, _swapped_weight],
                         ids=lambda f: f.__name__)
def test_momentum_closed_form_catches_planted_mistakes(mistake):
    beta = 0.9
    g = RNG.standard_normal((8, 24)).astype(np.float32)
    buf = np.zeros_like(g)
    worst = 0.0
    for k in range(1, 6):
        buf, u = mistake(g, buf, beta, True)
        worst = max(worst, np.abs(u - (1.0 - beta ** (k + 1)) * g).max())
    assert worst > 1e-2


def test_decay_closed_form_catches_planted_mistake():
    p = RNG.standard_normal((6, 10)).astype(np.float32)
    lr, wd = 0.1, 0.2
    wrong = p * np.float32(1.0 - wd)  # decay without the learning rate
    assert not np.array_equal(wrong, p * np.float32(1.0 - lr * wd))


@pytest.mark.parametrize("alpha_of", [lambda lr, s: +lr * s, lambda lr, s: -lr / s],
                         ids=["sign_flip", "inverted_scale"])
def test_svd_closed_form_catches_planted_update_mistakes(alpha_of):
    g, *_ = svd_input(24, 70, rng=RNG, lo=0.1, hi=1.0)
    g = g.astype(np.float32)
    lr, scale = 0.1, 1.7
    _, _, o = O.muon_update_fused(np.zeros_like(g), g, np.zeros_like(g), 0.0, True,
                                  O.COEFFICIENTS, lr, 0.0, scale)
    wrong = np.float32(alpha_of(lr, scale)) * o.astype(np.float32)
    xb = O.bf16_round(g).astype(np.float64)
    u, s, vt = np.linalg.svd(xb, full_matrices=False)
    d = np.sqrt((xb * xb).sum()) * 1.01 + 1e-6
    expected = (u * O.scalar_polynomial(s / d, O.COEFFICIENTS)) @ vt
    assert O.rel_frobenius(-wrong.astype(np.float64) / (lr * scale), expected) > 0.3
