"""CPU oracle for one Polar Express step — TEST INFRASTRUCTURE ONLY.

This module restates the reference's algorithm on the CPU so that tests can
check the HIP path against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
or the reported CPU baseline; the product path (``muon_fusion_ascend950_amd``)
never calls it and has no CPU fallback.

What it restates (reference file:line):

* ``reference_formula`` — the reference's own oracle, ``tests/test_polar_step.py:22-28``:
  ``gram = x @ x.mT; polynomial = b*gram + c*(gram@gram); out = a*out + polynomial@out``,
  looped over coefficient triples.  ``reference_formula_torch`` runs it in torch with the
  caller's dtype (bf16 like the reference test, or fp32); ``polar_step_f64`` runs one step
  in float64 numpy.
* ``make_input`` — the input recipe of ``tests/test_polar_step.py:38-39`` (bf16 N(0,1),
  divided per matrix by ``‖x‖_F·1.01 + 1e-6``) with a seeded CPU generator.
* ``polar_step_fused`` — the rounding points the kernels implement, which follow the
  reference kernels' storage choices (``csrc/muon_polar_step_binding.cpp:641-664``: A and P
  are bf16 tensors; ``.asc:407`` RNE cast of A; ``.asc:929-940`` P = RNE(b·A + c·A²) in
  fp32) and, for Y, one rounding of ``a·X + P·X`` (the reference instead rounds P·X, a·X and
  the sum separately in bf16, ``.asc:1472-1476``).  Products are summed exactly (float64),
  so it differs from a kernel only by the kernel's fp32 accumulation error.
* ``bf16_round`` / ``f32_to_bf16_bits`` — round-to-nearest-even from the IEEE definition,
  as ``FloatToBf16Bits`` (``csrc/muon_polar_step_binding.cpp:156-162``), plus NaN/inf
  handling.
* ``pad_crop_step`` — the reference binding's pad-to-128/16 + crop semantics
  (``csrc/muon_polar_step_binding.cpp:630-672``), to show masking equals padding.
* ``wrapper_step`` — the Python wrapper's M > N transpose policy (``muon_ascend950/ops.py:24-33``).
* ``normalize_reference_rounding`` — the normalisation of ``tests/test_polar_step.py:39`` and
  ``examples/five_steps.py:18`` with torch's bf16 rounding points (for ``polar_express``).
* ``sparse_sign_input`` / ``polar_step_fused_sparse`` — ``polar_step_fused`` on sparse ±1
  inputs whose sums are exact in fp32 in any order, so a kernel must match it bit for bit
  at full size whatever its K split (no reference counterpart: a test device).
* ``lerp_f32`` / ``muon_momentum`` / ``muon_param_update`` / ``muon_update_fused`` — the
  Muon optimizer update around the iteration, which the reference leaves to its caller
  (README.md:130) and whose algorithm lives in a dependency absent from the reference
  tree: nanochat's ``Muon.step`` (karpathy/nanochat ``nanochat/muon.py``; the reference
  was extracted from SwanHubX/nanochat-ascend PR #15, commit ae3d3a6b, README.md:247;
  no pinned copy is available here).  Restated from the published Muon step (momentum
  ``buf.lerp_(g, 1 - β)``, Nesterov ``g.lerp_(buf, β)``, orthogonalisation, ``p.add_(O,
  alpha=-lr·sqrt(max(1, rows/cols)))``) plus decoupled weight decay ``p·(1 − lr·wd)``, in
  float32 with every operation rounded on its own (torch.lerp's two-branch form, ATen
  Lerp.h), the iteration with the rounding points above.

How each function is pinned (``tests/test_oracle.py``, ``tests/test_muon_oracle.py``): SVD
closed form (one step maps singular values σ -> aσ + bσ³ + cσ⁵, five steps compose),
textbook special cases of each stage, brute-force loops on tiny inputs, bf16 rounding
against torch's RNE conversion, for the Muon update the closed forms of momentum under a
constant gradient, weight decay alone and the update's singular values, torch.lerp within
one ulp, and planted mistakes that must fail those checks.
"""

from __future__ import annotations

import numpy as np

# tests/test_polar_step.py:13-19 (= examples/five_steps.py:7-13 = README.md:101-107)
COEFFICIENTS = (
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
)


# ----------------------------------------------------------------------------- bf16
def f32_to_bf16_bits(x) -> np.ndarray:
    """Round float32 values to bf16 (nearest, ties to even); returns uint16 bit patterns.

    binding.cpp:156-162 adds 0x7FFF + lsb to the raw bits; NaNs are kept quiet NaNs
    (a plain add could carry a NaN payload into infinity).
    """
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = f.view(np.uint32)
    # u + 0x7FFF + lsb stays below 2^32 for every non-NaN pattern (the largest,
    # -inf = 0xFF800000, gives 0xFF807FFF); NaN lanes are replaced below.
    t = u >> 16
    t &= 1
    t += np.uint32(0x7FFF)
    t += u
    t >>= 16
    rounded = t.astype(np.uint16)
    nan = np.isnan(f)
    if np.any(nan):
        rounded = np.where(nan, ((u >> 16).astype(np.uint16) | np.uint16(0x0040)), rounded)
    return rounded


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16)).astype(np.uint32)
    b <<= 16
    return b.view(np.float32)


def bf16_round(x) -> np.ndarray:
    """Value of x (any float dtype) after float32 then bf16 RNE rounding, as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


# ----------------------------------------------------------------------------- inputs
def make_input(shape, seed: int = 0):
    """bf16 torch CPU tensor per tests/test_polar_step.py:38-39, seeded.

    randn in bf16 from a CPU generator, then x / (‖x‖_F(last two dims)·1.01 + 1e-6),
    evaluated in bf16 on the CPU so every box gets the same bits.
    """
    import torch

    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, dtype=torch.bfloat16, generator=gen)
    return x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)


def normalize_reference_rounding(x: np.ndarray) -> np.ndarray:
    """x / (‖x‖_F·1.01 + 1e-6) per matrix with the rounding points of the reference
    recipe as torch evaluates it on bf16 tensors (tests/test_polar_step.py:39,
    examples/five_steps.py:18): the norm rounded to bf16, the product with 1.01 (as
    fp32) rounded to bf16, the sum with 1e-6 (as fp32) rounded to bf16, then an fp32
    division rounded to bf16.  The sum of squares is exact (float64) here; a kernel
    summing in fp32 can differ only where the norm sits at a bf16 rounding boundary.
    x must hold bf16 values (float64 array)."""
    x = np.asarray(x, dtype=np.float64)
    norm = bf16_round(np.sqrt((x * x).sum(axis=(-2, -1), keepdims=True)))
    d = bf16_round(norm * np.float32(1.01))
    d = bf16_round(d + np.float32(1e-6))
    return bf16_round(x.astype(np.float32) / d).astype(np.float64)


def to_numpy_f64(t) -> np.ndarray:
    return t.detach().to("cpu").float().numpy().astype(np.float64)


# ----------------------------------------------------------------------------- formula
def _mT(x: np.ndarray) -> np.ndarray:
    return np.swapaxes(x, -1, -2)


def gram_f64(x: np.ndarray) -> np.ndarray:
    """A = X·Xᵀ (tests/test_polar_step.py:25)."""
    x = np.asarray(x, dtype=np.float64)
    return x @ _mT(x)


def poly_f64(gram: np.ndarray, b: float, c: float) -> np.ndarray:
    """P = b·A + c·A·A (tests/test_polar_step.py:26)."""
    g = np.asarray(gram, dtype=np.float64)
    return b * g + c * (g @ g)


def apply_f64(poly: np.ndarray, x: np.ndarray, a: float) -> np.ndarray:
    """Y = a·X + P·X (tests/test_polar_step.py:27)."""
    x = np.asarray(x, dtype=np.float64)
    return a * x + np.asarray(poly, dtype=np.float64) @ x


def polar_step_f64(x: np.ndarray, a: float, b: float, c: float) -> np.ndarray:
    """One step in float64 (the formula of tests/test_polar_step.py:22-28)."""
    return apply_f64(poly_f64(gram_f64(x), b, c), x, a)


def reference_formula_f64(x: np.ndarray, coefficients) -> np.ndarray:
    out = np.asarray(x, dtype=np.float64)
    for a, b, c in coefficients:
        out = polar_step_f64(out, a, b, c)
    return out


def reference_formula_torch(x, coefficients):
    """tests/test_polar_step.py:22-28, in x's dtype and on x's device.

    The transposed operand is materialised (``.contiguous()``) before the product:
    same values, but batched bf16 products with a transposed right operand have
    faulted ROCm GPUs, so no such call is made.
    """
    import torch

    out = x
    for a, b, c in coefficients:
        gram = torch.matmul(out, out.mT.contiguous())
        polynomial = b * gram + c * torch.matmul(gram, gram)
        out = a * out + torch.matmul(polynomial, out)
    return out


# ----------------------------------------------------------------------------- kernel rounding points
def polar_step_fused(x: np.ndarray, a: float, b: float, c: float, return_stages: bool = False):
    """One step with the kernels' rounding points, exact sums.

    A = bf16(X·Xᵀ); P = bf16(b·A + c·(A·A)) with b, c as fp32; Y = bf16(a·X + P·X) with
    a as fp32.  X must hold bf16 values.
    """
    x = np.asarray(x, dtype=np.float64)
    a32, b32, c32 = (float(np.float32(v)) for v in (a, b, c))
    gram = bf16_round(gram_f64(x)).astype(np.float64)
    poly = bf16_round(b32 * gram + c32 * (gram @ gram)).astype(np.float64)
    y = bf16_round(a32 * x + poly @ x).astype(np.float64)
    if return_stages:
        return y, gram, poly
    return y


def five_step_fused(x: np.ndarray, coefficients=COEFFICIENTS) -> np.ndarray:
    out = np.asarray(x, dtype=np.float64)
    for a, b, c in coefficients:
        out = polar_step_fused(out, a, b, c)
    return out


# ----------------------------------------------------------------------------- exact-sum inputs
def sparse_sign_input(shape, nnz_per_row: int, seed: int = 0):
    """Sparse X with entries in {-1, 0, +1}: ``nnz_per_row`` distinct random columns per
    row, random signs.  Returns a list of scipy CSR matrices, one per batch matrix.

    With such inputs (and small integer coefficients) every sum a kernel forms is an
    integer far below 2^24, so its fp32 accumulation is exact in any order: split-K,
    tile shape and summation order cannot change a single bit, and the kernel output
    must equal ``polar_step_fused`` exactly.
    """
    import scipy.sparse as sp

    *lead, m, n = shape
    batch = int(np.prod(lead)) if lead else 1
    rng = np.random.default_rng(seed)
    mats = []
    for _ in range(batch):
        cols = np.argsort(rng.random((m, n)), axis=1)[:, :nnz_per_row] if n <= 4096 else \
            np.stack([rng.choice(n, nnz_per_row, replace=False) for _ in range(m)])
        vals = rng.choice(np.array([-1.0, 1.0]), size=(m, nnz_per_row))
        rows = np.repeat(np.arange(m), nnz_per_row)
        mats.append(sp.csr_matrix((vals.ravel(), (rows, cols.ravel())), shape=(m, n)))
    return mats


def _bf16_round_sparse(mat):
    out = mat.tocsr(copy=True)
    out.data = bf16_round(out.data).astype(np.float64)
    out.eliminate_zeros()
    return out


def polar_step_fused_sparse(x_csr, a: float, b: float, c: float, return_stages: bool = False):
    """``polar_step_fused`` for one sparse matrix (scipy CSR, float64 values).

    Same rounding points (A = bf16(X·Xᵀ), P = bf16(b·A + c·A·A), Y = bf16(a·X + P·X),
    coefficients rounded to fp32), exact float64 sums.  Returns (Y as a dense float64
    array, max_sum), where max_sum bounds every partial sum a kernel accumulates (the sum
    of |terms| of any output), so the caller can check that fp32 accumulation is exact
    (max_sum < 2^24 with integer data).  With ``return_stages`` also A and P (dense).
    """
    a32, b32, c32 = (float(np.float32(v)) for v in (a, b, c))
    x = x_csr.tocsr().astype(np.float64)
    ax = abs(x)
    gram = _bf16_round_sparse(x @ x.T)
    ag = abs(gram)
    poly = _bf16_round_sparse(b32 * gram + c32 * (gram @ gram)).toarray()
    # P·X as (Xᵀ·Pᵀ)ᵀ: sparse times dense, cost nnz(X)·m; rounded in that
    # (contiguous) transposed layout, transposed once at the end
    yt = bf16_round(a32 * x.T.toarray() + x.T @ poly.T)
    y = np.ascontiguousarray(yt.T).astype(np.float64)
    max_col = np.diff(x.tocsc().indptr).max()
    max_sum = max(
        (ax @ ax.T).max(),
        (ag @ ag).max() * abs(c32) + ag.max() * abs(b32),
        np.abs(poly).max() * max_col + abs(a32),
    )
    if return_stages:
        return y, float(max_sum), gram.toarray(), poly
    return y, float(max_sum)


# ----------------------------------------------------------------------------- boundary semantics
def pad_crop_step(x: np.ndarray, a: float, b: float, c: float, step=polar_step_fused):
    """Reference binding semantics (binding.cpp:630-672): zero-pad rows to a multiple of
    128 and columns to max(multiple of 16, padded rows), run, crop."""
    x = np.asarray(x, dtype=np.float64)
    *lead, m, n = x.shape
    rows = -(-m // 128) * 128
    cols = max(-(-n // 16) * 16, rows)
    padded = np.zeros((*lead, rows, cols), dtype=np.float64)
    padded[..., :m, :n] = x
    return step(padded, a, b, c)[..., :m, :n]


def wrapper_step(x: np.ndarray, a: float, b: float, c: float, step=polar_step_fused):
    """ops.py:24-33: [M,N] -> [1,M,N]; transpose when M > N; undo both afterwards."""
    x = np.asarray(x, dtype=np.float64)
    squeeze = x.ndim == 2
    work = x[None] if squeeze else x
    transposed = work.shape[-2] > work.shape[-1]
    if transposed:
        work = _mT(work)
    out = step(work, a, b, c)
    if transposed:
        out = _mT(out)
    return out[0] if squeeze else out


# ----------------------------------------------------------------------------- metrics
def rel_frobenius(actual, expected) -> float:
    """‖actual − expected‖_F / ‖expected‖_F over the whole tensor."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    den = np.linalg.norm(expected.ravel())
    return float(np.linalg.norm((actual - expected).ravel()) / (den if den > 0 else 1.0))


def bf16_ulp_distance(a_bits, b_bits) -> np.ndarray:
    """Distance in bf16 units in the last place between two arrays of bf16 bit patterns."""

    def ordered(bits):
        v = np.asarray(bits, dtype=np.uint16).astype(np.int32)
        return np.where(v & 0x8000, 0x8000 - v, v)  # monotone map of bf16 to integers

    return np.abs(ordered(a_bits) - ordered(b_bits))


def scalar_polynomial(sigma, coefficients) -> np.ndarray:
    """Singular-value map of the steps: σ -> aσ + bσ³ + cσ⁵, composed over triples."""
    s = np.asarray(sigma, dtype=np.float64)
    for a, b, c in coefficients:
        s = a * s + b * s**3 + c * s**5
    return s



# ----------------------------------------------------------------------------- Muon update
def lerp_f32(start, end, w) -> np.ndarray:
    """torch.lerp's two-branch form (ATen Lerp.h) in float32, each operation rounded on its
    own: start + w·(end − start) for |w| < 0.5, else end − (end − start)·(1 − w)."""
    start = np.asarray(start, dtype=np.float32)
    end = np.asarray(end, dtype=np.float32)
    w = np.float32(w)
    if abs(w) < np.float32(0.5):
        return start + w * (end - start)
    return end - (end - start) * (np.float32(1.0) - w)


def muon_momentum(grad, buf, momentum: float, nesterov: bool):
    """nanochat Muon.step: ``buf.lerp_(g, 1 - momentum)``; the iteration's input is
    ``g.lerp(buf, momentum)`` (Nesterov) or ``buf``.  Weights rounded to fp32 as
    torch does with Python floats: (float)(1 − momentum), (float)momentum.
    Returns (new buf, iteration input), float32."""
    new_buf = lerp_f32(buf, grad, np.float32(1.0 - momentum))
    u = lerp_f32(grad, new_buf, np.float32(momentum)) if nesterov else new_buf
    return new_buf, u


def muon_param_update(param, o, lr: float, weight_decay: float, lr_scale: float) -> np.ndarray:
    """param·(float)(1 − lr·wd) + (float)(−lr·lr_scale)·O in float32, each operation
    rounded on its own (``p.mul_(1 - lr*wd); p.add_(O, alpha=-lr*scale)``)."""
    decay = np.float32(1.0 - lr * weight_decay)
    alpha = np.float32(-lr * lr_scale)
    return np.asarray(param, dtype=np.float32) * decay + alpha * np.asarray(o, dtype=np.float32)


def muon_update_fused(param, grad, buf, momentum: float, nesterov: bool, coefficients, lr: float,
                      weight_decay: float, lr_scale: float):
    """One Muon update of float32 [..., M, N] arrays: momentum, bf16 input, normalisation
    and steps with the kernels' rounding points (M > N through the wrapper's transpose,
    which the right-Gram form equals), then the parameter update.
    Returns (new param, new buf, O) as float32, float32, float64."""
    new_buf, u = muon_momentum(grad, buf, momentum, nesterov)
    x = normalize_reference_rounding(bf16_round(u).astype(np.float64))
    for a, b, c in coefficients:
        x = wrapper_step(x, a, b, c)
    return muon_param_update(param, x, lr, weight_decay, lr_scale), new_buf, x
