"""Python surface of the operator (reference: ``muon_ascend950/ops.py:6-33``)."""

from __future__ import annotations

import torch


# The five coefficient triples of the reference (tests/test_polar_step.py:13-19,
# examples/five_steps.py:7-13).
COEFFICIENTS = (
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
)


def _check(x) -> None:
    if not isinstance(x, torch.Tensor):
        raise TypeError("x must be a torch.Tensor")
    if x.device.type != "cuda":
        raise ValueError(f"x must be on a ROCm GPU, got {x.device}")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x must use torch.bfloat16, got {x.dtype}")
    if x.ndim not in (2, 3):
        raise ValueError(f"x must have shape [M,N] or [B,M,N], got {tuple(x.shape)}")
    if any(size <= 0 for size in x.shape):
        raise ValueError("all input dimensions must be positive")


def polar_express(x: torch.Tensor, coefficients=COEFFICIENTS, normalize: bool = True) -> torch.Tensor:
    """Normalise (optionally) and run one Polar Express step per coefficient triple.

    The loop of the reference's ``examples/five_steps.py:17-20`` in one call::

        x = x / (x.norm(dim=(-2, -1), keepdim=True) * 1.01 + 1e-6)   # if normalize
        for a, b, c in coefficients:
            x = polar_step(x, a, b, c)

    with the same rounding points for the normalisation (bf16 norm, bf16 product and
    sum, fp32 division rounded to bf16) and the same steps as ``polar_step``; the
    workspace and launch plans are shared by all steps.  Shapes and the ``M > N``
    policy are those of ``polar_step`` (the iteration commutes with transposition,
    and so does the Frobenius norm).
    """
    _check(x)
    flat = [float(v) for triple in coefficients for v in triple]
    if len(flat) % 3 != 0:
        raise ValueError("coefficients must be (a, b, c) triples")
    if not flat and not normalize:
        raise ValueError("nothing to do: no coefficients and normalize=False")
    squeeze_batch = x.ndim == 2
    work = x.unsqueeze(0) if squeeze_batch else x
    tall = work.size(-2) > work.size(-1)
    if tall and work.size(-1) % 8 == 0:  # right-Gram form, no transposed copies
        out = torch.ops.muon_ascend950.polar_express(work, flat, bool(normalize))
        return out.squeeze(0) if squeeze_batch else out
    transposed = tall
    if transposed:
        work = work.mT.contiguous()
    out = torch.ops.muon_ascend950.polar_express(work, flat, bool(normalize))
    if transposed:
        out = out.mT.contiguous()
    return out.squeeze(0) if squeeze_batch else out


def polar_step(x: torch.Tensor, a: float, b: float, c: float) -> torch.Tensor:
    """Run one Polar Express iteration and return a tensor with the same shape.

    ``x`` must be a BF16 ROCm (HIP) tensor with shape ``[M,N]`` or ``[B,M,N]``.
    ``M > N`` runs the right-Gram form (``N % 8 == 0``) or, otherwise, transposes
    around the native operator as the reference's wrapper does (ops.py:26-32).
    Non-aligned dimensions are handled by masked edge tiles inside the kernels.
    """
    _check(x)
    squeeze_batch = x.ndim == 2
    work = x.unsqueeze(0) if squeeze_batch else x
    tall = work.size(-2) > work.size(-1)
    if tall and work.size(-1) % 8 == 0:
        # M > N in the right-Gram form Y = a·X + X·(b·G + c·G²), G = XᵀX: the same
        # step without the two transposed copies (equal to them bit for bit when no
        # stage is cut by stream-K; to bf16 precision otherwise, since which tiles are
        # cut follows each form's tile order)
        out = torch.ops.muon_ascend950.polar_step_tall(work, float(a), float(b), float(c))
        return out.squeeze(0) if squeeze_batch else out
    transposed = tall
    if transposed:
        work = work.mT.contiguous()

    out = torch.ops.muon_ascend950.polar_step(work, float(a), float(b), float(c))
    if transposed:
        out = out.mT.contiguous()
    return out.squeeze(0) if squeeze_batch else out
