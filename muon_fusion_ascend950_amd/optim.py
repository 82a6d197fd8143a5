"""Muon optimizer update around the Polar Express iteration.

The reference provides the orthogonalisation only and leaves momentum, weight decay
and the parameter update to its caller (README.md:130), nanochat's Muon optimizer
(README.md:247).  This module runs that update on the GPU in one native call per
parameter (``torch.ops.muon_ascend950.muon_update``), following the published Muon
step as nanochat's ``Muon.step`` writes it:

    buf.lerp_(g, 1 - momentum)
    g = g.lerp(buf, momentum) if nesterov else buf
    X = polar_express(bf16(g))          # normalise, then one step per triple
    p.mul_(1 - lr * weight_decay)
    p.add_(X, alpha=-lr * max(1, rows / cols) ** 0.5)

in fp32 for the parameter, gradient and momentum buffer, with the iteration in bf16.
"""

from __future__ import annotations

import math

import torch

from .ops import COEFFICIENTS

# Muon.step batches parameters of one shape into one native call when each matrix is
# small (at most _GROUP_MAX_NUMEL elements): a small matrix alone leaves most CUs idle
# and its steps are latency-bound, while a batch of them runs in about the time of one.
# Batches hold at most _GROUP_BATCH_NUMEL elements (bounding the stacked copies).
_GROUP_MAX_NUMEL = 1 << 22
_GROUP_BATCH_NUMEL = 1 << 24


def default_lr_scale(rows: int, cols: int) -> float:
    """nanochat's shape factor of the learning rate: sqrt(max(1, rows / cols))."""
    return math.sqrt(max(1.0, rows / cols))


def _flat(coefficients, steps: int):
    triples = tuple(coefficients)[:steps]
    if len(triples) != steps:
        raise ValueError(f"{steps} steps need {steps} coefficient triples, got {len(triples)}")
    flat = [float(v) for t in triples for v in t]
    if len(flat) != 3 * steps:
        raise ValueError("coefficients must be (a, b, c) triples")
    return flat


@torch.no_grad()
def muon_update(param: torch.Tensor, grad: torch.Tensor, momentum_buffer: torch.Tensor, *,
                lr: float, momentum: float = 0.95, nesterov: bool = True,
                weight_decay: float = 0.0, ns_steps: int = 5, coefficients=COEFFICIENTS,
                lr_scale: float | None = None) -> None:
    """One Muon update of ``param`` (in place) and ``momentum_buffer`` (in place).

    param, momentum_buffer: float32 ``[..., M, N]`` on the GPU (leading dimensions are
    a batch of matrices); grad: same shape, float32 or bfloat16.  ``lr_scale``
    defaults to ``sqrt(max(1, M / N))``.
    """
    for name, t in (("param", param), ("grad", grad), ("momentum_buffer", momentum_buffer)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be on a ROCm GPU, got {t.device}")
    if param.dtype != torch.float32 or momentum_buffer.dtype != torch.float32:
        raise TypeError("param and momentum_buffer must be float32")
    if grad.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"grad must be float32 or bfloat16, got {grad.dtype}")
    if param.ndim < 2:
        raise ValueError(f"Muon updates matrices (ndim >= 2), got shape {tuple(param.shape)}")
    if grad.shape != param.shape or momentum_buffer.shape != param.shape:
        raise ValueError("param, grad and momentum_buffer must have one shape")
    if any(size <= 0 for size in param.shape):
        raise ValueError("all dimensions must be positive")
    rows, cols = param.shape[-2], param.shape[-1]
    scale = default_lr_scale(rows, cols) if lr_scale is None else float(lr_scale)
    flat = _flat(coefficients, ns_steps)

    def as3d(t):
        return t.reshape(-1, rows, cols)

    # the right-Gram form runs M > N when N % 8 == 0; otherwise the update runs on
    # the transposed matrices (the iteration commutes with transposition)
    transposed = rows > cols and cols % 8 != 0
    g_work = as3d(grad.float())
    if transposed:
        p_work, b_work, g_work = (as3d(t).mT.contiguous() for t in (param, momentum_buffer, g_work))
    else:
        # a contiguous tensor reshapes to a view, updated in place; others go
        # through a contiguous copy that is written back
        p_work = as3d(param) if param.is_contiguous() else as3d(param).contiguous()
        b_work = (as3d(momentum_buffer) if momentum_buffer.is_contiguous()
                  else as3d(momentum_buffer).contiguous())
    torch.ops.muon_ascend950.muon_update(p_work, g_work, b_work, float(momentum), bool(nesterov),
                                         flat, float(lr), float(weight_decay), scale)
    for work, dst in ((p_work, param), (b_work, momentum_buffer)):
        if transposed:
            dst.copy_(work.mT.reshape(dst.shape))
        elif not dst.is_contiguous():
            dst.copy_(work.reshape(dst.shape))


class Muon(torch.optim.Optimizer):
    """Muon: momentum, Polar Express orthogonalisation and a shape-scaled update, per
    matrix parameter, on the native ``muon_update`` (one call per parameter).

    Arguments as nanochat's Muon (lr, momentum, nesterov, ns_steps) plus decoupled
    weight decay and the coefficient triples of the iteration (default: the
    reference's five).  Parameters must be float32 matrices (ndim >= 2) on the GPU;
    the momentum buffer is float32, created at the first step.

    ``group_shapes``: parameters of one group that share a shape and a device, each of
    at most 4M elements, are stacked and updated in one batched call (as nanochat's
    Muon stacks same-shape parameters), in batches of at most 16M elements; each is
    updated exactly as alone except that the batch's launch plan may cut the
    iteration's sums differently (fp32 rounding of O; the momentum buffers are the
    same bits).
    """

    def __init__(self, params, lr: float = 0.02, momentum: float = 0.95, nesterov: bool = True,
                 ns_steps: int = 5, weight_decay: float = 0.0, coefficients=COEFFICIENTS,
                 group_shapes: bool = True):
        if lr < 0.0:
            raise ValueError(f"invalid learning rate {lr}")
        if not 0.0 <= momentum <= 1.0:
            raise ValueError(f"invalid momentum {momentum}")
        if weight_decay < 0.0:
            raise ValueError(f"invalid weight_decay {weight_decay}")
        if ns_steps < 1:
            raise ValueError(f"invalid ns_steps {ns_steps}")
        _flat(coefficients, ns_steps)
        defaults = dict(lr=lr, momentum=momentum, nesterov=nesterov, ns_steps=ns_steps,
                        weight_decay=weight_decay, coefficients=tuple(coefficients))
        super().__init__(params, defaults)
        self.group_shapes = bool(group_shapes)

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            kw = dict(lr=group["lr"], momentum=group["momentum"], nesterov=group["nesterov"],
                      weight_decay=group["weight_decay"], ns_steps=group["ns_steps"],
                      coefficients=group["coefficients"])
            batches = {}
            for p in group["params"]:
                if p.grad is None:
                    continue
                state = self.state[p]
                if "momentum_buffer" not in state:
                    state["momentum_buffer"] = torch.zeros_like(
                        p, dtype=torch.float32, memory_format=torch.contiguous_format)
                if not self.group_shapes or p.numel() > _GROUP_MAX_NUMEL:
                    muon_update(p, p.grad, state["momentum_buffer"], **kw)
                    continue
                key = (tuple(p.shape), p.device)
                batch = batches.setdefault(key, [[]])
                if batch[-1] and (len(batch[-1]) + 1) * p.numel() > _GROUP_BATCH_NUMEL:
                    batch.append([])
                batch[-1].append(p)
            for chunks in batches.values():
                for ps in chunks:
                    self._update_stacked(ps, kw)
        return loss

    def _update_stacked(self, ps, kw) -> None:
        """One batched update of same-shape parameters: stacked copies of the
        parameters, gradients and buffers go through one native call and are copied
        back (a single parameter is updated in place)."""
        bufs = [self.state[p]["momentum_buffer"] for p in ps]
        if len(ps) == 1:
            muon_update(ps[0], ps[0].grad, bufs[0], **kw)
            return
        params = torch.stack([p.detach() for p in ps])
        grads = torch.stack([p.grad.float() for p in ps])
        buf = torch.stack(bufs)
        muon_update(params, grads, buf, **kw)
        for i, p in enumerate(ps):
            p.copy_(params[i])
            bufs[i].copy_(buf[i])
