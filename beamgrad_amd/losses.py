# SPDX-License-Identifier: MIT
"""Sequence-level objectives on a :class:`BeamSearchResult`, differentiable
through its scores (the interface of reference python/beamgrad/losses.py:
139-169: name, arguments, reductions and error texts).

``minimum_risk`` is the expected cost of the beams under a softmax of their
scores. Its gradient has a closed form, so it is one autograd node instead
of a chain of elementwise operators: with ``p = softmax(s / t)`` over an
example's live beams (finite scores) and ``r = sum_k p_k c_k``,

    d r / d s_k = p_k (c_k - r) / t        (live beams; 0 for dead ones)

An example without a live beam has risk 0 and no gradient, and the costs of
dead beams are never read (NaN there is harmless).
"""

from __future__ import annotations

import torch

from ._search import BeamSearchResult

__all__ = ["minimum_risk"]

_REDUCTIONS = ("none", "mean", "sum")  # the operator's reduction codes 0, 1, 2


class _ExpectedCost(torch.autograd.Function):
    """The loss (per-example risk [B], or its mean or sum) of scores [B, K]
    under costs [B, K], and the factor [B, K] that turns the loss's incoming
    gradient into the scores' gradient (the reduction's scale included). On
    the GPU both, the reduction too, come from one HIP launch
    (``beamgrad::minimum_risk``); CPU tensors take the same formula in torch
    operations. The backward is one multiplication."""

    generate_vmap_rule = True  # elementwise and last-dim reductions only

    @staticmethod
    def forward(scores: torch.Tensor, costs: torch.Tensor, temperature: float, reduction: str):
        if scores.is_cuda:
            return torch.ops.beamgrad.minimum_risk(scores.float(), costs, temperature, _REDUCTIONS.index(reduction))
        scale = 1.0 / scores.shape[0] if reduction == "mean" else 1.0
        live = torch.isfinite(scores)
        z = torch.where(live, scores / temperature, float("-inf"))
        top = z.amax(-1, keepdim=True)
        # rows without a live beam: every weight is 0 (exp(-inf - 0))
        w = torch.exp(z - torch.where(torch.isfinite(top), top, 0.0))
        total = w.sum(-1, keepdim=True)
        p = w / torch.where(total > 0, total, 1.0)
        c = torch.where(live, costs.to(device=p.device, dtype=p.dtype), 0.0)
        risk = (p * c).sum(-1)
        factor = (scale / temperature) * p * (c - risk[:, None])
        loss = risk if reduction == "none" else (risk.sum() if reduction == "sum" else risk.mean())
        return loss, factor

    @staticmethod
    def setup_context(ctx, inputs, output):
        _loss, factor = output
        ctx.save_for_backward(factor)
        ctx.mark_non_differentiable(factor)
        ctx.set_materialize_grads(False)

    @staticmethod
    def backward(ctx, grad_loss, _grad_factor):
        (factor,) = ctx.saved_tensors
        if grad_loss is None:
            return None, None, None, None
        g = grad_loss[:, None] if grad_loss.dim() == 1 else grad_loss
        return g * factor, None, None, None


def minimum_risk(result: BeamSearchResult, costs: torch.Tensor, temperature: float = 1.0,
                 reduction: str = "mean") -> torch.Tensor:
    """Expected cost of the beams under ``softmax(scores / temperature)``.

    ``costs[b, k]`` is the cost of beam ``k`` (no gradient needed); dead beams
    (``-inf`` scores) get no probability and their costs are ignored. The
    gradient reaches the scores, and through them the inputs of the search,
    along the paths of the beams found."""
    if not temperature > 0:
        raise ValueError(f"temperature must be positive, got {temperature}")
    scores = result.scores
    if scores.dim() == 1:
        scores = scores[None]
    if tuple(costs.shape) != tuple(scores.shape):
        raise ValueError(f"costs must have the scores' shape {tuple(scores.shape)}, got {tuple(costs.shape)}")
    if reduction not in _REDUCTIONS:
        raise ValueError(f"reduction must be 'mean', 'sum' or 'none', got {reduction!r}")
    return _ExpectedCost.apply(scores, costs, float(temperature), reduction)[0]
