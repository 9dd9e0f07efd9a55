# SPDX-License-Identifier: MIT
"""Sequence-level objectives on a :class:`BeamSearchResult`, differentiable
through its scores (reference python/beamgrad/losses.py)."""

from __future__ import annotations

import torch

from ._search import BeamSearchResult

__all__ = ["minimum_risk"]


def _reduce(loss: torch.Tensor, reduction: str) -> torch.Tensor:
    if reduction == "mean":
        return loss.mean()
    if reduction == "sum":
        return loss.sum()
    if reduction == "none":
        return loss
    raise ValueError(f"reduction must be 'mean', 'sum' or 'none', got {reduction!r}")


def minimum_risk(result: BeamSearchResult, costs: torch.Tensor, temperature: float = 1.0,
                 reduction: str = "mean") -> torch.Tensor:
    """Expected cost of the beams under ``softmax(scores / temperature)``; dead
    beams (-inf scores) get no probability and their costs are ignored
    (reference python/beamgrad/losses.py:139-169)."""
    if not temperature > 0:
        raise ValueError(f"temperature must be positive, got {temperature}")
    scores = result.scores if result.scores.dim() == 2 else result.scores[None]
    if tuple(costs.shape) != tuple(scores.shape):
        raise ValueError(f"costs must have the scores' shape {tuple(scores.shape)}, got {tuple(costs.shape)}")
    live = torch.isfinite(scores)
    any_live = live.any(-1, keepdim=True)
    logits = torch.where(live, scores / temperature, float("-inf"))
    logits = torch.where(any_live, logits, torch.zeros_like(logits))
    probs = torch.softmax(logits, dim=-1)
    costs = torch.where(live, costs.to(probs), 0.0)
    loss = (probs * costs).sum(-1) * any_live[:, 0]
    return _reduce(loss, reduction)
