"""Reduction of the layer axis of multi-layer encoder features (the LayerPooling module of
src/molpot/pooling/layer_pooling.py:18-54): (atoms, layers, features) -> (atoms, features);
(atoms, features) passes through.  Reductions: mean, sum, or the last layer."""

from __future__ import annotations

import torch
import torch.nn as nn


def _mean(f: torch.Tensor) -> torch.Tensor:
    return f.mean(dim=1)


def _sum(f: torch.Tensor) -> torch.Tensor:
    return f.sum(dim=1)


def _last(f: torch.Tensor) -> torch.Tensor:
    return f.select(1, f.shape[1] - 1)


_REDUCTIONS = {"mean": _mean, "sum": _sum, "last": _last}


class LayerPooling(nn.Module):
    def __init__(self, reduction: str = "mean"):
        super().__init__()
        if reduction not in _REDUCTIONS:
            raise ValueError(f"LayerPooling: unknown reduction {reduction!r} (one of {', '.join(_REDUCTIONS)})")
        self.reduction = reduction

    def forward(self, features: torch.Tensor) -> torch.Tensor:
        rank = features.dim()
        if rank == 3:
            return _REDUCTIONS[self.reduction](features)
        if rank == 2:
            return features
        raise ValueError(f"LayerPooling takes (atoms, features) or (atoms, layers, features), got shape "
                         f"{tuple(features.shape)}")

    def extra_repr(self) -> str:
        return f"reduction={self.reduction!r}"
