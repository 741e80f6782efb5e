"""Layer pooling (src/molpot/pooling/layer_pooling.py:18-54)."""

import torch
import torch.nn as nn


class LayerPooling(nn.Module):
    def __init__(self, reduction: str = "mean"):
        super().__init__()
        if reduction not in ("mean", "sum", "last"):
            raise ValueError(f"reduction must be 'mean', 'sum', or 'last', got '{reduction}'")
        self.reduction = reduction

    def forward(self, features: torch.Tensor) -> torch.Tensor:
        if features.ndim == 2:
            return features
        if features.ndim != 3:
            raise ValueError(f"Expected 2D or 3D tensor, got {features.ndim}D.")
        if self.reduction == "mean":
            return features.mean(dim=1)
        if self.reduction == "sum":
            return features.sum(dim=1)
        return features[:, -1]
