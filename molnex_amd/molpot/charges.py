"""Charge head with per-molecule neutrality (src/molpot/composition/heads.py:120-171)."""

from __future__ import annotations

import torch
import torch.nn as nn


class ChargeHead(nn.Module):
    def __init__(self, feature_dim: int, hidden_dim: int = 64, total_charge: float = 0.0):
        super().__init__()
        self.total_charge = total_charge
        self.mlp = nn.Sequential(nn.Linear(feature_dim, hidden_dim), nn.SiLU(), nn.Linear(hidden_dim, 1))

    def forward(self, node_features: torch.Tensor, *, batch: torch.Tensor, num_graphs: int | None = None,
                **kwargs) -> dict[str, torch.Tensor]:
        raw = self.mlp(node_features).squeeze(-1)
        if num_graphs is None:
            num_graphs = int(batch.max().item()) + 1
        s = torch.zeros(num_graphs, dtype=raw.dtype, device=raw.device).index_add_(0, batch, raw)
        cnt = torch.zeros(num_graphs, dtype=raw.dtype, device=raw.device).index_add_(0, batch, torch.ones_like(raw))
        shift = (self.total_charge - s) / cnt.clamp(min=1)
        return {"charge": raw + shift[batch]}
