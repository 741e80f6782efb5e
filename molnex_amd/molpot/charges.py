"""Charge head with per-molecule neutrality (src/molpot/composition/heads.py:120-171)."""

from __future__ import annotations

import torch
import torch.nn as nn

from .derivation import _graph_totals


class _PerGraph(torch.autograd.Function):
    """``values[batch]`` whose backward is an ``index_add_`` (atomic) instead of the sort-based
    accumulate of advanced indexing (~0.8 ms for 50k atoms into one graph)."""

    @staticmethod
    def forward(ctx, values, batch):
        ctx.save_for_backward(batch)
        ctx.n = values.shape[0]
        return values.index_select(0, batch)

    @staticmethod
    def backward(ctx, g):
        (batch,) = ctx.saved_tensors
        return g.new_zeros(ctx.n).index_add_(0, batch, g), None


class ChargeHead(nn.Module):
    def __init__(self, feature_dim: int, hidden_dim: int = 64, total_charge: float = 0.0):
        super().__init__()
        self.total_charge = total_charge
        self.mlp = nn.Sequential(nn.Linear(feature_dim, hidden_dim), nn.SiLU(), nn.Linear(hidden_dim, 1))

    def forward(self, node_features: torch.Tensor, *, batch: torch.Tensor, num_graphs: int | None = None,
                **kwargs) -> dict[str, torch.Tensor]:
        raw = self.mlp(node_features).squeeze(-1)
        trusted = num_graphs is not None  # given: no host synchronisation, batch ids trusted
        if not trusted:
            num_graphs = int(batch.max().item()) + 1
        # per-graph raw total and atom count in one segment-sum pass
        r = raw.unsqueeze(-1)
        both = _graph_totals(torch.cat([r, torch.ones_like(r)], dim=1), batch, num_graphs, trusted)
        shift = (self.total_charge - both[:, 0]) / both[:, 1].clamp(min=1)
        return {"charge": raw + _PerGraph.apply(shift, batch)}
