"""Energy aggregation and autograd forces (src/molpot/derivation/energy_aggregation.py:40-67,
force_derivation.py:28-45)."""

from __future__ import annotations

import torch
import torch.nn as nn


class EnergyAggregation(nn.Module):
    def __init__(self, pooling: str = "sum"):
        super().__init__()
        if pooling not in ("sum", "mean"):
            raise ValueError(f"pooling must be 'sum' or 'mean', got '{pooling}'")
        self.pooling = pooling

    def forward(self, node_energy: torch.Tensor, batch: torch.Tensor, num_graphs: int | None = None) -> torch.Tensor:
        if num_graphs is None:
            num_graphs = int(batch.max().item()) + 1
        energy = torch.zeros(num_graphs, dtype=node_energy.dtype, device=node_energy.device)
        energy.index_add_(0, batch, node_energy)
        if self.pooling == "mean":
            counts = torch.zeros(num_graphs, dtype=node_energy.dtype, device=node_energy.device)
            counts.index_add_(0, batch, torch.ones_like(node_energy))
            energy = energy / counts.clamp(min=1)
        return energy


class ForceDerivation(nn.Module):
    """forces = -dE/dpos by autograd; the backward through every HIP op stays on the GPU."""

    def forward(self, energy: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        return -torch.autograd.grad(energy.sum(), pos, create_graph=self.training, retain_graph=self.training)[0]
