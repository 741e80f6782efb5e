"""Per-atom energy MLP (src/molpot/heads/heads.py:13-41)."""

import torch
import torch.nn as nn


class AtomicEnergyMLP(nn.Module):
    def __init__(self, hidden_dim: int = 64):
        super().__init__()
        self.mlp = nn.Sequential(nn.Linear(hidden_dim, hidden_dim), nn.SiLU(), nn.Linear(hidden_dim, 1))

    def forward(self, atoms_h: torch.Tensor) -> torch.Tensor:
        return self.mlp(atoms_h).squeeze(-1)
