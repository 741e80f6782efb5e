"""Energy + forces composition around an encoder, as the reference composes it
(tests/test_molzoo/test_symmetry.py:88-124): recompute bond vectors from
positions (so autograd reaches them), encode, mean over layers, per-atom energy
MLP, per-graph sum, forces = -dE/dpos.  The bond vectors come from
``molix::bond_vectors`` (one gather kernel forward, one kernel backward)."""

from __future__ import annotations

import torch
import torch.nn as nn

from .. import kernels
from .derivation import EnergyAggregation, ForceDerivation
from .heads import AtomicEnergyMLP
from .pooling import LayerPooling


class EnergyForceModel(nn.Module):
    def __init__(self, encoder: nn.Module, hidden_dim: int):
        super().__init__()
        self.encoder = encoder
        self.pool = LayerPooling("mean")
        self.energy = AtomicEnergyMLP(hidden_dim=hidden_dim)
        self.aggregate = EnergyAggregation("sum")
        self.forces = ForceDerivation()

    def forward(self, Z, pos, edge_index, batch, num_graphs: int, compute_forces: bool = True):
        if compute_forces and not pos.requires_grad:
            pos = pos.requires_grad_(True)
        bond_diff = kernels.bond_vectors(pos, edge_index)
        bond_dist = bond_diff.norm(dim=-1).clamp(min=1e-6)
        feats = self.encoder(Z=Z, bond_dist=bond_dist, bond_diff=bond_diff, edge_index=edge_index)
        energy = self.aggregate(self.energy(self.pool(feats)), batch, num_graphs)
        if not compute_forces:
            return energy, None
        return energy, self.forces(energy, pos)
