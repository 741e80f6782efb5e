"""Product head (src/molrep/readout/product_head.py:45-142): symmetric contraction ->
identity projection -> nn.Linear(hidden_dim, out_dim).

``EquivariantProductHead`` is the literal MACE product block: the equivariant
symmetric contraction (irreps_in -> irreps_out, per element, correlation <= 3)
followed by an equivariant linear on irreps_out."""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, Field

from ...config import config
from ..interaction.linear import Linear
from ..interaction.symmetric_contraction import EquivariantSymmetricContraction, SymmetricContraction
from .basis_projection import BasisProjection


class ProductHeadSpec(BaseModel):
    hidden_dim: int = Field(..., gt=0)
    out_dim: int = Field(..., gt=0)
    num_radial: int = Field(8, gt=0)
    l_max: int = Field(2, ge=0)
    max_body_order: int = Field(2, ge=1, le=3)
    num_species: int = Field(118, gt=0)


class ProductHead(nn.Module):
    def __init__(self, *, hidden_dim: int, out_dim: int, num_radial: int = 8, l_max: int = 2,
                 max_body_order: int = 2, num_species: int = 118):
        super().__init__()
        self.config = ProductHeadSpec(hidden_dim=hidden_dim, out_dim=out_dim, num_radial=num_radial, l_max=l_max,
                                      max_body_order=max_body_order, num_species=num_species)
        self.symmetric_contraction = SymmetricContraction(hidden_dim=hidden_dim, num_species=num_species,
                                                          max_body_order=max_body_order)
        self.basis_projection = BasisProjection(hidden_dim=hidden_dim, num_radial=num_radial, l_max=l_max,
                                                max_body_order=max_body_order)
        self.linear = nn.Linear(hidden_dim, out_dim, dtype=config.ftype)

    def forward(self, node_features: torch.Tensor, atom_types: torch.Tensor) -> torch.Tensor:
        basis = self.symmetric_contraction(node_features, atom_types)
        return self.linear(self.basis_projection(basis))


class EquivariantProductHead(nn.Module):
    def __init__(self, *, irreps_in: str, irreps_out: str, max_body_order: int, num_species: int):
        super().__init__()
        self.symmetric_contraction = EquivariantSymmetricContraction(irreps_in, irreps_out, max_body_order,
                                                                     num_species, dtype=config.ftype)
        self.linear = Linear(irreps_out, irreps_out, dtype=config.ftype)

    def forward(self, node_features: torch.Tensor, atom_types: torch.Tensor) -> torch.Tensor:
        return self.linear(self.symmetric_contraction(node_features, atom_types))
