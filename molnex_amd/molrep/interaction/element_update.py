"""Element-specific residual update (src/molrep/interaction/element_update.py:44-158):
``h_new = h_prev + W[z] m`` through the indexed linear (one D x D matrix per element,
``weight (S, D*D)`` initialised ``randn / sqrt(D)``, element_update.py:112-118).

With ``irreps`` given (the literal MACE configuration) the per-element map is the
equivariant indexed linear over those irreps (channel mixing within each irrep,
``weight (S, weight_numel)`` ~ N(0, 1), normalised by fan-in inside ``Linear``)."""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, ConfigDict, Field

from ...config import config
from .linear import Linear


class ElementUpdateSpec(BaseModel):
    model_config = ConfigDict(arbitrary_types_allowed=True)
    hidden_dim: int = Field(..., gt=0)
    num_species: int = Field(..., gt=0)


class ElementUpdate(nn.Module):
    def __init__(self, *, hidden_dim: int, num_species: int, irreps: str | None = None):
        super().__init__()
        self.config = ElementUpdateSpec(hidden_dim=hidden_dim, num_species=num_species)
        if irreps is None:
            self.linear = Linear(f"{hidden_dim}x0e", f"{hidden_dim}x0e", internal_weights=False,
                                 weight_classes=num_species, method="indexed_linear", dtype=config.ftype)
            w = torch.randn(num_species, hidden_dim * hidden_dim, dtype=config.ftype) / (hidden_dim ** 0.5)
        else:
            self.linear = Linear(irreps, irreps, internal_weights=False, weight_classes=num_species,
                                 method="indexed_linear", dtype=config.ftype)
            w = torch.randn(num_species, self.linear.weight_numel, dtype=config.ftype)
        self.register_parameter("weight", nn.Parameter(w))

    def forward(self, h_prev: torch.Tensor, m_curr: torch.Tensor, atom_types: torch.Tensor) -> torch.Tensor:
        return h_prev + self.linear(m_curr, weight=self.weight, weight_indices=atom_types)
