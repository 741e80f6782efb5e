"""Radial weight MLP (src/molrep/interaction/radial_mlp.py:38-93): [Linear -> SiLU] x L -> Linear."""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, ConfigDict, Field


class RadialWeightMLPSpec(BaseModel):
    model_config = ConfigDict(arbitrary_types_allowed=True)
    in_dim: int = Field(..., gt=0)
    hidden_dim: int = Field(..., gt=0)
    out_dim: int = Field(..., gt=0)
    num_layers: int = Field(2, ge=1)


class RadialWeightMLP(nn.Module):
    def __init__(self, *, in_dim: int, hidden_dim: int, out_dim: int, num_layers: int = 2):
        super().__init__()
        self.config = RadialWeightMLPSpec(in_dim=in_dim, hidden_dim=hidden_dim, out_dim=out_dim,
                                          num_layers=num_layers)
        layers: list[nn.Module] = []
        cur = in_dim
        for _ in range(num_layers):
            layers += [nn.Linear(cur, hidden_dim), nn.SiLU()]
            cur = hidden_dim
        layers.append(nn.Linear(cur, out_dim))
        self.mlp = nn.Sequential(*layers)

    def forward(self, edge_feats: torch.Tensor) -> torch.Tensor:
        return self.mlp(edge_feats)
