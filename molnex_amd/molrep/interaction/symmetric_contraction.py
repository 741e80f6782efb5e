"""Symmetric contraction (src/molrep/interaction/symmetric_contraction.py:42-130).

As the reference configures it -- ``"{D}x0e" -> "{D}x0e"``, contraction degree
``max_body_order``, per-element weights (``original_mace=True``, :90-109) --
the product basis of scalar channels reduces to a per-channel polynomial,
``out[n, c] = sum_{k=1..nu} W[z_n, k, c] x[n, c]^k``, computed by the HIP kernel
``molix::symmetric_contraction_scalar``.  Weight layout ``(S, nu, D)``, N(0, 1)
initialisation (cuequivariance's own layout and scaling are not reachable here).
"""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, ConfigDict, Field

from ... import kernels  # noqa: F401
from ...config import config


class SymmetricContractionSpec(BaseModel):
    model_config = ConfigDict(arbitrary_types_allowed=True)
    hidden_dim: int = Field(..., gt=0)
    num_species: int = Field(..., gt=0)
    max_body_order: int = Field(2, ge=1, le=3)


class _ScalarSymmetricContraction(nn.Module):
    """Inner module standing in for cuet.SymmetricContraction (exposes contraction_degree,
    num_elements, tests/test_molzoo/test_mace.py:712-721)."""

    def __init__(self, dim: int, contraction_degree: int, num_elements: int, dtype=None):
        super().__init__()
        self.contraction_degree = contraction_degree
        self.num_elements = num_elements
        self.weight = nn.Parameter(torch.randn(num_elements, contraction_degree, dim,
                                               dtype=dtype if dtype is not None else config.ftype))

    def forward(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        return torch.ops.molix.symmetric_contraction_scalar(x, indices, self.weight)


class SymmetricContraction(nn.Module):
    def __init__(self, *, hidden_dim: int, num_species: int, max_body_order: int = 2):
        super().__init__()
        self.config = SymmetricContractionSpec(hidden_dim=hidden_dim, num_species=num_species,
                                               max_body_order=max_body_order)
        self.symmetric_contraction = _ScalarSymmetricContraction(hidden_dim, max_body_order, num_species,
                                                                 dtype=config.ftype)

    def forward(self, node_features: torch.Tensor, atom_types: torch.Tensor) -> torch.Tensor:
        return self.symmetric_contraction(node_features, atom_types)
