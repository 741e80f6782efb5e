"""Symmetric contraction (src/molrep/interaction/symmetric_contraction.py:42-130).

As the reference configures it -- ``"{D}x0e" -> "{D}x0e"``, contraction degree
``max_body_order``, per-element weights (``original_mace=True``, :90-109) --
the product basis of scalar channels reduces to a per-channel polynomial,
``out[n, c] = sum_{k=1..nu} W[z_n, k, c] x[n, c]^k``, computed by the HIP kernel
``molix::symmetric_contraction_scalar``.  Weight layout ``(S, nu, D)``, N(0, 1)
initialisation (cuequivariance's own layout and scaling are not reachable here).

``EquivariantSymmetricContraction`` is the general product basis that the
reference's cuet call computes for non-scalar irreps (``irreps_in`` =
C x (0e + 1o + .. + l_in), ``irreps_out`` = C x 0e or C x (0e + 1o), correlation
<= 3): ``B = sum_nu U_nu . W[z] (A^{(x) nu})`` with the basis of
``molnex_amd.symmetric``, run by ``molix::symmetric_contraction``.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, ConfigDict, Field

from ... import kernels  # noqa: F401
from ...config import config
from ...irreps import Irreps


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


def _chain_l(irreps: Irreps, what: str) -> tuple[int, int]:
    """(multiplicity, l_max) of ``C x (0e + 1o + .. + l_max)``; anything else is rejected."""
    muls = {b.mul for b in irreps}
    ls = [(b.ir.l, b.ir.p) for b in irreps]
    l_max = len(ls) - 1
    if len(muls) != 1 or ls != [(l, (-1) ** l) for l in range(l_max + 1)]:
        raise ValueError(f"{what} must be C x (0e + 1o + ...) with one block per l in order, got {irreps}")
    return muls.pop(), l_max


class EquivariantSymmetricContraction(nn.Module):
    """Per-element symmetric contraction of equivariant features (mirrors the arguments of
    cuet.SymmetricContraction(irreps_in, irreps_out, contraction_degree, num_elements),
    symmetric_contraction.py:100-109).  ``weight`` is ``(num_elements, paths, C)``, N(0, 1)."""

    def __init__(self, irreps_in, irreps_out, contraction_degree: int, num_elements: int, dtype=None):
        super().__init__()
        from ... import kernels as K

        self.irreps_in, self.irreps_out = Irreps(irreps_in), Irreps(irreps_out)
        C, self.l_in = _chain_l(self.irreps_in, "irreps_in")
        C_out, self.l_out = _chain_l(self.irreps_out, "irreps_out")
        if C_out != C:
            raise ValueError("irreps_in and irreps_out must have the same multiplicity")
        self.contraction_degree = contraction_degree
        self.num_elements = num_elements
        self.config_id = K.sc_config_id(self.l_in, self.l_out, contraction_degree)
        self.num_paths = K.sc_config_info(self.config_id)[2]
        self.weight = nn.Parameter(torch.randn(num_elements, self.num_paths, C,
                                               dtype=dtype if dtype is not None else config.ftype))

    def forward(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        return torch.ops.molix.symmetric_contraction(x, indices, self.weight, self.l_in, self.l_out,
                                                     self.contraction_degree)
