"""Spherical harmonics module (src/molrep/embedding/angular.py:48-104) on the HIP kernel.

Real harmonics l <= 3 in component normalisation of the normalised input
vectors, concatenated ``[Y^0, Y^1, ..., Y^l_max]``; the l = 1 block is
``sqrt(3) (x, y, z)``.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, Field

from ... import kernels  # noqa: F401


class SphericalHarmonicsSpec(BaseModel):
    l_max: int = Field(..., ge=0)
    normalize: bool = True

    @property
    def ls(self) -> list[int]:
        return list(range(self.l_max + 1))

    @property
    def output_dim(self) -> int:
        return (self.l_max + 1) ** 2


class SphericalHarmonics(nn.Module):
    def __init__(self, *, l_max: int, normalize: bool = True):
        super().__init__()
        self.config = SphericalHarmonicsSpec(l_max=l_max, normalize=normalize)
        if not self.config.normalize:
            raise ValueError("only normalize=True harmonics are implemented (the reference's setting)")
        if self.config.l_max > 3:
            raise ValueError("l_max <= 3 is supported")
        self.l_max = int(self.config.l_max)

    def forward(self, vectors: torch.Tensor) -> torch.Tensor:
        return torch.ops.molix.spherical_harmonics(vectors, self.l_max)
