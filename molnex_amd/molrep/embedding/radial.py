"""Bessel radial basis (src/molrep/embedding/radial.py:36-148).

phi_n(r) = sqrt(2/r_cut) sin(n pi r / r_cut) / (r + eps), optionally shifted and
scaled by per-channel mean / std of r ~ U[eps, r_cut] from a 4096-point grid
(radial.py:117-147).  Elementwise on E x num_radial values: torch ops on the
GPU tensors it is given.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
from pydantic import BaseModel, Field


class BesselRBFSpec(BaseModel):
    r_cut: float = Field(..., gt=0)
    num_radial: int = Field(..., gt=0)
    eps: float = 1e-8
    normalize: bool = True
    normalize_samples: int = Field(4096, gt=0)


class BesselRBF(nn.Module):
    def __init__(self, *, r_cut: float, num_radial: int, eps: float = 1e-8, normalize: bool = True,
                 normalize_samples: int = 4096) -> None:
        super().__init__()
        self.config = BesselRBFSpec(r_cut=r_cut, num_radial=num_radial, eps=eps, normalize=normalize,
                                    normalize_samples=normalize_samples)
        self.r_cut = float(self.config.r_cut)
        num = int(self.config.num_radial)
        self.register_buffer("freqs", torch.arange(1, num + 1, dtype=torch.float32) * (math.pi / self.r_cut),
                             persistent=False)
        self.register_buffer("prefactor", torch.tensor(math.sqrt(2.0 / self.r_cut), dtype=torch.float32),
                             persistent=False)
        self.eps = float(self.config.eps)
        self.normalize = bool(self.config.normalize)
        if self.normalize:
            mu, sigma = self._compute_stats(self.config.normalize_samples)
        else:
            mu, sigma = torch.zeros(num), torch.ones(num)
        self.register_buffer("mu", mu, persistent=False)
        self.register_buffer("sigma", sigma, persistent=False)

    def _raw_basis(self, r: torch.Tensor) -> torch.Tensor:
        rr = r.unsqueeze(-1)
        return self.prefactor * torch.sin(rr * self.freqs) / (rr + self.eps)

    @torch.no_grad()
    def _compute_stats(self, n_samples: int):
        r = torch.linspace(self.eps, self.r_cut, n_samples, dtype=torch.float32)
        phi = self._raw_basis(r)
        return phi.mean(dim=0), phi.std(dim=0).clamp(min=1e-8)

    def forward(self, r: torch.Tensor) -> torch.Tensor:
        r = r.float()
        phi = self._raw_basis(r)
        if self.normalize:
            phi = (phi - self.mu) / self.sigma
        return phi
