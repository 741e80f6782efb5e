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


def radial_edge_features(rbf: "BesselRBF", cutoff_fn: nn.Module, r: torch.Tensor) -> torch.Tensor:
    """``rbf(r) * cutoff_fn(r)[..., None]`` (MACE's edge features, src/molzoo/mace.py:180-182): one
    HIP kernel each way (``molix::bessel_cutoff``) for a BesselRBF with a cosine or polynomial
    cutoff of the same radius on float32 GPU distances; the torch composition otherwise."""
    from ... import kernels as K
    from .cutoff import CosineCutoff, PolynomialCutoff

    kind = 1 if isinstance(cutoff_fn, CosineCutoff) else 2 if isinstance(cutoff_fn, PolynomialCutoff) else -1
    if (kind > 0 and isinstance(rbf, BesselRBF) and r.is_cuda and r.dtype == torch.float32
            and rbf.config.num_radial <= 32 and float(cutoff_fn.config.r_cut) == rbf.r_cut):
        # the radius is compared on the spec, not on the module's device buffer: reading a GPU
        # scalar back would synchronise the host once per forward
        exponent = cutoff_fn.exponent if kind == 2 else 0
        mu, sigma = (rbf.mu, rbf.sigma) if rbf.normalize else (None, None)
        return torch.ops.molix.bessel_cutoff(r, int(rbf.config.num_radial), rbf.r_cut, rbf.eps, mu, sigma, kind,
                                             exponent)
    return rbf(r) * cutoff_fn(r).unsqueeze(-1)

