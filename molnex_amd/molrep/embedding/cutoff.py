"""Cutoff envelopes (src/molrep/embedding/cutoff.py:23-161)."""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, Field


class CosineCutoffSpec(BaseModel):
    r_cut: float = Field(..., gt=0)


class CosineCutoff(nn.Module):
    """c(r) = 0.5 (cos(pi r / r_cut) + 1) for r < r_cut, else 0 (cutoff.py:56-75)."""

    def __init__(self, *, r_cut: float):
        super().__init__()
        self.config = CosineCutoffSpec(r_cut=r_cut)
        self.register_buffer("r_cut", torch.tensor(float(self.config.r_cut)), persistent=False)

    def forward(self, r: torch.Tensor) -> torch.Tensor:
        r = r.float()
        c = 0.5 * (torch.cos(torch.pi * (r / self.r_cut)) + 1.0)
        return torch.where(r < self.r_cut, c, torch.zeros_like(c))


class PolynomialCutoffSpec(BaseModel):
    r_cut: float = Field(..., gt=0)
    exponent: int = Field(6, gt=0)


class PolynomialCutoff(nn.Module):
    """1 - (p+1)(p+2)/2 x^p + p(p+2) x^(p+1) - p(p+1)/2 x^(p+2) for x = r/r_cut < 1 (cutoff.py:138-161)."""

    def __init__(self, *, r_cut: float, exponent: int = 6):
        super().__init__()
        self.config = PolynomialCutoffSpec(r_cut=r_cut, exponent=exponent)
        self.register_buffer("r_cut", torch.tensor(float(self.config.r_cut)), persistent=False)
        self.exponent = int(self.config.exponent)

    def forward(self, r: torch.Tensor) -> torch.Tensor:
        r = r.float()
        x = r / self.r_cut
        p = float(self.exponent)
        x_p = torch.pow(x, p)
        x_p1 = x_p * x
        x_p2 = x_p1 * x
        c = 1.0 - (p + 1.0) * (p + 2.0) / 2.0 * x_p + p * (p + 2.0) * x_p1 - p * (p + 1.0) / 2.0 * x_p2
        return torch.where(x < 1.0, c, torch.zeros_like(c))
