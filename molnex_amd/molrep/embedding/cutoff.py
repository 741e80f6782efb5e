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
    """u(x) = 1 - (p+1)(p+2)/2 x^p + p(p+2) x^(p+1) - p(p+1)/2 x^(p+2) for x = r/r_cut < 1, else 0
    (cutoff.py:138-161).

    The envelope has a triple root at x = 1 (u, u', u'' vanish there), and for integer p it equals
    (1 - x)^3 * sum_{k<p} C(k+2, 2) x^k exactly; it is evaluated in that form.  The expanded sum
    cancels near the cutoff (terms of size ~50 summing to ~1e-5 at p = 6), so in fp32 it carries
    absolute errors up to ~6e-6 in u and ~3e-5 in u', against ~1e-8 for the factored form."""

    def __init__(self, *, r_cut: float, exponent: int = 6):
        super().__init__()
        self.config = PolynomialCutoffSpec(r_cut=r_cut, exponent=exponent)
        self.register_buffer("r_cut", torch.tensor(float(self.config.r_cut)), persistent=False)
        self.exponent = int(self.config.exponent)

    def forward(self, r: torch.Tensor) -> torch.Tensor:
        r = r.float()
        x = r / self.r_cut
        p = self.exponent
        # Horner form of sum_{k<p} C(k+2, 2) x^k, highest coefficient first
        g = torch.full_like(x, float((p + 1) * p // 2))
        for k in range(p - 2, -1, -1):
            g = g * x + float((k + 2) * (k + 1) // 2)
        c = (1.0 - x) ** 3 * g
        return torch.where(x < 1.0, c, torch.zeros_like(c))
