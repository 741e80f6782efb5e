"""Particle-mesh Ewald potential term (new: the reference has the ops but no module
that combines them, src/molix/F/pot.py:11-14).

E = E_direct(pairs within the real-space cutoff, minimum image)
  + E_reciprocal(B-spline order p on a gx x gy x gz mesh)
  - k alpha / sqrt(pi) sum_i q_i^2                      (Ewald self term)
with the influence-function moduli |b(m)|^2 of smooth PME (Essmann et al.,
J. Chem. Phys. 103, 8577 (1995), eq. 4.4) computed here once per mesh.
All three terms run on the HIP kernels; forces come from autograd through the
ops' analytic gradients.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn as nn

from .. import kernels  # noqa: F401

COULOMB_EV_A = 14.399645478425668  # e^2 / (4 pi eps0) in eV * Angstrom


def _cardinal_bspline_knots(order: int) -> np.ndarray:
    """M_order(k) at k = 1 .. order-1 by the Cox-de Boor recursion on whole arrays."""
    x = np.arange(1, order, dtype=np.float64)
    # M_2 on the integer grid 0..order
    grid = np.arange(0, order + 1, dtype=np.float64)
    m = np.maximum(0.0, 1.0 - np.abs(grid - 1.0))
    for n in range(3, order + 1):
        shifted = np.concatenate([[0.0], m[:-1]])  # M_{n-1}(x - 1)
        m = (grid * m + (n - grid) * shifted) / (n - 1)
    return m[x.astype(int)]


def bspline_moduli(K: int, order: int) -> np.ndarray:
    w = _cardinal_bspline_knots(order)
    f = np.fft.fft(np.concatenate([w, np.zeros(K - len(w))]))
    mod = (f.real ** 2 + f.imag ** 2)
    for i in range(K):
        if mod[i] < 1e-7:
            mod[i] = 0.5 * (mod[(i - 1) % K] + mod[(i + 1) % K])
    return mod


class PMEPotential(nn.Module):
    def __init__(self, *, alpha: float = 0.3, grid: tuple[int, int, int] = (128, 128, 128), order: int = 6,
                 cutoff: float = 5.0, coulomb: float = COULOMB_EV_A):
        super().__init__()
        self.alpha, self.grid, self.order, self.cutoff, self.coulomb = alpha, tuple(grid), order, cutoff, coulomb
        for name, g in zip(("xmoduli", "ymoduli", "zmoduli"), self.grid):
            self.register_buffer(name, torch.tensor(bspline_moduli(g, order), dtype=torch.float64),
                                 persistent=False)

    def forward(self, positions: torch.Tensor, charges: torch.Tensor, box: torch.Tensor,
                exclusions: torch.Tensor | None = None, pairs=None) -> torch.Tensor:
        dt = positions.dtype
        ops = torch.ops.molix
        if pairs is None:
            i, j, _, d, r = ops.neighbor_list(positions.detach(), self.cutoff, box.detach(), False)
            nb = torch.stack([i, j])
        else:
            nb, d, r = pairs
        if exclusions is None:
            exclusions = torch.full((positions.shape[0], 1), -1, dtype=torch.int32, device=positions.device)
        e_dir = ops.pme_direct(positions, charges, nb, d, r, exclusions, self.alpha, self.coulomb)
        mods = [m.to(dt) for m in (self.xmoduli, self.ymoduli, self.zmoduli)]
        # the spectrum variant of molix::pme_reciprocal keeps the convolved spectrum for the
        # backward, which then skips the second spread and forward transform
        e_rec, _ = ops.pme_reciprocal_spectrum(positions, charges, box.to(dt), *self.grid, self.order, self.alpha,
                                               self.coulomb, *mods)
        e_self = self.coulomb * self.alpha / math.sqrt(math.pi) * (charges * charges).sum()
        return e_dir + e_rec - e_self
