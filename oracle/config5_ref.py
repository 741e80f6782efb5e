"""fp64 CPU restatement of the config-5 energy + forces composition -- TEST INFRASTRUCTURE ONLY.

MACE encoder (``oracle.mace_ref``) -> layer mean -> per-atom energy MLP, summed per graph
(src/molpot/heads/heads.py:13-41, src/molpot/derivation/energy_aggregation.py:40-67), plus the
long-range term: per-atom charges from the layer-mean features with per-graph neutrality
(ChargeHead, src/molpot/composition/heads.py:120-171) fed to particle-mesh Ewald
(direct + reciprocal - self; the reciprocal and direct sums of ``oracle.pme``, which restate
src/molix/op/src/pme/pme_cpu.cpp:95-431, with this oracle's own B-spline moduli).
Forces = -dE/dpos by torch autograd in float64; the PME sums enter autograd through their
analytic gradients (energy, d/dpos, d/dq) like the reference op (pme_cpu.cpp:168-215).

Pinned by: its pieces (mace_ref: config-1 parity, O(3) invariance, finite differences, periodic
image consistency; pme: the reference op's outputs and the NaCl Madelung constant), and
end to end by finite differences of this function's own energy (tests/test_oracle_config5.py).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import mace_ref
from . import pme as PME


def charges(t: dict, feats: torch.Tensor, batch: torch.Tensor, num_graphs: int, total_charge: float = 0.0,
            prefix: str = "") -> torch.Tensor:
    """Raw per-atom charges MLP(feats) shifted per graph so each graph sums to ``total_charge``
    (heads.py:158-171): q = raw + (Q - sum_graph raw) / n_graph."""
    h = torch.nn.functional.silu(feats @ t[prefix + "mlp.0.weight"].T + t[prefix + "mlp.0.bias"])
    raw = (h @ t[prefix + "mlp.2.weight"].T + t[prefix + "mlp.2.bias"]).squeeze(-1)
    s = torch.zeros(num_graphs, dtype=raw.dtype).index_add(0, batch, raw)
    n = torch.zeros(num_graphs, dtype=raw.dtype).index_add(0, batch, torch.ones_like(raw))
    return raw + ((total_charge - s) / n.clamp(min=1))[batch]


class _PMEEnergy(torch.autograd.Function):
    """direct + reciprocal - self in fp64 NumPy, with the analytic position / charge gradients."""

    @staticmethod
    def forward(ctx, pos, q, pairs, box, grid, order, alpha, coulomb, moduli):
        nb, deltas, dist = pairs
        p = pos.detach().numpy()
        qq = q.detach().numpy()
        e_d, gp_d, gq_d = PME.direct(p, qq, nb, deltas, dist, np.zeros((p.shape[0], 0), np.int32), alpha, coulomb)
        e_r, gp_r, gq_r = PME.reciprocal(p, qq, box, grid, order, alpha, coulomb, moduli)
        self_k = coulomb * alpha / math.sqrt(math.pi)
        e = e_d + e_r - self_k * float(np.sum(qq * qq))
        ctx.save_for_backward(torch.from_numpy(gp_d + gp_r), torch.from_numpy(gq_d + gq_r - 2 * self_k * qq))
        return pos.new_tensor(e)

    @staticmethod
    def backward(ctx, g):
        gp, gq = ctx.saved_tensors
        return g * gp, g * gq, None, None, None, None, None, None, None


def half_pair_geometry(pos: torch.Tensor, rows: np.ndarray, cols: np.ndarray, shifts: np.ndarray):
    """Half-list deltas pos[row] - (pos[col] + shift) and distances in fp64 for a fixed pair list."""
    p = pos.detach().numpy()
    d = p[rows] - p[cols] - shifts
    return np.stack([rows, cols]).astype(np.int32), d, np.sqrt((d * d).sum(1))


def energy_forces(sd_model: dict, sd_charge: dict, cfg: dict, Z, pos, edge_index, shifts, batch, num_graphs: int,
                  box: np.ndarray, half_pairs, grid, order: int, alpha: float, coulomb: float):
    """Per-graph total energies and forces (fp64) of MACE + ChargeHead + PME.

    ``edge_index`` (E, 2) [source, target] with ``shifts`` (E, 3) so the bond vector is
    pos[target] - pos[source] - shift; ``half_pairs = (rows, cols, shifts)`` is the PME
    real-space pair list (row > col) with its image offsets.  Returns
    (energies (G,), forces (N, 3), charges (N,), mace energies (G,), pme energy)."""
    t = mace_ref._f64(sd_model)
    tq = mace_ref._f64(sd_charge)
    pos = pos.detach().to(torch.float64).requires_grad_(True)
    sh = torch.as_tensor(shifts, dtype=torch.float64)
    feats = torch.stack(mace_ref.mace_layers(t, cfg, Z, pos, edge_index, sh), dim=1).mean(1)
    e_atoms = mace_ref.atom_energies(t, feats)
    e_mace = torch.zeros(num_graphs, dtype=torch.float64).index_add(0, batch, e_atoms)
    q = charges(tq, feats, batch, num_graphs)
    rows, cols, pshift = half_pairs
    pairs = half_pair_geometry(pos, rows, cols, pshift)
    moduli = [PME.bspline_moduli(g, order) for g in grid]
    e_pme = _PMEEnergy.apply(pos, q, pairs, np.asarray(box, np.float64), tuple(grid), order, alpha, coulomb, moduli)
    total = e_mace.sum() + e_pme
    (g,) = torch.autograd.grad(total, pos)
    e = e_mace.detach().clone()
    e[0] += e_pme.detach()  # one periodic system: the long-range term belongs to graph 0
    return e, -g, q.detach(), e_mace.detach(), e_pme.detach()
