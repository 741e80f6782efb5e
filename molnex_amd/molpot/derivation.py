"""Per-graph energies and autograd forces (the roles of src/molpot/derivation/energy_aggregation.py:40-67
and force_derivation.py:28-45).

``EnergyAggregation`` reduces per-atom energies to one value per graph of the batch on the
``molix::segment_sum`` HIP kernel: the atoms are grouped by graph through a CSR of ``batch`` and each
graph's atoms are added in ascending atom order into one output row (no atomics, bitwise
reproducible).  For ``"mean"`` the atom count of every graph rides along as a second column of the
same pass.  Energies of another dtype than float32 (a float64 model) are added by torch's
``index_add`` on their device instead."""

from __future__ import annotations

import torch
import torch.nn as nn

_POOLINGS = ("sum", "mean")


def _graph_totals(values: torch.Tensor, batch: torch.Tensor, num_graphs: int, trusted: bool) -> torch.Tensor:
    """Column sums of ``values`` (N, k) per graph id in ``batch``: (num_graphs, k)."""
    if values.dtype == torch.float32 and values.is_cuda:
        return torch.ops.molix.segment_sum(values, batch, num_graphs, None, not trusted)
    return values.new_zeros(num_graphs, values.shape[1]).index_add(0, batch, values)


class EnergyAggregation(nn.Module):
    """``E[b] = reduce_{i : batch[i] = b} e[i]`` with reduce = sum or mean.

    ``num_graphs`` given: no host synchronisation, and ``batch`` is trusted to lie in
    ``[0, num_graphs)`` (atoms with other ids are left out), the convention the reference's native
    ops follow for their inputs.  Without it the count is ``batch.max() + 1`` (one synchronisation)
    and the ids are checked."""

    def __init__(self, pooling: str = "sum"):
        super().__init__()
        if pooling not in _POOLINGS:
            raise ValueError(f"pooling must be 'sum' or 'mean', got '{pooling}'")
        self.pooling = pooling

    def forward(self, node_energy: torch.Tensor, batch: torch.Tensor, num_graphs: int | None = None) -> torch.Tensor:
        trusted = num_graphs is not None
        if not trusted:
            num_graphs = int(batch.max().item()) + 1 if batch.numel() else 0
        e = node_energy.reshape(-1, 1)
        if self.pooling == "sum":
            return _graph_totals(e, batch, num_graphs, trusted).reshape(num_graphs)
        # one pass for the sums and the atom counts (exact in fp32 below 2^24 atoms per graph)
        both = _graph_totals(torch.cat([e, torch.ones_like(e)], dim=1), batch, num_graphs, trusted)
        return both[:, 0] / both[:, 1].clamp(min=1)


class ForceDerivation(nn.Module):
    """forces = -dE/dpos by autograd; the backward through every HIP op stays on the GPU."""

    def forward(self, energy: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        return -torch.autograd.grad(energy.sum(), pos, create_graph=self.training, retain_graph=self.training)[0]
