"""Message aggregation: neighbour sum of per-edge messages into their target nodes, optionally
weighted by a per-edge cutoff value, followed by an equivariant linear
(src/molrep/interaction/aggregation.py:36-117, the A-feature construction of MACE).

The sum is the ``molix::segment_sum`` HIP kernel over the targets' CSR (cutoff weights folded into
the same pass, each node row summed in a fixed order and written once); the linear is
``EquivariantLinear`` on the block-linear kernel.  Edges are ``edge_index`` rows
[source, target]."""

from __future__ import annotations

import torch
from pydantic import BaseModel
from torch import nn

from .linear import EquivariantLinear


class MessageAggregationSpec(BaseModel):
    irreps: str
    apply_cutoff: bool = True


class MessageAggregation(nn.Module):
    def __init__(self, *, irreps: str, apply_cutoff: bool = True):
        super().__init__()
        self.config = MessageAggregationSpec(irreps=irreps, apply_cutoff=apply_cutoff)
        self.linear = EquivariantLinear(irreps_in=irreps, irreps_out=irreps)

    def forward(self, messages: torch.Tensor, edge_index: torch.Tensor, edge_cutoff: torch.Tensor | None = None,
                n_nodes: int | None = None) -> torch.Tensor:
        if n_nodes is None:
            # the reference sizes the output by the largest node id in either column
            n_nodes = int(edge_index.max().item()) + 1 if edge_index.numel() else 0
        weights = edge_cutoff.reshape(-1) if (self.config.apply_cutoff and edge_cutoff is not None) else None
        summed = torch.ops.molix.segment_sum(messages, edge_index[:, 1], int(n_nodes), weights)
        return self.linear(summed)
