"""Message aggregation: neighbour sum of per-edge messages into their target nodes, optionally
weighted by a per-edge cutoff value, followed by an equivariant linear
(src/molrep/interaction/aggregation.py:36-117, the A-feature construction of MACE).

The sum is the ``molix::segment_sum`` HIP kernel over the targets' CSR (cutoff weights folded into
the same pass, each node row summed in a fixed order and written once); the linear is
``EquivariantLinear`` on the block-linear kernel.  Edges are ``edge_index`` rows
[source, target].  Messages of another dtype than float32 (a float64 model) are summed by torch's
``index_add`` on their device.  With ``n_nodes`` given there is no host synchronisation and the
targets are trusted to lie in ``[0, n_nodes)``; without it the size is the largest node id + 1 and
the ids are checked."""

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
        trusted = n_nodes is not None
        if not trusted:
            # the reference sizes the output by the largest node id in either column
            n_nodes = int(edge_index.max().item()) + 1 if edge_index.numel() else 0
        weights = edge_cutoff.reshape(-1) if (self.config.apply_cutoff and edge_cutoff is not None) else None
        target = edge_index[:, 1]
        if messages.dtype == torch.float32 and messages.is_cuda:
            summed = torch.ops.molix.segment_sum(messages, target, int(n_nodes), weights, not trusted)
        else:
            scaled = messages if weights is None else messages * weights.to(messages.dtype).unsqueeze(-1)
            summed = messages.new_zeros(int(n_nodes), messages.shape[1]).index_add(0, target, scaled)
        return self.linear(summed)
