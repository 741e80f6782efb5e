"""Module wrapper (src/molix/nn/locality.py:10-20)."""

import torch.nn as nn

from ..F import locality as F


class NeighborList(nn.Module):
    def __init__(self, cutoff, pbc=True):
        super().__init__()
        self.cutoff = cutoff
        self.pbc = pbc

    def forward(self, positions, cell):
        # the reference passes the cell whatever pbc says (pbc only appears in the repr)
        return F.get_neighbor_pairs(positions, self.cutoff, box_vectors=cell)

    def extra_repr(self):
        return f"cutoff={self.cutoff}, pbc={self.pbc}"
