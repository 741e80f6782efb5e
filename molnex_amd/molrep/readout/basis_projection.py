"""Identity basis projection (src/molrep/readout/basis_projection.py:93-108)."""

import torch
import torch.nn as nn


class BasisProjection(nn.Module):
    def __init__(self, *, hidden_dim: int, num_radial: int = 8, l_max: int = 2, max_body_order: int = 2):
        super().__init__()
        self.hidden_dim = hidden_dim

    def forward(self, basis_tensor: torch.Tensor) -> torch.Tensor:
        return basis_tensor
