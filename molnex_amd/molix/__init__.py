"""molix (hot-path subset): op registration, functional ops, NeighborList task.

Mirrors src/molix/__init__.py:14-63: importing registers the ``torch.ops.molix``
library (here the HIP ops of molnex_amd.kernels instead of libmolnex_opLib.so).
"""

import torch

from .. import kernels as _kernels  # noqa: F401  registers torch.ops.molix.*
from ..config import config

_OPS = ("get_neighbor_pairs", "neighbor_list", "pme_direct", "pme_reciprocal", "spherical_harmonics",
        "edge_csr", "tp_scatter", "symmetric_contraction_scalar")


def ensure_op_registered(name: str) -> None:
    """Raise if ``torch.ops.molix.<name>`` is missing (src/molix/__init__.py:40-60)."""
    if not hasattr(torch.ops.molix, name):
        raise RuntimeError(f"torch.ops.molix.{name} is not registered; build with `python -m molnex_amd.build`")


__all__ = ["config", "ensure_op_registered"]
