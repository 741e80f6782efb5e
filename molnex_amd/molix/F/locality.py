"""Functional locality ops (src/molix/F/locality.py:14-44): thin wrappers over torch.ops.molix."""

from __future__ import annotations

from torch import Tensor, empty, ops

from .. import ensure_op_registered


def get_neighbor_pairs(positions: Tensor, cutoff: float, max_num_pairs: int = -1,
                       box_vectors: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Half pair list (row > col) within ``cutoff``: ``(neighbors (2, W) int32, deltas, distances,
    num_pairs)``, padded with -1 / NaN to width ``max_num_pairs`` (``N(N-1)/2`` for -1)."""
    ensure_op_registered("get_neighbor_pairs")
    if box_vectors is None:
        box_vectors = empty((0, 0), device=positions.device, dtype=positions.dtype)
    return ops.molix.get_neighbor_pairs(positions, cutoff, max_num_pairs, box_vectors)


def neighbor_list(positions: Tensor, cutoff: float, box_vectors: Tensor | None = None, full: bool = True):
    """Exact-size directed (``full``) or half cell list sorted by (i, j):
    ``(i, j, shifts, deltas, distances)`` with ``deltas = pos[i] - (pos[j] + shifts)``."""
    ensure_op_registered("neighbor_list")
    if box_vectors is None:
        box_vectors = empty((0, 0), device=positions.device, dtype=positions.dtype)
    return ops.molix.neighbor_list(positions, float(cutoff), box_vectors, bool(full))
