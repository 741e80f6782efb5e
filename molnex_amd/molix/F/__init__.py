from .locality import get_neighbor_pairs, neighbor_list
from .pot import pme_direct, pme_reciprocal
from .scatter import batch_add, scatter_sum

__all__ = ["get_neighbor_pairs", "neighbor_list", "pme_direct", "pme_reciprocal", "scatter_sum", "batch_add"]
