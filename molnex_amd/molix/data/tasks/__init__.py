from .neighbor_list import NeighborList

__all__ = ["NeighborList"]
