from .locality import NeighborList

__all__ = ["NeighborList"]
