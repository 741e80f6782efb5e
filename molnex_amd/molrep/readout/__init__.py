from .basis_projection import BasisProjection
from .product_head import EquivariantProductHead, ProductHead

__all__ = ["ProductHead", "EquivariantProductHead", "BasisProjection"]
