from .basis_projection import BasisProjection
from .product_head import ProductHead

__all__ = ["ProductHead", "BasisProjection"]
