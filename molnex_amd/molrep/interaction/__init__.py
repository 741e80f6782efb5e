from .aggregation import MessageAggregation, MessageAggregationSpec
from .element_update import ElementUpdate, ElementUpdateSpec
from .linear import EquivariantLinear, EquivariantLinearSpec, Linear
from .radial_mlp import RadialWeightMLP, RadialWeightMLPSpec
from .symmetric_contraction import (EquivariantSymmetricContraction, SymmetricContraction,
                                   SymmetricContractionSpec)
from .tensor_product import ConvTP, ConvTPSpec, irreps_from_l_max, sh_irreps_from_l_max

__all__ = ["ConvTP", "ConvTPSpec", "irreps_from_l_max", "sh_irreps_from_l_max", "RadialWeightMLP",
           "RadialWeightMLPSpec", "EquivariantLinear", "EquivariantLinearSpec", "Linear", "SymmetricContraction",
           "SymmetricContractionSpec", "EquivariantSymmetricContraction", "ElementUpdate", "ElementUpdateSpec",
           "MessageAggregation", "MessageAggregationSpec"]
