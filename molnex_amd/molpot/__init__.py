"""molpot (hot-path subset): energy / force derivation, pooling, heads, PME potential."""

from .charges import ChargeHead
from .derivation import EnergyAggregation, ForceDerivation
from .heads import AtomicEnergyMLP
from .pme import PMEPotential, bspline_moduli
from .pooling import LayerPooling

__all__ = ["EnergyAggregation", "ForceDerivation", "AtomicEnergyMLP", "LayerPooling", "ChargeHead", "PMEPotential",
           "bspline_moduli"]
