from .angular import SphericalHarmonics, SphericalHarmonicsSpec
from .cutoff import CosineCutoff, CosineCutoffSpec, PolynomialCutoff, PolynomialCutoffSpec
from .node import ContinuousEmbeddingSpec, DiscreteEmbeddingSpec, JointEmbedding, JointEmbeddingSpec
from .radial import BesselRBF, BesselRBFSpec, radial_edge_features

__all__ = ["SphericalHarmonics", "SphericalHarmonicsSpec", "CosineCutoff", "CosineCutoffSpec", "PolynomialCutoff",
           "PolynomialCutoffSpec", "BesselRBF", "BesselRBFSpec", "JointEmbedding", "JointEmbeddingSpec",
           "DiscreteEmbeddingSpec", "ContinuousEmbeddingSpec", "radial_edge_features"]
