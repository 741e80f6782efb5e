"""MACE encoder (src/molzoo/mace.py:65-576) assembled from the HIP-backed modules.

Same constructor, attribute names (``embedding``, ``initial_projection``,
``interactions.i.{conv_tp, node_linear, radial_mlp, linear}``, ``products``,
``projections``, ``element_updates``, ``layer_norms``), in/out keys and
per-layer output ``(n_nodes, num_interactions, num_features)`` as the
reference.  ``forward`` takes the reference's GraphBatch (any mapping that
answers ``td["atoms", "Z"]`` or ``td["atoms"]["Z"]``) or keyword tensors.

``hidden_irreps`` (default None = the reference as coded, mace.py:256,428-430)
selects the literal MACE: node features carry ``hidden_irreps`` (e.g.
``"128x0e+128x1o"``; scalars only at the first layer's input), messages carry
``F x (0e+1o+..+l_max)``, the product is the equivariant symmetric contraction
onto ``hidden_irreps`` (scalars only after the last layer) followed by
equivariant linears, and the residual is the equivariant per-element linear.
Every map is then O(3)-equivariant and the energy rotation-invariant.  The
per-layer output stacked for the readout is the scalar block ``(N, F)``.
"""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, ConfigDict, Field

from ..config import config
from ..irreps import Irreps
from ..molrep.embedding.angular import SphericalHarmonics
from ..molrep.embedding.cutoff import CosineCutoff, PolynomialCutoff
from ..molrep.embedding.node import ContinuousEmbeddingSpec, DiscreteEmbeddingSpec, JointEmbedding
from ..molrep.embedding.radial import BesselRBF, radial_edge_features
from ..molrep.interaction.element_update import ElementUpdate
from ..molrep.interaction.linear import Linear
from ..molrep.interaction.radial_mlp import RadialWeightMLP
from ..molrep.interaction.tensor_product import ConvTP, irreps_from_l_max, sh_irreps_from_l_max
from ..molrep.readout.product_head import EquivariantProductHead, ProductHead


def _get(td, group: str, key: str):
    try:
        return td[group, key]
    except (KeyError, TypeError):
        return td[group][key]


def _set(td, group: str, key: str, value):
    if isinstance(td, dict):  # nested plain mappings: a tuple key would be stored as such
        td[group][key] = value
        return
    try:
        td[group, key] = value
    except (KeyError, TypeError):
        td[group][key] = value


class EmbeddingSpec(BaseModel):
    model_config = ConfigDict(arbitrary_types_allowed=True)
    node_attr_specs: list[DiscreteEmbeddingSpec | ContinuousEmbeddingSpec] = Field(..., min_length=1)
    num_features: int = Field(..., gt=0)
    r_max: float = Field(..., gt=0.0)
    num_bessel: int = Field(8, gt=0)
    l_max: int = Field(2, ge=0)


class EmbeddingBlock(nn.Module):
    """Node embedding, harmonics of the edge direction, Bessel x cutoff (mace.py:88-184)."""

    def __init__(self, *, node_attr_specs, num_features: int, r_max: float, num_bessel: int = 8, l_max: int = 2,
                 cutoff: str = "cosine"):
        super().__init__()
        self.config = EmbeddingSpec(node_attr_specs=node_attr_specs, num_features=num_features, r_max=r_max,
                                    num_bessel=num_bessel, l_max=l_max)
        self.node_embedding = JointEmbedding(embedding_specs=node_attr_specs, out_dim=num_features)
        self.radial_embedding = BesselRBF(r_cut=r_max, num_radial=num_bessel)
        self.spherical_harmonics = SphericalHarmonics(l_max=l_max)
        self.cutoff_fn = CosineCutoff(r_cut=r_max) if cutoff == "cosine" else PolynomialCutoff(r_cut=r_max)

    def forward(self, Z, bond_dist, bond_diff):
        node_feats = self.node_embedding(Z=Z)
        edge_dir = bond_diff / (bond_dist.unsqueeze(-1) + 1e-8)
        edge_attrs = self.spherical_harmonics(edge_dir)
        edge_feats = radial_edge_features(self.radial_embedding, self.cutoff_fn, bond_dist)
        return node_feats, edge_attrs, edge_feats


class InteractionSpec(BaseModel):
    model_config = ConfigDict(arbitrary_types_allowed=True)
    num_features: int = Field(..., gt=0)
    num_bessel: int = Field(8, gt=0)
    l_max: int = Field(2, ge=0)
    avg_num_neighbors: float = Field(1.0, gt=0.0)


class InteractionBlock(nn.Module):
    """node_linear -> radial MLP -> ConvTP (gather, TP, scatter) -> / avg_num_neighbors -> linear
    (mace.py:210-337)."""

    def __init__(self, *, num_features: int, num_bessel: int = 8, l_max: int = 2, avg_num_neighbors: float = 1.0,
                 irreps_in: str | None = None):
        super().__init__()
        self.config = InteractionSpec(num_features=num_features, num_bessel=num_bessel, l_max=l_max,
                                      avg_num_neighbors=avg_num_neighbors)
        irreps_str = irreps_from_l_max(l_max, num_features)
        in_str = irreps_str if irreps_in is None else irreps_in
        self.conv_tp = ConvTP(in_irreps=in_str, out_irreps=irreps_str, sh_irreps=sh_irreps_from_l_max(l_max))
        tp_out_irreps = str(self.conv_tp.cue_tp.irreps_out)
        self.node_linear = Linear(Irreps(in_str), Irreps(in_str), dtype=config.ftype)
        self.radial_mlp = RadialWeightMLP(in_dim=num_bessel, hidden_dim=num_features,
                                          out_dim=self.conv_tp.weight_numel, num_layers=2)
        self.linear = Linear(Irreps(tp_out_irreps), Irreps(irreps_str), dtype=config.ftype)
        # linear(messages) / avg_num_neighbors, with the division folded into the linear's weights
        self.linear.output_scale = 1.0 / avg_num_neighbors
        self.avg_num_neighbors = avg_num_neighbors

    def forward(self, node_feats, edge_attrs, edge_feats, edge_index):
        sc = node_feats
        node_feats_up = self.node_linear(node_feats)
        messages = self.conv_tp.forward_radial(node_feats_up, edge_attrs, edge_index, self.radial_mlp, edge_feats)
        # linear(messages / avg) == linear(messages) / avg == linear with weights / avg
        return self.linear(messages), sc


class MACESpec(BaseModel):
    model_config = ConfigDict(arbitrary_types_allowed=True)
    node_attr_specs: list[DiscreteEmbeddingSpec | ContinuousEmbeddingSpec] = Field(..., min_length=1)
    num_elements: int = Field(..., gt=0)
    num_features: int = Field(..., gt=0)
    r_max: float = Field(..., gt=0.0)
    num_bessel: int = Field(8, gt=0)
    l_max: int = Field(2, ge=0)
    num_interactions: int = Field(2, gt=0)
    correlation: int = Field(2, ge=1, le=3)
    avg_num_neighbors: float = Field(1.0, gt=0.0)
    layer_norm: bool = False
    hidden_irreps: str | None = None


class MACE(nn.Module):
    in_keys = [("atoms", "Z"), ("atoms", "pos"), ("edges", "edge_index"), ("edges", "bond_diff"),
               ("edges", "bond_dist")]
    out_keys = [("atoms", "node_features")]

    def __init__(self, *, node_attr_specs, num_elements: int, num_features: int, r_max: float, num_bessel: int = 8,
                 l_max: int = 2, num_interactions: int = 2, correlation: int = 2, avg_num_neighbors: float = 1.0,
                 layer_norm: bool = False, cutoff: str = "cosine", hidden_irreps: str | None = None):
        super().__init__()
        self.config = MACESpec(node_attr_specs=node_attr_specs, num_elements=num_elements,
                               num_features=num_features, r_max=r_max, num_bessel=num_bessel, l_max=l_max,
                               num_interactions=num_interactions, correlation=correlation,
                               avg_num_neighbors=avg_num_neighbors, layer_norm=layer_norm,
                               hidden_irreps=hidden_irreps)
        self.embedding = EmbeddingBlock(node_attr_specs=node_attr_specs, num_features=num_features, r_max=r_max,
                                        num_bessel=num_bessel, l_max=l_max, cutoff=cutoff)
        if hidden_irreps is not None:
            self._build_literal(num_features, num_elements, num_bessel, l_max, num_interactions, correlation,
                                avg_num_neighbors, hidden_irreps)
            return
        irreps_dim = Irreps(irreps_from_l_max(l_max, num_features)).dim
        self.initial_projection = nn.Linear(num_features, irreps_dim, dtype=config.ftype)
        self.interactions = nn.ModuleList([
            InteractionBlock(num_features=num_features, num_bessel=num_bessel, l_max=l_max,
                             avg_num_neighbors=avg_num_neighbors) for _ in range(num_interactions)])
        self.products = nn.ModuleList([
            ProductHead(hidden_dim=irreps_dim, out_dim=num_features, num_radial=num_bessel, l_max=l_max,
                        max_body_order=correlation, num_species=num_elements) for _ in range(num_interactions)])
        self.projections = nn.ModuleList([
            nn.Linear(num_features, irreps_dim, dtype=config.ftype) for _ in range(num_interactions)])
        self.element_updates = nn.ModuleList([
            ElementUpdate(hidden_dim=irreps_dim, num_species=num_elements)
            for _ in range(max(num_interactions - 1, 0))])
        self.layer_norms = nn.ModuleList([
            nn.LayerNorm(irreps_dim) if layer_norm else nn.Identity() for _ in range(max(num_interactions - 1, 0))])

    def _build_literal(self, F, S, num_bessel, l_max, L, correlation, avg_num_neighbors, hidden_irreps):
        hidden = Irreps(hidden_irreps)
        if {b.mul for b in hidden} != {F}:
            raise ValueError(f"hidden_irreps must have multiplicity num_features={F}, got {hidden_irreps}")
        scalars = f"{F}x0e"
        target = irreps_from_l_max(l_max, F)
        outs = [str(hidden) if i < L - 1 else scalars for i in range(L)]
        ins = [scalars] + outs[:-1]
        self.initial_projection = Linear(scalars, scalars, dtype=config.ftype)
        self.interactions = nn.ModuleList([
            InteractionBlock(num_features=F, num_bessel=num_bessel, l_max=l_max, avg_num_neighbors=avg_num_neighbors,
                             irreps_in=ins[i]) for i in range(L)])
        self.products = nn.ModuleList([
            EquivariantProductHead(irreps_in=target, irreps_out=outs[i], max_body_order=correlation, num_species=S)
            for i in range(L)])
        self.projections = nn.ModuleList([Linear(outs[i], outs[i], dtype=config.ftype) for i in range(L)])
        self.element_updates = nn.ModuleList([
            ElementUpdate(hidden_dim=F, num_species=S, irreps=outs[i]) for i in range(max(L - 1, 0))])
        self.layer_norms = nn.ModuleList([nn.Identity() for _ in range(max(L - 1, 0))])
        self._literal_dims = [(Irreps(ins[i]).dim, Irreps(outs[i]).dim) for i in range(L)]

    def _encode_literal(self, Z, bond_dist, bond_diff, edge_index) -> torch.Tensor:
        node_feats_init, edge_attrs, edge_feats = self.embedding(Z=Z, bond_dist=bond_dist, bond_diff=bond_diff)
        node_feats = self.initial_projection(node_feats_init)
        F = self.config.num_features
        per_layer = []
        for i in range(self.config.num_interactions):
            msg, sc = self.interactions[i](node_feats=node_feats, edge_attrs=edge_attrs, edge_feats=edge_feats,
                                           edge_index=edge_index)
            h = self.products[i](node_features=msg, atom_types=Z)
            per_layer.append(h[:, :F])  # the 0e block (ir_mul: its F channels come first)
            h_proj = self.projections[i](h)
            if i < self.config.num_interactions - 1:
                d_in, d_out = self._literal_dims[i]
                if d_in != d_out:  # scalars-only input: embed into the 0e block of hidden_irreps
                    sc = torch.nn.functional.pad(sc, (0, d_out - d_in))
                node_feats = self.element_updates[i](h_prev=sc, m_curr=h_proj, atom_types=Z)
            else:
                node_feats = h_proj
        return torch.stack(per_layer, dim=1)

    def encode(self, Z, bond_dist, bond_diff, edge_index) -> torch.Tensor:
        if self.config.hidden_irreps is not None:
            return self._encode_literal(Z, bond_dist, bond_diff, edge_index)
        node_feats_init, edge_attrs, edge_feats = self.embedding(Z=Z, bond_dist=bond_dist, bond_diff=bond_diff)
        node_feats = self.initial_projection(node_feats_init)
        per_layer = []
        for i in range(self.config.num_interactions):
            msg, sc = self.interactions[i](node_feats=node_feats, edge_attrs=edge_attrs, edge_feats=edge_feats,
                                           edge_index=edge_index)
            h = self.products[i](node_features=msg, atom_types=Z)
            per_layer.append(h)
            h_proj = self.projections[i](h)
            if i < self.config.num_interactions - 1:
                node_feats = self.layer_norms[i](self.element_updates[i](h_prev=sc, m_curr=h_proj, atom_types=Z))
            else:
                node_feats = h_proj
        return torch.stack(per_layer, dim=1)

    def forward(self, td=None, *, Z=None, bond_dist=None, bond_diff=None, edge_index=None):
        if td is None:
            return self.encode(Z, bond_dist, bond_diff, edge_index)
        feats = self.encode(_get(td, "atoms", "Z"), _get(td, "edges", "bond_dist"), _get(td, "edges", "bond_diff"),
                            _get(td, "edges", "edge_index"))
        _set(td, "atoms", "node_features", feats)
        return td
