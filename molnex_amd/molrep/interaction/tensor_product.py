"""Channelwise tensor-product convolution (src/molrep/interaction/tensor_product.py:33-149)
on the fused HIP gather / TP / scatter kernels.

``ConvTP`` keeps the reference constructor, ``forward(node_features,
edge_angular, edge_index, tp_weights)``, ``weight_numel``, ``config`` and a
``cue_tp`` attribute with ``irreps_in1`` / ``irreps_in2`` / ``irreps_out`` /
``weight_numel`` (tests/test_molzoo/test_mace.py:412-422).
"""

from __future__ import annotations

import warnings

import torch
import torch.nn as nn
from pydantic import BaseModel

from ... import kernels as K
from ...config import config
from ...irreps import ChannelwiseTPDescriptor, Irrep, Irreps
from ...irreps import irreps_from_l_max as _irreps_from_l_max
from ...irreps import sh_irreps_from_l_max as _sh_irreps_from_l_max


class ConvTPSpec(BaseModel):
    in_irreps: str
    out_irreps: str
    sh_irreps: str


def _compiled_ls(irreps: Irreps) -> list[int] | None:
    """The l's of ``irreps`` when it has the form of the compiled configurations (natural parity,
    ascending l, one block per l), else None."""
    ls = [b.ir.l for b in irreps]
    if any(b.ir.p != (-1) ** b.ir.l for b in irreps) or ls != sorted(set(ls)):
        return None
    return ls


class EdgeGraph:
    """Receiver CSR of one edge list, built once and reused by every layer (its indices are
    validated once, here: one host synchronisation per graph, when ``config.validate_edges``);
    the sender CSR (for the atomic-free backward, ``config.deterministic``) is built on first
    use."""

    def __init__(self, edge_index: torch.Tensor, num_nodes: int):
        self.edge_index = edge_index
        self.num_nodes = num_nodes
        self.row_ptr, self.perm, self.senders = torch.ops.molix.edge_csr(edge_index, num_nodes,
                                                                         config.validate_edges)
        self._sender_csr = None
        self._pairs = None  # (features tensor, its version, EdgePairs or None)
        self._gh_batches = None

    def pairs(self, feats: torch.Tensor):
        """The undirected pairs of this graph whose two edges have bit-identical rows of ``feats``
        (``kernels.EdgePairs``; None when some edge has no such partner).  Built on the first
        features tensor; for later ones (new positions on the same edge list) the pairing is kept
        if the features of every pair still agree, else rebuilt: one host synchronisation per new
        features tensor, or none with ``config.verify_pairs = False``, which trusts the first
        pairing for later positions."""
        p = self._pairs
        if p is None or p[0] is not feats or p[1] != feats._version:
            prev = p[2] if p is not None else None
            if prev is not None and feats.shape[0] == prev.wrow.shape[0] and (
                    not config.verify_pairs or prev.holds_for(feats)):
                built = prev
            else:
                built = K.EdgePairs.build(self.edge_index, self.num_nodes, self.row_ptr, self.perm, self.senders,
                                          feats.detach())
            self._pairs = p = (feats, feats._version, built)
        return p[2]

    def gh_batches(self):
        """Work list of the fused output-layer gradient (``kernels.tp_gh_batches``), built on first
        use (one host synchronisation per graph)."""
        if self._gh_batches is None:
            self._gh_batches = K.tp_gh_batches(self.row_ptr)
        return self._gh_batches

    def sender_csr(self):
        if self._sender_csr is None:
            # same edges as the receiver CSR, already validated
            self._sender_csr = torch.ops.molix.edge_csr(self.edge_index.flip(1), self.num_nodes, False)
        return self._sender_csr


_graph_cache: dict = {}


def _key(t: torch.Tensor):
    return (t.data_ptr(), t.shape, t.stride(), t._version, t.device)


def _cached_graph(key, sources, make) -> EdgeGraph:
    g = _graph_cache.get(key)
    if g is None or any(a is not b for a, b in zip(g._sources, sources)):
        _graph_cache.clear()
        g = make()
        g._sources = sources
        _graph_cache[key] = g
    return g


def edge_graph(edge_index: torch.Tensor, num_nodes: int) -> EdgeGraph:
    """The EdgeGraph of ``edge_index``, cached on the tensor's storage and version so every layer of
    one step shares it.  Under torch.compile / torch.export the CSR is built in the traced graph."""
    if torch.compiler.is_compiling():
        return EdgeGraph(edge_index, num_nodes)
    return _cached_graph(("ei", _key(edge_index), num_nodes), (edge_index,),
                         lambda: EdgeGraph(edge_index, num_nodes))


def edge_graph_from_indices(indices_1: torch.Tensor, indices_out: torch.Tensor, num_nodes: int) -> EdgeGraph:
    """The EdgeGraph of separate sender / receiver index vectors (the cuet call form), cached on
    both tensors so repeated calls with the same indices share one CSR."""
    if torch.compiler.is_compiling():
        return EdgeGraph(torch.stack([indices_1, indices_out], dim=1), num_nodes)
    return _cached_graph(("pair", _key(indices_1), _key(indices_out), num_nodes), (indices_1, indices_out),
                         lambda: EdgeGraph(torch.stack([indices_1, indices_out], dim=1), num_nodes))


class ChannelWiseTensorProduct(nn.Module):
    """Channelwise TP x (mul x ir1) (x) Y (1 x ir2) -> mul x ir3 with per-edge weights,
    gathered from senders and summed into receivers (ir_mul layout)."""

    def __init__(self, irreps_in1, irreps_in2, irreps_out_filter):
        super().__init__()
        self.descriptor = ChannelwiseTPDescriptor(irreps_in1, irreps_in2, irreps_out_filter)
        self.irreps_in1 = self.descriptor.irreps_in1
        self.irreps_in2 = self.descriptor.irreps_in2
        self.irreps_out = self.descriptor.irreps_out
        self.weight_numel = self.descriptor.weight_numel
        self.channels = self.descriptor.mul
        # the straight-line kernels compiled per configuration (uniform multiplicity, natural parity,
        # one block per l), else the table-driven kernels of molix::tp_any (any irreps, l <= 3)
        self.config_id = -1
        self.any_table = None
        in_ls, sh_ls = _compiled_ls(self.irreps_in1), _compiled_ls(self.irreps_in2)
        out_irs = {b.ir for b in self.irreps_out}
        if self.channels is not None and in_ls is not None and sh_ls is not None and all(
                ir.p == (-1) ** ir.l for ir in out_irs):
            out_ls = sorted({ir.l for ir in out_irs})
            self.config_id = K.tp_config_id(in_ls, sh_ls, out_ls) if out_ls else -1
        if self.config_id >= 0:
            num_paths, nx, ny, no = K.tp_config_info(self.config_id)
            if num_paths != self.descriptor.num_paths or no * self.channels != self.irreps_out.dim:
                raise RuntimeError("compiled tensor-product configuration does not match the path descriptor")
        else:
            self.any_table = K.tp_any_table(self.descriptor)

    def forward(self, x, y, weight, indices_1=None, indices_out=None, size_out=None):
        num_nodes = int(size_out) if size_out is not None else x.shape[0]
        return self.apply_graph(x, y, weight, edge_graph_from_indices(indices_1, indices_out, num_nodes))

    def apply_graph(self, x, y, weight, g: EdgeGraph):
        if self.config_id < 0:
            if config.deterministic:
                warnings.warn("config.deterministic: the table-driven tensor product (irreps outside the compiled "
                              "configurations) accumulates grad_x and grad_Y with atomics; its gradients are not "
                              "bitwise reproducible", stacklevel=2)
            return torch.ops.molix.tp_any(x, y, weight, g.row_ptr, g.perm, g.senders, self.any_table)
        extra = g.sender_csr() if config.deterministic else ()
        return torch.ops.molix.tp_scatter(x, y, weight, g.row_ptr, g.perm, g.senders, self.config_id, self.channels,
                                          *extra)


class ConvTP(nn.Module):
    """Channelwise tensor product for equivariant message passing, fused with the
    gather from senders (edge_index[:, 0]) and the scatter-sum into receivers
    (edge_index[:, 1])."""

    def __init__(self, *, in_irreps: str, out_irreps: str, sh_irreps: str):
        super().__init__()
        self.config = ConvTPSpec(in_irreps=in_irreps, out_irreps=out_irreps, sh_irreps=sh_irreps)
        self.cue_tp = ChannelWiseTensorProduct(Irreps(in_irreps), Irreps(sh_irreps), Irreps(out_irreps))
        self.weight_numel = self.cue_tp.weight_numel

    def forward(self, node_features: torch.Tensor, edge_angular: torch.Tensor, edge_index: torch.Tensor,
                tp_weights: torch.Tensor) -> torch.Tensor:
        g = edge_graph(edge_index, node_features.shape[0])
        return self.cue_tp.apply_graph(node_features, edge_angular, tp_weights, g)

    def forward_radial(self, node_features: torch.Tensor, edge_angular: torch.Tensor, edge_index: torch.Tensor,
                       radial_mlp, edge_feats: torch.Tensor) -> torch.Tensor:
        """``forward(..., tp_weights=radial_mlp(edge_feats))`` (the composition of mace.py:321-332).
        When the MLP's parameters need no gradient (energy + forces with a fixed model) and no second
        derivatives are taken (eval mode), and every edge has an opposite edge with bit-identical
        radial features (a neighbor list's pairs), the MLP runs once per undirected pair and the
        product reads each pair's weights for both directions (``molix::radial_tp_pairs``): the same
        weights as per edge, half the MLP work and half the weight tensor.  Otherwise, with
        ``config.fused_weight_grad``, the output layer and the product run as ``molix::radial_tp``,
        whose backward forms the per-edge weight gradient in registers (``molix::tp_weight_grad``)."""
        last = radial_mlp.mlp[-1]
        x = node_features
        if self.cue_tp.config_id < 0:  # table-driven product: no fused forms
            return self.forward(x, edge_angular, edge_index, radial_mlp(edge_feats))
        if (config.paired_radial and not self.training and x.is_cuda and x.dtype == torch.float32
                and edge_feats.dim() == 2 and not config.deterministic and not torch.compiler.is_compiling()
                and not any(p.requires_grad for p in radial_mlp.parameters())
                and K.edge_weights_supported(last.in_features, last.out_features)):
            g = edge_graph(edge_index, x.shape[0])
            pairs = g.pairs(edge_feats)
            if pairs is not None:
                h = radial_mlp.hidden(torch.ops.molix.gather_rows(edge_feats, pairs.lead))
                batches = None
                fuse = config.fused_weight_grad
                if fuse is None:  # automatic: products of scalar inputs only (see config.py)
                    fuse = all(b.ir.l == 0 for b in self.cue_tp.irreps_in1)
                if fuse and K.tp_weight_grad_supported(self.cue_tp.config_id, self.cue_tp.channels,
                                                       last.in_features):
                    batches = g.gh_batches()
                out, _ = torch.ops.molix.radial_tp_pairs(x, edge_angular, h, last.weight, last.bias, g.row_ptr,
                                                         g.perm, g.senders, pairs.wrow, pairs.pairs,
                                                         self.cue_tp.config_id, self.cue_tp.channels, batches)
                return out
        if (config.fused_weight_grad is True and not self.training and x.is_cuda and x.dtype == torch.float32
                and not config.deterministic and not last.weight.requires_grad
                and (last.bias is None or not last.bias.requires_grad)
                and K.tp_weight_grad_supported(self.cue_tp.config_id, self.cue_tp.channels, last.in_features)
                and K.edge_weights_supported(last.in_features, last.out_features)):
            h = radial_mlp.hidden(edge_feats)
            g = edge_graph(edge_index, x.shape[0])
            out, _ = torch.ops.molix.radial_tp(x, edge_angular, h, last.weight, last.bias, g.row_ptr, g.perm,
                                               g.senders, g.edge_index, self.cue_tp.config_id,
                                               self.cue_tp.channels)
            return out
        return self.forward(x, edge_angular, edge_index, radial_mlp(edge_feats))


def irreps_from_l_max(l_max: int, hidden_dim: int) -> str:
    return _irreps_from_l_max(l_max, hidden_dim)


def sh_irreps_from_l_max(l_max: int) -> str:
    return _sh_irreps_from_l_max(l_max)


__all__ = ["ConvTP", "ConvTPSpec", "ChannelWiseTensorProduct", "irreps_from_l_max", "sh_irreps_from_l_max",
           "EdgeGraph", "edge_graph", "edge_graph_from_indices", "Irrep"]
