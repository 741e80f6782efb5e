"""Radial weight MLP (src/molrep/interaction/radial_mlp.py:38-93): [Linear -> SiLU] x L -> Linear.

The last layer maps every edge to ``weight_numel`` tensor-product weights (at 2.6 M edges
and 2944 outputs a 30.8 GB result).  For many rows it runs as row chunks of 2^18 written
straight into one output (hipBLASLt picks a faster kernel for chunk-sized problems: 11.4 ms
instead of 14.0 ms at that size on MI355X), with an explicit backward doing the same.
``.mlp`` stays the reference's ``Sequential`` so parameters and their names are unchanged.

On the GPU in float32 the last Linear runs as ``molix::edge_weights`` (fp32-accurate products
from three-way bf16 splits on the matrix cores, bound by the store of its output rather than by
the fp32 matrix-core rate) for input widths 16/32/64/128.

When the hidden Linears' parameters need no gradient (energy + forces with fixed weights)
the hidden stack ``[Linear -> SiLU] x num_layers`` runs as one fused HIP kernel
(``molix::radial_hidden``, gradient w.r.t. the edge features only); otherwise, and for
shapes the kernel does not cover, it runs layer by layer, the Linears over many rows with their
weight gradients (and those of second derivatives) on ``molix::tall_tn`` and the SiLUs' second
derivatives in one fused pass (``kernels.silu_bwd2``).
"""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, ConfigDict, Field

from ... import kernels
from ...config import config

_CHUNK = 1 << 18


class RadialWeightMLPSpec(BaseModel):
    model_config = ConfigDict(arbitrary_types_allowed=True)
    in_dim: int = Field(..., gt=0)
    hidden_dim: int = Field(..., gt=0)
    out_dim: int = Field(..., gt=0)
    num_layers: int = Field(2, ge=1)


class _ChunkedLinear(torch.autograd.Function):
    """``x @ W^T + b`` over row chunks of ``_CHUNK``, each GEMM writing its slice of one output."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        out = x.new_empty(x.shape[0], weight.shape[0])
        wt = weight.t()
        for i in range(0, x.shape[0], _CHUNK):
            if bias is None:
                torch.mm(x[i:i + _CHUNK], wt, out=out[i:i + _CHUNK])
            else:
                torch.addmm(bias, x[i:i + _CHUNK], wt, out=out[i:i + _CHUNK])
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, g):
        x, weight = ctx.saved_tensors
        need_x, need_w, need_b = ctx.needs_input_grad
        gx = x.new_empty(x.shape) if need_x else None
        gw = torch.zeros_like(weight) if need_w else None
        g = g.contiguous()
        for i in range(0, x.shape[0], _CHUNK):
            gi = g[i:i + _CHUNK]
            if need_x:
                torch.mm(gi, weight, out=gx[i:i + _CHUNK])
            if need_w:
                gw.addmm_(gi.t(), x[i:i + _CHUNK])
        gb = g.sum(0) if (need_b and ctx.has_bias) else None
        return gx, gw, gb


_ROWS_MIN = 1 << 16


class _RowsLinear(torch.autograd.Function):
    """``x @ W^T + b`` over many rows (one per edge) whose weight gradient, summed over all rows, is
    ``molix::tall_tn`` instead of one long hipBLASLt reduction.  The input gradient is this function
    again (``g @ W``), so that second derivatives (force-matching training) also take the weight
    gradient of that product through ``tall_tn``."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        return torch.addmm(bias, x, weight.t()) if bias is not None else x @ weight.t()

    @staticmethod
    def backward(ctx, g):
        x, weight = ctx.saved_tensors
        need_x, need_w, need_b = ctx.needs_input_grad
        g = g.contiguous()
        gx = _RowsLinear.apply(g, weight.t(), None) if need_x else None
        gw = gb = None
        want_b = need_b and ctx.has_bias
        if need_w and want_b:
            gw, gb = kernels.tall_tn_colsum(g, x)
        elif need_w:
            gw = kernels.tall_tn(g, x)
        elif want_b:
            gb = g.sum(0)
        return gx, gw, gb


class _SiLU(torch.autograd.Function):
    """SiLU whose input gradient is ``_SiLUGrad``: the second derivatives of a force loss then take
    one fused HIP pass (``kernels.silu_bwd2``) instead of torch's chain of elementwise kernels."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return torch.nn.functional.silu(x)

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        return _SiLUGrad.apply(x, g)


class _SiLUGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, g):
        ctx.save_for_backward(x, g)
        return torch.ops.aten.silu_backward(g, x)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, gg):
        x, g = ctx.saved_tensors
        return kernels.silu_bwd2(x, g, gg)


def _big_rows(h: torch.Tensor) -> bool:
    return (h.is_cuda and h.dim() == 2 and h.shape[0] >= _ROWS_MIN and h.dtype == torch.float32
            and torch.is_grad_enabled())


def _linear(layer: nn.Linear, h: torch.Tensor) -> torch.Tensor:
    if _big_rows(h) and layer.weight.dtype == torch.float32 and layer.weight.requires_grad:
        return _RowsLinear.apply(h, layer.weight, layer.bias)
    return layer(h)


def _act(layer: nn.Module, h: torch.Tensor) -> torch.Tensor:
    if isinstance(layer, nn.SiLU) and _big_rows(h) and h.requires_grad:
        return _SiLU.apply(h)
    return layer(h)


class RadialWeightMLP(nn.Module):
    def __init__(self, *, in_dim: int, hidden_dim: int, out_dim: int, num_layers: int = 2):
        super().__init__()
        self.config = RadialWeightMLPSpec(in_dim=in_dim, hidden_dim=hidden_dim, out_dim=out_dim,
                                          num_layers=num_layers)
        layers: list[nn.Module] = []
        cur = in_dim
        for _ in range(num_layers):
            layers += [nn.Linear(cur, hidden_dim), nn.SiLU()]
            cur = hidden_dim
        layers.append(nn.Linear(cur, out_dim))
        self.mlp = nn.Sequential(*layers)

    def _fused_hidden(self, h: torch.Tensor) -> bool:
        if not (config.fused_radial and h.is_cuda and h.dim() == 2 and h.dtype == torch.float32):
            return False
        hidden = list(self.mlp[:-1])
        if not all(isinstance(m, nn.SiLU) for m in hidden[1::2]) or any(
                not isinstance(m, nn.Linear) or m.bias is None for m in hidden[0::2]):
            return False
        if torch.is_grad_enabled() and any(p.requires_grad for p in self.mlp[:-1].parameters()):
            return False
        c = self.config
        return kernels.radial_supported(c.in_dim, c.hidden_dim, c.num_layers)

    def hidden(self, edge_feats: torch.Tensor) -> torch.Tensor:
        """The activations fed to the output layer: ``mlp[:-1](edge_feats)``."""
        h = edge_feats
        if self._fused_hidden(h):
            c = self.config
            raw = torch.cat([t.detach().reshape(-1) for m in self.mlp[:-1:2] for t in (m.weight, m.bias)])
            return kernels.radial_hidden(h, raw, c.in_dim, c.hidden_dim, c.num_layers)
        for layer in self.mlp[:-1]:
            h = _linear(layer, h) if isinstance(layer, nn.Linear) else _act(layer, h)
        return h

    def forward(self, edge_feats: torch.Tensor) -> torch.Tensor:
        h = self.hidden(edge_feats)
        last = self.mlp[-1]
        if (config.edge_weights_kernel and h.is_cuda and h.dim() == 2 and h.dtype == torch.float32
                and last.weight.dtype == torch.float32
                and kernels.edge_weights_supported(last.in_features, last.out_features)):
            return kernels.edge_weights(h, last.weight, last.bias)
        if h.dim() == 2 and h.shape[0] > _CHUNK and h.is_cuda:
            return _ChunkedLinear.apply(h, last.weight, last.bias)
        return last(h)
