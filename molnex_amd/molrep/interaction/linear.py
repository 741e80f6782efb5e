"""Equivariant linear layers (src/molrep/interaction/linear.py:43-105 and the
cuet.Linear calls of mace.py:270-291, element_update.py:101-109, node.py:153-159).

``Linear`` mixes channels within each irrep type: for an output block
``mul_o x ir`` and every input block ``mul_b x ir`` of the same irrep,
``out[m, o] += sum_c W_bo[c, o] x_b[m, c] / sqrt(fan_in)`` with ``fan_in`` the
total input multiplicity of that irrep (ir_mul layout, weights ~ N(0, 1)).
With ``weight_classes`` the weights are external, one set per class, selected
per row by ``weight_indices`` (cuet's indexed_linear).  Both run as GEMMs on
the GPU (hipBLASLt through torch.matmul) over the ir_mul views.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
from pydantic import BaseModel

from ...config import config
from ...irreps import Irreps


class Linear(nn.Module):
    def __init__(self, irreps_in, irreps_out, *, layout=None, internal_weights: bool = True,
                 weight_classes: int | None = None, method: str | None = None, dtype=None):
        super().__init__()
        self.irreps_in = Irreps(irreps_in)
        self.irreps_out = Irreps(irreps_out)
        self.weight_classes = weight_classes
        self.method = method
        in_off, out_off = self.irreps_in.offsets(), self.irreps_out.offsets()
        # one entry per output block: (out offset, out mul, dim, [(in offset, in mul, weight offset)], fan_in)
        self.plan = []
        woff = 0
        for ob, o in enumerate(self.irreps_out):
            srcs = []
            for ib, b in enumerate(self.irreps_in):
                if b.ir == o.ir:
                    srcs.append((in_off[ib], b.mul, woff))
                    woff += b.mul * o.mul
            fan_in = sum(s[1] for s in srcs)
            self.plan.append((out_off[ob], o.mul, o.ir.dim, srcs, fan_in))
        self.weight_numel = woff
        dt = dtype if dtype is not None else config.ftype
        if internal_weights and weight_classes is None:
            self.weight = nn.Parameter(torch.randn(1, self.weight_numel, dtype=dt))
        else:
            self.register_parameter("weight", None)

    def _mix(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """x (R, dim_in), w (weight_numel,) -> (R, dim_out)."""
        R = x.shape[0]
        outs = []
        for off_o, mul_o, d, srcs, fan_in in self.plan:
            if not srcs:
                outs.append(x.new_zeros(R, d * mul_o))
                continue
            acc = None
            for off_i, mul_i, wo in srcs:
                xb = x[:, off_i:off_i + d * mul_i].reshape(R, d, mul_i)
                wb = w[wo:wo + mul_i * mul_o].view(mul_i, mul_o)
                y = torch.matmul(xb, wb)
                acc = y if acc is None else acc + y
            outs.append((acc * (1.0 / math.sqrt(fan_in))).reshape(R, d * mul_o))
        return torch.cat(outs, dim=1) if len(outs) > 1 else outs[0]

    def forward(self, x: torch.Tensor, weight: torch.Tensor | None = None,
                weight_indices: torch.Tensor | None = None) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.irreps_in.dim)
        if self.weight_classes is None:
            w = self.weight if weight is None else weight
            out = self._mix(x2, w.reshape(-1))
        else:
            if weight is None or weight_indices is None:
                raise ValueError("indexed linear needs weight and weight_indices")
            out = x2.new_empty(x2.shape[0], self.irreps_out.dim)
            idx = weight_indices.reshape(-1)
            for cls, rows in _class_rows(idx, self.weight_classes):
                out[rows] = self._mix(x2[rows], weight[cls].reshape(-1))
        return out.reshape(*shape[:-1], self.irreps_out.dim)


def _class_rows(idx: torch.Tensor, num_classes: int):
    """Row indices of each class present (one host sync per call)."""
    order = torch.argsort(idx, stable=True)
    counts = torch.bincount(idx, minlength=num_classes).tolist()
    if len(counts) > num_classes:
        raise ValueError(f"weight_indices has a value >= weight_classes ({num_classes})")
    start = 0
    for cls, c in enumerate(counts):
        if c:
            yield cls, order[start:start + c]
        start += c


class EquivariantLinearSpec(BaseModel):
    irreps_in: str
    irreps_out: str


class EquivariantLinear(nn.Module):
    def __init__(self, *, irreps_in: str, irreps_out: str):
        super().__init__()
        self.config = EquivariantLinearSpec(irreps_in=irreps_in, irreps_out=irreps_out)
        self.irreps_in = Irreps(self.config.irreps_in)
        self.irreps_out = Irreps(self.config.irreps_out)
        self.linear = Linear(self.irreps_in, self.irreps_out, dtype=config.ftype)

    def forward(self, features: torch.Tensor) -> torch.Tensor:
        return self.linear(features)
