"""Segment sums for molix's functional API: ``scatter_sum`` and ``batch_add`` with the signatures of
src/molix/F/scatter.py:13-51, computed by the ``molix::segment_sum`` HIP kernel (rows grouped by
segment id through a CSR, each output row summed in a fixed order and written once) instead of an
atomic ``scatter_add_``.

The reduction axis is moved to the front and the remaining axes flattened into columns, so any
``dim`` reduces as one (rows, columns) segment sum.  ``index`` is the 1-D segment id of every slice
along ``dim``; an index of ``src``'s rank whose entries only vary along ``dim`` (a broadcast view,
or singleton axes elsewhere) is reduced to that 1-D form.  A full-rank index that varies along other
axes is an element-wise scatter, not a segment sum: it goes to torch's GPU ``scatter_add``, and so
does a ``src`` that is not float32 (float64 models, half precision, integer counts), which the fp32
kernel does not compute.  GPU tensors only (the HIP op raises for CPU tensors)."""

from __future__ import annotations

import math

import torch
from torch import Tensor


def _segment_ids(index: Tensor, src: Tensor, dim: int) -> Tensor | None:
    """The 1-D segment id per slice along ``dim``, or None when ``index`` varies along other axes."""
    if index.dim() == 1:
        return index
    if index.dim() != src.dim():
        raise ValueError(f"index of rank {index.dim()} does not broadcast against src of rank {src.dim()}")
    others = [a for a in range(index.dim()) if a != dim]
    if all(index.shape[a] == 1 or index.stride(a) == 0 for a in others):
        return index[tuple(slice(None) if a == dim else 0 for a in range(index.dim()))]
    return None


def scatter_sum(src: Tensor, index: Tensor, dim: int = 0, dim_size: int | None = None) -> Tensor:
    """Sum the slices of ``src`` along ``dim`` into ``dim_size`` buckets given by ``index``
    (``dim_size`` defaults to ``index.max() + 1``)."""
    dim = dim % src.dim() if src.dim() else 0
    if dim_size is None:
        dim_size = int(index.max().item()) + 1 if index.numel() else 0
    ids = _segment_ids(index, src, dim)
    if ids is None or src.dtype != torch.float32:
        if src.device.type != "cuda":
            raise RuntimeError(f"scatter_sum runs on the GPU only (got a {src.device} tensor)")
        out_shape = list(src.shape)
        out_shape[dim] = dim_size
        if ids is not None:  # a 1-D segment id per slice: broadcast it over the other axes
            shape = [1] * src.dim()
            shape[dim] = ids.shape[0]
            index = ids.reshape(shape)
        return src.new_zeros(out_shape).scatter_add(dim, index.expand_as(src), src)
    moved = src.movedim(dim, 0)
    rows = moved.reshape(moved.shape[0], math.prod(moved.shape[1:]))
    summed = torch.ops.molix.segment_sum(rows, ids.reshape(-1).to(torch.int64), int(dim_size))
    return summed.reshape(dim_size, *moved.shape[1:]).movedim(0, dim)


def batch_add(src: Tensor, batch: Tensor, dim_size: int | None = None) -> Tensor:
    """Per-graph sums of per-item rows: ``out[b] = sum_{i: batch[i] = b} src[i]``."""
    return scatter_sum(src, batch, dim=0, dim_size=dim_size)
