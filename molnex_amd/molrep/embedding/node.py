"""Node embeddings (src/molrep/embedding/node.py:96-187): per-spec nn.Embedding / Linear,
concatenated and projected by a scalar equivariant Linear (node.py:153-159)."""

from __future__ import annotations

import torch
import torch.nn as nn
from pydantic import BaseModel, Field

from ..interaction.linear import Linear


class DiscreteEmbeddingSpec(BaseModel):
    input_key: str | tuple[str, ...]
    num_classes: int = Field(..., gt=0)
    emb_dim: int = Field(..., gt=0)


class ContinuousEmbeddingSpec(BaseModel):
    input_key: str | tuple[str, ...]
    in_dim: int = Field(..., gt=0)
    emb_dim: int = Field(..., gt=0)
    use_bias: bool = True


class JointEmbeddingSpec(BaseModel):
    specs: list[DiscreteEmbeddingSpec | ContinuousEmbeddingSpec] = Field(..., min_length=1)
    out_dim: int = Field(..., gt=0)
    output_key: str | tuple[str, ...] = "_unused"


class JointEmbedding(nn.Module):
    def __init__(self, *, embedding_specs, out_dim: int):
        super().__init__()
        self.config = JointEmbeddingSpec(specs=embedding_specs, out_dim=out_dim)
        self.embedders = nn.ModuleList()
        for spec in self.config.specs:
            if isinstance(spec, DiscreteEmbeddingSpec):
                self.embedders.append(nn.Embedding(spec.num_classes, spec.emb_dim))
            else:
                self.embedders.append(nn.Sequential(nn.Linear(spec.in_dim, spec.emb_dim, bias=spec.use_bias)))
        total = sum(s.emb_dim for s in self.config.specs)
        self.project = nn.Sequential(Linear(f"{total}x0e", f"{out_dim}x0e"))

    def forward(self, **features: torch.Tensor) -> torch.Tensor:
        embs = []
        for i, spec in enumerate(self.config.specs):
            key = "_".join(spec.input_key) if isinstance(spec.input_key, tuple) else spec.input_key
            embs.append(self.embedders[i](features[key]))
        return self.project(torch.cat(embs, dim=-1))
