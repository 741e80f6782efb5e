"""fp64 CPU restatement of the Allegro edge encoder -- TEST INFRASTRUCTURE ONLY.

Follows src/molzoo/allegro.py: pair embedding (:137-249: Bessel x polynomial cutoff, harmonics of
the bond direction, concatenated source / destination type embeddings, scalar MLP with SiLU after
every Linear, per-channel environment weights times the harmonics), then per layer (:407-480)
env-scaled tensor track, harmonics summed onto each source node and normalised (1/sqrt of the
constant average or of the node's out-degree), the channelwise product of the scaled track with
the source's aggregated harmonics (shared weights, one per path and channel), the equivariant
projection back to the tensor irreps, the latent MLP on [scalars, l = 0 block] with the residual
a x + b MLP, and the output env scaling; per-layer scalars times the cutoff, stacked (:606-642).

Written with this oracle's pieces (harmonics as explicit polynomials, coupling tensors from the
null-space construction of ``oracle.equivariant``, the product as one einsum per path, the
equivariant linear per irrep block from ``oracle.mace_ref``); parameters are read by name from
the product model's ``state_dict``.  Pinned by: the pieces' own checks (``oracle.equivariant``,
``oracle.mace_ref``), rotation invariance of the scalar edge features in float64 for l_max 1-3, and
a planted output-block-order mistake that breaks it (tests/test_allegro_cpu.py).  Only the product's paths whose output irrep is an input
irrep feed the projection (the reference's ``cuet.Linear(tp.irreps_out, irreps_in)`` connects
nothing else), so only those are evaluated here; the weight rows are picked from the full path
enumeration (input block, harmonics block, l3 ascending).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import equivariant as EQ
from .mace_ref import _irr_str, linear, sh_torch


def bessel_normalised(r, r_max, num, samples=4096):
    """sqrt(2/rc) sin(n pi r / rc) / r, standardised by its mean / std over a uniform fp32 grid
    on (0, rc] (the BesselRBF normalisation)."""
    freqs = torch.arange(1, num + 1, dtype=torch.float64) * (math.pi / r_max)
    pref = math.sqrt(2.0 / r_max)
    rs = torch.linspace(1e-8, r_max, samples, dtype=torch.float32)
    raw = pref * torch.sin(rs[:, None] * freqs.float()) / (rs[:, None] + 1e-8)
    mu, sig = raw.mean(0).double(), raw.std(0).clamp(min=1e-8).double()
    return (pref * torch.sin(r[:, None] * freqs) / (r[:, None] + 1e-8) - mu) / sig


def polynomial_cutoff(r, r_max, p):
    x = r / r_max
    c = 1.0 - (p + 1) * (p + 2) / 2 * x ** p + p * (p + 2) * x ** (p + 1) - p * (p + 1) / 2 * x ** (p + 2)
    return torch.where(x < 1.0, c, torch.zeros_like(c))


def _mlp(t, prefix, x, n_linear, act_after_last):
    for j in range(n_linear):
        x = x @ t[f"{prefix}.{2 * j}.weight"].T + t[f"{prefix}.{2 * j}.bias"]
        if j < n_linear - 1 or act_after_last:
            x = torch.nn.functional.silu(x)
    return x


def _n_linear(t, prefix):
    return sum(1 for k in t if k.startswith(prefix + ".") and k.endswith(".weight"))


def edge_tp(V, Ye, weight, l_max, F):
    """Per-edge channelwise product of V (E, D*F) with Ye (E, D): kept paths only, outputs
    sorted by irrep (stable), weights (1, P_full*F) in full path order."""
    ls = list(range(l_max + 1))
    tp = EQ.ChannelwiseTP(_irr_str(ls, F), _irr_str(ls), _irr_str(ls, F), F)
    full = [(l1, l2, l3) for l1 in ls for l2 in ls for l3 in range(abs(l1 - l2), l1 + l2 + 1)]
    kept = [k for k, (l1, l2, l3) in enumerate(full) if (l1 + l2 + l3) % 2 == 0 and l3 <= l_max]
    assert len(kept) == len(tp.paths)
    w = weight.reshape(len(full), F)[kept]
    E = V.shape[0]
    xs = V.reshape(E, tp.nx, F)
    out = V.new_zeros(E, tp.no, F)
    for k, p in enumerate(tp.paths):
        s1, s2, s3 = tp._blocks(k)
        cf = torch.from_numpy(np.ascontiguousarray(tp._coef(p)))
        out[:, s3] = torch.einsum("abc,eaC,eb,C->ecC", cf, xs[:, s1], Ye[:, s2], w[k])
    blocks = [(F, tp.paths[k][4], tp.paths[k][5]) for k in sorted(range(len(tp.paths)),
                                                                     key=lambda k: tp.out_pos[k])]
    return out.reshape(E, -1), blocks


def allegro_features(sd: dict, cfg: dict, Z, bond_dist, bond_diff, edge_index):
    """(E, num_layers, num_scalar_features) in float64 from the model's state_dict.  Entries that
    already are float64 CPU tensors requiring grad are used as given (so autograd reaches them)."""
    t = {k: v if (v.dtype == torch.float64 and v.device.type == "cpu" and v.requires_grad) else
         v.detach().double().cpu() for k, v in sd.items()}
    l_max, F, nl = cfg["l_max"], cfg["num_tensor_features"], cfg["num_layers"]
    rc, nb, pp = cfg["r_max"], cfg["num_bessel"], cfg.get("poly_p", 6)
    alpha = cfg.get("residual_alpha", 0.5)
    avg = cfg.get("avg_num_neighbors")
    src, dst = edge_index[:, 0], edge_index[:, 1]
    N, E = Z.shape[0], edge_index.shape[0]
    D = (l_max + 1) ** 2
    fcut = polynomial_cutoff(bond_dist, rc, pp)
    radial = bessel_normalised(bond_dist, rc, nb) * fcut[:, None]
    Y = sh_torch(l_max, bond_diff / (bond_dist[:, None] + 1e-8))
    emb = t["embedding.type_embedding.weight"]
    s = _mlp(t, "embedding.scalar_mlp", torch.cat([radial, emb[Z[src]], emb[Z[dst]]], 1),
             _n_linear(t, "embedding.scalar_mlp"), True)
    env = s @ t["embedding.tensor_env.weight"].T + t["embedding.tensor_env.bias"]
    V = (Y[:, :, None] * env[:, None, :]).reshape(E, D * F)
    a, b = 1 / math.sqrt(1 + alpha * alpha), alpha / math.sqrt(1 + alpha * alpha)
    out = []
    for i in range(nl):
        p = f"layers.{i}"
        env_w = s @ t[f"{p}.env_embed.weight"].T + t[f"{p}.env_embed.bias"]
        Vs = (V.reshape(E, D, F) * env_w[:, None, :]).reshape(E, D * F)
        nodeY = torch.zeros(N, D, dtype=torch.float64).index_add(0, src, Y)
        if avg is not None:
            nodeY = nodeY / math.sqrt(avg)
        else:
            deg = torch.zeros(N, dtype=torch.float64).index_add(0, src, torch.ones(E, dtype=torch.float64))
            nodeY = nodeY / deg.clamp(min=1).sqrt()[:, None]
        tp_out, blocks = edge_tp(Vs, nodeY[src], t[f"{p}.tp.weight"], l_max, F)
        new = linear(tp_out, t[f"{p}.tp_linear.weight"], blocks, [(F, l, (-1) ** l) for l in range(l_max + 1)])
        mlp = _mlp(t, f"{p}.latent_mlp", torch.cat([s, new[:, :F]], 1), _n_linear(t, f"{p}.latent_mlp"), False)
        s = a * s + b * mlp
        env_o = s @ t[f"{p}.tensor_env.weight"].T + t[f"{p}.tensor_env.bias"]
        V = (new.reshape(E, D, F) * env_o[:, None, :]).reshape(E, D * F)
        out.append(s * fcut[:, None])
    return torch.stack(out, 1)
