"""fp64 CPU restatement of the MACE energy + forces pipeline -- TEST INFRASTRUCTURE ONLY.

Follows the reference's composition (src/molzoo/mace.py:151-184, 295-337,
487-544; src/molrep/readout/product_head.py:119-142;
src/molrep/interaction/element_update.py:147-158; tests/test_molzoo/
test_symmetry.py:88-124): embedding -> initial projection -> [interaction ->
product head -> projection -> element update] x L -> layer mean -> per-atom
energy MLP -> per-graph sum; forces = -dE/dpos by torch autograd in float64.

Written from the mathematics with this oracle's own pieces (not the product
modules): harmonics as explicit polynomials checked against the scipy-based
``oracle.equivariant.real_sh``; coupling tensors from ``oracle.equivariant``
(null-space construction); the channelwise product as an einsum per path;
equivariant linears per irrep block.  Parameters are read by name from the
product model's ``state_dict`` (the weights are the model's; the arithmetic is
this file's).  Parity status: the cuequivariance conventions of the reference
are unreachable, so this pins the product to the documented conventions;
energy/force consistency is pinned by finite differences (tests).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import equivariant as EQ

S3, S5, S7, S15 = math.sqrt(3), math.sqrt(5), math.sqrt(7), math.sqrt(15)


def sh_torch(l_max: int, v: torch.Tensor) -> torch.Tensor:
    r = torch.linalg.vector_norm(v, dim=-1, keepdim=True)
    u = torch.where(r > 0, v / torch.where(r > 0, r, torch.ones_like(r)), torch.zeros_like(v))
    x, y, z = u.unbind(-1)
    cols = [torch.ones_like(x)]
    if l_max >= 1:
        cols += [S3 * x, S3 * y, S3 * z]
    if l_max >= 2:
        cols += [S15 * x * y, S15 * y * z, 0.5 * S5 * (2 * z * z - x * x - y * y), S15 * x * z,
                 0.5 * S15 * (x * x - y * y)]
    if l_max >= 3:
        a, b, c = math.sqrt(35 / 8), math.sqrt(105), math.sqrt(21 / 8)
        cols += [a * y * (3 * x * x - y * y), b * x * y * z, c * y * (4 * z * z - x * x - y * y),
                 0.5 * S7 * z * (2 * z * z - 3 * x * x - 3 * y * y), c * x * (4 * z * z - x * x - y * y),
                 0.5 * b * z * (x * x - y * y), a * x * (x * x - 3 * y * y)]
    return torch.stack(cols, dim=-1)


def _irr(l_max, mul):
    return [(mul, l, (-1) ** l) for l in range(l_max + 1)]


def _irr_str(ls, C=None):
    return "+".join(f"{C}x{l}{'e' if l % 2 == 0 else 'o'}" if C else f"{l}{'e' if l % 2 == 0 else 'o'}"
                    for l in ls)


def conv_tp(x, Y, w, edge_index, num_nodes, l_max, C, in_ls=None):
    """Channelwise TP + scatter in fp64 (einsum per path; paths / layout per oracle.equivariant);
    input irreps ``C x in_ls`` (default l <= l_max), harmonics and output filter l <= l_max."""
    ls = list(range(l_max + 1))
    tp = EQ.ChannelwiseTP(_irr_str(in_ls if in_ls is not None else ls, C), _irr_str(ls), _irr_str(ls, C), C)
    E = Y.shape[0]
    xs = x.reshape(-1, tp.nx, C)
    w3 = w.reshape(E, len(tp.paths), C)
    s, r = edge_index[:, 0], edge_index[:, 1]
    out = x.new_zeros(num_nodes, tp.no, C)
    for k, p in enumerate(tp.paths):
        s1, s2, s3 = tp._blocks(k)
        cf = torch.from_numpy(np.ascontiguousarray(tp._coef(p))).to(x.dtype)
        msg = torch.einsum("abc,eaC,eb,eC->ecC", cf, xs[:, s1][s], Y[:, s2], w3[:, k])
        out[:, s3] = out[:, s3].index_add(0, r, msg)
    return out.reshape(num_nodes, -1), tp


def linear(x, weight, blocks_in, blocks_out):
    """Equivariant linear: per output block, sum over input blocks of the same irrep of
    x_b @ W / sqrt(fan_in); blocks are (mul, l, p) in ir_mul layout."""
    N = x.shape[0]
    offs_in = np.cumsum([0] + [m * (2 * l + 1) for m, l, _ in blocks_in])
    outs, woff = [], 0
    w = weight.reshape(-1)
    for mo, lo, po in blocks_out:
        d = 2 * lo + 1
        acc, fan = None, 0
        for bi, (mi, li, pi) in enumerate(blocks_in):
            if (li, pi) != (lo, po):
                continue
            xb = x[:, offs_in[bi]:offs_in[bi + 1]].reshape(N, d, mi)
            Wb = w[woff:woff + mi * mo].reshape(mi, mo)
            woff += mi * mo
            y = xb @ Wb
            acc = y if acc is None else acc + y
            fan += mi
        outs.append((acc / math.sqrt(fan)).reshape(N, d * mo))
    return torch.cat(outs, dim=1)


def bond_vectors(pos, edge_index, shifts=None):
    """pos[target] - pos[source] (src/molix/data/tasks/neighbor_list.py:86-89), minus the periodic
    image offset of the source when ``shifts`` is given (bond = pos[i] - (pos[j] + shift))."""
    d = pos[edge_index[:, 1]] - pos[edge_index[:, 0]]
    return d if shifts is None else d - shifts


def _edge_embedding(cfg, pos, edge_index, l_max, shifts=None):
    rc, nb_ = cfg["r_max"], cfg["num_bessel"]
    bond_diff = bond_vectors(pos, edge_index, shifts)
    bond_dist = bond_diff.norm(dim=-1).clamp(min=1e-6)
    edge_dir = bond_diff / (bond_dist.unsqueeze(-1) + 1e-8)
    Y = sh_torch(l_max, edge_dir)
    return Y, radial_features(bond_dist, rc, nb_, cfg.get("cutoff", "cosine"))


def bessel_stats(rc, nb_):
    """Shift / scale of the Bessel basis: mean and std of its fp32 values on 4096 points of
    [1e-8, r_cut] (radial.py:117-147)."""
    freqs = torch.arange(1, nb_ + 1, dtype=torch.float64) * (math.pi / rc)
    pref = math.sqrt(2.0 / rc)
    rs = torch.linspace(1e-8, rc, 4096, dtype=torch.float32)
    raw = (pref * torch.sin(rs[:, None] * freqs.float()) / (rs[:, None] + 1e-8))
    return raw.mean(0).double(), raw.std(0).clamp(min=1e-8).double()


def radial_features(bond_dist, rc, nb_, cutoff="cosine", p=6, normalize=True):
    """MACE's edge features: the (normalised) Bessel basis times the cutoff envelope
    (radial.py:36-148, cutoff.py:56-75 / 138-161, mace.py:180-182), in the dtype of bond_dist.  The
    polynomial envelope in the expanded form of the reference,
    1 - (p+1)(p+2)/2 x^p + p(p+2) x^(p+1) - p(p+1)/2 x^(p+2)."""
    freqs = torch.arange(1, nb_ + 1, dtype=torch.float64) * (math.pi / rc)
    pref = math.sqrt(2.0 / rc)
    phi = pref * torch.sin(bond_dist[:, None] * freqs) / (bond_dist[:, None] + 1e-8)
    if normalize:
        mu, sig = bessel_stats(rc, nb_)
        phi = (phi - mu) / sig
    if cutoff == "polynomial":
        x = bond_dist / rc
        u = (1.0 - (p + 1) * (p + 2) / 2 * x ** p + p * (p + 2) * x ** (p + 1) - p * (p + 1) / 2 * x ** (p + 2))
        fcut = torch.where(x < 1.0, u, torch.zeros_like(x))
    elif cutoff == "cosine":
        fcut = torch.where(bond_dist < rc, 0.5 * (torch.cos(math.pi * bond_dist / rc) + 1.0),
                           torch.zeros_like(bond_dist))
    else:
        fcut = torch.ones_like(bond_dist)
    return phi * fcut[:, None]


def _radial(t, p, edge_feats):
    a = edge_feats
    for j in (0, 2):
        a = torch.nn.functional.silu(a @ t[p + f"radial_mlp.mlp.{j}.weight"].T + t[p + f"radial_mlp.mlp.{j}.bias"])
    return a @ t[p + "radial_mlp.mlp.4.weight"].T + t[p + "radial_mlp.mlp.4.bias"]


def atom_energies(t, feats):
    """Per-atom energy MLP on the layer-mean features (src/molpot/heads/heads.py:13-41)."""
    e_atom = torch.nn.functional.silu(feats @ t["energy.mlp.0.weight"].T + t["energy.mlp.0.bias"])
    return (e_atom @ t["energy.mlp.2.weight"].T + t["energy.mlp.2.bias"]).squeeze(-1)


def _readout(t, per_layer, batch, num_graphs):
    feats = torch.stack(per_layer, dim=1).mean(1)
    return torch.zeros(num_graphs, dtype=torch.float64).index_add(0, batch, atom_energies(t, feats))


def _f64(sd: dict) -> dict:
    return {k: v.detach().to("cpu", torch.float64) for k, v in sd.items()}


def mace_energy_literal(sd: dict, cfg: dict, Z, pos, edge_index, batch, num_graphs, shifts=None):
    """Per-graph energies (fp64) of the literal MACE configuration (hidden irreps
    ``F x hidden_ls``, equivariant product basis and linears throughout)."""
    t = _f64(sd)
    return _readout(t, _layers_literal(t, cfg, Z, pos, edge_index, shifts), batch, num_graphs)


def _layers_literal(t: dict, cfg: dict, Z, pos, edge_index, shifts=None):
    from . import symcon as SC

    F, L, l_max, nu = cfg["num_features"], cfg["num_interactions"], cfg["l_max"], cfg["correlation"]
    hid = list(cfg["hidden_ls"])
    blk = lambda ls: [(F, l, (-1) ** l) for l in ls]  # noqa: E731
    Y, edge_feats = _edge_embedding(cfg, pos, edge_index, l_max, shifts)
    emb = t["embedding.node_embedding.embedders.0.weight"][Z]
    node = linear(emb, t["embedding.node_embedding.project.0.weight"], [(emb.shape[1], 0, 1)], [(F, 0, 1)])
    h = linear(node, t["initial_projection.weight"], blk([0]), blk([0]))
    target = list(range(l_max + 1))
    per_layer = []
    for i in range(L):
        p = f"interactions.{i}."
        in_ls = [0] if i == 0 else hid
        out_ls = hid if i < L - 1 else [0]
        sc = h
        up = linear(h, t[p + "node_linear.weight"], blk(in_ls), blk(in_ls))
        w = _radial(t, p, edge_feats)
        msg, tp = conv_tp(up, Y, w, edge_index, pos.shape[0], l_max, F, in_ls=in_ls)
        msg = msg / cfg["avg_num_neighbors"]
        order = sorted(tp.out_pos, key=tp.out_pos.get)
        m = linear(msg, t[p + "linear.weight"], [(F, tp.paths[k][4], tp.paths[k][5]) for k in order], blk(target))
        B = SC.contract(m, Z, t[f"products.{i}.symmetric_contraction.weight"], l_max, max(out_ls), nu)
        hp = linear(B, t[f"products.{i}.linear.weight"], blk(out_ls), blk(out_ls))
        per_layer.append(hp[:, :F])
        proj = linear(hp, t[f"projections.{i}.weight"], blk(out_ls), blk(out_ls))
        if i < L - 1:
            sc = torch.nn.functional.pad(sc, (0, proj.shape[1] - sc.shape[1]))
            Wu = t[f"element_updates.{i}.weight"]
            upd = torch.zeros_like(proj)
            for s_ in range(Wu.shape[0]):
                sel = Z == s_
                if sel.any():
                    upd[sel] = linear(proj[sel], Wu[s_], blk(out_ls), blk(out_ls))
            h = sc + upd
        else:
            h = proj
    return per_layer


def mace_energy(sd: dict, cfg: dict, Z, pos, edge_index, batch, num_graphs, shifts=None):
    """Per-graph energies (fp64) of the MACE-as-coded pipeline with the parameters ``sd``
    (the literal configuration when ``cfg`` names ``hidden_ls``)."""
    t = _f64(sd)
    return _readout(t, mace_layers(t, cfg, Z, pos, edge_index, shifts), batch, num_graphs)


def mace_layers(t: dict, cfg: dict, Z, pos, edge_index, shifts=None):
    """Per-layer scalar features (the encoder output, mace.py:487-544) in fp64, from fp64
    parameters ``t``; the literal configuration when ``cfg`` names ``hidden_ls``."""
    if cfg.get("hidden_ls") is not None:
        return _layers_literal(t, cfg, Z, pos, edge_index, shifts)
    F, L, l_max = cfg["num_features"], cfg["num_interactions"], cfg["l_max"]
    rc, nb_, nu = cfg["r_max"], cfg["num_bessel"], cfg["correlation"]
    D = F * (l_max + 1) ** 2
    blocks = _irr(l_max, F)
    bond_diff = bond_vectors(pos, edge_index, shifts)
    bond_dist = bond_diff.norm(dim=-1).clamp(min=1e-6)
    # embedding (mace.py:170-184)
    emb = t["embedding.node_embedding.embedders.0.weight"][Z]
    node = linear(emb, t["embedding.node_embedding.project.0.weight"], [(emb.shape[1], 0, 1)], [(F, 0, 1)])
    edge_dir = bond_diff / (bond_dist.unsqueeze(-1) + 1e-8)
    Y = sh_torch(l_max, edge_dir)
    freqs = torch.arange(1, nb_ + 1, dtype=torch.float64) * (math.pi / rc)
    pref = math.sqrt(2.0 / rc)
    rs = torch.linspace(1e-8, rc, 4096, dtype=torch.float32)
    raw = (pref * torch.sin(rs[:, None] * freqs.float()) / (rs[:, None] + 1e-8))
    mu, sig = raw.mean(0).double(), raw.std(0).clamp(min=1e-8).double()
    phi = (pref * torch.sin(bond_dist[:, None] * freqs) / (bond_dist[:, None] + 1e-8) - mu) / sig
    fcut = torch.where(bond_dist < rc, 0.5 * (torch.cos(math.pi * bond_dist / rc) + 1.0),
                       torch.zeros_like(bond_dist))
    edge_feats = phi * fcut[:, None]
    h = node @ t["initial_projection.weight"].T + t["initial_projection.bias"]
    per_layer = []
    for i in range(L):
        p = f"interactions.{i}."
        sc = h
        up = linear(h, t[p + "node_linear.weight"], blocks, blocks)
        a = edge_feats
        for j in (0, 2):
            a = torch.nn.functional.silu(a @ t[p + f"radial_mlp.mlp.{j}.weight"].T + t[p + f"radial_mlp.mlp.{j}.bias"])
        w = a @ t[p + "radial_mlp.mlp.4.weight"].T + t[p + "radial_mlp.mlp.4.bias"]
        msg, tp = conv_tp(up, Y, w, edge_index, pos.shape[0], l_max, F)
        msg = msg / cfg["avg_num_neighbors"]
        order = sorted(tp.out_pos, key=tp.out_pos.get)
        tp_blocks = [(F, tp.paths[k][4], tp.paths[k][5]) for k in order]
        m = linear(msg, t[p + "linear.weight"], tp_blocks, blocks)
        # product head: per-element polynomial of scalar channels, then nn.Linear (product_head.py:119-142)
        W = t[f"products.{i}.symmetric_contraction.symmetric_contraction.weight"][Z]  # (N, nu, D)
        powers = torch.stack([m ** (k + 1) for k in range(nu)], dim=1)
        basis = (W * powers).sum(1)
        hp = basis @ t[f"products.{i}.linear.weight"].T + t[f"products.{i}.linear.bias"]
        per_layer.append(hp)
        proj = hp @ t[f"projections.{i}.weight"].T + t[f"projections.{i}.bias"]
        if i < L - 1:
            Wu = t[f"element_updates.{i}.weight"]  # (S, D*D)
            upd = torch.zeros_like(proj)
            for s in range(Wu.shape[0]):
                sel = Z == s
                if sel.any():
                    upd[sel] = proj[sel] @ Wu[s].reshape(D, D) / math.sqrt(D)
            h = sc + upd
        else:
            h = proj
    return per_layer


def energy_forces(sd, cfg, Z, pos, edge_index, batch, num_graphs, shifts=None):
    pos = pos.detach().to(torch.float64).requires_grad_(True)
    e = mace_energy(sd, cfg, Z, pos, edge_index, batch, num_graphs, shifts)
    (g,) = torch.autograd.grad(e.sum(), pos)
    return e.detach(), -g
