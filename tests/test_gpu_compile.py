"""The custom ops under torch.compile / torch.export (the drop-in boundary requires both, like the
reference's tests/utils.py:23-106 checks): torch.library.opcheck of every op (schema, fake/meta
implementation, autograd registration, AOT dispatch with dynamic shapes), a compiled MACE energy +
forces step equal to eager, and an exported ConvTP and Linear equal to eager."""

import numpy as np
import pytest
import torch
from torch.library import opcheck

import molnex_amd.kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"
ops = torch.ops.molix


def _graph(n=60, L=9.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    pos = (torch.rand(n, 3, generator=g) * L).to(DEV)
    box = torch.eye(3, device=DEV) * L
    i, j, shifts, deltas, dist = ops.neighbor_list(pos, 3.0, box, True)
    ei = torch.stack([j.long(), i.long()], 1)
    return pos, box, ei, shifts, deltas


def test_opcheck_spherical_harmonics():
    v = torch.randn(50, 3, device=DEV, requires_grad=True)
    opcheck(ops.spherical_harmonics.default, (v, 3))


def test_opcheck_bond_vectors():
    pos, box, ei, shifts, _ = _graph()
    opcheck(ops.bond_vectors.default, (pos.clone().requires_grad_(True), ei, shifts))


def test_opcheck_radial_hidden():
    kin, H, L = 8, 32, 2
    params = torch.randn(K._lib.load().mnx_radial_raw_floats(kin, H, L), device=DEV) * 0.1
    f = torch.randn(40, kin, device=DEV, requires_grad=True)
    opcheck(ops.radial_hidden.default, (f, params, kin, H, L))


def test_opcheck_tp_scatter():
    pos, box, ei, _, deltas = _graph()
    N, C = pos.shape[0], 8
    cfg = K.tp_config_id([0, 1], [0, 1], [0, 1])
    P, nx, ny, no = K.tp_config_info(cfg)
    row_ptr, perm, snd = ops.edge_csr(ei, N)
    x = torch.randn(N, nx * C, device=DEV, requires_grad=True)
    Y = torch.randn(ei.shape[0], ny, device=DEV, requires_grad=True)
    w = torch.randn(ei.shape[0], P * C, device=DEV, requires_grad=True)
    opcheck(ops.tp_scatter.default, (x, Y, w, row_ptr, perm, snd, cfg, C))


def test_opcheck_tp_any():
    from molnex_amd.irreps import ChannelwiseTPDescriptor

    pos, box, ei, _, deltas = _graph()
    N = pos.shape[0]
    d = ChannelwiseTPDescriptor("8x0e + 4x1o + 4x1e", "0e + 1o", "0e + 0o + 1o + 1e")
    table = K.tp_any_table(d)
    row_ptr, perm, snd = ops.edge_csr(ei, N)
    x = torch.randn(N, d.irreps_in1.dim, device=DEV, requires_grad=True)
    Y = torch.randn(ei.shape[0], d.irreps_in2.dim, device=DEV, requires_grad=True)
    w = torch.randn(ei.shape[0], d.weight_numel, device=DEV, requires_grad=True)
    opcheck(ops.tp_any.default, (x, Y, w, row_ptr, perm, snd, table))


def test_opcheck_pairs():
    """The undirected-pair ops: edge_reverse, tp_scatter with a weight-row map, the pair-summing
    output-layer backward, and radial_tp_pairs in pair and edge mode."""
    pos, box, ei, shifts, _ = _graph()
    N, C, Kh = pos.shape[0], 8, 16
    bond = ops.bond_vectors(pos, ei, shifts)
    feats = bond.norm(dim=-1, keepdim=True)
    row_ptr, perm, snd = ops.edge_csr(ei, N)
    opcheck(ops.edge_reverse.default, (ei, N, row_ptr, perm, snd, feats), test_utils=("test_schema", "test_faketensor"))
    pr = K.EdgePairs.build(ei, N, row_ptr, perm, snd, feats)
    assert pr is not None
    E = ei.shape[0]
    cfg = K.tp_config_id([0, 1], [0, 1], [0, 1])
    P, nx, ny, no = K.tp_config_info(cfg)
    x = torch.randn(N, nx * C, device=DEV, requires_grad=True)
    Y = torch.randn(E, ny, device=DEV, requires_grad=True)
    w = torch.randn(E // 2, P * C, device=DEV, requires_grad=True)
    opcheck(ops.tp_scatter.default, (x, Y, w, row_ptr, perm, snd, cfg, C, None, None, None, pr.wrow))
    W = torch.randn(P * C, Kh, device=DEV) * 0.3
    gw = torch.randn(E, P * C, device=DEV)
    opcheck(ops.edge_weights_backward_pairs.default, (gw, pr.pairs, W), test_utils=("test_schema", "test_faketensor"))
    b = torch.randn(P * C, device=DEV)
    f2 = torch.randn(E, 8, device=DEV, requires_grad=True)
    opcheck(ops.gather_rows.default, (f2, pr.lead))
    opcheck(ops.scatter_rows.default, (torch.randn(E // 2, 8, device=DEV, requires_grad=True), pr.lead, E))
    for rows in (E // 2, E):  # pair mode, edge mode
        h = torch.randn(rows, Kh, device=DEV, requires_grad=True)
        opcheck(ops.radial_tp_pairs.default, (x, Y, h, W, b, row_ptr, perm, snd, pr.wrow, pr.pairs, cfg, C))
    # the fused input gradient (receiver batches; channels a multiple of 16)
    C2 = 16
    batches = K.tp_gh_batches(row_ptr)
    x2 = torch.randn(N, nx * C2, device=DEV, requires_grad=True)
    W2 = torch.randn(P * C2, Kh, device=DEV) * 0.3
    b2 = torch.randn(P * C2, device=DEV)
    for rows in (E // 2, E):
        h = torch.randn(rows, Kh, device=DEV, requires_grad=True)
        opcheck(ops.radial_tp_pairs.default, (x2, Y, h, W2, b2, row_ptr, perm, snd, pr.wrow, pr.pairs, cfg, C2,
                                              batches))
    g = torch.randn(N, no * C2, device=DEV)
    opcheck(ops.tp_weight_grad_batched.default, (x2.detach(), Y.detach(), g, row_ptr, perm, snd, batches, W2, cfg,
                                                 C2), test_utils=("test_schema", "test_faketensor"))


def test_opcheck_class_groups():
    z = torch.randint(-1, 7, (3000,), device=DEV)
    opcheck(ops.class_groups.default, (z, 6), test_utils=("test_schema", "test_faketensor"))


def test_opcheck_segment_sum():
    idx = torch.randint(0, 40, (500,), device=DEV)
    v = torch.randn(500, 12, device=DEV, requires_grad=True)
    w = torch.randn(500, device=DEV, requires_grad=True)
    opcheck(ops.segment_sum.default, (v, idx, 40, w, False))


def test_opcheck_edge_csr():
    pos, box, ei, _, _ = _graph()
    opcheck(ops.edge_csr.default, (ei, pos.shape[0]), test_utils=("test_schema", "test_faketensor"))


def test_opcheck_symmetric_contraction():
    N, C, S = 30, 8, 3
    x = torch.randn(N, 16 * C, device=DEV, requires_grad=True)
    z = torch.randint(0, S, (N,), device=DEV)
    paths = K.sc_config_info(K.sc_config_id(3, 1, 3))[2]
    w = torch.randn(S, paths, C, device=DEV, requires_grad=True)
    opcheck(ops.symmetric_contraction.default, (x, z, w, 3, 1, 3))
    xs = torch.randn(N, C, device=DEV, requires_grad=True)
    ws = torch.randn(S, 3, C, device=DEV, requires_grad=True)
    opcheck(ops.symmetric_contraction_scalar.default, (xs, z, ws))


def test_opcheck_pme():
    from oracle import pme as P

    pos, box, _, _, _ = _graph(n=40, L=12.0)
    pos64 = pos.double().requires_grad_(True)
    q = torch.randn(40, dtype=torch.float64, device=DEV)
    q = (q - q.mean()).requires_grad_(True)
    nb, d, dist, _ = ops.get_neighbor_pairs(pos64.detach(), 4.0, -1, box.double())
    keep = nb[0] >= 0
    excl = torch.full((40, 1), -1, dtype=torch.int32, device=DEV)
    opcheck(ops.pme_direct.default, (pos64, q, nb[:, keep].contiguous(), d[keep].contiguous(),
                                     dist[keep].contiguous(), excl, 0.3, 14.399645))
    mods = [torch.tensor(P.bspline_moduli(16, 5), device=DEV) for _ in range(3)]
    opcheck(ops.pme_reciprocal.default, (pos64, q, box.double(), 16, 16, 16, 5, 0.3, 14.399645, *mods))
    # the spectrum variant: the AOT check is left out, as its harness sums the real energy and
    # the complex spectrum outputs into one accumulator
    opcheck(ops.pme_reciprocal_spectrum.default, (pos64, q, box.double(), 16, 16, 16, 5, 0.3, 14.399645, *mods),
            test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


def test_opcheck_get_neighbor_pairs():
    """Schema, fake and autograd registration through opcheck.  Its AOT check is left out: that
    harness sums every output into one accumulator, which the int64 neighbour list (the first
    output) makes an integer tensor that the float64 distances cannot be added to in place.  The
    compiled-gradient test below covers AOT dispatch instead."""
    pos = torch.rand(30, 3, dtype=torch.float64, device=DEV) * 6
    box = torch.eye(3, dtype=torch.float64, device=DEV) * 6
    opcheck(ops.get_neighbor_pairs.default, (pos.requires_grad_(True), 2.5, 200, box),
            test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))


def test_compiled_get_neighbor_pairs_gradient():
    """A pair energy over get_neighbor_pairs under torch.compile (AOT autograd, dynamic shapes):
    energy and position gradient equal to eager."""
    g = torch.Generator().manual_seed(7)
    pos0 = (torch.rand(40, 3, generator=g, dtype=torch.float64) * 6).to(DEV)
    box = torch.eye(3, dtype=torch.float64, device=DEV) * 6

    def energy(p):
        nb, d, r, _ = ops.get_neighbor_pairs(p, 2.5, 400, box)
        keep = nb[0] >= 0  # padding slots carry NaN
        r = torch.where(keep, r, torch.full_like(r, 2.5))
        d = torch.where(keep[:, None], d, torch.zeros_like(d))
        return ((r - 2.5) ** 2).sum() + 0.1 * (d ** 2).sum()

    def run(fn):
        p = pos0.clone().requires_grad_(True)
        e = fn(p)
        (gp,) = torch.autograd.grad(e, p)
        return e.detach(), gp

    e0, g0 = run(energy)
    e1, g1 = run(torch.compile(energy, backend="aot_eager", dynamic=True))
    assert torch.allclose(e0, e1, rtol=1e-12, atol=1e-12)
    assert torch.allclose(g0, g1, rtol=1e-12, atol=1e-12)


def test_opcheck_block_linear():
    from molnex_amd.molrep.interaction.linear import Linear

    lin = Linear("16x0e+8x0e+16x1o", "32x0e+8x1o").to(DEV)
    x = torch.randn(37, lin.irreps_in.dim, device=DEV)
    w = lin.weight.detach().reshape(-1)
    ws = w.index_select(0, lin._hip_idx_f) * lin._hip_sc_f
    opcheck(ops.block_linear.default, (x, ws, lin._hip_plan["fwd"], lin.irreps_out.dim))


def test_compiled_mace_matches_eager():
    from tests.test_gpu_mace import CFG1_LITERAL, build, molecules
    from oracle import nlist as NL

    pos, Z, batch = molecules(seed=3, n_mol=4)
    ii, jj, _, _ = NL.directed_pairs(pos.astype(np.float32), 5.0, None)
    ei = torch.tensor(np.stack([jj, ii], 1).astype(np.int64), device=DEV)
    model = build(CFG1_LITERAL, seed=3)
    Zt, bt = torch.tensor(Z, device=DEV), torch.tensor(batch, device=DEV)
    p = torch.tensor(pos, dtype=torch.float32, device=DEV)

    def run(m):
        e, f = m(Zt, p.clone(), ei, bt, 4)
        return e.detach(), f.detach()

    e0, f0 = run(model)
    e1, f1 = run(torch.compile(model, backend="eager", fullgraph=False))
    assert torch.allclose(e0, e1, rtol=1e-6, atol=1e-6)
    assert torch.allclose(f0, f1, rtol=1e-5, atol=1e-6)


def test_exported_conv_tp_matches_eager():
    from molnex_amd.molrep.interaction import ConvTP

    pos, box, ei, _, deltas = _graph(n=80, L=10.0, seed=4)
    N, C = pos.shape[0], 8
    conv = ConvTP(in_irreps=f"{C}x0e+{C}x1o", out_irreps=f"{C}x0e+{C}x1o", sh_irreps="0e+1o").to(DEV)
    x = torch.randn(N, 4 * C, device=DEV)
    Y = ops.spherical_harmonics(deltas, 1)
    w = torch.randn(ei.shape[0], conv.weight_numel, device=DEV)
    ref = conv(node_features=x, edge_angular=Y, edge_index=ei, tp_weights=w)

    class Wrap(torch.nn.Module):
        def __init__(self, m):
            super().__init__()
            self.m = m

        def forward(self, x, Y, ei, w):
            return self.m(node_features=x, edge_angular=Y, edge_index=ei, tp_weights=w)

    ep = torch.export.export(Wrap(conv), (x, Y, ei, w), strict=False)
    out = ep.module()(x, Y, ei, w)
    assert torch.allclose(out, ref, rtol=1e-6, atol=1e-6)


def test_exported_linear_matches_eager():
    """An exported equivariant Linear runs the HIP block op with its weight tables as constants."""
    from molnex_amd.molrep.interaction.linear import Linear

    lin = Linear("16x0e+16x1o+8x2e", "32x0e+16x1o+8x2e").to(DEV)
    x = torch.randn(45, lin.irreps_in.dim, device=DEV)
    ref = lin(x)
    ep = torch.export.export(lin, (x,), strict=False)
    assert any("block_linear" in str(n.target) for n in ep.graph.nodes)
    assert torch.allclose(ep.module()(x), ref, rtol=1e-6, atol=1e-6)


def test_opcheck_edge_tp():
    cfg = K.tp_config_id([0, 1, 2], [0, 1, 2], [0, 1, 2])
    P, NX, NY, NO = K.tp_config_info(cfg)
    E, C = 70, 16
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn(E, NX * C, device=DEV, generator=g).requires_grad_(True)
    Y = torch.randn(E, NY, device=DEV, generator=g).requires_grad_(True)
    w = torch.randn(P, C, device=DEV, generator=g).requires_grad_(True)
    s = torch.randn(E, C, device=DEV, generator=g).requires_grad_(True)
    opcheck(ops.edge_tp.default, (x, Y, w, cfg, C, s))
    opcheck(ops.edge_tp.default, (x, Y, w, cfg, C))
    gout = torch.randn(E, NO * C, device=DEV, generator=g)
    opcheck(ops.edge_tp_backward.default, (gout, x.detach(), Y.detach(), w.detach(), cfg, C, True, True, True,
                                           s.detach(), True))


def test_compiled_allegro_matches_eager():
    """The Allegro encoder's energy + forces under torch.compile equal eager (the reference's
    tests/test_molzoo/test_allegro.py:232-254 compile check)."""
    from molnex_amd.molzoo.allegro import Allegro

    pos, box, ei, shifts, deltas = _graph(n=50, L=8.0, seed=4)
    Z = torch.randint(0, 3, (pos.shape[0],), device=DEV)
    torch.manual_seed(5)
    model = Allegro(num_elements=3, num_scalar_features=16, num_tensor_features=8, r_max=3.0, l_max=2,
                    num_layers=2).to(DEV)
    readout = torch.randn(2, 16, device=DEV)

    def run(m):
        p = pos.clone().requires_grad_(True)
        diff = ops.bond_vectors(p, ei, shifts)
        feats = m(Z=Z, bond_dist=diff.norm(dim=-1), bond_diff=diff, edge_index=ei)
        e = (feats * readout).sum()
        (f,) = torch.autograd.grad(e, p)
        return e.detach(), f.detach()

    e0, f0 = run(model)
    e1, f1 = run(torch.compile(model, backend="eager", fullgraph=False))
    rel_e = float((e0 - e1).abs() / e0.abs())
    rel_f = float((f0 - f1).norm() / f0.norm())
    # the source-harmonics and force scatters use atomics (summation order differs run to run); the
    # energy is a sum over every edge's features with cancellation, so its relative spread between
    # runs reaches ~1e-6 of fp32 rounding
    assert rel_e <= 5e-6 and rel_f <= 1e-5, (rel_e, rel_f, float((f0 - f1).abs().max()))
