"""Allegro encoder on the HIP kernels (molzoo.allegro) vs its fp64 restatement
(oracle/allegro_ref.py), plus the reference's own module checks
(tests/test_molzoo/test_allegro.py: shapes, encoder contract, rotation invariance, compile).

Tolerance: edge features and forces (-d/dpos of a fixed linear readout of the features) within
1e-5 norm-wise relative error of float64.
"""

import math

import numpy as np
import pytest
import torch

from oracle import allegro_ref as AR
from oracle import equivariant as EQ

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _system(n=40, rc=5.0, seed=0, box=9.0):
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand(n, 3, generator=g, dtype=torch.float64) * box
    Z = torch.randint(0, 3, (n,), generator=g)
    d = pos[None, :, :] - pos[:, None, :]
    r = d.norm(dim=-1)
    src, dst = torch.nonzero((r < rc) & (r > 0), as_tuple=True)
    return pos, Z, torch.stack([src, dst], 1), rc


def _geometry(pos, edge_index):
    diff = pos[edge_index[:, 1]] - pos[edge_index[:, 0]]
    return diff, diff.norm(dim=-1)


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm())


def _model(l_max, F, S, layers, avg=None, seed=1):
    from molnex_amd.molzoo.allegro import Allegro

    torch.manual_seed(seed)
    m = Allegro(num_elements=3, num_scalar_features=S, num_tensor_features=F, r_max=5.0, l_max=l_max,
                num_layers=layers, avg_num_neighbors=avg)
    cfg = dict(l_max=l_max, num_tensor_features=F, num_layers=layers, r_max=5.0, num_bessel=8, poly_p=6,
               residual_alpha=0.5, avg_num_neighbors=avg)
    return m, cfg


@pytest.mark.parametrize("l_max,F,S,layers,avg", [(2, 8, 16, 3, None), (2, 16, 64, 2, 12.0), (1, 16, 32, 2, None),
                                                  (3, 8, 16, 2, None)])
def test_allegro_matches_fp64_oracle(l_max, F, S, layers, avg):
    pos, Z, ei, rc = _system()
    m, cfg = _model(l_max, F, S, layers, avg)
    mg = m.to(DEV)
    readout = torch.randn(layers, S, dtype=torch.float64, generator=torch.Generator().manual_seed(2))

    pg = pos.float().to(DEV).requires_grad_(True)
    diff, dist = _geometry(pg, ei.to(DEV))
    feats = mg(Z=Z.to(DEV), bond_dist=dist, bond_diff=diff, edge_index=ei.to(DEV))
    (fg,) = torch.autograd.grad((feats * readout.float().to(DEV)).sum(), pg)

    p64 = pos.clone().requires_grad_(True)
    diff64, dist64 = _geometry(p64, ei)
    ref = AR.allegro_features(m.state_dict(), cfg, Z, dist64, diff64, ei)
    (f64,) = torch.autograd.grad((ref * readout).sum(), p64)
    assert feats.shape == ref.shape == (ei.shape[0], layers, S)
    assert _rel(feats, ref) <= 1e-5, _rel(feats, ref)
    assert _rel(fg, f64) <= 1e-5, _rel(fg, f64)


@pytest.mark.parametrize("l_max,F,S,layers,avg", [(2, 16, 64, 2, 12.0), (1, 16, 32, 2, None)])
def test_allegro_frozen_fused_scalar_mlp_vs_fp64_oracle(l_max, F, S, layers, avg):
    """Parameters frozen (energy + forces in eval): the pair embedding's scalar MLP runs as the
    fused hidden-stack kernel (molix::radial_hidden, 40 -> S -> S -> S with SiLU); features and
    forces against the fp64 oracle and against the torch form."""
    import molnex_amd.kernels as K
    from molnex_amd.config import config

    pos, Z, ei, rc = _system()
    m, cfg = _model(l_max, F, S, layers, avg)
    mg = m.to(DEV)
    for p in mg.parameters():
        p.requires_grad_(False)
    assert K.radial_supported(8 + 2 * 16, S, 3)
    readout = torch.randn(layers, S, dtype=torch.float64, generator=torch.Generator().manual_seed(2))

    def run():
        pg = pos.float().to(DEV).requires_grad_(True)
        diff, dist = _geometry(pg, ei.to(DEV))
        feats = mg(Z=Z.to(DEV), bond_dist=dist, bond_diff=diff, edge_index=ei.to(DEV))
        (fg,) = torch.autograd.grad((feats * readout.float().to(DEV)).sum(), pg)
        return feats, fg

    feats, fg = run()
    prev = config.fused_radial
    config.fused_radial = False
    try:
        feats_t, fg_t = run()
    finally:
        config.fused_radial = prev
    p64 = pos.clone().requires_grad_(True)
    diff64, dist64 = _geometry(p64, ei)
    ref = AR.allegro_features(m.state_dict(), cfg, Z, dist64, diff64, ei)
    (f64,) = torch.autograd.grad((ref * readout).sum(), p64)
    for a, b in ((feats, ref), (fg, f64), (feats_t, ref), (fg_t, f64)):
        assert _rel(a, b) <= 1e-5, _rel(a, b)
    assert _rel(feats, feats_t) <= 1e-5


def test_allegro_frozen_tail_second_order_matches_module_form():
    """Frozen parameters run each layer's tail as one autograd Function with a hand-written
    backward; differentiating the forces again (create_graph) recomputes it in tracked ops.  The
    forces and the position gradient of <forces, v> must match the module form (parameters
    requiring gradients), and the first-order forces the fp64 oracle."""
    pos, Z, ei, rc = _system(seed=3)
    m, cfg = _model(2, 16, 64, 2, 12.0)
    m = m.to(DEV)
    readout = torch.randn(2, 64, generator=torch.Generator().manual_seed(4)).to(DEV)
    v = torch.randn(pos.shape[0], 3, generator=torch.Generator().manual_seed(5)).to(DEV)

    def run(frozen):
        for p in m.parameters():
            p.requires_grad_(not frozen)
        pg = pos.float().to(DEV).requires_grad_(True)
        diff, dist = _geometry(pg, ei.to(DEV))
        feats = m(Z=Z.to(DEV), bond_dist=dist, bond_diff=diff, edge_index=ei.to(DEV))
        (f,) = torch.autograd.grad((feats * readout).sum(), pg, create_graph=True)
        (h,) = torch.autograd.grad((f * v).sum(), pg)
        return f.detach(), h

    f_fast, h_fast = run(True)
    f_mod, h_mod = run(False)
    assert _rel(f_fast, f_mod) <= 1e-5, _rel(f_fast, f_mod)
    assert _rel(h_fast, h_mod) <= 1e-5, _rel(h_fast, h_mod)
    p64 = pos.clone().requires_grad_(True)
    diff64, dist64 = _geometry(p64, ei)
    sd = {k: t.detach().cpu() for k, t in m.state_dict().items()}
    ref = AR.allegro_features(sd, cfg, Z, dist64, diff64, ei)
    (f64,) = torch.autograd.grad((ref * readout.double().cpu()).sum(), p64)
    assert _rel(f_fast, f64) <= 1e-5, _rel(f_fast, f64)


def test_channel_scale_first_and_second_order_vs_fp64():
    """molix::channel_scale (Allegro's output env scaling) against float64 torch: forward, both
    gradients, and the second-order terms of the gradient (force-matching training)."""
    import molnex_amd.kernels as K

    g = torch.Generator().manual_seed(4)
    E, D, F = 1037, 9, 16
    t64, s64, w64 = (torch.randn(*sh, generator=g, dtype=torch.float64) for sh in ((E, D * F), (E, F), (E, D * F)))
    r1, r2 = torch.randn(E, D * F, generator=g, dtype=torch.float64), torch.randn(E, F, generator=g,
                                                                                   dtype=torch.float64)

    def run(fn, t, s, w):
        t, s, w = (a.clone().requires_grad_(True) for a in (t, s, w))
        out = fn(t, s)
        gt, gs = torch.autograd.grad((out * w).sum(), (t, s), create_graph=True)
        tot = (gt * r1.to(gt)).sum() + (gs * r2.to(gs)).sum()
        return (out,) + (gt, gs) + torch.autograd.grad(tot, (t, s, w))

    ref = run(lambda t, s: (t.view(E, D, F) * s.unsqueeze(1)).reshape(E, -1), t64, s64, w64)
    got = run(lambda t, s: K.channel_scale(t, s, D), *(a.float().to(DEV) for a in (t64, s64, w64)))
    for name, a, b in zip(("out", "grad_t", "grad_s", "d2/dt", "d2/ds", "d2/dw"), got, ref):
        assert _rel(a, b) <= 1e-6, (name, _rel(a, b))


def test_channel_outer_first_and_second_order_vs_fp64():
    """molix::channel_outer (the pair embedding's env-weighted harmonics) against float64 torch:
    forward, both gradients and the second-order terms, D = 1, 4, 9, 16 and F = 4 .. 64."""
    import molnex_amd.kernels as K

    g = torch.Generator().manual_seed(5)
    for E, D, F in ((517, 9, 16), (301, 16, 8), (64, 4, 64), (33, 1, 4)):
        y64, s64, w64 = (torch.randn(*sh, generator=g, dtype=torch.float64) for sh in ((E, D), (E, F), (E, D * F)))
        r1, r2 = torch.randn(E, D, generator=g, dtype=torch.float64), torch.randn(E, F, generator=g,
                                                                                dtype=torch.float64)

        def run(fn, y, s, w):
            y, s, w = (a.clone().requires_grad_(True) for a in (y, s, w))
            out = fn(y, s)
            gy, gs = torch.autograd.grad((out * w).sum(), (y, s), create_graph=True)
            tot = (gy * r1.to(gy)).sum() + (gs * r2.to(gs)).sum()
            return (out, gy, gs) + torch.autograd.grad(tot, (y, s, w))

        ref = run(lambda y, s: (y.unsqueeze(-1) * s.unsqueeze(-2)).reshape(E, -1), y64, s64, w64)
        got = run(K.channel_outer, *(a.float().to(DEV) for a in (y64, s64, w64)))
        for name, a, b in zip(("out", "grad_y", "grad_s", "d2/dy", "d2/ds", "d2/dw"), got, ref):
            assert _rel(a, b) <= 1e-6, (E, D, F, name, _rel(a, b))


def test_envelope_stack_first_and_second_order_vs_fp64():
    """The cutoff envelope written into the per-layer stack in one pass (molix::channel_outer_stack
    and its one-pass backward, via the encoder's Function) against float64 torch: forward, the
    gradients of the envelope and of every layer's features (non-contiguous and offset inputs
    included), and the second-order terms (tracked backward); L = 1 .. 8, F = 4 .. 256."""
    import molnex_amd.kernels as K
    from molnex_amd.molzoo.allegro import _envelope_stack

    g = torch.Generator().manual_seed(6)
    for E, L, F in ((517, 2, 64), (301, 3, 16), (64, 1, 4), (33, 8, 256), (1, 2, 8)):
        u64 = torch.rand(E, 1, generator=g, dtype=torch.float64)
        xs64 = [torch.randn(E, F, generator=g, dtype=torch.float64) for _ in range(L)]
        w64 = torch.randn(E, L, F, generator=g, dtype=torch.float64)
        r = [torch.randn(E, F, generator=g, dtype=torch.float64) for _ in range(L)]
        ru = torch.randn(E, 1, generator=g, dtype=torch.float64)

        def run(fn, u, xs, w, second):
            u = u.clone().requires_grad_(True)
            xs = [x.clone().requires_grad_(True) for x in xs]
            out = fn(xs, u)
            grads = torch.autograd.grad((out * w).sum(), [u] + xs, create_graph=second)
            if not second:
                return (out,) + grads
            tot = (grads[0] * ru.to(u)).sum() + sum((gx * rr.to(gx)).sum() for gx, rr in zip(grads[1:], r))
            return (out,) + grads + torch.autograd.grad(tot, [u] + xs)

        ref_fn = lambda xs, u: torch.stack(xs, 1) * u.unsqueeze(-1)  # noqa: E731
        dev = (u64.float().to(DEV), [x.float().to(DEV) for x in xs64], w64.float().to(DEV))
        for second in (False, True):
            ref = run(ref_fn, u64, xs64, w64, second)
            got = run(_envelope_stack, *dev, second)
            assert len(got) == len(ref)
            for k, (a, b) in enumerate(zip(got, ref)):
                assert _rel(a, b) <= 2e-6, (E, L, F, second, k, _rel(a, b))
        # inputs that are strided or offset views go through a contiguous, aligned copy
        base = torch.randn(E, 2 * F + 1, generator=g).to(DEV)
        xv = [base[:, 1:F + 1], base[:, F + 1:]] * ((L + 1) // 2)
        xv = xv[:L]
        out = K.channel_outer_stack(dev[0], xv)
        assert _rel(out, torch.stack([x.double().cpu() for x in xv], 1) * u64.unsqueeze(-1)) <= 1e-6
        res = K.channel_outer_stack_backward(dev[2], dev[0], xv, True, False)
        assert res[0].shape == (E, 1) and all(t.numel() == 0 for t in res[1:])
        ref_u = sum((w64[:, l] * xv[l].double().cpu()).sum(-1, keepdim=True) for l in range(L))
        assert _rel(res[0], ref_u) <= 1e-6


def test_envelope_stack_opcheck_and_errors():
    import molnex_amd.kernels as K

    g = torch.Generator().manual_seed(7)
    u = torch.rand(37, 1, generator=g).to(DEV)
    xs = [torch.randn(37, 16, generator=g).to(DEV) for _ in range(3)]
    gr = torch.randn(37, 3, 16, generator=g).to(DEV)
    torch.library.opcheck(torch.ops.molix.channel_outer_stack, (u, xs))
    torch.library.opcheck(torch.ops.molix.channel_outer_stack_backward, (gr, u, xs, True, True))
    empty = K.channel_outer_stack(u[:0], [x[:0] for x in xs])
    assert empty.shape == (0, 3, 16)
    with pytest.raises(ValueError):
        K.channel_outer_stack(u, xs * 3)  # 9 inputs
    with pytest.raises(ValueError):
        K.channel_outer_stack(u, [torch.randn(37, 12, device=DEV)])  # F / 4 not a power of two
    with pytest.raises(ValueError):
        K.channel_outer_stack(u, [xs[0], xs[1][:36]])


def test_allegro_rotation_invariant_and_contract():
    """Scalar edge features are invariant under a rotation of the positions (the reference checks
    rtol = atol = 1e-4; fp32 here stays far inside), and the GraphBatch contract writes
    ``edges.edge_features`` of shape (n_edges, num_layers, num_scalar)."""
    pos, Z, ei, rc = _system(seed=3)
    m, _ = _model(2, 8, 16, 3)
    m = m.to(DEV)
    R = torch.from_numpy(EQ.random_rotation(np.random.default_rng(4)))
    td = {"atoms": {"Z": Z.to(DEV)}, "edges": {"edge_index": ei.to(DEV)}}
    diff, dist = _geometry(pos.float().to(DEV), ei.to(DEV))
    td["edges"]["bond_diff"], td["edges"]["bond_dist"] = diff, dist
    base = m(td)["edges"]["edge_features"]
    assert base.shape == (ei.shape[0], 3, 16)
    diff_r, dist_r = _geometry((pos @ R.T).float().to(DEV), ei.to(DEV))
    rot = m(Z=Z.to(DEV), bond_dist=dist_r, bond_diff=diff_r, edge_index=ei.to(DEV))
    assert _rel(rot, base) <= 1e-5
    assert torch.allclose(base, rot, rtol=1e-4, atol=1e-4)


def test_allegro_layer_shapes_and_compile():
    from molnex_amd.molzoo.allegro import AllegroLayer, PairEmbedding

    pos, Z, ei, rc = _system(seed=5)
    diff, dist = _geometry(pos.float().to(DEV), ei.to(DEV))
    torch.manual_seed(0)
    emb = PairEmbedding(num_elements=3, num_scalar_features=16, num_tensor_features=8, r_max=5.0, l_max=2).to(DEV)
    s, t, ang, cut = emb(Z.to(DEV), dist, diff, ei.to(DEV))
    E = ei.shape[0]
    assert s.shape == (E, 16) and t.shape == (E, emb.irreps_dim) and ang.shape == (E, 9) and cut.shape == (E,)
    # the reference's polynomial in fp32 (same arithmetic here) cancels to about -2e-6 just inside
    # r_cut (x = 0.999); it is exactly 0 from r_cut on
    assert bool((cut >= -1e-5).all()) and bool((cut <= 1).all())
    layer = AllegroLayer(num_scalar_features=16, num_tensor_features=8, l_max=2).to(DEV)
    s2, t2 = layer(s, t, ang, ei.to(DEV), Z.shape[0])
    assert s2.shape == s.shape and t2.shape == t.shape
    compiled = torch.compile(layer, fullgraph=False)
    s3, t3 = compiled(s, t, ang, ei.to(DEV), Z.shape[0])
    assert _rel(s3, s2) <= 1e-6 and _rel(t3, t2) <= 1e-6


def test_allegro_layer_called_alone_frozen_matches_module_form():
    """One AllegroLayer called directly (its reference interface): frozen, it runs the whole-layer
    Function and forms its tensor output from the returned env weights; outputs and the gradients
    of scalars, tensor track and harmonics must match the module form (parameters requiring
    gradients)."""
    from molnex_amd.molzoo.allegro import AllegroLayer

    pos, Z, ei, rc = _system(seed=6)
    torch.manual_seed(3)
    layer = AllegroLayer(num_scalar_features=32, num_tensor_features=16, l_max=2, avg_num_neighbors=10.0).to(DEV)
    E, n = ei.shape[0], pos.shape[0]
    g = torch.Generator().manual_seed(7)
    s0 = torch.randn(E, 32, generator=g).to(DEV)
    V0 = torch.randn(E, 9 * 16, generator=g).to(DEV)
    Y0 = torch.randn(E, 9, generator=g).to(DEV)
    rs = torch.randn(E, 32, generator=g).to(DEV)
    rv = torch.randn(E, 9 * 16, generator=g).to(DEV)

    def run(frozen):
        for p in layer.parameters():
            p.requires_grad_(not frozen)
        s, V, Y = (t.clone().requires_grad_(True) for t in (s0, V0, Y0))
        us, uv = layer(s, V, Y, ei.to(DEV), n)
        grads = torch.autograd.grad((us * rs).sum() + (uv * rv).sum(), (s, V, Y))
        return us.detach(), uv.detach(), grads

    a = run(True)
    b = run(False)
    for x, y in zip(a[:2] + tuple(a[2]), b[:2] + tuple(b[2])):
        assert _rel(x, y) <= 1e-5, _rel(x, y)
