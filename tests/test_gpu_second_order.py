"""Second derivatives through the molix ops (force-matching training: the forces are taken with
create_graph=True, as ForceDerivation does in training mode, force_derivation.py:38-43).

Per op, with first-order gradients G = dL1/dθ of L1 = <g, op(θ)> and seeds s, the derivatives of
L2 = <s, G> with respect to g and θ are compared with a float64 reference: for the multilinear ops
(tensor product, block linear, output layer, bond vectors) the exact identities of multilinearity
evaluated with the fp64 oracle / torch float64; for the pointwise polynomial ops (harmonics,
contractions) torch float64 autograd of their restatements, whose forward is first checked against
the kernel.  End to end: the gradient of an energy + force loss of MACE (as coded and literal)
for every parameter against torch float64 autograd of the oracle restatements.
Tolerance 1e-5 relative (norm-wise) throughout.
"""

import copy

import numpy as np
import pytest
import torch

from oracle import equivariant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
ag = torch.autograd


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


@pytest.fixture(scope="module")
def ops():
    import molnex_amd.kernels  # noqa: F401

    return torch.ops.molix


def test_harmonics_second_order(ops):
    from molnex_amd.second_order import sh_torch

    g0 = torch.Generator().manual_seed(0)
    v = torch.randn(300, 3, generator=g0, dtype=torch.float64)
    v[0] = 0.0
    g = torch.randn(300, 16, generator=g0, dtype=torch.float64)
    s = torch.randn(300, 3, generator=g0, dtype=torch.float64)
    assert _rel(ops.spherical_harmonics(v.float().to(DEV), 3), sh_torch(v, 3)) <= 1e-6
    vd, gd = v.float().to(DEV).requires_grad_(True), g.float().to(DEV).requires_grad_(True)
    (gv,) = ag.grad(ops.spherical_harmonics(vd, 3), vd, gd, create_graph=True)
    dv, dg = ag.grad((gv * s.float().to(DEV)).sum(), (vd, gd))
    v64, g64 = v.clone().requires_grad_(True), g.clone().requires_grad_(True)
    (gv64,) = ag.grad(sh_torch(v64, 3), v64, g64, create_graph=True)
    rv, rg = ag.grad((gv64 * s).sum(), (v64, g64))
    assert _rel(dv, rv) <= 1e-5 and _rel(dg, rg) <= 1e-5


def test_bond_vectors_second_order(ops):
    g0 = torch.Generator().manual_seed(1)
    pos = torch.randn(50, 3, generator=g0).to(DEV).requires_grad_(True)
    ei = torch.randint(0, 50, (400, 2), generator=g0).to(DEV)
    g = torch.randn(400, 3, generator=g0).to(DEV).requires_grad_(True)
    s = torch.randn(50, 3, generator=g0).to(DEV)
    (gp,) = ag.grad(ops.bond_vectors(pos, ei), pos, g, create_graph=True)
    (dg,) = ag.grad((gp * s).sum(), g)
    assert _rel(dg, s[ei[:, 1]] - s[ei[:, 0]]) <= 1e-6


def test_segment_sum_second_order(ops):
    """Weighted segment sum: second derivatives of <s, (gv, gw)> with respect to the output
    gradient g, the values and the weights against float64 autograd of index_add."""
    g0 = torch.Generator().manual_seed(12)
    R, D, S = 700, 5, 31
    idx = torch.randint(0, S, (R,), generator=g0)
    v, w = torch.randn(R, D, generator=g0, dtype=torch.float64), torch.rand(R, generator=g0, dtype=torch.float64)
    g = torch.randn(S, D, generator=g0, dtype=torch.float64)
    sv, sw = torch.randn(R, D, generator=g0, dtype=torch.float64), torch.randn(R, generator=g0, dtype=torch.float64)
    vd, wd, gd = (t.float().to(DEV).requires_grad_(True) for t in (v, w, g))
    gv, gw = ag.grad(ops.segment_sum(vd, idx.to(DEV), S, wd), (vd, wd), gd, create_graph=True)
    dv, dw, dg = ag.grad((gv * sv.float().to(DEV)).sum() + (gw * sw.float().to(DEV)).sum(), (vd, wd, gd))
    v64, w64, g64 = (t.clone().requires_grad_(True) for t in (v, w, g))
    out = torch.zeros(S, D, dtype=torch.float64).index_add(0, idx, v64 * w64[:, None])
    gv64, gw64 = ag.grad(out, (v64, w64), g64, create_graph=True)
    rv, rw, rg = ag.grad((gv64 * sv).sum() + (gw64 * sw).sum(), (v64, w64, g64))
    assert _rel(dv, rv) <= 1e-6 and _rel(dw, rw) <= 1e-6 and _rel(dg, rg) <= 1e-6


def test_edge_weights_second_order():
    import molnex_amd.kernels as K

    g0 = torch.Generator().manual_seed(2)
    h, W = torch.randn(500, 64, generator=g0), torch.randn(96, 64, generator=g0) / 8
    g, s = torch.randn(500, 96, generator=g0), torch.randn(500, 64, generator=g0)
    hd, Wd, gd = (t.to(DEV).requires_grad_(True) for t in (h, W, g))
    (gh,) = ag.grad(K.edge_weights(hd, Wd), hd, gd, create_graph=True)
    dg, dW = ag.grad((gh * s.to(DEV)).sum(), (gd, Wd))
    assert _rel(dg, s.double() @ W.double().t()) <= 1e-5
    assert _rel(dW, g.double().t() @ s.double()) <= 1e-5


@pytest.mark.parametrize("sender", [False, True])
def test_tensor_product_second_order(ops, sender):
    import molnex_amd.kernels as K

    C, N, E = 8, 40, 300
    ls = [0, 1, 2, 3]
    irr = "0e + 1o + 2e + 3o"
    tp = O.ChannelwiseTP(" + ".join(f"{C}x{t}" for t in irr.split(" + ")), irr, irr, C)
    rng = np.random.default_rng(3)
    x, Y, w = (rng.normal(size=s).astype(np.float32) for s in ((N, tp.nx * C), (E, tp.ny), (E, len(tp.paths) * C)))
    g = rng.normal(size=(N, tp.no * C)).astype(np.float32)
    sx, sY, sw = (rng.normal(size=a.shape).astype(np.float32) for a in (x, Y, w))
    ei = rng.integers(0, N, (E, 2))
    config = K.tp_config_id(ls, ls, ls)
    eit = torch.tensor(ei, device=DEV)
    csr = ops.edge_csr(eit, N)
    extra = ops.edge_csr(eit.flip(1), N) if sender else ()
    xt, Yt, wt, gt = (torch.tensor(a, device=DEV, requires_grad=True) for a in (x, Y, w, g))
    out = ops.tp_scatter(xt, Yt, wt, *csr, config, C, *extra)
    gx, gY, gw = ag.grad(out, (xt, Yt, wt), gt, create_graph=True)
    L2 = sum((a * torch.tensor(b, device=DEV)).sum() for a, b in ((gx, sx), (gY, sY), (gw, sw)))
    dg, dx, dY, dw = ag.grad(L2, (gt, xt, Yt, wt))
    f = lambda a, b, c: tp.forward(a, b, c, ei, N)  # noqa: E731
    b = lambda a, bb, c: tp.backward(a, bb, c, ei, g)  # noqa: E731
    ref_g = f(sx, Y, w) + f(x, sY, w) + f(x, Y, sw)
    ref_x = b(x, sY, w)[0] + b(x, Y, sw)[0]
    ref_Y = b(sx, Y, w)[1] + b(x, Y, sw)[1]
    ref_w = b(sx, Y, w)[2] + b(x, sY, w)[2]
    for name, got, ref in (("g", dg, ref_g), ("x", dx, ref_x), ("Y", dY, ref_Y), ("w", dw, ref_w)):
        assert _rel(got, torch.tensor(ref)) <= 1e-5, name


def test_block_linear_second_order():
    from molnex_amd.molrep.interaction.linear import Linear

    torch.manual_seed(4)
    lin = Linear("16x0e+8x0e+16x1o+8x2e", "32x0e+16x1o+8x2e").to(DEV)
    x = torch.randn(70, lin.irreps_in.dim, device=DEV, requires_grad=True)
    g = torch.randn(70, lin.irreps_out.dim, device=DEV, requires_grad=True)
    s = torch.randn(70, lin.irreps_in.dim, device=DEV)
    (gx,) = ag.grad(lin(x), x, g, create_graph=True)
    dg, dw = ag.grad((gx * s).sum(), (g, lin.weight))
    ref = copy.deepcopy(lin).double().cpu()
    x64, g64 = x.detach().double().cpu().requires_grad_(True), g.detach().double().cpu().requires_grad_(True)
    (gx64,) = ag.grad(ref(x64), x64, g64, create_graph=True)
    rg, rw = ag.grad((gx64 * s.double().cpu()).sum(), (g64, ref.weight))
    assert _rel(dg, rg) <= 1e-5 and _rel(dw, rw) <= 1e-5


def test_scalar_contraction_second_order(ops):
    from molnex_amd.second_order import sc_scalar_torch

    g0 = torch.Generator().manual_seed(5)
    x = torch.randn(60, 32, generator=g0)
    z = torch.randint(0, 3, (60,), generator=g0)
    w = torch.randn(3, 3, 32, generator=g0) * 0.3
    g, sx, sw = torch.randn(60, 32, generator=g0), torch.randn(60, 32, generator=g0), torch.randn(3, 3, 32, generator=g0)
    assert _rel(ops.symmetric_contraction_scalar(x.to(DEV), z.to(DEV), w.to(DEV)), sc_scalar_torch(x.double(), z, w.double())) <= 1e-6
    xd, wd, gd = (t.to(DEV).requires_grad_(True) for t in (x, w, g))
    gx, gw = ag.grad(ops.symmetric_contraction_scalar(xd, z.to(DEV), wd), (xd, wd), gd, create_graph=True)
    d = ag.grad((gx * sx.to(DEV)).sum() + (gw * sw.to(DEV)).sum(), (gd, xd, wd))
    x64, w64, g64 = (t.double().requires_grad_(True) for t in (x, w, g))
    rx, rw = ag.grad(sc_scalar_torch(x64, z, w64), (x64, w64), g64, create_graph=True)
    r = ag.grad((rx * sx.double()).sum() + (rw * sw.double()).sum(), (g64, x64, w64))
    for a, b in zip(d, r):
        assert _rel(a, b) <= 1e-5


@pytest.mark.parametrize("l_in,l_out,nu", [(1, 1, 3), (3, 1, 3), (2, 0, 2)])
def test_equivariant_contraction_second_order(ops, l_in, l_out, nu):
    import molnex_amd.kernels as K
    from molnex_amd.second_order import sc_torch

    C, N, S = 8, 40, 3
    paths = K.sc_config_info(K.sc_config_id(l_in, l_out, nu))[2]
    g0 = torch.Generator().manual_seed(6 + l_in)
    x = torch.randn(N, (l_in + 1) ** 2 * C, generator=g0) * 0.7
    z = torch.randint(0, S, (N,), generator=g0)
    w = torch.randn(S, paths, C, generator=g0) * 0.3
    g = torch.randn(N, (l_out + 1) ** 2 * C, generator=g0)
    sx, sw = torch.randn_like(x), torch.randn_like(w)
    fwd = ops.symmetric_contraction(x.to(DEV), z.to(DEV), w.to(DEV), l_in, l_out, nu)
    assert _rel(fwd, sc_torch(x.double(), z, w.double(), l_in, l_out, nu)) <= 1e-5
    xd, wd, gd = (t.to(DEV).requires_grad_(True) for t in (x, w, g))
    gx, gw = ag.grad(ops.symmetric_contraction(xd, z.to(DEV), wd, l_in, l_out, nu), (xd, wd), gd, create_graph=True)
    d = ag.grad((gx * sx.to(DEV)).sum() + (gw * sw.to(DEV)).sum(), (gd, xd, wd))
    x64, w64, g64 = (t.double().requires_grad_(True) for t in (x, w, g))
    rx, rw = ag.grad(sc_torch(x64, z, w64, l_in, l_out, nu), (x64, w64), g64, create_graph=True)
    r = ag.grad((rx * sx.double()).sum() + (rw * sw.double()).sum(), (g64, x64, w64))
    for name, a, b in zip(("g", "x", "w"), d, r):
        assert _rel(a, b) <= 1e-5, name


def _compare_param_grads(got: dict, ref: dict, what: str):
    """Parameter gradients of the GPU path (fp32) against fp64 autograd: norm-wise over all
    parameters at 1e-5, and for every tensor that carries at least 1e-3 of the gradient's norm,
    norm-wise and max-abs (against that tensor's own RMS: tensors differ in scale by orders of
    magnitude, a final bias collects the sum over every atom) at 1e-5."""
    names = sorted(got)
    a = torch.cat([got[n].reshape(-1) for n in names])
    b = torch.cat([ref[n].reshape(-1) for n in names])
    rel = _rel(a, b)
    total = float(b.norm())
    worst_rel, worst_mx = (0.0, ""), (0.0, "")
    for n in names:
        nb = float(ref[n].norm())
        if nb < 1e-3 * total:
            continue
        r = _rel(got[n], ref[n])
        m = float((got[n] - ref[n]).abs().max()) / (nb / ref[n].numel() ** 0.5)
        worst_rel, worst_mx = max(worst_rel, (r, n)), max(worst_mx, (m, n))
    print(f"{what}: parameter gradients rel err {rel:.2e}; worst tensor rel {worst_rel[0]:.2e} ({worst_rel[1]}), "
          f"max-abs {worst_mx[0]:.2e} of its RMS ({worst_mx[1]})")
    assert rel <= 1e-5 and worst_rel[0] <= 1e-5 and worst_mx[0] <= 1e-5, (rel, worst_rel, worst_mx)


@pytest.mark.parametrize("literal", [False, True])
def test_mace_force_loss_gradient_vs_fp64_oracle(literal):
    """Training step of a force-matching loss L = sum E^2 + sum F^2 (forces with create_graph
    through every HIP op's second-order formula): dL/dθ for every parameter against torch
    float64 autograd of the oracle restatement (oracle/mace_ref.py) with the same parameters."""
    from oracle import mace_ref
    from oracle import nlist as NL
    from tests.test_gpu_mace import CFG1, CFG1_LITERAL, build, molecules

    cfg = CFG1_LITERAL if literal else CFG1
    pos, Z, batch = molecules(seed=7, n_mol=2)
    ii, jj, _, _ = NL.directed_pairs(pos.astype(np.float32), 5.0, None)
    ei = np.stack([jj, ii], 1).astype(np.int64)
    model = build(cfg, seed=7)
    model.train()
    Zt, bt = torch.tensor(Z, device=DEV), torch.tensor(batch, device=DEV)
    e, f = model(Zt, torch.tensor(pos, dtype=torch.float32, device=DEV), torch.tensor(ei, device=DEV), bt, 2)
    model.zero_grad()
    ((e ** 2).sum() + (f ** 2).sum()).backward()
    named = {n: q for n, q in model.named_parameters() if q.requires_grad}
    got = {n: (q.grad if q.grad is not None else torch.zeros_like(q)).detach().double().cpu()
           for n, q in named.items()}

    t = {k.removeprefix("encoder."): v.detach().double().cpu() for k, v in model.state_dict().items()}
    leaves = {n: t[n.removeprefix("encoder.")].requires_grad_(True) for n in named}
    p64 = torch.tensor(pos.astype(np.float32), dtype=torch.float64, requires_grad=True)
    E = mace_ref._readout(t, mace_ref.mace_layers(t, cfg, torch.tensor(Z), p64, torch.tensor(ei)),
                          torch.tensor(batch), 2)
    (gpos,) = ag.grad(E.sum(), p64, create_graph=True)
    loss = (E ** 2).sum() + (gpos ** 2).sum()
    grads = ag.grad(loss, list(leaves.values()), allow_unused=True)
    ref = {n: (g if g is not None else torch.zeros_like(leaves[n])).detach() for n, g in zip(leaves, grads)}
    _compare_param_grads(got, ref, f"MACE {'literal' if literal else 'as coded'} force loss")


def test_edge_tp_second_order_identities_vs_fp64_restatement():
    """Second derivatives of the per-edge product with a channel scale (Allegro's layer product)
    against torch float64 autograd of the einsum restatement in the oracle (allegro_ref.edge_tp):
    d<r, grad(<g, TP(s x, Y; w)>)>/d(g, x, Y, w, s) for random cotangents r of every gradient."""
    import molnex_amd.kernels as K
    from oracle import allegro_ref as AR

    E, C, l_max = 300, 8, 2
    ls = list(range(l_max + 1))
    config = K.tp_config_id(ls, ls, ls)
    P, NX, NY, NO = K.tp_config_info(config)
    full = [(l1, l2, l3) for l1 in ls for l2 in ls for l3 in range(abs(l1 - l2), l1 + l2 + 1)]
    kept = [k for k, (l1, l2, l3) in enumerate(full) if (l1 + l2 + l3) % 2 == 0 and l3 <= l_max]
    gen = torch.Generator().manual_seed(3)
    x, Y, s, g = (torch.randn(*shape, generator=gen, dtype=torch.float64)
                  for shape in ((E, NX * C), (E, NY), (E, C), (E, NO * C)))
    wk = torch.randn(P, C, generator=gen, dtype=torch.float64)
    rs = [torch.randn(*t.shape, generator=gen, dtype=torch.float64) for t in (x, Y, wk, s)]

    def second(fn, prims):
        prims = [p.clone().requires_grad_(True) for p in prims]
        gg = g.clone().requires_grad_(True)
        out = fn(*prims)
        first = torch.autograd.grad((out * gg).sum(), prims, create_graph=True)
        tot = sum((f * r).sum() for f, r in zip(first, rs))
        return torch.autograd.grad(tot, [gg] + prims)

    def ref_fn(xx, YY, ww, ss):
        wfull = torch.zeros(len(full), C, dtype=torch.float64)
        wfull = wfull.index_copy(0, torch.tensor(kept), ww)
        xs = (xx.view(E, NX, C) * ss.unsqueeze(1)).reshape(E, -1)
        return AR.edge_tp(xs, YY, wfull.reshape(1, -1), l_max, C)[0]

    rows = torch.tensor(K.edge_tp_out_rows(ls), device=DEV)

    def hip_fn(xx, YY, ww, ss):
        # the kernel's rows (one block per output irrep) read back in the oracle's per-path order
        return K.edge_tp(xx, YY, ww, config, C, ss).view(E, NO, C)[:, rows].reshape(E, -1)

    ref = second(ref_fn, [x, Y, wk, s])
    # the HIP path in fp32 on the GPU: cotangents and primals cast once
    g32 = g.float().to(DEV).requires_grad_(True)
    prims = [t.float().to(DEV).requires_grad_(True) for t in (x, Y, wk, s)]
    out = hip_fn(*prims)
    first = torch.autograd.grad((out * g32).sum(), prims, create_graph=True)
    tot = sum((f * r.float().to(DEV)).sum() for f, r in zip(first, rs))
    got = torch.autograd.grad(tot, [g32] + prims)
    for name, a, b in zip(("g", "x", "Y", "w", "s"), got, ref):
        assert _rel(a, b) <= 1e-5, (name, _rel(a, b))


def test_allegro_force_loss_gradient_vs_fp64_oracle():
    """Force-matching training of the Allegro encoder: d(sum E^2 + sum F^2)/dθ (forces with
    create_graph through molix::edge_tp's second-order formulas) for every parameter against
    torch float64 autograd of the oracle restatement (oracle/allegro_ref.py)."""
    from molnex_amd.molzoo.allegro import Allegro
    from oracle import allegro_ref as AR

    g = torch.Generator().manual_seed(11)
    n = 30
    pos = torch.rand(n, 3, generator=g, dtype=torch.float64) * 8.0
    Z = torch.randint(0, 3, (n,), generator=g)
    r = (pos[None] - pos[:, None]).norm(dim=-1)
    src, dst = torch.nonzero((r < 5.0) & (r > 0), as_tuple=True)
    ei = torch.stack([src, dst], 1)
    torch.manual_seed(12)
    cfg = dict(l_max=2, num_tensor_features=8, num_layers=2, r_max=5.0, num_bessel=8, poly_p=6)
    model = Allegro(num_elements=3, num_scalar_features=16, num_tensor_features=8, r_max=5.0, l_max=2,
                    num_layers=2).to(DEV)
    readout = torch.randn(2, 16, generator=torch.Generator().manual_seed(13), dtype=torch.float64) / 4

    p = pos.float().to(DEV).requires_grad_(True)
    diff = p[ei[:, 1].to(DEV)] - p[ei[:, 0].to(DEV)]
    feats = model(Z=Z.to(DEV), bond_dist=diff.norm(dim=-1), bond_diff=diff, edge_index=ei.to(DEV))
    e = (feats * readout.float().to(DEV)).sum()
    (fg,) = ag.grad(e, p, create_graph=True)
    model.zero_grad()
    (e ** 2 + (fg ** 2).sum()).backward()
    named = {k: q for k, q in model.named_parameters() if q.requires_grad}
    got = {k: (q.grad if q.grad is not None else torch.zeros_like(q)).detach().double().cpu()
           for k, q in named.items()}

    t = {k: v.detach().double().cpu() for k, v in model.state_dict().items()}
    leaves = {k: t[k].requires_grad_(True) for k in named}
    p64 = pos.float().double().requires_grad_(True)
    d64 = p64[ei[:, 1]] - p64[ei[:, 0]]
    cfg["avg_num_neighbors"] = getattr(model, "avg_num_neighbors", None)
    f64 = AR.allegro_features(t, cfg, Z, d64.norm(dim=-1), d64, ei)
    e64 = (f64 * readout).sum()
    (gp64,) = ag.grad(e64, p64, create_graph=True)
    grads = ag.grad(e64 ** 2 + (gp64 ** 2).sum(), list(leaves.values()), allow_unused=True)
    ref = {k: (gg if gg is not None else torch.zeros_like(leaves[k])).detach() for k, gg in zip(leaves, grads)}
    _compare_param_grads(got, ref, "Allegro force loss")
