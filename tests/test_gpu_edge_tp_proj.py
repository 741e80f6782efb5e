"""molix::edge_tp_proj: Allegro's per-edge product fused with the projection after it
(src/molzoo/allegro.py:352-367,465-466; 16 channels) against the fp64 restatement of the two steps
(oracle/allegro_ref.py: the product of every kept path, then oracle.mace_ref's equivariant linear
on its irrep blocks), on the module's own parameters: forward, every first-order gradient (x, Y,
the shared path weights, the per-channel scale of x), the projection's weight gradient and the
second derivatives through the tracked form; the fixed-order weight-gradient sum is bitwise
reproducible.

Tolerance: 1e-5 norm-wise relative error of float64 (fp32 products and sums of at most 7 x 16
terms per projected output).
"""

import math

import pytest
import torch
from torch.library import opcheck

import molnex_amd.kernels as K
from oracle import allegro_ref as AR
from oracle.mace_ref import linear as lin_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
ops = torch.ops.molix


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-300))


def _layer(l_max, seed=0):
    from molnex_amd.molzoo.allegro import AllegroLayer

    torch.manual_seed(seed)
    layer = AllegroLayer(num_scalar_features=8, num_tensor_features=16, l_max=l_max).to(DEV)
    assert layer._proj_scale is not None
    return layer


def _inputs(layer, E, seed):
    g = torch.Generator().manual_seed(seed)
    D = (layer.l_max + 1) ** 2
    x = torch.randn(E, D * 16, generator=g)
    Y = torch.randn(E, D, generator=g)
    s = torch.rand(E, 16, generator=g) + 0.5
    return x, Y, s


def _ref(layer, x, Y, s, w_full, lin_w):
    """fp64: project(TP(s x, Y; w)) with the oracle's product and linear."""
    E, l_max = x.shape[0], layer.l_max
    D = (l_max + 1) ** 2
    xs = x.reshape(E, D, 16) * s[:, None, :] if s is not None else x.reshape(E, D, 16)
    out, blocks = AR.edge_tp(xs.reshape(E, D * 16), Y, w_full, l_max, 16)
    return lin_ref(out, lin_w, blocks, [(16, l, (-1) ** l) for l in range(l_max + 1)])


def _fused(layer, x, Y, s, w_full):
    tp, lin = layer.tp, layer.tp_linear
    w = w_full.reshape(tp.num_paths_full, 16).index_select(0, tp.kept_paths)
    proj = lin.weight.detach().reshape(-1, 16) * layer._proj_scale
    return K.edge_tp_proj(x, Y, w, tp.config_id, proj, s)


@pytest.mark.parametrize("l_max", [0, 1, 2, 3])
@pytest.mark.parametrize("E", [1, 7, 333])
@pytest.mark.parametrize("scaled", [True, False])
def test_edge_tp_proj_forward_and_gradients_vs_fp64(l_max, E, scaled):
    layer = _layer(l_max, seed=l_max)
    x, Y, s = _inputs(layer, E, seed=10 * l_max + E)
    s = s if scaled else None
    wf = layer.tp.weight.detach()
    # fp64 oracle with autograd
    x64, Y64 = x.double().requires_grad_(True), Y.double().requires_grad_(True)
    s64 = s.double().requires_grad_(True) if scaled else None
    w64 = wf.double().cpu().requires_grad_(True)
    ref = _ref(layer, x64, Y64, s64, w64, layer.tp_linear.weight.detach().double().cpu())
    R = torch.randn(ref.shape, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    leaves64 = [x64, Y64, w64] + ([s64] if scaled else [])
    g64 = torch.autograd.grad((ref * R).sum(), leaves64)
    # fused op on the GPU
    xg, Yg = x.to(DEV).requires_grad_(True), Y.to(DEV).requires_grad_(True)
    sg = s.to(DEV).requires_grad_(True) if scaled else None
    wg = wf.clone().requires_grad_(True)
    out = _fused(layer, xg, Yg, sg, wg)
    assert out.shape == ref.shape
    assert _rel(out, ref) <= 1e-5, _rel(out, ref)
    leaves = [xg, Yg, wg] + ([sg] if scaled else [])
    gg = torch.autograd.grad((out * R.float().to(DEV)).sum(), leaves)
    for name, a, b in zip(("x", "Y", "w", "x_scale"), gg, g64):
        assert _rel(a.reshape(b.shape), b) <= 1e-5, (name, _rel(a.reshape(b.shape), b))


def test_edge_tp_proj_matches_unfused_layer_path():
    """The layer's product + projection: fused (projection weights frozen) against molix::edge_tp
    followed by the block-linear projection, outputs and input gradients."""
    layer = _layer(2, seed=5)
    x, Y, s = (t.to(DEV) for t in _inputs(layer, 1001, seed=6))
    from molnex_amd.molzoo.allegro import _product_and_projection

    def run(frozen_proj):
        layer.tp_linear.weight.requires_grad_(not frozen_proj)
        xs = [t.clone().requires_grad_(True) for t in (x, Y, s)]
        out = _product_and_projection(layer, *xs)
        R = torch.randn(out.shape, generator=torch.Generator(device=DEV).manual_seed(8), device=DEV)
        g = torch.autograd.grad((out * R).sum(), xs + [layer.tp.weight])
        return out.detach(), g

    out_f, g_f = run(True)
    out_u, g_u = run(False)
    assert _rel(out_f, out_u) <= 1e-5
    for a, b in zip(g_f, g_u):
        assert _rel(a, b) <= 1e-5, _rel(a, b)


def test_edge_tp_proj_projection_gradient_and_second_order_vs_fp64():
    """proj requiring a gradient, and differentiating the input gradient again (create_graph): both
    take the tracked form (projection adjoint in torch, molix::edge_tp's backward)."""
    layer = _layer(2, seed=7)
    x, Y, s = _inputs(layer, 50, seed=11)
    tp, lin = layer.tp, layer.tp_linear
    lw64 = lin.weight.detach().double().cpu().requires_grad_(True)
    x64, Y64, s64 = x.double().requires_grad_(True), Y.double().requires_grad_(True), s.double().requires_grad_(True)
    w64 = tp.weight.detach().double().cpu().requires_grad_(True)
    ref = _ref(layer, x64, Y64, s64, w64, lw64)
    R = torch.randn(ref.shape, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    V = torch.randn(x.shape, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    (gx64, glw64) = torch.autograd.grad((ref * R).sum(), (x64, lw64), create_graph=True)
    h64 = torch.autograd.grad((gx64 * V).sum(), (Y64, s64, w64))

    xg, Yg, sg = (t.to(DEV).requires_grad_(True) for t in (x, Y, s))
    wg = tp.weight.detach().clone().requires_grad_(True)
    lwg = lin.weight.detach().clone().requires_grad_(True)
    w = wg.reshape(tp.num_paths_full, 16).index_select(0, tp.kept_paths)
    proj = lwg.reshape(-1, 16) * layer._proj_scale
    out = K.edge_tp_proj(xg, Yg, w, tp.config_id, proj, sg)
    gx, glw = torch.autograd.grad((out * R.float().to(DEV)).sum(), (xg, lwg), create_graph=True)
    assert _rel(gx, gx64) <= 1e-5, _rel(gx, gx64)
    assert _rel(glw, glw64) <= 1e-5, _rel(glw, glw64)
    h = torch.autograd.grad((gx * V.float().to(DEV)).sum(), (Yg, sg, wg))
    for a, b in zip(h, h64):
        assert _rel(a, b) <= 1e-5, _rel(a, b)


def test_edge_tp_proj_no_edges_and_reproducible_weight_gradient():
    layer = _layer(2, seed=2)
    tp = layer.tp
    proj = layer.tp_linear.weight.detach().reshape(-1, 16) * layer._proj_scale
    w = tp.weight.detach().reshape(tp.num_paths_full, 16).index_select(0, tp.kept_paths)
    P, NX, NY, NO = K.tp_config_info(tp.config_id)
    ni = sum(2 * l + 1 for l, _, _, _ in K.edge_tp_proj_blocks(tp.config_id))
    x0, Y0 = torch.zeros(0, NX * 16, device=DEV), torch.zeros(0, NY, device=DEV)
    assert K.edge_tp_proj(x0, Y0, w, tp.config_id, proj).shape == (0, ni * 16)
    _, _, gw, _, _ = K.edge_tp_proj_backward(torch.zeros(0, ni * 16, device=DEV), x0, Y0, w, tp.config_id, proj,
                                             False, False, True)
    assert gw.shape == w.shape and not gw.any()
    g = torch.Generator(device=DEV).manual_seed(4)
    E = 200_003
    x = torch.randn(E, NX * 16, device=DEV, generator=g)
    Y = torch.randn(E, NY, device=DEV, generator=g)
    go = torch.randn(E, ni * 16, device=DEV, generator=g)
    a = K.edge_tp_proj_backward(go, x, Y, w, tp.config_id, proj, True, True, True)
    b = K.edge_tp_proj_backward(go, x, Y, w, tp.config_id, proj, True, True, True)
    for u, v in zip(a[:3], b[:3]):
        assert torch.equal(u, v)
    # against the unfused backward at full size (the product's gradient from the projection's adjoint)
    gt = K.edge_tp_proj_adjoint(go, proj, K.edge_tp_proj_blocks(tp.config_id))
    c = K.edge_tp_backward(gt.contiguous(), x, Y, w, tp.config_id, 16, True, True, True)
    for u, v in zip(a[:3], c[:3]):
        assert _rel(u, v) <= 1e-5, _rel(u, v)


def test_opcheck_edge_tp_proj():
    layer = _layer(2, seed=3)
    tp = layer.tp
    P, NX, NY, NO = K.tp_config_info(tp.config_id)
    g = torch.Generator(device=DEV).manual_seed(9)
    E = 70
    x = torch.randn(E, NX * 16, device=DEV, generator=g).requires_grad_(True)
    Y = torch.randn(E, NY, device=DEV, generator=g).requires_grad_(True)
    w = torch.randn(P, 16, device=DEV, generator=g).requires_grad_(True)
    s = torch.randn(E, 16, device=DEV, generator=g).requires_grad_(True)
    proj = (layer.tp_linear.weight.detach().reshape(-1, 16) * layer._proj_scale).requires_grad_(True)
    opcheck(ops.edge_tp_proj.default, (x, Y, w, tp.config_id, proj, s))
    opcheck(ops.edge_tp_proj.default, (x, Y, w, tp.config_id, proj.detach()))
    ni = sum(2 * l + 1 for l, _, _, _ in K.edge_tp_proj_blocks(tp.config_id))
    gout = torch.randn(E, ni * 16, device=DEV, generator=g)
    opcheck(ops.edge_tp_proj_backward.default, (gout, x.detach(), Y.detach(), w.detach(), tp.config_id,
                                                proj.detach(), True, True, True, s.detach(), True))
    s2 = (torch.rand(E, 16, device=DEV, generator=g) + 0.5).requires_grad_(True)
    opcheck(ops.edge_tp_proj.default, (x, Y, w, tp.config_id, proj.detach(), s, s2))
    opcheck(ops.edge_tp_proj_backward.default, (gout, x.detach(), Y.detach(), w.detach(), tp.config_id,
                                                proj.detach(), True, True, True, s.detach(), True, s2.detach(),
                                                True))
    assert math.isfinite(float(gout.sum()))


@pytest.mark.parametrize("l_max", [1, 2, 3])
def test_edge_tp_proj_shared_x_matches_expanded(l_max):
    """x given as (E, NX), one value per component shared by the 16 channels (the first layer's
    harmonics, their channel weights in x_scale): forward and every gradient equal the op on the
    expanded (E, NX*16) rows, x's gradient being the channel sum; also through the tracked form
    (create_graph)."""
    layer = _layer(l_max, seed=20 + l_max)
    tp = layer.tp
    P, NX, NY, NO = K.tp_config_info(tp.config_id)
    E = 517
    g = torch.Generator().manual_seed(30 + l_max)
    xb = torch.randn(E, NX, generator=g).to(DEV)
    Y = torch.randn(E, NY, generator=g).to(DEV)
    s = (torch.rand(E, 16, generator=g) + 0.5).to(DEV)
    w = tp.weight.detach().reshape(tp.num_paths_full, 16).index_select(0, tp.kept_paths)
    proj = layer.tp_linear.weight.detach().reshape(-1, 16) * layer._proj_scale
    R = torch.randn(E, (l_max + 1) ** 2 * 16, generator=g).to(DEV)

    def run(shared, create_graph=False):
        xa, Ya, sa, wa = (t.clone().requires_grad_(True) for t in (xb, Y, s, w))
        x = xa if shared else xa.unsqueeze(-1).expand(E, NX, 16).reshape(E, NX * 16)
        out = K.edge_tp_proj(x, Ya, wa, tp.config_id, proj, sa)
        gr = torch.autograd.grad((out * R).sum(), (xa, Ya, sa, wa), create_graph=create_graph)
        return out.detach(), gr

    o1, g1 = run(True)
    o2, g2 = run(False)
    assert _rel(o1, o2) <= 1e-6
    for a, b in zip(g1, g2):
        assert a.shape == b.shape
        assert _rel(a, b) <= 1e-5, _rel(a, b)
    # second order through the tracked form: d<grad_x, v>/dY
    v = torch.randn(E, NX, generator=g).to(DEV)
    hs = []
    for shared in (True, False):
        xa, Ya = xb.clone().requires_grad_(True), Y.clone().requires_grad_(True)
        x = xa if shared else xa.unsqueeze(-1).expand(E, NX, 16).reshape(E, NX * 16)
        out = K.edge_tp_proj(x, Ya, w, tp.config_id, proj, s)
        (gx,) = torch.autograd.grad((out * R).sum(), xa, create_graph=True)
        (h,) = torch.autograd.grad((gx * v).sum(), Ya)
        hs.append(h)
    assert _rel(hs[0], hs[1]) <= 1e-5, _rel(hs[0], hs[1])


def test_edge_tp_proj_two_channel_scales_match_their_product():
    """x_scale2 multiplies x_scale inside the kernels: forward and every gradient (both scales'
    included) equal the op with the product as its one scale, first order and through the tracked
    form (create_graph)."""
    layer = _layer(2, seed=12)
    tp = layer.tp
    P, NX, NY, NO = K.tp_config_info(tp.config_id)
    E = 733
    g = torch.Generator().manual_seed(13)
    x = torch.randn(E, NX * 16, generator=g).to(DEV)
    Y = torch.randn(E, NY, generator=g).to(DEV)
    s1 = (torch.rand(E, 16, generator=g) + 0.5).to(DEV)
    s2 = (torch.rand(E, 16, generator=g) + 0.5).to(DEV)
    w = tp.weight.detach().reshape(tp.num_paths_full, 16).index_select(0, tp.kept_paths)
    proj = layer.tp_linear.weight.detach().reshape(-1, 16) * layer._proj_scale
    R = torch.randn(E, 9 * 16, generator=g).to(DEV)
    for create_graph in (False, True):
        xa, Ya, a1, a2 = (t.clone().requires_grad_(True) for t in (x, Y, s1, s2))
        out2 = K.edge_tp_proj(xa, Ya, w, tp.config_id, proj, a1, a2)
        g2 = torch.autograd.grad((out2 * R).sum(), (xa, Ya, a1, a2), create_graph=create_graph)
        xb, Yb, b1, b2 = (t.clone().requires_grad_(True) for t in (x, Y, s1, s2))
        out1 = K.edge_tp_proj(xb, Yb, w, tp.config_id, proj, b1 * b2)
        g1 = torch.autograd.grad((out1 * R).sum(), (xb, Yb, b1, b2), create_graph=create_graph)
        assert _rel(out2, out1) <= 1e-6
        for a, b in zip(g2, g1):
            assert _rel(a, b) <= 1e-5, _rel(a, b)
