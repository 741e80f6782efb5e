"""Radial-MLP output layer (molix::edge_weights) vs the same Linear in float64.

The kernel computes near-fp32 products on the fp16 matrix cores (operands scaled by powers of two
per row / output column and split into two fp16 parts, three partial products).  Tolerance: norm-wise relative error at most 4x that of torch's own fp32 GEMM on
the same inputs (and at most 1e-5), max-abs at most 4x torch's or 1e-5 x RMS of the result, for the forward,
the input gradient and the training gradients of weight and bias.
"""

import pytest
import torch

import molnex_amd.kernels as K
from molnex_amd.config import config
from molnex_amd.molrep.interaction.radial_mlp import RadialWeightMLP

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    return float((a.detach().double() - b.detach().double()).norm() / b.double().norm().clamp_min(1e-300))


def _check(got, ref64, torch32):
    got, ref64 = got.detach().double().cpu(), ref64.detach().double().cpu()
    rel, rel32 = _rel(got, ref64), _rel(torch32.cpu(), ref64)
    assert rel <= max(4 * rel32, 2e-7) and rel <= 1e-5, (rel, rel32)
    rms = float(ref64.pow(2).mean().sqrt())
    worst32 = float((torch32.detach().cpu().double() - ref64).abs().max())
    assert float((got - ref64).abs().max()) <= max(4 * worst32, 1e-5 * rms)


@pytest.mark.parametrize("k,n,e", [(64, 2944, 1000), (128, 512, 777), (32, 736, 100), (16, 184, 33),
                                   (64, 40, 1), (128, 1280, 4099), (64, 8, 129)])
def test_edge_weights_matches_fp64(k, n, e):
    g = torch.Generator().manual_seed(k * 7 + n + e)
    h = torch.randn(e, k, generator=g)
    W = torch.randn(n, k, generator=g) / k ** 0.5
    b = torch.randn(n, generator=g)
    gout = torch.randn(e, n, generator=g)
    hd, Wd, bd = (t.to(DEV).requires_grad_(True) for t in (h, W, b))
    out = K.edge_weights(hd, Wd, bd)
    gh, gW, gb = torch.autograd.grad(out, (hd, Wd, bd), gout.to(DEV))

    h64, W64, b64 = (t.double().requires_grad_(True) for t in (h, W, b))
    out64 = h64 @ W64.t() + b64
    gh64, gW64, gb64 = torch.autograd.grad(out64, (h64, W64, b64), gout.double())
    h32, W32, b32 = (t.to(DEV).requires_grad_(True) for t in (h, W, b))
    out32 = torch.addmm(b32, h32, W32.t())
    gh32, gW32, gb32 = torch.autograd.grad(out32, (h32, W32, b32), gout.to(DEV))

    _check(out, out64, out32)
    _check(gh, gh64, gh32)
    _check(gW, gW64, gW32)
    _check(gb, gb64, gb32)


def test_edge_weights_without_bias_and_wide_range():
    """No bias; rows spanning 30 orders of magnitude (the split is relative to each value)."""
    g = torch.Generator().manual_seed(5)
    e, k, n = 300, 64, 96
    scale = 10.0 ** torch.linspace(-15, 15, e, dtype=torch.float64).unsqueeze(1)
    h = (torch.randn(e, k, generator=g, dtype=torch.float64) * scale).float()
    W = torch.randn(n, k, generator=g) / 8
    out = K.edge_weights(h.to(DEV), W.to(DEV)).cpu().double()
    ref = h.double() @ W.double().t()
    row_rel = (out - ref).norm(dim=1) / ref.norm(dim=1)
    assert float(row_rel.max()) <= 1e-6
    gout = (torch.randn(e, n, generator=g, dtype=torch.float64) * scale).float()
    gh = K.edge_weights_backward(gout.to(DEV), W.to(DEV)).cpu().double()
    ref_g = gout.double() @ W.double()
    assert float(((gh - ref_g).norm(dim=1) / ref_g.norm(dim=1)).max()) <= 1e-6


def test_edge_weights_empty_and_unsupported():
    W = torch.randn(64, 32, device=DEV)
    assert K.edge_weights(torch.empty(0, 32, device=DEV), W).shape == (0, 64)
    assert not K.edge_weights_supported(48, 64)
    assert not K.edge_weights_supported(64, 60)
    with pytest.raises(Exception):
        K.edge_weights(torch.zeros(4, 48, device=DEV), torch.zeros(64, 48, device=DEV))


@pytest.mark.parametrize("hidden,out", [(64, 2944), (128, 512)])
def test_module_matches_hipblaslt_path(hidden, out):
    """RadialWeightMLP with the kernel vs the hipBLASLt last layer, both against the module in
    float64: outputs and input gradients."""
    import copy

    torch.manual_seed(1)
    m = RadialWeightMLP(in_dim=8, hidden_dim=hidden, out_dim=out, num_layers=2).to(DEV)
    for p in m.parameters():
        p.requires_grad_(False)
    m64 = copy.deepcopy(m).double()
    feats = (torch.rand(2001, 8, device=DEV) * 2 - 1).requires_grad_(True)
    gout = torch.randn(2001, out, device=DEV)
    w1 = m(feats)
    (g1,) = torch.autograd.grad(w1, feats, gout)
    config.edge_weights_kernel = False
    try:
        w0 = m(feats)
        (g0,) = torch.autograd.grad(w0, feats, gout)
    finally:
        config.edge_weights_kernel = True
    f64 = feats.detach().double().requires_grad_(True)
    w64 = m64(f64)
    (g64,) = torch.autograd.grad(w64, f64, gout.double())
    _check(w1, w64, w0)
    _check(g1, g64, g0)


def test_edge_weights_config3_scale_sampled_rows():
    """BASELINE config-3 shape (2.6 M edges, 64 -> 2944): sampled rows of the forward and of the
    input gradient against float64."""
    E, k, n = 2_618_418, 64, 2944
    g = torch.Generator(device=DEV).manual_seed(3)
    h = torch.randn(E, k, device=DEV, generator=g)
    W = torch.randn(n, k, device=DEV, generator=g) / 8
    b = torch.randn(n, device=DEV, generator=g)
    rows = torch.randint(0, E, (256,), device=DEV, generator=g)
    rows[-1] = E - 1
    out = K.edge_weights(h, W, b)
    ref = h[rows].double() @ W.double().t() + b.double()
    _check(out[rows], ref, h[rows] @ W.t() + b)
    del out
    gw = torch.randn(E, n, device=DEV, generator=g)
    gh = K.edge_weights_backward(gw, W)
    ref = gw[rows].double() @ W.double()
    _check(gh[rows], ref, gw[rows] @ W)


@pytest.mark.parametrize("n,k,e", [(64, 64, 1000), (16, 64, 777), (64, 16, 333), (16, 16, 5)])
def test_edge_weights_backward_accumulating_matches_fp64(n, k, e):
    """``out += grad @ weight`` in place (molix::edge_weights_backward_acc) against fp64, on an
    ``out`` that already holds a gradient; the same product as edge_weights_backward, added."""
    g = torch.Generator(device=DEV).manual_seed(n + k + e)
    grad = torch.randn(e, n, device=DEV, generator=g)
    weight = torch.randn(n, k, device=DEV, generator=g) / 4
    out = torch.randn(e, k, device=DEV, generator=g)
    ref = out.double() + grad.double() @ weight.double()
    K.edge_weights_backward_acc(grad, weight, out)
    err = float((out.double() - ref).norm() / ref.norm())
    assert err <= 1e-6, err
    prod = K.edge_weights_backward(grad, weight)
    assert float((prod.double() - grad.double() @ weight.double()).norm() / (grad.double() @ weight.double()).norm()) <= 1e-6
    with pytest.raises(ValueError):
        K.edge_weights_backward_acc(grad, weight, torch.empty(e, k + 1, device=DEV))
    # into a column block of a wider tensor (rows k + 12 floats apart, columns 4 .. 4 + k): the
    # block takes the product, the columns either side stay as they were
    wide = torch.randn(e, k + 12, device=DEV, generator=g)
    before = wide.clone()
    K.edge_weights_backward_acc(grad, weight, wide[:, 4:4 + k])
    ref = before[:, 4:4 + k].double() + grad.double() @ weight.double()
    err = float((wide[:, 4:4 + k].double() - ref).norm() / ref.norm())
    assert err <= 1e-6, err
    assert torch.equal(wide[:, :4], before[:, :4]) and torch.equal(wide[:, 4 + k:], before[:, 4 + k:])
    with pytest.raises(ValueError):
        K.edge_weights_backward_acc(grad, weight, wide[:, 2:2 + k])  # rows not 16-byte aligned
