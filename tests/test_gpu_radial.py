"""Fused radial-MLP hidden stack (molix::radial_hidden) vs a float64 torch MLP.

The kernel computes in fp32 with MFMA; the reference is the same Linear/SiLU stack in
float64 on the same (fp32-representable) inputs and weights.  Tolerance: 1e-5 relative
(Frobenius) for the output and for the gradient w.r.t. the edge features.
"""

import pytest
import torch

import molnex_amd.kernels as K
from molnex_amd.config import config
from molnex_amd.molrep.interaction.radial_mlp import RadialWeightMLP

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-300))


def _mlp_params(kin, H, L, g):
    Ws, bs = [], []
    for j in range(L):
        fan = kin if j == 0 else H
        Ws.append(torch.randn(H, fan, generator=g) / fan ** 0.5)
        bs.append(torch.randn(H, generator=g) * 0.1)
    return Ws, bs


def _ref(feats, Ws, bs):
    h = feats
    for W, b in zip(Ws, bs):
        h = torch.nn.functional.silu(h @ W.t() + b)
    return h


# input widths up to 16 run the LDS-resident grid-strided kernels (the large-E cases walk many
# edge groups per wavefront), wider inputs the per-layer staged ones
@pytest.mark.parametrize("kin,H,L,E", [(8, 64, 2, 1000), (8, 128, 2, 4099), (8, 128, 1, 77), (5, 32, 1, 33),
                                       (13, 64, 3, 31), (64, 32, 4, 100), (8, 64, 4, 257), (40, 64, 1, 64),
                                       (8, 32, 2, 1), (8, 128, 2, 300_007), (16, 64, 2, 200_003),
                                       (24, 128, 2, 5000), (40, 64, 3, 5003), (33, 32, 2, 77),
                                       (56, 64, 2, 20_011)])
def test_radial_hidden_matches_fp64(kin, H, L, E):
    g = torch.Generator().manual_seed(kin * 1000 + H * 10 + L)
    Ws, bs = _mlp_params(kin, H, L, g)
    feats = torch.randn(E, kin, generator=g) * 2.0
    gout = torch.randn(E, H, generator=g)
    raw = torch.cat([t.reshape(-1) for W, b in zip(Ws, bs) for t in (W, b)])
    f = feats.to(DEV).requires_grad_(True)
    h = K.radial_hidden(f, raw.to(DEV), kin, H, L)
    (gf,) = torch.autograd.grad(h, f, gout.to(DEV))
    f64 = feats.double().requires_grad_(True)
    h64 = _ref(f64, [W.double() for W in Ws], [b.double() for b in bs])
    (gf64,) = torch.autograd.grad(h64, f64, gout.double())
    assert _rel(h.cpu(), h64) <= 1e-5
    assert _rel(gf.cpu(), gf64) <= 1e-5
    for a, r in ((h.detach().cpu().double(), h64.detach()), (gf.cpu().double(), gf64)):
        assert (a - r).abs().max() <= 1e-5 * r.pow(2).mean().sqrt()


def test_radial_hidden_empty_and_unsupported():
    raw = torch.zeros(8 * 64 + 64 + 64 * 64 + 64, device=DEV)
    out = K.radial_hidden(torch.empty(0, 8, device=DEV), raw, 8, 64, 2)
    assert out.shape == (0, 64)
    assert not K.radial_supported(8, 48, 2)
    assert not K.radial_supported(8, 128, 3)
    with pytest.raises(Exception):
        K.radial_hidden(torch.zeros(4, 8, device=DEV), raw, 8, 48, 2)


@pytest.mark.parametrize("hidden,layers", [(64, 2), (128, 2)])
def test_module_fused_matches_sequential(hidden, layers):
    """RadialWeightMLP with frozen parameters: fused hidden stack vs the Sequential path,
    outputs and input gradients, both in fp32 on the GPU."""
    torch.manual_seed(0)
    m = RadialWeightMLP(in_dim=8, hidden_dim=hidden, out_dim=96, num_layers=layers).to(DEV)
    for p in m.parameters():
        p.requires_grad_(False)
    feats = (torch.rand(3001, 8, device=DEV) * 2 - 1).requires_grad_(True)
    gout = torch.randn(3001, 96, device=DEV)
    assert m._fused_hidden(feats)
    w1 = m(feats)
    (g1,) = torch.autograd.grad(w1, feats, gout)
    config.fused_radial = False
    try:
        assert not m._fused_hidden(feats)
        w0 = m(feats)
        (g0,) = torch.autograd.grad(w0, feats, gout)
    finally:
        config.fused_radial = True
    assert _rel(w1, w0) <= 1e-5
    assert _rel(g1, g0) <= 1e-5


def test_module_trains_through_sequential():
    """Parameters that need gradients take the Sequential path (the fused kernel has no
    parameter gradient)."""
    m = RadialWeightMLP(in_dim=8, hidden_dim=64, out_dim=32).to(DEV)
    feats = torch.randn(100, 8, device=DEV)
    assert not m._fused_hidden(feats)
    m(feats).sum().backward()
    assert m.mlp[0].weight.grad is not None


def test_module_last_layer_trained_hidden_fused():
    """Frozen hidden Linears with a trainable last Linear: hidden stack fused, last layer in torch,
    its weight gradient intact."""
    torch.manual_seed(0)
    m = RadialWeightMLP(in_dim=8, hidden_dim=64, out_dim=40, num_layers=2).to(DEV)
    for p in m.mlp[:-1].parameters():
        p.requires_grad_(False)
    feats = torch.randn(500, 8, device=DEV)
    assert m._fused_hidden(feats)
    out = m(feats)
    out.square().sum().backward()
    g1 = m.mlp[-1].weight.grad.clone()
    m.mlp[-1].weight.grad = None
    config.fused_radial = False
    try:
        m(feats).square().sum().backward()
    finally:
        config.fused_radial = True
    assert _rel(g1, m.mlp[-1].weight.grad) <= 1e-5
