"""Per-edge channelwise tensor product with shared weights (molix::edge_tp, Allegro's layer
product) vs the fp64 oracle, forward and backward.

The oracle is the channelwise TP + scatter of ``oracle/equivariant.py`` with each edge its own
sender and receiver and the shared weights broadcast to every edge; the shared weight gradient is
the oracle's per-edge gradient summed over edges.  Tolerance as for the scatter kernel:
norm-wise relative error <= 1e-5, max-abs <= 1e-4 x RMS of the reference.
"""

import numpy as np
import pytest
import torch

from oracle import equivariant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def irr(ls, mul=None):
    return " + ".join(f"{mul}x{l}{'e' if l % 2 == 0 else 'o'}" if mul else f"{l}{'e' if l % 2 == 0 else 'o'}"
                      for l in ls)


def assert_close(got, ref, what, rtol=1e-5):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    nref = np.linalg.norm(ref)
    if nref == 0:
        assert np.abs(got).max(initial=0) == 0, what
        return
    err = np.linalg.norm(got - ref) / nref
    rms = nref / np.sqrt(ref.size)
    mx = np.abs(got - ref).max()
    assert err <= rtol and mx <= rtol * rms, f"{what}: rel {err:.2e}, max-abs {mx:.2e} (rms {rms:.2e})"


def oracle_case(l_max, C, E, seed):
    ls = list(range(l_max + 1))
    rng = np.random.default_rng(seed)
    tp = O.ChannelwiseTP(irr(ls, C), irr(ls), irr(ls), C)
    x = rng.normal(size=(E, tp.nx * C)).astype(np.float32)
    Y = rng.normal(size=(E, tp.ny)).astype(np.float32)
    w = rng.normal(size=(len(tp.paths), C)).astype(np.float32)
    g = rng.normal(size=(E, tp.no * C)).astype(np.float32)
    ei = np.stack([np.arange(E), np.arange(E)], 1)
    wb = np.broadcast_to(w.reshape(1, -1), (E, w.size))
    ref = tp.forward(x, Y, wb, ei, E)
    rx, rY, rw = tp.backward(x, Y, wb, ei, g)
    rw = rw.reshape(E, len(tp.paths), C).sum(0)
    return ls, x, Y, w, to_kernel_rows(g, ls, C), to_kernel_rows(ref, ls, C), rx, rY, rw


def to_kernel_rows(a, ls, C):
    """The oracle's per-path output rows in molix::edge_tp's layout (the paths of one output
    irrep merged into one block, kernels.edge_tp_out_rows)."""
    import molnex_amd.kernels as K

    rows = K.edge_tp_out_rows(ls)
    a = np.asarray(a).reshape(a.shape[0], len(rows), C)
    out = np.empty_like(a)
    out[:, rows] = a
    return out.reshape(a.shape[0], -1)


@pytest.mark.parametrize("l_max", [0, 1, 2, 3])
@pytest.mark.parametrize("C", [8, 16, 32, 64, 128])
def test_edge_tp_matches_oracle(l_max, C):
    import molnex_amd.kernels as K

    E = 389 if C >= 64 else 1237  # not a multiple of the edges per wavefront
    ls, x, Y, w, g, ref, rx, rY, rw = oracle_case(l_max, C, E, seed=10 * l_max + C)
    config = K.tp_config_id(ls, ls, ls)
    assert K.edge_tp_supported(config, C)
    xd, Yd, wd = (torch.from_numpy(a).to(DEV).requires_grad_(True) for a in (x, Y, w))
    out = K.edge_tp(xd, Yd, wd, config, C)
    assert_close(out.detach().cpu().numpy(), ref, f"out l<={l_max} C={C}")
    gx, gY, gw = torch.autograd.grad(out, (xd, Yd, wd), torch.from_numpy(g).to(DEV))
    assert_close(gx.cpu().numpy(), rx, "grad_x")
    assert_close(gY.cpu().numpy(), rY, "grad_Y")
    assert_close(gw.cpu().numpy(), rw, "grad_w")


def test_edge_tp_many_edges_and_reproducible_weight_gradient():
    """More edges than one sweep of the backward grid (grid-stride loop), against the oracle;
    the weight gradient is summed in a fixed order, so two runs agree bitwise."""
    import molnex_amd.kernels as K

    E, C = 40_000, 16
    ls, x, Y, w, g, ref, rx, rY, rw = oracle_case(2, C, E, seed=5)
    config = K.tp_config_id(ls, ls, ls)
    xd, Yd, wd, gd = (torch.from_numpy(a).to(DEV) for a in (x, Y, w, g))
    out = K.edge_tp(xd, Yd, wd, config, C)
    assert_close(out.cpu().numpy(), ref, "out")
    a = K.edge_tp_backward(gd, xd, Yd, wd, config, C, True, True, True)
    b = K.edge_tp_backward(gd, xd, Yd, wd, config, C, True, True, True)
    assert_close(a[0].cpu().numpy(), rx, "grad_x")
    assert_close(a[1].cpu().numpy(), rY, "grad_Y")
    assert_close(a[2].cpu().numpy(), rw, "grad_w")
    assert torch.equal(a[2], b[2])


def test_edge_tp_empty_and_unsupported():
    import molnex_amd.kernels as K

    config = K.tp_config_id([0, 1], [0, 1], [0, 1])
    P, NX, NY, NO = K.tp_config_info(config)
    x = torch.zeros(0, NX * 16, device=DEV)
    Y = torch.zeros(0, NY, device=DEV)
    w = torch.randn(P, 16, device=DEV)
    assert K.edge_tp(x, Y, w, config, 16).shape == (0, NO * 16)
    gx, gY, gw, _ = K.edge_tp_backward(torch.zeros(0, NO * 16, device=DEV), x, Y, w, config, 16, True, True, True)
    assert gx.shape == (0, NX * 16) and gY.shape == (0, NY) and torch.equal(gw, torch.zeros_like(w))
    assert not K.edge_tp_supported(config, 24)
    with pytest.raises(Exception):
        K.edge_tp(torch.zeros(4, NX * 24, device=DEV), torch.zeros(4, NY, device=DEV), torch.zeros(P, 24, device=DEV),
                  config, 24)
    other = K.tp_config_id([0, 1], [0, 1, 2, 3], [0, 1])  # output filter differs from the input irreps
    assert not K.edge_tp_supported(other, 16)


@pytest.mark.parametrize("l_max,C", [(2, 16), (1, 8), (3, 64)])
def test_edge_tp_fused_channel_scale(l_max, C):
    """``x_scale`` (E, C): the forward equals the product of the pre-scaled x bitwise (the same fp32
    multiply in the kernel), the gradients match torch's scaling + unscaled product within 1e-6."""
    import molnex_amd.kernels as K

    E = 777
    ls = list(range(l_max + 1))
    config = K.tp_config_id(ls, ls, ls)
    P, NX, NY, NO = K.tp_config_info(config)
    g = torch.Generator(device=DEV).manual_seed(l_max + C)
    x = torch.randn(E, NX * C, device=DEV, generator=g).requires_grad_(True)
    s = torch.randn(E, C, device=DEV, generator=g).requires_grad_(True)
    Y = torch.randn(E, NY, device=DEV, generator=g).requires_grad_(True)
    w = torch.randn(P, C, device=DEV, generator=g).requires_grad_(True)
    gout = torch.randn(E, NO * C, device=DEV, generator=g)
    fused = K.edge_tp(x, Y, w, config, C, s)
    ref = K.edge_tp((x.view(E, NX, C) * s.unsqueeze(1)).reshape(E, -1), Y, w, config, C)
    assert torch.equal(fused, ref)
    a = torch.autograd.grad(fused, (x, s, Y, w), gout)
    b = torch.autograd.grad(ref, (x, s, Y, w), gout)
    for name, u, v in zip(("x", "scale", "Y", "w"), a, b):
        rel = float((u - v).norm() / v.norm())
        assert rel <= 1e-6, (name, rel)
