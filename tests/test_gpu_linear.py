"""Equivariant Linear on the GPU (hipBLASLt GEMMs, split-K weight gradient for tall inputs)
against the fp64 oracle linear (oracle/mace_ref.py) and its autograd gradients.
Tolerance: norm-wise relative error <= 1e-5."""

import numpy as np
import pytest
import torch

from oracle import mace_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300)


@pytest.mark.parametrize("rows", [100, 70001])
def test_linear_forward_backward_vs_oracle(rows):
    from molnex_amd.molrep.interaction import Linear

    torch.manual_seed(0)
    lin = Linear("16x0e+16x1o", "8x0e+8x1o").to(DEV)
    x = torch.randn(rows, 64, device=DEV, requires_grad=True)
    g = torch.randn(rows, 32, device=DEV)
    out = lin(x)
    gx, gw = torch.autograd.grad(out, (x, lin.weight), g)
    xd = x.detach().cpu().double().requires_grad_(True)
    wd = lin.weight.detach().cpu().double().requires_grad_(True)
    ref = mace_ref.linear(xd, wd, [(16, 0, 1), (16, 1, -1)], [(8, 0, 1), (8, 1, -1)])
    rgx, rgw = torch.autograd.grad(ref, (xd, wd), g.cpu().double())
    assert _rel(out.detach().cpu(), ref.detach()) <= 1e-5
    assert _rel(gx.cpu(), rgx) <= 1e-5
    assert _rel(gw.cpu(), rgw) <= 1e-5


@pytest.mark.parametrize("irr_in,irr_out,rows", [
    ("16x0e+16x1o", "8x0e+8x1o", 1000),
    ("128x0e+128x1o+128x2e+128x3o", "128x0e+128x1o", 5003),          # unused input blocks
    ("128x0e+128x1o+128x0e+128x1o+64x2e", "128x0e+128x1o+32x2e", 777),  # two sources per output
    ("40x0e+24x1o", "24x0e+40x1o+16x2e", 333),                        # output block without source
    ("8x3o+16x3o", "200x3o", 65),                                      # N > 128: second column tile
    ("128x0e+128x1o", "128x0e+128x1o", 120_001),     # weights resident in LDS, many row groups per workgroup
    ("256x0e+256x1o+128x1o", "128x0e+128x1o", 60_000),  # K = 256 / 384: weight chunks streamed
])
def test_hip_block_linear_matches_torch_blocks(irr_in, irr_out, rows):
    """The HIP block kernel (forward, input gradient) and the torch block GEMMs agree; weight
    gradients go through the torch path in both."""
    from molnex_amd.molrep.interaction import Linear
    from molnex_amd.molrep.interaction import linear as L

    torch.manual_seed(1)
    lin = Linear(irr_in, irr_out).to(DEV)
    assert lin._hip_ok()
    x = torch.randn(rows, lin.irreps_in.dim, device=DEV, requires_grad=True)
    g = torch.randn(rows, lin.irreps_out.dim, device=DEV)
    out = lin(x)
    gx, gw = torch.autograd.grad(out, (x, lin.weight), g)
    out0 = L._BlockLinear.apply(x, lin.weight.reshape(-1), lin.plan, lin.irreps_out.dim)
    gx0, gw0 = torch.autograd.grad(out0, (x, lin.weight), g)
    assert _rel(out.detach().cpu(), out0.detach().cpu()) <= 1e-5
    assert _rel(gx.cpu(), gx0.cpu()) <= 1e-5
    assert _rel(gw.cpu(), gw0.cpu()) <= 1e-5
    # fp64 reference of the same math
    xd, wd = x.detach().double(), lin.weight.detach().double().reshape(-1)
    ref = L._block_forward(xd, wd, lin.plan, lin.irreps_out.dim)
    assert _rel(out.detach().cpu(), ref.cpu()) <= 1e-5
    o = out.detach().cpu().double()
    assert (o - ref.cpu()).abs().max() <= 1e-5 * ref.cpu().pow(2).mean().sqrt()


def test_hip_block_linear_zero_rows_and_views():
    from molnex_amd.molrep.interaction import Linear

    lin = Linear("16x0e+16x1o", "16x0e+16x1o").to(DEV)
    assert lin(torch.empty(0, 64, device=DEV)).shape == (0, 64)
    base = torch.randn(50, 65, device=DEV)
    xv = base[:, 1:]  # misaligned, strided view
    assert torch.allclose(lin(xv), lin(xv.contiguous()), rtol=1e-6, atol=1e-6)


def test_hip_block_linear_dynamic_range():
    """Rows of the input spanning 40 decades and weight columns spanning 24: every output element
    (forward and input gradient) stays within the error bound of an fp32 GEMM, K u sum |a| |w|
    (K <= 64 here, u = 2^-24), since each bf16 part of the three-way split carries the full fp32
    exponent range (a scaled fp16 split would lose the small entries of a column that spans
    many decades)."""
    from molnex_amd.molrep.interaction import Linear
    from molnex_amd.molrep.interaction import linear as L

    torch.manual_seed(3)
    lin = Linear("64x0e+32x1o", "32x0e+64x1o").to(DEV)
    with torch.no_grad():
        for off_o, mul_o, d, srcs, _ in lin.plan:
            for o, m, wo in srcs:
                blk = lin.weight.view(-1)[wo:wo + m * mul_o].view(m, mul_o)
                blk *= torch.logspace(-12, 12, mul_o, device=DEV)
    rows = 3000
    x = torch.randn(rows, lin.irreps_in.dim, device=DEV)
    x *= torch.logspace(-20, 20, rows, device=DEV)[torch.randperm(rows, device=DEV)].unsqueeze(1)
    x.requires_grad_(True)
    g = torch.randn(rows, lin.irreps_out.dim, device=DEV) * torch.logspace(-15, 15, rows, device=DEV).unsqueeze(1)
    out = lin(x)
    (gx,) = torch.autograd.grad(out, x, g)
    xd, wd = x.detach().double(), lin.weight.detach().double().reshape(-1)
    ref = L._block_forward(xd, wd, lin.plan, lin.irreps_out.dim)
    gref = L._block_backward(xd, wd, g.double(), lin.plan, True, False)[0]
    # per element, against the scale of an fp32 GEMM's rounding: the sum of |a| |w| products
    bound = L._block_forward(xd.abs(), wd.abs(), lin.plan, lin.irreps_out.dim)
    gbound = L._block_backward(xd.abs(), wd.abs(), g.double().abs(), lin.plan, True, False)[0]
    for got, want, b in ((out.detach().double(), ref, bound), (gx.double(), gref, gbound)):
        assert torch.isfinite(got).all()
        err = ((got - want).abs() / b.clamp_min(1e-300)).max().item()
        assert err <= 64 * 2.0 ** -24, err
