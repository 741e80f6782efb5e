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
