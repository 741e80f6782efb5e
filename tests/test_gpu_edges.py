"""molix::bond_vectors vs torch advanced indexing (the reference pipeline's formulation)."""

import pytest
import torch

import molnex_amd.kernels  # noqa: F401

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _graph(shuffle: bool):
    g = torch.Generator().manual_seed(7 + int(shuffle))
    n, L = 3000, 31.0
    pos = (torch.rand(n, 3, generator=g) * L).to(DEV)
    box = torch.eye(3, device=DEV) * L
    i, j, shifts, _, _ = torch.ops.molix.neighbor_list(pos, 5.0, box, True)
    ei = torch.stack([j.long(), i.long()], 1)
    if shuffle:
        p = torch.randperm(ei.shape[0], generator=g).to(DEV)
        ei, shifts = ei[p].contiguous(), shifts[p].contiguous()
    return pos, ei, shifts


@pytest.mark.parametrize("shuffle", [False, True])
def test_bond_vectors_forward_and_gradient(shuffle):
    pos, ei, shifts = _graph(shuffle)
    gout = torch.randn(ei.shape[0], 3, device=DEV)
    p1 = pos.clone().requires_grad_(True)
    d1 = torch.ops.molix.bond_vectors(p1, ei, shifts)
    (g1,) = torch.autograd.grad(d1, p1, gout)
    p0 = pos.clone().requires_grad_(True)
    d0 = p0[ei[:, 1]] - p0[ei[:, 0]] - shifts
    (g0,) = torch.autograd.grad(d0, p0, gout)
    assert torch.equal(d1, d0)
    assert float((g1 - g0).norm() / g0.norm()) <= 1e-6
    # no shifts
    d2 = torch.ops.molix.bond_vectors(pos, ei)
    assert torch.equal(d2, pos[ei[:, 1]] - pos[ei[:, 0]])


def test_bond_vectors_empty_and_shift_gradient():
    pos = torch.randn(5, 3, device=DEV, requires_grad=True)
    ei = torch.empty(0, 2, dtype=torch.long, device=DEV)
    d = torch.ops.molix.bond_vectors(pos, ei)
    assert d.shape == (0, 3)
    (g,) = torch.autograd.grad(d.sum(), pos, allow_unused=True)
    assert g is None or float(g.abs().sum()) == 0.0
    ei = torch.tensor([[0, 1], [2, 1], [1, 4]], device=DEV)
    sh = torch.randn(3, 3, device=DEV, requires_grad=True)
    d = torch.ops.molix.bond_vectors(pos, ei, sh)
    gp, gs = torch.autograd.grad(d.sum(), (pos, sh))
    assert torch.equal(gs, -torch.ones_like(sh))
    # per component: +1 for each incoming edge, -1 for each outgoing one
    assert torch.equal(gp, torch.tensor([[-1.] * 3, [1.] * 3, [-1.] * 3, [0.] * 3, [1.] * 3], device=DEV))
