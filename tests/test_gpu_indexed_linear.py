"""The element-indexed linear of ElementUpdate (cuet.Linear(weight_classes=S,
method="indexed_linear"), src/molrep/interaction/element_update.py:101-109,147-158) on the HIP
indexed block kernel: per class against the fp64 oracle linear (oracle/mace_ref.py), gradients
against fp64 autograd, nodes with an out-of-range class give zeros, and the forward + input
gradient (the energy + forces path, weights frozen) run without a host synchronisation."""

import numpy as np
import pytest
import torch

from oracle import mace_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _blocks(s):
    out = []
    for tok in s.split("+"):
        mul, ir = tok.strip().split("x")
        out.append((int(mul), int(ir[:-1]), 1 if ir[-1] == "e" else -1))
    return out


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def _max_rms(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.pow(2).mean().sqrt().clamp_min(1e-300))


@pytest.mark.parametrize("irreps,S,R", [("128x0e+128x1o", 10, 3000), ("256x0e", 4, 1500), ("32x0e+16x1o+8x2e", 3, 777),
                                        ("64x0e", 16, 40)])
def test_indexed_linear_vs_oracle(irreps, S, R):
    from molnex_amd.molrep.interaction.linear import Linear

    torch.manual_seed(S + R)
    lin = Linear(irreps, irreps, internal_weights=False, weight_classes=S, method="indexed_linear")
    assert lin._hip_ok()
    W = torch.randn(S, lin.weight_numel)
    x = torch.randn(R, lin.irreps_in.dim)
    z = torch.randint(0, S, (R,))
    if S > 3:
        z[z == 2] = 1  # a class with no nodes
    z[:3] = torch.tensor([-1, S, S + 7])  # out of range: zero output
    out = lin.to(DEV)(x.to(DEV), weight=W.to(DEV), weight_indices=z.to(DEV))
    blocks = _blocks(irreps)
    ref = torch.zeros(R, lin.irreps_out.dim, dtype=torch.float64)
    for s in range(S):
        sel = z == s
        if sel.any():
            ref[sel] = mace_ref.linear(x[sel].double(), W[s].double(), blocks, blocks)
    print(f"{irreps} S={S}: rel err {_rel(out, ref):.2e}, max-abs {_max_rms(out, ref):.2e} RMS")
    assert torch.equal(out[:3].cpu(), torch.zeros(3, lin.irreps_out.dim))
    assert _rel(out, ref) <= 1e-6 and _max_rms(out, ref) <= 1e-5

    # gradients of x and W against fp64 autograd of the per-class oracle
    xg = x.to(DEV).requires_grad_(True)
    Wg = W.to(DEV).requires_grad_(True)
    go = torch.randn(R, lin.irreps_out.dim)
    gx, gW = torch.autograd.grad(lin(xg, weight=Wg, weight_indices=z.to(DEV)), (xg, Wg), go.to(DEV))
    x64, W64 = x.double().requires_grad_(True), W.double().requires_grad_(True)
    parts = torch.zeros(R, lin.irreps_out.dim, dtype=torch.float64)
    for s in range(S):
        sel = z == s
        if sel.any():
            parts = parts.index_put((sel.nonzero()[:, 0],), mace_ref.linear(x64[sel], W64[s], blocks, blocks))
    rx, rW = torch.autograd.grad(parts, (x64, W64), go.double())
    assert _rel(gx, rx) <= 1e-6 and _max_rms(gx, rx) <= 1e-5
    assert _rel(gW, rW) <= 1e-6


def test_element_update_has_no_host_sync():
    """ElementUpdate forward and input gradient with frozen weights: no device-to-host copy or
    synchronisation (torch's sync debug mode raises on one)."""
    from molnex_amd.molrep.interaction import ElementUpdate

    torch.manual_seed(0)
    eu = ElementUpdate(hidden_dim=128, num_species=10, irreps="128x0e+128x1o").to(DEV)
    eu.weight.requires_grad_(False)
    R = 5000
    h = torch.randn(R, 512, device=DEV)
    m = torch.randn(R, 512, device=DEV, requires_grad=True)
    z = torch.randint(0, 10, (R,), device=DEV)
    out = eu(h, m, z)  # warm-up (lazy buffers, library load)
    torch.autograd.grad(out.sum(), m)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        out = eu(h, m, z)
        (gm,) = torch.autograd.grad(out, m, torch.ones_like(out))
    finally:
        torch.cuda.set_sync_debug_mode(0)
    assert torch.isfinite(gm).all()
