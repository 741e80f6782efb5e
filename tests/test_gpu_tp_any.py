"""GPU table-driven channelwise tensor product (``molix::tp_any``: irreps outside the compiled
configurations) vs the fp64 oracle ``ChannelwiseTPMul``, forward and backward, and through the
``ChannelWiseTensorProduct`` / ``ConvTP`` modules.

Tolerance (fp32 kernels vs fp64 oracle): norm-wise relative error <= 1e-5 and max-abs error
<= 1e-5 * RMS(reference) for every output and gradient.
"""

import numpy as np
import pytest
import torch

from oracle import equivariant as O
from tests.test_gpu_tp import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # non-uniform multiplicities, natural parity
    ("16x0e + 8x1o + 24x2e", "0e + 1o + 2e", "0e + 1o + 2e + 3o"),
    # non-natural parities with odd couplings (1o x 1o -> 1e, 1e x 1o -> 0o, 2o ...)
    ("8x0e + 8x1o + 8x1e + 4x2o", "0e + 1o + 1e", "0e + 0o + 1o + 1e + 2e + 2o"),
    # two blocks of one l, l = 3 everywhere
    ("8x0e + 8x0e + 8x1o + 8x3o", "0e + 1o + 2e + 3o", "0e + 1o + 2e + 3o + 3e"),
    # multiplicities above one 64-channel chunk, ragged
    ("96x0e + 70x1o", "0e + 1o + 2e", "0e + 1o + 2e"),
    # the full uniform configuration (also compiled: the two kernels are compared below)
    ("16x0e + 16x1o + 16x2e + 16x3o", "0e + 1o + 2e + 3o", "0e + 1o + 2e + 3o"),
]


@pytest.fixture(scope="module")
def ops():
    import molnex_amd.kernels  # noqa: F401

    return torch.ops.molix


def _data(tp, N, E, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(N, tp.nx)).astype(np.float32)
    Y = rng.normal(size=(E, tp.ny)).astype(np.float32)
    w = rng.normal(size=(E, tp.nw)).astype(np.float32)
    ei = rng.integers(0, N - 1, (E, 2))  # node N-1 isolated
    if E >= 10:
        ei[: E // 10, 1] = 0  # one heavy receiver
    g = rng.normal(size=(N, tp.no)).astype(np.float32)
    return x, Y, w, ei, g


def _check(ops, in1, in2, filt, N, E, seed):
    from molnex_amd import kernels as K
    from molnex_amd.irreps import ChannelwiseTPDescriptor

    tp = O.ChannelwiseTPMul(in1, in2, filt)
    table = K.tp_any_table(ChannelwiseTPDescriptor(in1, in2, filt))
    x, Y, w, ei, g = _data(tp, N, E, seed)
    xt, Yt, wt = (torch.tensor(a, device=DEV, requires_grad=True) for a in (x, Y, w))
    csr = ops.edge_csr(torch.tensor(ei, device=DEV), N)
    out = ops.tp_any(xt, Yt, wt, *csr, table)
    what = f"{in1} x {in2} -> {filt}, N={N} E={E}"
    assert_close(out.detach().cpu().numpy(), tp.forward(x, Y, w, ei, N), f"fwd {what}")
    if E == 0:
        return
    gx, gY, gw = torch.autograd.grad(out, (xt, Yt, wt), torch.tensor(g, device=DEV))
    rx, rY, rw = tp.backward(x, Y, w, ei, g)
    assert_close(gx.cpu().numpy(), rx, f"grad_x {what}")
    assert_close(gY.cpu().numpy(), rY, f"grad_Y {what}")
    assert_close(gw.cpu().numpy(), rw, f"grad_w {what}")


@pytest.mark.parametrize("case", range(len(CASES)))
def test_tp_any_vs_oracle(ops, case):
    print(f"tp_any case {case}: {CASES[case]}", flush=True)
    _check(ops, *CASES[case], N=40, E=400, seed=case)


def test_tp_any_edge_cases(ops):
    in1, in2, filt = CASES[1]
    _check(ops, in1, in2, filt, N=5, E=0, seed=10)  # no edges: zero output
    _check(ops, in1, in2, filt, N=3, E=1, seed=11)  # one edge
    _check(ops, "1x0e + 1x1e", "1o", "1o + 0o", N=4, E=9, seed=12)  # multiplicity 1


def test_tp_any_matches_compiled_kernel(ops):
    """Where a compiled configuration exists, the two product paths agree (fp32 summation order
    aside: 2e-6 forward; 1e-5 for the gradients, whose atomic sums run in different orders),
    forward and backward."""
    from molnex_amd import kernels as K
    from molnex_amd.irreps import ChannelwiseTPDescriptor

    in1, in2, filt = CASES[4]
    d = ChannelwiseTPDescriptor(in1, in2, filt)
    cfg = K.tp_config_id([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3])
    tp = O.ChannelwiseTPMul(in1, in2, filt)
    x, Y, w, ei, g = _data(tp, 60, 900, 13)
    xt, Yt, wt = (torch.tensor(a, device=DEV, requires_grad=True) for a in (x, Y, w))
    gt = torch.tensor(g, device=DEV)
    csr = ops.edge_csr(torch.tensor(ei, device=DEV), 60)
    a = ops.tp_any(xt, Yt, wt, *csr, K.tp_any_table(d))
    b = ops.tp_scatter(xt, Yt, wt, *csr, cfg, 16)
    assert_close(a.detach().cpu().numpy(), b.detach().cpu().numpy(), "fwd any vs compiled", rtol=2e-6)
    for u, v, name in zip(torch.autograd.grad(a, (xt, Yt, wt), gt), torch.autograd.grad(b, (xt, Yt, wt), gt),
                          ("x", "Y", "w")):
        assert_close(u.cpu().numpy(), v.cpu().numpy(), f"grad_{name} any vs compiled", rtol=1e-5)


def test_conv_tp_module_any_irreps(ops):
    """ConvTP with non-compiled irreps runs the table-driven kernels, forward and autograd."""
    from molnex_amd.molrep.interaction.tensor_product import ConvTP

    in1, in2, filt = CASES[1]
    conv = ConvTP(in_irreps=in1, out_irreps=filt, sh_irreps=in2)
    assert conv.cue_tp.config_id < 0 and conv.cue_tp.any_table is not None
    tp = O.ChannelwiseTPMul(in1, in2, filt)
    assert conv.weight_numel == tp.nw
    x, Y, w, ei, g = _data(tp, 30, 300, 14)
    xt, Yt, wt = (torch.tensor(a, device=DEV, requires_grad=True) for a in (x, Y, w))
    out = conv(xt, Yt, torch.tensor(ei, device=DEV), wt)
    assert_close(out.detach().cpu().numpy(), tp.forward(x, Y, w, ei, 30), "ConvTP fwd")
    gx, gY, gw = torch.autograd.grad(out, (xt, Yt, wt), torch.tensor(g, device=DEV))
    rx, rY, rw = tp.backward(x, Y, w, ei, g)
    for got, ref, name in ((gx, rx, "x"), (gY, rY, "Y"), (gw, rw, "w")):
        assert_close(got.cpu().numpy(), ref, f"ConvTP grad_{name}")


def test_tp_any_second_order(ops):
    """Second derivatives by trilinearity against the fp64 oracle (as for tp_scatter)."""
    import molnex_amd.second_order  # noqa: F401
    from molnex_amd import kernels as K
    from molnex_amd.irreps import ChannelwiseTPDescriptor

    in1, in2, filt = CASES[1]
    tp = O.ChannelwiseTPMul(in1, in2, filt)
    table = K.tp_any_table(ChannelwiseTPDescriptor(in1, in2, filt))
    N, E = 30, 250
    x, Y, w, ei, g = _data(tp, N, E, 15)
    rng = np.random.default_rng(16)
    sx, sY, sw = (rng.normal(size=a.shape).astype(np.float32) for a in (x, Y, w))
    xt, Yt, wt, gt = (torch.tensor(a, device=DEV, requires_grad=True) for a in (x, Y, w, g))
    csr = ops.edge_csr(torch.tensor(ei, device=DEV), N)
    out = ops.tp_any(xt, Yt, wt, *csr, table)
    gx, gY, gw = torch.autograd.grad(out, (xt, Yt, wt), gt, create_graph=True)
    L2 = sum((a * torch.tensor(b, device=DEV)).sum() for a, b in ((gx, sx), (gY, sY), (gw, sw)))
    dg, dx, dY, dw = torch.autograd.grad(L2, (gt, xt, Yt, wt))
    f = lambda a, b, c: tp.forward(a, b, c, ei, N)  # noqa: E731
    bw = lambda a, b, c: tp.backward(a, b, c, ei, g)  # noqa: E731
    refs = {"g": f(sx, Y, w) + f(x, sY, w) + f(x, Y, sw), "x": bw(x, sY, w)[0] + bw(x, Y, sw)[0],
            "Y": bw(sx, Y, w)[1] + bw(x, Y, sw)[1], "w": bw(sx, Y, w)[2] + bw(x, sY, w)[2]}
    for name, got in (("g", dg), ("x", dx), ("Y", dY), ("w", dw)):
        assert_close(got.cpu().numpy(), refs[name], f"second order d{name}")


def test_tp_any_config3_scale_matches_compiled(ops):
    """At the config-3 graph size (50k atoms, rc 5 A, ~2.6 M edges; 32 channels to bound memory) the
    table-driven product equals the compiled one, forward (2e-6) and all three gradients (1e-5)."""
    from molnex_amd import kernels as K
    from molnex_amd.irreps import ChannelwiseTPDescriptor

    g0 = torch.Generator().manual_seed(17)
    n, C = 50_000, 32
    L = (n / 0.1) ** (1.0 / 3.0)
    pos = (torch.rand((n, 3), generator=g0) * L).to(DEV)
    i, j, _, deltas, _ = ops.neighbor_list(pos, 5.0, torch.eye(3, device=DEV) * L, True)
    ei = torch.stack([j.long(), i.long()], 1)
    E = ei.shape[0]
    print(f"tp_any at scale: {E} edges", flush=True)
    irr = "0e + 1o + 2e + 3o"
    in1 = " + ".join(f"{C}x{t}" for t in irr.split(" + "))
    d = ChannelwiseTPDescriptor(in1, irr, irr)
    cfg = K.tp_config_id([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3])
    g = torch.Generator(device=DEV).manual_seed(18)
    x = torch.randn(n, d.irreps_in1.dim, device=DEV, generator=g, requires_grad=True)
    Y = ops.spherical_harmonics(deltas, 3).detach().requires_grad_(True)
    w = torch.randn(E, d.weight_numel, device=DEV, generator=g, requires_grad=True)
    go = torch.randn(n, d.irreps_out.dim, device=DEV, generator=g)
    csr = ops.edge_csr(ei, n)
    a = ops.tp_any(x, Y, w, *csr, K.tp_any_table(d))
    b = ops.tp_scatter(x, Y, w, *csr, cfg, C)
    assert_close(a.detach().cpu().numpy(), b.detach().cpu().numpy(), "fwd at scale", rtol=2e-6)
    ga = torch.autograd.grad(a, (x, Y, w), go)
    gb = torch.autograd.grad(b, (x, Y, w), go)
    for u, v, name in zip(ga, gb, ("x", "Y", "w")):
        assert_close(u.cpu().numpy(), v.cpu().numpy(), f"grad_{name} at scale", rtol=1e-5)


@pytest.mark.parametrize("in1,in2,filt", [
    # harmonics-like operand with odd parity blocks only, outputs of both parities per l
    ("4x1o + 6x2e", "1o + 2o", "0e + 0o + 1e + 1o + 2e + 2o + 3e + 3o"),
    # one block of 200 channels (4 chunks of 64, ragged) next to a multiplicity-1 block
    ("200x1e + 1x0o", "0e + 1o", "0o + 1o + 1e + 2o"),
])
def test_tp_any_more_irreps(ops, in1, in2, filt):
    print(f"tp_any {in1} x {in2} -> {filt}", flush=True)
    _check(ops, in1, in2, filt, N=30, E=250, seed=20)
