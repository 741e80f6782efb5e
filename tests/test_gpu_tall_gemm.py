"""``molix::tall_tn``: a.T @ b for tall operands (the per-edge layers' weight gradients when
training) against float64 torch, fp32-accurate: norm-wise relative error and max-abs / RMS of the
reference <= 1e-5, and the norm-wise error no worse than twice torch's own fp32 GEMM's on the same
inputs (or 1e-6); shapes with ragged tiles, strided rows, no rows; its autograd and opcheck."""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, ref, what, tol=1e-5, mtol=1e-5):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    n = ref.norm()
    if n == 0:
        assert got.abs().max() == 0, what
        return
    rms = n / ref.numel() ** 0.5
    err, mx = float((got - ref).norm() / n), float((got - ref).abs().max())
    assert err <= tol and mx <= mtol * rms, f"{what}: rel {err:.2e}, max-abs {mx:.2e} (rms {float(rms):.2e})"
    return err


@pytest.fixture(scope="module")
def K():
    from molnex_amd import kernels

    return kernels


@pytest.mark.parametrize("rows,M,N", [(1, 1, 1), (15, 31, 33), (17, 64, 128), (1000, 1280, 128), (4096, 300, 70),
                                      (300_000, 512, 128), (2_607_384, 1280, 128)])
def test_tall_tn_vs_float64(K, rows, M, N):
    print(f"tall_tn {rows} x {M} x {N}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(rows + M)
    a = torch.randn(rows, M, device=DEV, generator=g)
    b = torch.randn(rows, N, device=DEV, generator=g)
    # a dynamic range across rows (edge weights near the cutoff are tiny): 2^±30, or 2^±8 at the full
    # 2.6 M rows, where fp32 accumulation itself (torch's GEMM included) reaches ~1e-5 at 2^±30
    span = 30 if rows <= 300_000 else 8
    a *= torch.exp2(torch.randint(-span, span + 1, (rows, 1), device=DEV, generator=g).float())
    ref = a.double().t() @ b.double()
    got = K.tall_tn(a, b)
    mm = a.t() @ b
    torch_err = float((mm.double() - ref).norm() / ref.norm())
    torch_mx = float((mm.double() - ref).abs().max())
    print(f"  rel error {float((got.double() - ref).norm() / ref.norm()):.2e}, torch fp32 {torch_err:.2e}", flush=True)
    if rows <= 300_000:
        err = _close(got, ref, f"{rows}x{M}x{N}")
    else:  # 2.6 M random-sign rows: the fp32 sum's own rounding is near 1e-5 of the result's RMS
        err = float((got.double() - ref).norm() / ref.norm())
        assert err <= 1e-5 and float((got.double() - ref).abs().max()) <= 2 * torch_mx
    assert err <= max(2 * torch_err, 1e-6), (err, torch_err)


def test_tall_tn_strided_rows_and_empty(K):
    g = torch.Generator(device=DEV).manual_seed(3)
    big = torch.randn(5000, 200, device=DEV, generator=g)
    a, b = big[:, 10:138], big[:, 150:190]  # row stride 200
    _close(K.tall_tn(a, b), a.double().t() @ b.double(), "strided")
    z = K.tall_tn(torch.empty(0, 7, device=DEV), torch.empty(0, 5, device=DEV))
    assert z.shape == (7, 5) and torch.all(z == 0)


def test_tall_tn_autograd_and_opcheck(K):
    from torch.library import opcheck

    g = torch.Generator(device=DEV).manual_seed(4)
    a = torch.randn(3000, 96, device=DEV, generator=g, requires_grad=True)
    b = torch.randn(3000, 40, device=DEV, generator=g, requires_grad=True)
    w = torch.randn(96, 40, device=DEV, generator=g)
    ga, gb = torch.autograd.grad((K.tall_tn(a, b) * w).sum(), (a, b))
    a64, b64 = a.detach().double().requires_grad_(True), b.detach().double().requires_grad_(True)
    ra, rb = torch.autograd.grad((a64.t() @ b64 * w.double()).sum(), (a64, b64))
    _close(ga, ra, "grad a", 1e-5)
    _close(gb, rb, "grad b", 1e-5)
    opcheck(torch.ops.molix.tall_tn.default, (a, b))


def test_rows_linear_first_and_second_derivatives():
    """The radial MLP's hidden Linear over many rows (weight gradients on tall_tn, also inside
    second derivatives) against float64 torch: output, first derivatives with create_graph, and the
    gradient of a loss on those derivatives."""
    from molnex_amd.molrep.interaction import radial_mlp as R

    g = torch.Generator(device=DEV).manual_seed(5)
    rows = R._ROWS_MIN + 1234
    lin = torch.nn.Linear(24, 40).to(DEV)
    x = torch.randn(rows, 24, device=DEV, generator=g, requires_grad=True)
    s = torch.randn(rows, 24, device=DEV, generator=g)
    ref = torch.nn.Linear(24, 40).double().to(DEV)
    ref.load_state_dict({k: v.double() for k, v in lin.state_dict().items()})
    x64 = x.detach().double().requires_grad_(True)

    def run(layer, xx, f):
        y = f(layer, xx)
        out = torch.nn.functional.silu(y)
        (gx,) = torch.autograd.grad(out.square().sum(), xx, create_graph=True)
        loss = (gx * s.to(gx.dtype)).sum() + out.sum()
        return y, torch.autograd.grad(loss, (layer.weight, layer.bias, xx))

    y, grads = run(lin, x, R._linear)
    y64, grads64 = run(ref, x64, lambda layer, xx: layer(xx))
    _close(y, y64, "rows linear output")
    for a, b, name in zip(grads, grads64, ("weight", "bias", "x")):
        _close(a, b, f"second-order grad {name}", 1e-5)


def test_silu_second_derivative_kernel(K):
    """kernels.silu_bwd2 against float64 autograd of SiLU's first derivative (odd size: tail path)."""
    g0 = torch.Generator(device=DEV).manual_seed(6)
    n = 100_003
    x, g, gg = (torch.randn(n, device=DEV, generator=g0) * 4 for _ in range(3))
    dx, dg = K.silu_bwd2(x, g, gg)
    x64, g64 = x.double().requires_grad_(True), g.double().requires_grad_(True)
    (gx,) = torch.autograd.grad(torch.nn.functional.silu(x64), x64, g64, create_graph=True)
    rx, rg = torch.autograd.grad(gx, (x64, g64), gg.double())
    sig = torch.sigmoid(x.double())
    for got, ref, scale, name in ((dx, rx, (gg * g).double().abs() * sig * (1 - sig), "d/dx"),
                                  (dg, rg, gg.double().abs(), "d/dg")):
        _close(got, ref, f"silu {name}", 1e-6)
        # elementwise, against the size of the terms (s'' crosses zero: no relative bound there); the
        # far tails (|x| up to ~20, 1 - sigma ~ 1e-9) are included
        err = (got.double() - ref).abs() / (scale * (1 + x.double().abs()) + 1e-30)
        assert float(err.max()) <= 1e-5, (name, float(err.max()))


def test_silu_second_derivative_offset_views(K):
    """Views starting one float into their storage (not 16-byte aligned) take the scalar path and
    agree bitwise with the aligned copies."""
    g0 = torch.Generator(device=DEV).manual_seed(7)
    base = [torch.randn(4099, device=DEV, generator=g0) for _ in range(3)]
    views = [t[1:] for t in base]
    assert all(v.data_ptr() % 16 for v in views)
    dx, dg = K.silu_bwd2(*views)
    ax, ag = K.silu_bwd2(*(v.clone() for v in views))
    assert torch.equal(dx, ax) and torch.equal(dg, ag)


def test_tall_tn_very_wide_row_stride(K):
    """A column slice of a tensor whose rows are 2^25 + 128 floats apart (beyond the kernel's row
    stride bound) is copied to contiguous rows instead of raising."""
    g0 = torch.Generator(device=DEV).manual_seed(8)
    rows = 16
    wide = torch.empty(rows, (1 << 25) + 128, device=DEV)
    a = wide[:, 64:128]
    a.copy_(torch.randn(rows, 64, device=DEV, generator=g0))
    b = torch.randn(rows, 32, device=DEV, generator=g0)
    assert a.stride(0) >= 1 << 25
    ref = a.double().t() @ b.double()
    out = K.tall_tn(a, b)
    _close(out, ref, "wide-stride tall_tn", 1e-6)
    out2, cs = K.tall_tn_colsum(a, b)
    _close(out2, ref, "wide-stride tall_tn_colsum", 1e-6)
    _close(cs, a.double().sum(0), "wide-stride column sums", 1e-6)
    del wide


def test_radial_mlp_hidden_second_order_many_rows():
    """RadialWeightMLP's hidden stack over many rows when training (Linears on tall_tn, SiLUs with the
    fused second derivative) against the same module in float64: a force-style loss on the input
    gradient, differentiated to every parameter and the input."""
    import copy

    from molnex_amd.molrep.interaction import radial_mlp as R

    torch.manual_seed(7)
    mlp = R.RadialWeightMLP(in_dim=8, hidden_dim=64, out_dim=32, num_layers=2).to(DEV)
    rows = R._ROWS_MIN + 999
    x = torch.randn(rows, 8, device=DEV, requires_grad=True)
    s = torch.randn(rows, 8, device=DEV)
    m64 = copy.deepcopy(mlp).double()
    x64 = x.detach().double().requires_grad_(True)

    def run(m, xx):
        h = m.hidden(xx)
        (gx,) = torch.autograd.grad(h.square().sum(), xx, create_graph=True)
        loss = (gx * s.to(gx.dtype)).sum() + h.sum()
        return torch.autograd.grad(loss, [*m.mlp[:-1].parameters(), xx])

    for a, b in zip(run(mlp, x), run(m64, x64)):
        _close(a, b, "hidden second order", 1e-5)


def test_tall_tn_colsum(K):
    """The column sums of a from the same pass (a layer's bias gradient) against float64, with a
    ragged tail and columns beyond one tile; autograd of both outputs and opcheck."""
    from torch.library import opcheck

    g0 = torch.Generator(device=DEV).manual_seed(8)
    for rows, M, N in ((300_001, 300, 64), (2_607_384, 1280, 128), (17, 5, 3)):
        a = torch.randn(rows, M, device=DEV, generator=g0) + 0.5
        b = torch.randn(rows, N, device=DEV, generator=g0)
        c, s = K.tall_tn_colsum(a, b)
        if rows <= 300_001:  # (the product at 2.6 M rows is checked by test_tall_tn_vs_float64)
            _close(c, a.double().t() @ b.double(), f"colsum product {rows}")
        _close(s, a.double().sum(0), f"colsum {rows}", 1e-6, 1e-6)
    a = torch.randn(3000, 40, device=DEV, generator=g0, requires_grad=True)
    b = torch.randn(3000, 24, device=DEV, generator=g0, requires_grad=True)
    wc, ws = torch.randn(40, 24, device=DEV, generator=g0), torch.randn(40, device=DEV, generator=g0)
    c, s = K.tall_tn_colsum(a, b)
    ga, gb = torch.autograd.grad((c * wc).sum() + (s * ws).sum(), (a, b))
    a64, b64 = a.detach().double().requires_grad_(True), b.detach().double().requires_grad_(True)
    ra, rb = torch.autograd.grad((a64.t() @ b64 * wc.double()).sum() + (a64.sum(0) * ws.double()).sum(), (a64, b64))
    _close(ga, ra, "colsum grad a", 1e-5)
    _close(gb, rb, "colsum grad b", 1e-5)
    opcheck(torch.ops.molix.tall_tn_colsum.default, (a, b))


def test_tall_tn_multi_tile_ragged_strided_colsum(K):
    """Several 256 x 128 output tiles in both directions with ragged edges, a row count that leaves a
    partial last step in every slab, row-strided views of both operands, and the column sums."""
    g0 = torch.Generator(device=DEV).manual_seed(9)
    rows = 100_003
    big = torch.randn(rows, 700, device=DEV, generator=g0)
    a, b = big[:, 3:336], big[:, 400:600]  # M = 333 (2 tiles), N = 200 (2 tiles), row stride 700
    c, s = K.tall_tn_colsum(a, b)
    _close(c, a.double().t() @ b.double(), "multi-tile product")
    _close(s, a.double().sum(0), "multi-tile colsum", 1e-6, 1e-6)
    _close(K.tall_tn(a, b), c, "tall_tn vs tall_tn_colsum product", 1e-7, 1e-7)
