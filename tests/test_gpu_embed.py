"""The radial edge embedding on the HIP path (molix::bessel_cutoff: the Bessel basis times the
cutoff envelope, src/molrep/embedding/radial.py:36-148, cutoff.py:23-161, mace.py:180-182) against
the fp64 oracle (oracle.mace_ref.radial_features, whose polynomial envelope is the reference's
expanded form while the kernel evaluates the factored one): values, dL/dr against fp64 autograd,
the second derivative (force-matching training) against fp64 double backward, and the module
path against the torch composition of the modules."""

import math

import pytest
import torch

from oracle import mace_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _stats(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    rms = b.pow(2).mean().sqrt()
    return float((a - b).norm() / b.norm()), float((a - b).abs().max() / rms)


def _distances(n=20_000, rc=5.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = torch.rand(n, generator=g, dtype=torch.float64) * (rc * 1.1)
    r[:4] = torch.tensor([1e-3, rc, rc * (1 - 1e-6), rc * 1.05], dtype=torch.float64)
    return r


@pytest.mark.parametrize("cutoff,p,nb,normalize", [("cosine", 6, 8, True), ("polynomial", 6, 8, True),
                                                   ("polynomial", 5, 16, False), ("none", 6, 8, True),
                                                   ("cosine", 6, 32, False)])
def test_bessel_cutoff_vs_fp64(cutoff, p, nb, normalize):
    import molnex_amd.kernels as K

    rc = 5.0
    r64 = _distances(rc=rc).requires_grad_(True)
    ref = mace_ref.radial_features(r64, rc, nb, cutoff, p=p, normalize=normalize)
    g = torch.randn(ref.shape, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    (rg,) = torch.autograd.grad(ref, r64, g)
    mu, sig = mace_ref.bessel_stats(rc, nb) if normalize else (None, None)
    cu = lambda t: None if t is None else t.float().to(DEV)  # noqa: E731
    r = r64.detach().float().to(DEV).requires_grad_(True)
    out = torch.ops.molix.bessel_cutoff(r, nb, rc, 1e-8, cu(mu), cu(sig), K.CUTOFF_KINDS[cutoff], p)
    (gr,) = torch.autograd.grad(out, r, g.float().to(DEV))
    for name, a, b in (("values", out, ref), ("dL/dr", gr, rg)):
        rel, mx = _stats(a, b)
        print(f"{cutoff} p={p} n={nb}: {name} rel {rel:.2e}, max-abs {mx:.2e} RMS")
        assert rel <= 1e-5 and mx <= 1e-5, name
    assert torch.equal(out[3].cpu(), torch.zeros(nb)) or cutoff == "none"  # beyond the cutoff


@pytest.mark.parametrize("cutoff", ["cosine", "polynomial"])
def test_bessel_cutoff_second_order_vs_fp64(cutoff):
    """d/dr and d/dg of <s, dL/dr> (the backward op's autograd, used by force-matching training)
    against fp64 double backward of the oracle."""
    import molnex_amd.kernels as K
    import molnex_amd.second_order  # noqa: F401  (registers the formulas)

    rc, nb = 5.0, 8
    r64 = _distances(5000, rc, seed=3).clamp(min=0.05).requires_grad_(True)
    gen = torch.Generator().manual_seed(4)
    g64 = torch.randn(5000, nb, dtype=torch.float64, generator=gen).requires_grad_(True)
    s64 = torch.randn(5000, dtype=torch.float64, generator=gen)
    ref = mace_ref.radial_features(r64, rc, nb, cutoff)
    (d1,) = torch.autograd.grad(ref, r64, g64, create_graph=True)
    rr, rgg = torch.autograd.grad(d1, (r64, g64), s64)
    mu, sig = (t.float().to(DEV) for t in mace_ref.bessel_stats(rc, nb))
    r = r64.detach().float().to(DEV).requires_grad_(True)
    g = g64.detach().float().to(DEV).requires_grad_(True)
    d = K.bessel_cutoff_backward(g, r, nb, rc, 1e-8, mu, sig, K.CUTOFF_KINDS[cutoff], 6)
    dr, dg = torch.autograd.grad(d, (r, g), s64.float().to(DEV))
    for name, a, b in (("d/dr", dr, rr), ("d/dg", dg, rgg)):
        rel, mx = _stats(a, b)
        print(f"{cutoff}: second order {name} rel {rel:.2e}, max-abs {mx:.2e} RMS")
        assert rel <= 1e-5 and mx <= 1e-5, name


def test_module_path_matches_torch_composition():
    """Values against the modules' torch composition; dL/dr against the fp64 oracle (torch's fp32
    autograd of sin(f r) / (r + eps) cancels for small r, which the kernel's backward avoids)."""
    from molnex_amd.molrep.embedding import BesselRBF, CosineCutoff, PolynomialCutoff, radial_edge_features

    r64 = _distances(30_000, 5.0, seed=7)
    r = r64.float().to(DEV).requires_grad_(True)
    for kind, cut in (("cosine", CosineCutoff(r_cut=5.0)), ("polynomial", PolynomialCutoff(r_cut=5.0, exponent=6))):
        rbf = BesselRBF(r_cut=5.0, num_radial=8).to(DEV)
        cut = cut.to(DEV)
        a = radial_edge_features(rbf, cut, r)
        b = rbf(r) * cut(r).unsqueeze(-1)
        assert _stats(a, b)[1] <= 1e-5
        ga = torch.autograd.grad(a.sum(), r)[0]
        rr = r64.clone().requires_grad_(True)
        ref = torch.autograd.grad(mace_ref.radial_features(rr, 5.0, 8, kind).sum(), rr)[0]
        rel, mx = _stats(ga, ref)
        assert rel <= 1e-5 and mx <= 1e-5, (kind, rel, mx)
    # a cutoff radius other than the basis' goes through the torch composition
    rbf = BesselRBF(r_cut=5.0, num_radial=8).to(DEV)
    c4 = CosineCutoff(r_cut=4.0).to(DEV)
    assert torch.equal(radial_edge_features(rbf, c4, r.detach()), rbf(r.detach()) * c4(r.detach()).unsqueeze(-1))
    assert math.isclose(float(rbf.r_cut), 5.0)
