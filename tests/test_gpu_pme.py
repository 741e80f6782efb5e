"""GPU PME ops (reference schemas) vs the reference op's outputs and the fp64 oracle."""

import math
import os

import numpy as np
import pytest
import torch

from oracle import pme as P

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden", "pme_golden.npz")
DEV = "cuda"


def _rel(a, b):
    return np.linalg.norm(np.asarray(a, np.float64) - np.asarray(b, np.float64)) / max(np.linalg.norm(b), 1e-300)


@pytest.fixture(scope="module")
def ops():
    import molnex_amd.kernels  # noqa: F401

    return torch.ops.molix


def _t(a, grad=False):
    return torch.tensor(a, device=DEV, requires_grad=grad)


def test_pme_against_reference_fixtures(ops):
    g = np.load(GOLD)
    for c in g["cases"]:
        pos = _t(g[c + "/positions"], True)
        q = _t(g[c + "/charges"], True)
        if c.startswith("recip"):
            grid = [int(v) for v in g[c + "/grid"]]
            e = ops.pme_reciprocal(pos, q, _t(g[c + "/box"]), *grid, int(g[c + "/order"]), float(g[c + "/alpha"]),
                                   float(g[c + "/coulomb"]), _t(g[c + "/xmoduli"]), _t(g[c + "/ymoduli"]),
                                   _t(g[c + "/zmoduli"]))
        else:
            e = ops.pme_direct(pos, q, _t(g[c + "/neighbors"]), _t(g[c + "/deltas"]), _t(g[c + "/distances"]),
                               _t(g[c + "/exclusions"]), float(g[c + "/alpha"]), float(g[c + "/coulomb"]))
        gp, gq = torch.autograd.grad(e, (pos, q))
        tol = 1e-10 if pos.dtype == torch.float64 else 2e-5
        ref_e = float(g[c + "/energy"])
        assert abs(float(e) - ref_e) <= tol * abs(ref_e), (c, float(e), ref_e)
        assert _rel(gp.cpu().numpy(), g[c + "/grad_positions"]) <= tol, c
        assert _rel(gq.cpu().numpy(), g[c + "/grad_charges"]) <= tol, c


def test_config5_pme_scale(ops):
    """BASELINE config 5 PME term: 50k atoms, 128^3 mesh, order 6, alpha 0.3, fp32 vs fp64 oracle."""
    rng = np.random.default_rng(5)
    n = 50_000
    L = (n / 0.1) ** (1 / 3)
    pos = rng.uniform(0, L, (n, 3))
    q = rng.normal(size=n) * 0.3
    q -= q.mean()
    box = np.eye(3) * L
    grid, order, alpha, k = (128, 128, 128), 6, 0.3, 14.399645
    mods = [P.bspline_moduli(g_, order) for g_ in grid]
    pt = torch.tensor(pos, dtype=torch.float32, device=DEV, requires_grad=True)
    qt = torch.tensor(q, dtype=torch.float32, device=DEV, requires_grad=True)
    e = ops.pme_reciprocal(pt, qt, torch.tensor(box, dtype=torch.float32, device=DEV), *grid, order, alpha, k,
                           *[torch.tensor(m, dtype=torch.float32, device=DEV) for m in mods])
    gp, gq = torch.autograd.grad(e, (pt, qt))
    # oracle on the fp32-rounded inputs
    p32 = pos.astype(np.float32).astype(np.float64)
    q32 = q.astype(np.float32).astype(np.float64)
    re, rp, rq = P.reciprocal(p32, q32, box.astype(np.float32).astype(np.float64), grid, order, alpha, k,
                              [m.astype(np.float32).astype(np.float64) for m in mods])
    assert abs(float(e) - re) <= 1e-5 * abs(re), (float(e), re)
    assert _rel(gp.cpu().numpy(), rp) <= 1e-5
    assert _rel(gq.cpu().numpy(), rq) <= 1e-5


def test_nacl_madelung_on_gpu(ops):
    from tests.test_oracle_pme import nacl

    pos, q, box = nacl(5)
    alpha, rc, grid, order, k = 1.2, 4.0, (48, 48, 48), 6, 14.399645
    pt = torch.tensor(pos, device=DEV)
    qt = torch.tensor(q, device=DEV)
    bt = torch.tensor(box, device=DEV)
    nb, d, dist, npairs = ops.get_neighbor_pairs(pt, rc, -1, bt)
    keep = nb[0] >= 0
    e_dir = ops.pme_direct(pt, qt, nb[:, keep].contiguous(), d[keep].contiguous(), dist[keep].contiguous(),
                           torch.full((len(q), 1), -1, dtype=torch.int32, device=DEV), alpha, k)
    mods = [torch.tensor(P.bspline_moduli(g_, order), device=DEV) for g_ in grid]
    e_rec = ops.pme_reciprocal(pt, qt, bt, *grid, order, alpha, k, *mods)
    e = float(e_dir) + float(e_rec) - k * alpha / math.sqrt(math.pi) * float(np.sum(q * q))
    madelung = -e / (len(q) / 2) / k
    assert abs(madelung - 1.747565) < 2e-5, madelung
