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


def _run_case(ops, g, c, dtype):
    pos = torch.tensor(g[c + "/positions"], dtype=dtype, device=DEV, requires_grad=True)
    q = torch.tensor(g[c + "/charges"], dtype=dtype, device=DEV, requires_grad=True)
    f = lambda k: torch.tensor(g[c + "/" + k], dtype=dtype, device=DEV)  # noqa: E731
    if c.startswith("recip"):
        grid = [int(v) for v in g[c + "/grid"]]
        e = ops.pme_reciprocal(pos, q, f("box"), *grid, int(g[c + "/order"]), float(g[c + "/alpha"]),
                               float(g[c + "/coulomb"]), f("xmoduli"), f("ymoduli"), f("zmoduli"))
    else:
        e = ops.pme_direct(pos, q, _t(g[c + "/neighbors"]), f("deltas"), f("distances"), _t(g[c + "/exclusions"]),
                           float(g[c + "/alpha"]), float(g[c + "/coulomb"]))
    gp, gq = torch.autograd.grad(e, (pos, q))
    return float(e.detach()), gp.cpu().numpy(), gq.cpu().numpy()


def _oracle_case(g, c):
    """The fp64 oracle (pinned to the fp64 fixtures at 1e-10 in tests/test_oracle_pme.py) on the
    case's inputs as stored."""
    a = lambda k: np.asarray(g[c + "/" + k], np.float64)  # noqa: E731
    if c.startswith("recip"):
        return P.reciprocal(a("positions"), a("charges"), a("box"), [int(v) for v in g[c + "/grid"]],
                            int(g[c + "/order"]), float(g[c + "/alpha"]), float(g[c + "/coulomb"]),
                            [a("xmoduli"), a("ymoduli"), a("zmoduli")])
    return P.direct(a("positions"), a("charges"), g[c + "/neighbors"], a("deltas"), a("distances"),
                    g[c + "/exclusions"], float(g[c + "/alpha"]), float(g[c + "/coulomb"]))


def test_pme_against_reference_fixtures(ops):
    """fp64 cases: the reference op's own fp64 outputs at 1e-10.  Every case again in fp32 (inputs
    rounded to fp32) against fp64 at 1e-5: the fp64 cases against the reference's fp64 outputs, the
    fp32 cases against the fp64 oracle on their inputs (the stored fp32 outputs are the
    reference's own fp32 evaluation and carry its rounding)."""
    g = np.load(GOLD)
    for c in g["cases"]:
        f64 = g[c + "/positions"].dtype == np.float64
        if f64:
            e, gp, gq = _run_case(ops, g, c, torch.float64)
            ref_e = float(g[c + "/energy"])
            assert abs(e - ref_e) <= 1e-10 * abs(ref_e), (c, e, ref_e)
            assert _rel(gp, g[c + "/grad_positions"]) <= 1e-10, c
            assert _rel(gq, g[c + "/grad_charges"]) <= 1e-10, c
            ref = (ref_e, g[c + "/grad_positions"], g[c + "/grad_charges"])
        else:
            ref = _oracle_case(g, c)
        e, gp, gq = _run_case(ops, g, c, torch.float32)
        errs = (abs(e - ref[0]) / abs(ref[0]), _rel(gp, ref[1]), _rel(gq, ref[2]))
        print(f"{c}: fp32 vs fp64 rel err energy {errs[0]:.2e}, d/dpos {errs[1]:.2e}, d/dq {errs[2]:.2e}")
        assert max(errs) <= 1e-5, (c, errs)


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


def _recip_gpu(ops, pos, q, box, grid, order, alpha, k, dtype):
    mods = [torch.tensor(P.bspline_moduli(g_, order), dtype=dtype, device=DEV) for g_ in grid]
    pt = torch.tensor(pos, dtype=dtype, device=DEV, requires_grad=True)
    qt = torch.tensor(q, dtype=dtype, device=DEV, requires_grad=True)
    e = ops.pme_reciprocal(pt, qt, torch.tensor(box, dtype=dtype, device=DEV), *grid, order, alpha, k, *mods)
    gp, gq = torch.autograd.grad(e, (pt, qt))
    return float(e), gp.cpu().numpy(), gq.cpu().numpy()


@pytest.mark.parametrize("grid,order", [((5, 6, 7), 4), ((8, 8, 8), 8), ((9, 17, 24), 6), ((15, 16, 33), 5),
                                        ((7, 30, 12), 3)])
def test_reciprocal_mesh_shapes(ops, grid, order):
    """Meshes smaller than one 8^3 brick, exact multiples, and partial last bricks (1..7 points),
    in a triclinic cell, fp64 against the oracle."""
    rng = np.random.default_rng(sum(grid) * 10 + order)
    n = 300
    box = np.array([[9.0, 0.0, 0.0], [1.5, 10.0, 0.0], [-2.0, 1.0, 11.0]])
    frac = rng.uniform(-0.2, 1.2, (n, 3))  # also outside the cell: wrapped by the kernels
    pos = frac @ box
    q = rng.normal(size=n)
    q -= q.mean()
    alpha, k = 0.35, 138.935
    e, gp, gq = _recip_gpu(ops, pos, q, box, grid, order, alpha, k, torch.float64)
    mods = [P.bspline_moduli(g_, order) for g_ in grid]
    re, rp, rq = P.reciprocal(pos, q, box, grid, order, alpha, k, mods)
    assert abs(e - re) <= 1e-10 * abs(re), (e, re)
    assert _rel(gp, rp) <= 1e-10
    assert _rel(gq, rq) <= 1e-10


def test_reciprocal_bitwise_reproducible(ops):
    """The spread sums each mesh point in a fixed order: repeated runs agree bit for bit."""
    rng = np.random.default_rng(11)
    n, L = 4000, 35.0
    pos = rng.uniform(0, L, (n, 3))
    q = rng.normal(size=n)
    q -= q.mean()
    box = np.eye(3) * L
    runs = [_recip_gpu(ops, pos, q, box, (40, 40, 40), 6, 0.3, 14.399645, torch.float32) for _ in range(3)]
    for e, gp, gq in runs[1:]:
        assert e == runs[0][0]
        assert np.array_equal(gp, runs[0][1]) and np.array_equal(gq, runs[0][2])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_reciprocal_spectrum_variant(ops, dtype):
    """molix::pme_reciprocal_spectrum (the module's op: the backward reuses the forward's convolved
    spectrum) gives the energy and both gradients of molix::pme_reciprocal (which recomputes it)
    bit for bit, in a triclinic cell with a ragged mesh; its spectrum output is the half spectrum
    and carries no gradient."""
    rng = np.random.default_rng(5)
    n, grid, order = 500, (12, 20, 15), 6
    box = np.array([[14.0, 0.0, 0.0], [2.0, 13.0, 0.0], [-1.0, 1.5, 15.0]])
    pos = rng.uniform(-0.1, 1.1, (n, 3)) @ box
    q = rng.normal(size=n)
    q -= q.mean()
    mods = [torch.tensor(P.bspline_moduli(g_, order), dtype=dtype, device=DEV) for g_ in grid]
    b = torch.tensor(box, dtype=dtype, device=DEV)
    res = []
    for op in (ops.pme_reciprocal, ops.pme_reciprocal_spectrum):
        pt = torch.tensor(pos, dtype=dtype, device=DEV, requires_grad=True)
        qt = torch.tensor(q, dtype=dtype, device=DEV, requires_grad=True)
        out = op(pt, qt, b, *grid, order, 0.3, 14.399645, *mods)
        e = out if op is ops.pme_reciprocal else out[0]
        if op is ops.pme_reciprocal_spectrum:
            assert out[1].shape == (grid[0], grid[1], grid[2] // 2 + 1) and out[1].is_complex()
            assert not out[1].requires_grad
        gp, gq = torch.autograd.grad(2.5 * e, (pt, qt))
        res.append((e.item(), gp.cpu().numpy(), gq.cpu().numpy()))
    assert res[0][0] == res[1][0]
    assert np.array_equal(res[0][1], res[1][1]) and np.array_equal(res[0][2], res[1][2])
    re, rp, rq = P.reciprocal(pos, q, box, grid, order, 0.3, 14.399645,
                              [P.bspline_moduli(g_, order) for g_ in grid])
    tol = 1e-10 if dtype == torch.float64 else 1e-5
    assert abs(res[1][0] - re) <= tol * abs(re) and _rel(res[1][1], 2.5 * rp) <= tol


def test_direct_against_oracle_with_exclusions_and_padding(ops):
    """Pair list in neighbor-list row order with -1 padding and exclusions; energy (energy-only
    forward) and both derivatives (backward) against the fp64 oracle, fp32 and fp64."""
    rng = np.random.default_rng(3)
    n, L, rc = 900, 22.0, 6.0
    pos = rng.uniform(0, L, (n, 3))
    q = rng.normal(size=n)
    q -= q.mean()
    pt = torch.tensor(pos, device=DEV)
    nb, d, dist, npairs = ops.get_neighbor_pairs(pt, rc, -1, torch.tensor(np.eye(3) * L, device=DEV))
    nb, d, dist = nb.cpu().numpy(), d.cpu().numpy(), dist.cpu().numpy()
    # symmetric exclusions from a random subset of listed pairs, descending, -1 padded
    listed = np.flatnonzero(nb[0] >= 0)
    sets = [set() for _ in range(n)]
    for s in rng.choice(listed, size=600, replace=False):
        a, b = int(nb[0][s]), int(nb[1][s])
        if len(sets[a]) < 4 and len(sets[b]) < 4:
            sets[a].add(b)
            sets[b].add(a)
    excl = -np.ones((n, 4), np.int32)
    for i, s in enumerate(sets):
        excl[i, :len(s)] = sorted(s, reverse=True)
    alpha, k = 0.3, 14.399645
    re, rp, rq = P.direct(pos, q, nb, d, dist, excl, alpha, k)
    for dtype, tol in ((torch.float64, 1e-10), (torch.float32, 1e-5)):
        p_ = torch.tensor(pos, dtype=dtype, device=DEV, requires_grad=True)
        q_ = torch.tensor(q, dtype=dtype, device=DEV, requires_grad=True)
        e = ops.pme_direct(p_, q_, torch.tensor(nb, device=DEV), torch.tensor(d, dtype=dtype, device=DEV),
                           torch.tensor(dist, dtype=dtype, device=DEV), torch.tensor(excl, device=DEV), alpha, k)
        gp, gq = torch.autograd.grad(e, (p_, q_))
        print(f"{dtype}: rel err energy {abs(float(e) - re) / abs(re):.2e}, d/dpos {_rel(gp.cpu().numpy(), rp):.2e}, "
              f"d/dq {_rel(gq.cpu().numpy(), rq):.2e}")
        assert abs(float(e) - re) <= tol * abs(re), (dtype, float(e), re)
        assert _rel(gp.cpu().numpy(), rp) <= tol, dtype
        assert _rel(gq.cpu().numpy(), rq) <= tol, dtype
