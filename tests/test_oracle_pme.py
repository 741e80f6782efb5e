"""PME oracle pinned against the reference op's outputs and textbook electrostatics (CPU)."""

import math
import os

import numpy as np
import pytest

from oracle import nlist as NL
from oracle import pme as P

GOLD = os.path.join(os.path.dirname(__file__), "golden", "pme_golden.npz")
K_COUL = 14.399645


def _rel(a, b):
    return np.linalg.norm(np.asarray(a) - np.asarray(b)) / max(np.linalg.norm(b), 1e-300)


def run_case(g, c):
    if c.startswith("recip"):
        return P.reciprocal(g[c + "/positions"], g[c + "/charges"], g[c + "/box"], g[c + "/grid"],
                            int(g[c + "/order"]), float(g[c + "/alpha"]), float(g[c + "/coulomb"]),
                            (g[c + "/xmoduli"], g[c + "/ymoduli"], g[c + "/zmoduli"]))
    return P.direct(g[c + "/positions"], g[c + "/charges"], g[c + "/neighbors"], g[c + "/deltas"],
                    g[c + "/distances"], g[c + "/exclusions"], float(g[c + "/alpha"]), float(g[c + "/coulomb"]))


def test_oracle_matches_reference_fixtures():
    g = np.load(GOLD)
    for c in g["cases"]:
        e, dp, dq = run_case(g, c)
        tol = 1e-12 if g[c + "/positions"].dtype == np.float64 else 2e-6  # fp32 reference vs fp64 oracle
        assert abs(e - g[c + "/energy"]) <= tol * abs(g[c + "/energy"]), c
        assert _rel(dp, g[c + "/grad_positions"]) <= tol, c
        assert _rel(dq, g[c + "/grad_charges"]) <= tol, c


def nacl(ncell):
    a = 2.0  # conventional cubic cell, nearest-neighbour distance 1
    base = np.array([[0, 0, 0], [1, 1, 0], [1, 0, 1], [0, 1, 1]], float)
    pts, qs = [], []
    for i in range(ncell):
        for j in range(ncell):
            for k in range(ncell):
                o = np.array([i, j, k]) * a
                for b in base:
                    pts.append(o + b)
                    qs.append(1.0)
                    pts.append(o + b + np.array([1.0, 0, 0]))
                    qs.append(-1.0)
    return np.array(pts), np.array(qs), np.eye(3) * a * ncell


def ewald_total(pos, q, box, alpha, rc, grid, order):
    rows, cols, d, dist = NL.half_pairs(pos, rc, box)
    nb = np.stack([rows, cols])
    excl = -np.ones((len(q), 1), np.int32)
    e_dir, _, _ = P.direct(pos, q, nb, d, dist, excl, alpha, K_COUL)
    mods = [P.bspline_moduli(g_, order) for g_ in grid]
    e_rec, _, _ = P.reciprocal(pos, q, box, grid, order, alpha, K_COUL, mods)
    e_self = K_COUL * alpha / math.sqrt(math.pi) * np.sum(q * q)
    return e_dir + e_rec - e_self


def test_nacl_madelung_constant():
    pos, q, box = nacl(5)  # L = 10, 1000 ions
    e = ewald_total(pos, q, box, alpha=1.2, rc=4.0, grid=(48, 48, 48), order=6)
    madelung = -e / (len(q) / 2) / K_COUL
    assert abs(madelung - 1.747565) < 2e-5, madelung


def test_ewald_sum_independent_of_alpha():
    rng = np.random.default_rng(3)
    L = 12.0
    pos = rng.uniform(0, L, (60, 3))
    q = rng.normal(size=60)
    q -= q.mean()
    e1 = ewald_total(pos, q, np.eye(3) * L, 0.9, 5.9, (40, 40, 40), 6)
    e2 = ewald_total(pos, q, np.eye(3) * L, 1.2, 5.9, (48, 48, 48), 6)
    assert abs(e1 - e2) <= 1e-5 * abs(e1)


@pytest.mark.parametrize("order", [4, 5, 6])
def test_reciprocal_gradients_finite_differences(order):
    rng = np.random.default_rng(order)
    box = np.array([[9.0, 0, 0], [1.0, 8.5, 0], [-0.5, 0.7, 9.2]])
    pos = rng.uniform(0, 1, (12, 3)) @ box
    q = rng.normal(size=12)
    grid = (16, 18, 20)
    mods = [P.bspline_moduli(g_, order) for g_ in grid]
    e, dp, dq = P.reciprocal(pos, q, box, grid, order, 0.4, K_COUL, mods)
    h = 1e-6
    for atom, k in [(0, 0), (3, 1), (7, 2)]:
        p1, p2 = pos.copy(), pos.copy()
        p1[atom, k] += h
        p2[atom, k] -= h
        fd = (P.reciprocal(p1, q, box, grid, order, 0.4, K_COUL, mods)[0]
              - P.reciprocal(p2, q, box, grid, order, 0.4, K_COUL, mods)[0]) / (2 * h)
        assert abs(fd - dp[atom, k]) < 1e-5 * max(1.0, abs(fd))
    q1 = q.copy()
    q1[5] += h
    q2 = q.copy()
    q2[5] -= h
    fd = (P.reciprocal(pos, q1, box, grid, order, 0.4, K_COUL, mods)[0]
          - P.reciprocal(pos, q2, box, grid, order, 0.4, K_COUL, mods)[0]) / (2 * h)
    assert abs(fd - dq[5]) < 1e-5 * max(1.0, abs(fd))


def test_bspline_moduli_known_values():
    # order 4 cardinal B-spline at knots 1, 2, 3: 1/6, 2/3, 1/6 -> modulus at m = 0 is 1
    m = P.bspline_moduli(16, 4)
    assert abs(m[0] - 1.0) < 1e-14
    # m = K/2: |1/6 - 2/3 + 1/6|^2 = 1/9
    assert abs(m[8] - 1.0 / 9.0) < 1e-14
