"""The oracle is pinned before it is trusted (CPU only).

* neighbor list: bit-exact against the reference op's own outputs
  (tests/golden/nlist_golden.npz, written by make_nlist_golden.py from the
  reference sources compiled by oracle/Makefile); brute force == cell list.
* harmonics: closed forms, orthonormality by quadrature, rotation equivariance.
* coupling tables: invariance, orthonormality, and agreement of two independent
  constructions (oracle null space vs product Gaunt integral).
* tensor product: gradients vs finite differences, rotation equivariance,
  linearity in w, invariance under edge permutation; a planted mistake fails.
"""

import itertools
import math
import os

import numpy as np
import pytest

from oracle import equivariant as O
from oracle import nlist as NL

GOLD = os.path.join(os.path.dirname(__file__), "golden", "nlist_golden.npz")


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def test_nlist_oracle_matches_reference_fixtures(gold):
    for c in gold["cases"]:
        box = gold[c + "/box"]
        nb, dd, ds, npairs = NL.get_neighbor_pairs(gold[c + "/positions"], float(gold[c + "/cutoff"]),
                                                   int(gold[c + "/max_num_pairs"]), box if box.size else None)
        assert np.array_equal(nb, gold[c + "/neighbors"]), c
        assert np.array_equal(_bits(dd), _bits(gold[c + "/deltas"])), c
        assert np.array_equal(_bits(ds), _bits(gold[c + "/distances"])), c
        assert np.array_equal(npairs, gold[c + "/num_pairs"]), c


def test_nlist_cells_equal_brute_force(gold):
    for c in gold["cases"]:
        box = gold[c + "/box"]
        b = box if box.size else None
        a = NL.half_pairs(gold[c + "/positions"], float(gold[c + "/cutoff"]), b, cells=False)
        z = NL.half_pairs(gold[c + "/positions"], float(gold[c + "/cutoff"]), b, cells=True)
        for u, v in zip(a, z):
            assert np.array_equal(_bits(u), _bits(v)), c


def test_nlist_oracle_planted_norm_mistake_fails(gold):
    # the plain (non-fma) norm differs from the reference on some pairs: the
    # fixture distinguishes the two roundings
    c = "cubic_f32_n1500"
    d = gold[c + "/deltas"]
    valid = ~np.isnan(gold[c + "/distances"])
    x, y, z = d[valid].T
    plain = np.sqrt((x * x + y * y) + z * z).astype(np.float32)
    assert not np.array_equal(_bits(plain), _bits(gold[c + "/distances"][valid]))


def test_nlist_directed_properties():
    rng = np.random.default_rng(3)
    L = 20.0
    pos = rng.uniform(0, L, (800, 3)).astype(np.float32)
    i, j, d, dist = NL.directed_pairs(pos, 5.0, np.eye(3, dtype=np.float32) * L)
    assert np.all(i != j)
    key = i.astype(np.int64) * 800 + j
    assert np.all(np.diff(key) > 0)  # sorted, unique
    rev = {(a, b): k for k, (a, b) in enumerate(zip(i, j))}
    k2 = np.array([rev[(b, a)] for a, b in zip(i, j)])
    assert np.array_equal(_bits(d[k2]), _bits(-d))
    # expected density: 4/3 pi r^3 rho per atom
    assert abs(len(i) / 800 - 4 / 3 * math.pi * 125 * 0.1) < 3


def _quadrature(n=12, nphi=30):
    t, wt = np.polynomial.legendre.leggauss(n)
    phi = 2 * np.pi * np.arange(nphi) / nphi
    st = np.sqrt(1 - t * t)
    pts = np.stack([(st[:, None] * np.cos(phi)).ravel(), (st[:, None] * np.sin(phi)).ravel(), np.repeat(t, nphi)], -1)
    return pts, np.repeat(wt, nphi) * 2 * np.pi / nphi


def test_sh_closed_forms_and_orthonormality():
    rng = np.random.default_rng(0)
    u = rng.normal(size=(20, 3))
    un = u / np.linalg.norm(u, axis=1, keepdims=True)
    np.testing.assert_allclose(O.real_sh(0, u), 1.0)
    np.testing.assert_allclose(O.real_sh(1, u), math.sqrt(3) * un, atol=1e-14)
    np.testing.assert_allclose(O.real_sh(2, u)[:, 0], math.sqrt(15) * un[:, 0] * un[:, 1], atol=1e-13)
    pts, w = _quadrature()
    for l in range(4):
        Y = O.real_sh(l, pts)
        gram = np.einsum("q,qa,qb->ab", w, Y, Y) / (4 * np.pi)
        np.testing.assert_allclose(gram, np.eye(2 * l + 1), atol=1e-12)
        np.testing.assert_allclose((Y * Y).sum(1), 2 * l + 1, atol=1e-12)
    assert np.all(O.real_sh(2, np.zeros((1, 3))) == 0)


def test_sh_equivariance():
    rng = np.random.default_rng(1)
    v = rng.normal(size=(30, 3))
    for _ in range(3):
        R = O.random_rotation(rng)
        for l in range(4):
            D = O.wigner_d(l, R)
            np.testing.assert_allclose(O.real_sh(l, v @ R.T), O.real_sh(l, v) @ D.T, atol=1e-12)
            np.testing.assert_allclose(D @ D.T, np.eye(2 * l + 1), atol=1e-12)
    np.testing.assert_allclose(O.wigner_d(1, R), R, atol=1e-12)


def test_coupling_tables_two_constructions_agree():
    from molnex_amd import irreps as P

    rng = np.random.default_rng(2)
    R = O.random_rotation(rng)
    for l1, l2, l3 in itertools.product(range(4), repeat=3):
        if not (abs(l1 - l2) <= l3 <= l1 + l2) or (l1 + l2 + l3) % 2:
            continue
        c = O.coupling(l1, l2, l3)
        np.testing.assert_allclose(c, P.coupling(l1, l2, l3), atol=1e-12)
        rot = np.einsum("ad,be,cf,def->abc", O.wigner_d(l1, R), O.wigner_d(l2, R), O.wigner_d(l3, R), c)
        np.testing.assert_allclose(rot, c, atol=1e-10)
        # isotropy: sum over (m1, m2) of c^2 is 1/(2 l3 + 1) for every m3
        np.testing.assert_allclose((c ** 2).sum((0, 1)), 1 / (2 * l3 + 1), atol=1e-12)
    # special case that reduces to a textbook form: (1, 1, 0) is delta_ab / sqrt(3)
    np.testing.assert_allclose(O.coupling(1, 1, 0)[:, :, 0], np.eye(3) / math.sqrt(3), atol=1e-12)


def _tp_case(rng, C=3, N=6, E=15, irr="0e+1o+2e+3o"):
    tp = O.ChannelwiseTP("+".join(f"{C}x{t}" for t in irr.split("+")), irr, irr, C)
    x = rng.normal(size=(N, tp.nx * C))
    Y = rng.normal(size=(E, tp.ny))
    w = rng.normal(size=(E, len(tp.paths) * C))
    ei = rng.integers(0, N, (E, 2))
    return tp, x, Y, w, ei, N


def test_tp_path_count_and_sizes():
    tp = O.ChannelwiseTP("128x0e+128x1o+128x2e+128x3o", "0e+1o+2e+3o", "0e+1o+2e+3o", 128)
    assert len(tp.paths) == 23 and tp.no == 99 and tp.nx == 16


def test_tp_gradients_finite_differences():
    rng = np.random.default_rng(4)
    tp, x, Y, w, ei, N = _tp_case(rng)
    g = rng.normal(size=(N, tp.no * tp.C))
    gx, gY, gw = tp.backward(x, Y, w, ei, g)
    f = lambda x_, Y_, w_: (tp.forward(x_, Y_, w_, ei, N) * g).sum()  # noqa: E731
    h = 1e-6
    for k, (arr, gr) in enumerate([(x, gx), (Y, gY), (w, gw)]):
        for _ in range(8):
            idx = tuple(rng.integers(0, s) for s in arr.shape)
            a, b = arr.copy(), arr.copy()
            a[idx] += h
            b[idx] -= h
            args_p = [x, Y, w]
            args_m = [x, Y, w]
            args_p[k], args_m[k] = a, b
            fd = (f(*args_p) - f(*args_m)) / (2 * h)
            assert abs(fd - gr[idx]) < 1e-6 * max(1, abs(fd))


def test_tp_rotation_equivariance_and_linearity():
    rng = np.random.default_rng(5)
    C, N, E = 4, 5, 20
    irr = "0e+1o+2e+3o"
    xirr = "+".join(f"{C}x{t}" for t in irr.split("+"))
    tp = O.ChannelwiseTP(xirr, irr, irr, C)
    vec = rng.normal(size=(E, 3))
    Y = O.sh(range(4), vec)
    x = rng.normal(size=(N, tp.nx * C))
    w = rng.normal(size=(E, len(tp.paths) * C))
    ei = rng.integers(0, N, (E, 2))
    out = tp.forward(x, Y, w, ei, N)
    R = O.random_rotation(rng)
    out_r = tp.forward(O.rotate_irreps(x, R, xirr, C), O.sh(range(4), vec @ R.T), w, ei, N)
    out_irr = " + ".join(f"{C}x{p[4]}{'e' if p[4] % 2 == 0 else 'o'}" for p in [tp.paths[k] for k in sorted(tp.out_pos, key=tp.out_pos.get)])
    np.testing.assert_allclose(out_r, O.rotate_irreps(out, R, out_irr, C), atol=1e-10)
    np.testing.assert_allclose(tp.forward(x, Y, 2.5 * w, ei, N), 2.5 * out, atol=1e-10)
    perm = rng.permutation(E)
    np.testing.assert_allclose(tp.forward(x, Y[perm], w[perm], ei[perm], N), out, atol=1e-10)


def test_tp_planted_mistakes_are_caught():
    rng = np.random.default_rng(6)
    C, N, E = 2, 4, 10
    irr = "0e+1o+2e+3o"
    xirr = "+".join(f"{C}x{t}" for t in irr.split("+"))
    tp = O.ChannelwiseTP(xirr, irr, irr, C)
    vec = rng.normal(size=(E, 3))
    x = rng.normal(size=(N, tp.nx * C))
    w = rng.normal(size=(E, len(tp.paths) * C))
    ei = rng.integers(0, N, (E, 2))
    R = O.random_rotation(rng)
    out_irr = " + ".join(f"{C}x{tp.paths[k][4]}{'e' if tp.paths[k][4] % 2 == 0 else 'o'}"
                         for k in sorted(tp.out_pos, key=tp.out_pos.get))

    def equivariant(f):
        out = f(x, O.sh(range(4), vec))
        out_r = f(O.rotate_irreps(x, R, xirr, C), O.sh(range(4), vec @ R.T))
        return np.allclose(out_r, O.rotate_irreps(out, R, out_irr, C), atol=1e-8)

    assert equivariant(lambda x_, Y_: tp.forward(x_, Y_, w, ei, N))
    # 1. a sign flipped on one path keeps equivariance, but the two independent
    #    table constructions then disagree
    from molnex_amd import irreps as P
    assert not np.allclose(-O.coupling(2, 1, 3), P.coupling(2, 1, 3))
    # 2. reading x in mul_ir instead of ir_mul order (a transposed operand) breaks equivariance
    misread = lambda x_: x_.reshape(N, C, tp.nx).transpose(0, 2, 1).reshape(N, -1)  # noqa: E731
    assert not equivariant(lambda x_, Y_: tp.forward(misread(x_), Y_, w, ei, N))
    # 3. a wrong l=1 harmonic order (e3nn's y, z, x) breaks equivariance
    yzx = lambda Y_: np.concatenate([Y_[:, :1], Y_[:, [2, 3, 1]], Y_[:, 4:]], 1)  # noqa: E731
    assert not equivariant(lambda x_, Y_: tp.forward(x_, yzx(Y_), w, ei, N))
