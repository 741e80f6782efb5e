"""GPU neighbor list vs the reference op's outputs and the C oracle (bit-exact)."""

import math
import os
import warnings

import numpy as np
import pytest
import torch

from oracle import nlist as NL

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden", "nlist_golden.npz")
DEV = "cuda"


def _bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


@pytest.fixture(scope="module")
def ops():
    import molnex_amd.kernels  # noqa: F401  registers torch.ops.molix.*

    return torch.ops.molix


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def test_get_neighbor_pairs_matches_reference_fixtures(ops, gold):
    for c in gold["cases"]:
        pos = torch.from_numpy(gold[c + "/positions"]).to(DEV)
        box = torch.from_numpy(gold[c + "/box"]).to(DEV)
        cut, mnp = float(gold[c + "/cutoff"]), int(gold[c + "/max_num_pairs"])
        with warnings.catch_warnings(record=True) as rec:
            warnings.simplefilter("always")
            nb, d, dist, npairs = ops.get_neighbor_pairs(pos, cut, mnp, box)
        ref_nb, ref_d, ref_dist = gold[c + "/neighbors"], gold[c + "/deltas"], gold[c + "/distances"]
        assert int(npairs.item()) == int(gold[c + "/num_pairs"][0]), c
        # more pairs than max_num_pairs: a RuntimeWarning says the outputs are cut to the width
        over = mnp != -1 and int(gold[c + "/num_pairs"][0]) > mnp
        assert any(issubclass(r.category, RuntimeWarning) for r in rec) == over, c
        w = nb.shape[1]
        # the reference CPU path widens past max_num_pairs on overflow; this op
        # keeps the schema width (like the CUDA/meta paths) with the first pairs
        assert w == (mnp if mnp != -1 else pos.shape[0] * (pos.shape[0] - 1) // 2), c
        assert np.array_equal(nb.cpu().numpy(), ref_nb[:, :w]), c
        assert np.array_equal(_bits(d.cpu().numpy()), _bits(ref_d[:w])), c
        assert np.array_equal(_bits(dist.cpu().numpy()), _bits(ref_dist[:w])), c


def _directed_check(ops, pos_np, box_np, cut):
    pos = torch.from_numpy(pos_np).to(DEV)
    box = torch.from_numpy(box_np).to(DEV) if box_np is not None else torch.empty((0, 0), dtype=pos.dtype, device=DEV)
    i, j, sh, d, dist = ops.neighbor_list(pos, cut, box, True)
    ri, rj, rd, rdist = NL.directed_pairs(pos_np, cut, box_np)
    assert np.array_equal(i.cpu().numpy(), ri)
    assert np.array_equal(j.cpu().numpy(), rj)
    assert np.array_equal(_bits(d.cpu().numpy()), _bits(rd))
    assert np.array_equal(_bits(dist.cpu().numpy()), _bits(rdist))
    return i, j, sh, d, dist


def test_directed_list_matches_oracle(ops, gold):
    for c in ["cubic_f32", "cubic_f32_n1500", "tric_f32", "tric_f64", "open_f32_m512", "cubic_unwrapped_f32",
              "edge_pbc_f32", "smallbox_f32"]:
        box = gold[c + "/box"]
        _directed_check(ops, gold[c + "/positions"], box if box.size else None, float(gold[c + "/cutoff"]))


def test_half_list_exact_size(ops, gold):
    c = "tric_f32"
    pos = torch.from_numpy(gold[c + "/positions"]).to(DEV)
    box = torch.from_numpy(gold[c + "/box"]).to(DEV)
    i, j, sh, d, dist = ops.neighbor_list(pos, 5.0, box, False)
    n = int(gold[c + "/num_pairs"][0])
    assert i.shape[0] == n
    assert np.array_equal(i.cpu().numpy(), gold[c + "/neighbors"][0, :n])
    assert np.array_equal(j.cpu().numpy(), gold[c + "/neighbors"][1, :n])


def test_config2_100k_atoms(ops):
    """100k atoms, periodic cube L=100 (rho=0.1), rc=5, directed list."""
    rng = np.random.default_rng(2)
    L = 100.0
    pos_np = rng.uniform(0, L, (100_000, 3)).astype(np.float32)
    box_np = np.eye(3, dtype=np.float32) * L
    i, j, sh, d, dist = _directed_check(ops, pos_np, box_np, 5.0)
    E = i.shape[0]
    assert abs(E / 100_000 - 4 / 3 * math.pi * 125 * 0.1) < 0.5
    s = sh.cpu().numpy()
    assert np.all(np.isin(s, [-L, 0.0, L]))
    pi, pj = pos_np[i.cpu().numpy()], pos_np[j.cpu().numpy()]
    np.testing.assert_allclose(pi - (pj + s), d.cpu().numpy(), atol=2e-5)
    # deterministic
    i2, j2, _, d2, _ = ops.neighbor_list(torch.from_numpy(pos_np).to(DEV), 5.0, torch.from_numpy(box_np).to(DEV), True)
    assert torch.equal(i, i2) and torch.equal(j, j2) and torch.equal(d, d2)


def test_get_neighbor_pairs_backward(ops):
    rng = np.random.default_rng(5)
    pos_np = rng.uniform(0, 12.0, (300, 3))
    pos = torch.tensor(pos_np, dtype=torch.float64, device=DEV, requires_grad=True)
    box = torch.eye(3, dtype=torch.float64, device=DEV) * 12.0
    nb, d, dist, npairs = ops.get_neighbor_pairs(pos, 4.0, 8000, box)
    valid = nb[0] >= 0
    a = torch.randn_like(d)
    b = torch.randn_like(dist)
    loss = (d[valid] * a[valid]).sum() + (dist[valid] * b[valid]).sum()
    (g,) = torch.autograd.grad(loss, pos)
    # explicit reference: per pair contribution (a + d/r b) to row, minus to col
    nbn, dn, rn = nb.cpu().numpy(), d.detach().cpu().numpy(), dist.detach().cpu().numpy()
    an, bn = a.cpu().numpy(), b.cpu().numpy()
    v = nbn[0] >= 0
    contrib = an[v] + dn[v] / rn[v, None] * bn[v, None]
    ref = np.zeros((300, 3))
    np.add.at(ref, nbn[0, v], contrib)
    np.add.at(ref, nbn[1, v], -contrib)
    np.testing.assert_allclose(g.cpu().numpy(), ref, rtol=1e-10, atol=1e-10)


def test_too_many_neighbours_raises(ops):
    pos = torch.rand(4200, 3, device=DEV)  # all within 1.8 A of each other
    with pytest.raises(RuntimeError, match="4096"):
        ops.neighbor_list(pos, 5.0, torch.empty((0, 0), device=DEV), True)


def test_empty_and_single(ops):
    for n in (0, 1):
        pos = torch.zeros((n, 3), device=DEV)
        nb, d, dist, npairs = ops.get_neighbor_pairs(pos, 5.0, 4, torch.empty((0, 0), device=DEV))
        assert int(npairs.item()) == 0
        assert torch.all(nb == -1) and torch.all(torch.isnan(dist))


def test_dense_cluster_beyond_cell_emit_buffer(ops):
    """Atoms with more than 1024 neighbours on a cell grid (a dense cluster inside a periodic box):
    their pair segments come from the per-atom emit, the rest from the cell emit; bit-exact."""
    rng = np.random.default_rng(11)
    L = 30.0
    bg = rng.uniform(0, L, (8000, 3))
    u = rng.normal(size=(1300, 3))
    cluster = L / 2 + 2.0 * u / np.linalg.norm(u, axis=1, keepdims=True) * rng.uniform(0, 1, (1300, 1)) ** (1 / 3)
    pos_np = np.concatenate([bg, cluster]).astype(np.float32)
    box_np = np.eye(3, dtype=np.float32) * L
    i, j, sh, d, dist = _directed_check(ops, pos_np, box_np, 5.0)
    counts = np.bincount(i.cpu().numpy(), minlength=pos_np.shape[0])
    assert counts.max() > 1024 and counts.max() <= 4096
    # half list too (the reference layout)
    ih, jh, _, _, _ = ops.neighbor_list(torch.from_numpy(pos_np).to(DEV), 5.0, torch.from_numpy(box_np).to(DEV), False)
    assert ih.shape[0] * 2 == i.shape[0]
