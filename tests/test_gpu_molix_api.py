"""molix's Python API on the HIP ops, against the neighbor-list oracle (itself bit-exact with the
reference op's outputs): the functional get_neighbor_pairs, the nn.NeighborList module and the
per-sample NeighborList data task (edge order, bond_diff sign and distances of
src/molix/data/tasks/neighbor_list.py:67-103)."""

import numpy as np
import pytest
import torch

from oracle import nlist as NL

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _sample(seed, n=60, L=9.0):
    rng = np.random.default_rng(seed)
    return rng.uniform(0, L, (n, 3)).astype(np.float32), np.eye(3, dtype=np.float32) * np.float32(L)


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype.kind == "f":
        return a.shape == b.shape and np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else np.uint64),
                                                     b.view(np.uint32 if b.dtype == np.float32 else np.uint64))
    return np.array_equal(a, b)


@pytest.mark.parametrize("periodic", [False, True])
@pytest.mark.parametrize("max_num_pairs", [-1, 5000, 10])
def test_functional_get_neighbor_pairs(periodic, max_num_pairs):
    from molnex_amd.molix import F

    pos, box = _sample(1)
    out = F.get_neighbor_pairs(torch.tensor(pos, device=DEV), 3.0, max_num_pairs,
                               torch.tensor(box, device=DEV) if periodic else None)
    ref = NL.get_neighbor_pairs(pos, 3.0, max_num_pairs, box if periodic else None)
    found = int(ref[3][0])
    assert int(out[3].item()) == found
    nb, d, dist = (t.cpu().numpy() for t in out[:3])
    if max_num_pairs != -1 and found > max_num_pairs:
        # fixed width (the CUDA / meta shape): the first max_num_pairs pairs in (row, col) order
        w = max_num_pairs
        assert nb.shape == (2, w)
        assert _same(nb, ref[0][:, :w]) and _same(d, ref[1][:w]) and _same(dist, ref[2][:w])
    else:
        assert _same(nb, ref[0]) and _same(d, ref[1]) and _same(dist, ref[2])


def test_nn_neighbor_list_module():
    from molnex_amd.molix.nn import NeighborList

    pos, box = _sample(2)
    mod = NeighborList(cutoff=3.5, pbc=True)
    assert "cutoff=3.5" in repr(mod)
    out = mod(torch.tensor(pos, device=DEV), torch.tensor(box, device=DEV))
    ref = NL.get_neighbor_pairs(pos, 3.5, -1, box)
    assert all(_same(o.cpu().numpy(), r) for o, r in zip(out, ref))


@pytest.mark.parametrize("pbc", [False, True])
@pytest.mark.parametrize("symmetry", [True, False])
@pytest.mark.parametrize("on_gpu", [False, True])
def test_neighbor_list_task_matches_reference_convention(pbc, symmetry, on_gpu):
    """edge_index rows [source, target] = the half list's (row, col), bond_diff = -deltas =
    pos[target] - pos[source] (neighbor_list.py:86-89), then the reversed edges with the opposite
    bond_diff (:91-96); outputs stay on the sample's device."""
    from molnex_amd.molix.data.tasks import NeighborList

    pos, box = _sample(3)
    data = {"pos": torch.tensor(pos), "cell": torch.tensor(box), "Z": torch.zeros(len(pos))}
    if on_gpu:
        data = {k: v.to(DEV) for k, v in data.items()}
    out = NeighborList(cutoff=3.0, pbc=pbc, symmetry=symmetry)(data)
    assert out["Z"] is data["Z"] and out["edge_index"].device == data["pos"].device
    rows, cols, d, dist = NL.half_pairs(pos, 3.0, box if pbc else None)
    ei = np.stack([rows, cols], 1).astype(np.int64)
    bd = -d
    if symmetry:
        ei = np.concatenate([ei, ei[:, ::-1]])
        bd = np.concatenate([bd, d])
        dist = np.concatenate([dist, dist])
    assert out["edge_index"].dtype == torch.int64 and out["bond_diff"].dtype == torch.float32
    assert _same(out["edge_index"].cpu().numpy(), ei)
    assert _same(out["bond_diff"].cpu().numpy(), bd) and _same(out["bond_dist"].cpu().numpy(), dist)
    if not pbc:  # open boundaries: the bond vector is literally pos[target] - pos[source]
        e = out["edge_index"].cpu().numpy()
        np.testing.assert_array_equal(out["bond_diff"].cpu().numpy(), pos[e[:, 1]] - pos[e[:, 0]])


def test_neighbor_list_task_receiver_sorted():
    """Every directed edge once, grouped by target in ascending (target, source) order, with the
    same bond vectors as the reference convention's."""
    from molnex_amd.molix.data.tasks import NeighborList

    pos, box = _sample(4)
    out = NeighborList(cutoff=3.0, pbc=True, receiver_sorted=True)({"pos": torch.tensor(pos, device=DEV),
                                                                      "cell": torch.tensor(box, device=DEV)})
    i, j, dd, dist = NL.directed_pairs(pos, 3.0, box)
    assert _same(out["edge_index"].cpu().numpy(), np.stack([j, i], 1).astype(np.int64))
    assert _same(out["bond_diff"].cpu().numpy(), dd) and _same(out["bond_dist"].cpu().numpy(), dist)
    ref = NeighborList(cutoff=3.0, pbc=True)({"pos": torch.tensor(pos), "cell": torch.tensor(box)})
    key = lambda e: set(map(tuple, e.cpu().numpy().tolist()))  # noqa: E731
    assert key(out["edge_index"]) == key(ref["edge_index"])
