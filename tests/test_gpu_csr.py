"""The receiver CSR (molix::edge_csr / mnx_csr_build) of edge lists in arbitrary order, with
receivers of every degree class the segment sort distinguishes: up to 64 edges (sorted in
registers), up to 4096 (merged in LDS) and beyond (merged in global memory through the senders
array, or -- without a senders array -- by one lane).  Against numpy's stable argsort by
receiver: rows grouped by receiver, ascending edge id within each receiver, exact."""

import numpy as np
import pytest
import torch

import molnex_amd.kernels  # noqa: F401  (registers torch.ops.molix.*)
from molnex_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _graph(seed, n=3000, light=40000, hubs=((7, 100), (11, 900), (1500, 4096), (2999, 4097), (5, 9000))):
    rng = np.random.default_rng(seed)
    recv = [rng.integers(0, n, light)]
    for r, deg in hubs:
        recv.append(np.full(deg, r))
    recv = np.concatenate(recv)
    send = rng.integers(0, n, recv.shape[0])
    ei = np.stack([send, recv], 1).astype(np.int64)
    return ei[rng.permutation(ei.shape[0])], n


def _expected(ei, n):
    order = np.argsort(ei[:, 1], kind="stable")
    row_ptr = np.concatenate([[0], np.cumsum(np.bincount(ei[:, 1], minlength=n))]).astype(np.int32)
    return row_ptr, order.astype(np.int32), ei[order, 0].astype(np.int32)


def test_edge_csr_heavy_receivers_unsorted():
    ei, n = _graph(1)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(torch.from_numpy(ei).to(DEV), n)
    r_ref, p_ref, s_ref = _expected(ei, n)
    assert np.array_equal(row_ptr.cpu().numpy(), r_ref)
    assert np.array_equal(perm.cpu().numpy(), p_ref)
    assert np.array_equal(snd.cpu().numpy(), s_ref)
    # the same edges again (sort result independent of the placement's atomic order)
    row_ptr2, perm2, snd2 = torch.ops.molix.edge_csr(torch.from_numpy(ei).to(DEV), n)
    assert torch.equal(perm, perm2) and torch.equal(snd, snd2)


def test_csr_build_without_senders_array():
    """mnx_csr_build with senders_sorted = NULL: segments longer than the LDS merge are merged
    by one lane in place; the permutation is the same."""
    lib = _lib.load()
    ei, n = _graph(2, hubs=((3, 70), (8, 5000)))
    eit = torch.from_numpy(ei).to(DEV)
    E = ei.shape[0]
    row_ptr = torch.empty(n + 1, dtype=torch.int32, device=DEV)
    perm = torch.empty(E, dtype=torch.int32, device=DEV)
    ws = torch.empty(int(lib.mnx_csr_workspace_bytes(n, E)), dtype=torch.uint8, device=DEV)
    _lib.check(lib.mnx_csr_build(eit.data_ptr(), E, n, row_ptr.data_ptr(), perm.data_ptr(), None, None,
                                 ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream), "csr build")
    r_ref, p_ref, _ = _expected(ei, n)
    assert np.array_equal(row_ptr.cpu().numpy(), r_ref)
    assert np.array_equal(perm.cpu().numpy(), p_ref)
