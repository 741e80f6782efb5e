"""The allocation-free CSR build (mnx_csr_build_noalloc) against the workspace entry point
(mnx_csr_build), both called through the C ABI: bit-equal row_ptr / perm / senders / invalid
count on two calls in a row, the second with a smaller input (the shared scratch keeps the
first call's contents, so its counters must be cleared)."""

import numpy as np
import pytest
import torch

from molnex_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"
MAX_NODES = 2097152  # MNX_CSR_NOALLOC_MAX_NODES


def _edges(rng, n, e, shuffle, n_invalid=0):
    recv = np.sort(rng.integers(0, n, e))
    send = rng.integers(0, n, e)
    ei = np.stack([send, recv], 1).astype(np.int64)
    if shuffle:
        ei = ei[rng.permutation(e)]
    if n_invalid:
        bad = rng.choice(e, n_invalid, replace=False)
        ei[bad[: n_invalid // 2], 0] = n + 3
        ei[bad[n_invalid // 2:], 1] = -1
    return torch.from_numpy(ei).to(DEV)


def _run(lib, ei, n, noalloc):
    E = ei.shape[0]
    row_ptr = torch.full((n + 1,), -7, dtype=torch.int32, device=DEV)
    perm = torch.full((max(E, 1),), -7, dtype=torch.int32, device=DEV)
    snd = torch.full((max(E, 1),), -7, dtype=torch.int32, device=DEV)
    inv = torch.full((1,), -7, dtype=torch.int32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.mnx_csr_build_noalloc(ei.data_ptr(), E, n, row_ptr.data_ptr(), perm.data_ptr(), snd.data_ptr(),
                                       inv.data_ptr(), stream)
    else:
        ws = torch.empty(int(lib.mnx_csr_workspace_bytes(n, E)), dtype=torch.uint8, device=DEV)
        rc = lib.mnx_csr_build(ei.data_ptr(), E, n, row_ptr.data_ptr(), perm.data_ptr(), snd.data_ptr(),
                               inv.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "csr build (noalloc)" if noalloc else "csr build")
    torch.cuda.synchronize()
    nv = int(row_ptr[n].item())
    return row_ptr.cpu(), perm[:nv].cpu(), snd[:nv].cpu(), int(inv.item())


@pytest.mark.parametrize("shuffle", [True, False])
def test_noalloc_csr_matches_workspace_entry_point(shuffle):
    lib = _lib.load()
    rng = np.random.default_rng(11 if shuffle else 12)
    # first call larger, second smaller: the second must not see the first's counters
    for n, e, bad in ((20000, 300000, 40), (700, 5000, 0), (1, 0, 0)):
        ei = _edges(rng, n, e, shuffle, bad) if e else torch.zeros((0, 2), dtype=torch.int64, device=DEV)
        ref = _run(lib, ei, n, noalloc=False)
        got = _run(lib, ei, n, noalloc=True)
        assert torch.equal(ref[0], got[0]), (n, e)
        assert torch.equal(ref[1], got[1]), (n, e)
        assert torch.equal(ref[2], got[2]), (n, e)
        assert ref[3] == got[3] == bad, (n, e, ref[3], got[3])
        if e:
            # and against numpy: receiver-grouped, ascending edge id per receiver
            h = ei.cpu().numpy()
            ok = (h[:, 0] >= 0) & (h[:, 0] < n) & (h[:, 1] >= 0) & (h[:, 1] < n)
            ids = np.nonzero(ok)[0]
            order = ids[np.argsort(h[ids, 1], kind="stable")]
            assert np.array_equal(got[1].numpy(), order.astype(np.int32))
            assert np.array_equal(got[2].numpy(), h[order, 0].astype(np.int32))


def test_noalloc_csr_rejects_oversized_graph():
    lib = _lib.load()
    ei = torch.zeros((1, 2), dtype=torch.int64, device=DEV)
    n = MAX_NODES + 1
    rc = lib.mnx_csr_build_noalloc(ei.data_ptr(), 1, n, None, None, None, None,
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == 1 and b"allocation-free limit" in lib.mnx_last_error()
