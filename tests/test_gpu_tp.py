"""GPU channelwise tensor product + scatter vs the fp64 oracle, forward and backward.

Tolerance (fp32 kernels vs fp64 oracle): norm-wise relative error <= 1e-5 and
max-abs error <= 1e-5 * RMS(reference) for every output and gradient.
"""

import numpy as np
import pytest
import torch

from oracle import equivariant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def irr(ls, mul=None):
    return " + ".join(f"{mul}x{l}{'e' if l % 2 == 0 else 'o'}" if mul else f"{l}{'e' if l % 2 == 0 else 'o'}"
                      for l in ls)


def assert_close(got, ref, what, rtol=1e-5):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    nref = np.linalg.norm(ref)
    if nref == 0:
        assert np.abs(got).max(initial=0) == 0, what
        return
    err = np.linalg.norm(got - ref) / nref
    rms = nref / np.sqrt(ref.size)
    mx = np.abs(got - ref).max()
    assert err <= rtol and mx <= rtol * rms, f"{what}: rel {err:.2e}, max-abs {mx:.2e} (rms {rms:.2e})"


CONFIGS = [
    ([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3]),
    ([0, 1, 2], [0, 1, 2], [0, 1, 2]),
    ([0, 1], [0, 1], [0, 1]),
    ([0], [0], [0]),
    ([0], [0, 1, 2, 3], [0, 1, 2, 3]),
    ([0, 1], [0, 1, 2, 3], [0, 1]),
    ([0], [0, 1], [0]),
    ([1], [0, 1], [1]),
]


def run_case(cfg, C, N, E, seed, ops):
    from molnex_amd import kernels as K

    in_ls, sh_ls, out_ls = cfg
    rng = np.random.default_rng(seed)
    tp = O.ChannelwiseTP(irr(in_ls, C), irr(sh_ls), irr(out_ls), C)
    x = rng.normal(size=(N, tp.nx * C)).astype(np.float32)
    Y = rng.normal(size=(E, tp.ny)).astype(np.float32)
    w = rng.normal(size=(E, len(tp.paths) * C)).astype(np.float32)
    ei = rng.integers(0, N, (E, 2))
    ei[: E // 10, 1] = 0  # one heavy receiver
    ei[E // 10: E // 5, 0] = 1  # one heavy sender
    g = rng.normal(size=(N, tp.no * C)).astype(np.float32)
    config = K.tp_config_id(in_ls, sh_ls, out_ls)
    assert config >= 0
    xt, Yt, wt = (torch.tensor(a, device=DEV, requires_grad=True) for a in (x, Y, w))
    eit = torch.tensor(ei, device=DEV)
    row_ptr, perm, snd = ops.edge_csr(eit, N)
    scsr = ops.edge_csr(eit.flip(1), N)
    ref = tp.forward(x, Y, w, ei, N)
    rx, rY, rw = tp.backward(x, Y, w, ei, g)
    # backward walked by receiver (grad_x atomics) and by sender (no atomics)
    for tag, extra in (("by receiver", ()), ("by sender", scsr)):
        out = ops.tp_scatter(xt, Yt, wt, row_ptr, perm, snd, config, C, *extra)
        assert_close(out.detach().cpu().numpy(), ref, f"fwd {cfg} C={C}")
        gx, gY, gw = torch.autograd.grad(out, (xt, Yt, wt), torch.tensor(g, device=DEV))
        assert_close(gx.cpu().numpy(), rx, f"grad_x {cfg} C={C} {tag}")
        assert_close(gY.cpu().numpy(), rY, f"grad_Y {cfg} C={C} {tag}")
        assert_close(gw.cpu().numpy(), rw, f"grad_w {cfg} C={C} {tag}")


@pytest.fixture(scope="module")
def ops():
    import molnex_amd.kernels  # noqa: F401

    return torch.ops.molix


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"{c}")
def test_tp_configs(ops, cfg):
    run_case(cfg, 16, 23, 180, 0, ops)


@pytest.mark.parametrize("C", [8, 32, 64, 96, 128])
def test_tp_channels(ops, C):
    run_case(CONFIGS[0], C, 37, 400, C, ops)


def test_tp_empty_receivers_and_no_edges(ops):
    from molnex_amd import kernels as K

    C, N = 16, 10
    config = K.tp_config_id([0, 1], [0, 1], [0, 1])
    ei = torch.zeros((0, 2), dtype=torch.int64, device=DEV)
    row_ptr, perm, snd = ops.edge_csr(ei, N)
    num_paths, nx, ny, no = K.tp_config_info(config)
    assert (num_paths, nx, ny, no) == (4, 4, 4, 8)
    x = torch.randn(N, nx * C, device=DEV)
    out = ops.tp_scatter(x, torch.zeros((0, ny), device=DEV), torch.zeros((0, num_paths * C), device=DEV), row_ptr,
                         perm, snd, config, C)
    assert out.shape == (N, no * C) and torch.all(out == 0)
    # backward with no edges, walked by sender: grad_x must come back all zero (stored, not accumulated)
    xg = x.clone().requires_grad_(True)
    out = ops.tp_scatter(xg, torch.zeros((0, ny), device=DEV), torch.zeros((0, num_paths * C), device=DEV), row_ptr,
                         perm, snd, config, C, *ops.edge_csr(ei.flip(1), N))
    (gx,) = torch.autograd.grad(out, (xg,), torch.ones_like(out))
    assert torch.all(gx == 0)


def test_edge_csr_rejects_out_of_range(ops):
    ei = torch.tensor([[0, 1], [2, 5]], device=DEV)
    with pytest.raises(ValueError):
        ops.edge_csr(ei, 3)


def test_tp_deterministic_forward(ops):
    from molnex_amd import kernels as K

    rng = np.random.default_rng(9)
    C, N, E = 64, 50, 900
    config = K.tp_config_id([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3])
    x = torch.tensor(rng.normal(size=(N, 16 * C)), dtype=torch.float32, device=DEV)
    Y = torch.tensor(rng.normal(size=(E, 16)), dtype=torch.float32, device=DEV)
    w = torch.tensor(rng.normal(size=(E, 23 * C)), dtype=torch.float32, device=DEV)
    csr = ops.edge_csr(torch.tensor(rng.integers(0, N, (E, 2)), device=DEV), N)
    a = ops.tp_scatter(x, Y, w, *csr, config, C)
    b = ops.tp_scatter(x, Y, w, *csr, config, C)
    assert torch.equal(a, b)


def test_tp_backward_by_sender_is_bitwise_reproducible(ops):
    """The sender-walked backward has no atomics: two runs give identical gradients."""
    from molnex_amd import kernels as K

    rng = np.random.default_rng(10)
    C, N, E = 128, 60, 1500
    config = K.tp_config_id([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3])
    x = torch.tensor(rng.normal(size=(N, 16 * C)), dtype=torch.float32, device=DEV)
    Y = torch.tensor(rng.normal(size=(E, 16)), dtype=torch.float32, device=DEV)
    w = torch.tensor(rng.normal(size=(E, 23 * C)), dtype=torch.float32, device=DEV)
    g = torch.tensor(rng.normal(size=(N, 99 * C)), dtype=torch.float32, device=DEV)
    ei = torch.tensor(rng.integers(0, N, (E, 2)), device=DEV)
    csr, scsr = ops.edge_csr(ei, N), ops.edge_csr(ei.flip(1), N)
    a = K.tp_scatter_backward(g, x, Y, w, *csr, config, C, True, True, True, *scsr)
    b = K.tp_scatter_backward(g, x, Y, w, *csr, config, C, True, True, True, *scsr)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.mark.parametrize("presorted", [True, False])
def test_edge_csr_matches_numpy(ops, presorted):
    """Receiver CSR on both paths: edges already grouped by receiver (identity fast path)
    and shuffled; perm holds edge ids ascending within each receiver."""
    rng = np.random.default_rng(21)
    N, E = 300, 5000
    ei = rng.integers(0, N, (E, 2))
    ei[:40, 1] = 7  # a heavy receiver
    if presorted:
        ei = ei[np.lexsort((ei[:, 0], ei[:, 1]))]
    row_ptr, perm, snd = ops.edge_csr(torch.tensor(ei, device=DEV), N)
    order = np.lexsort((np.arange(E), ei[:, 1]))  # by receiver, then edge id
    ref_ptr = np.concatenate([[0], np.cumsum(np.bincount(ei[:, 1], minlength=N))])
    np.testing.assert_array_equal(row_ptr.cpu().numpy(), ref_ptr)
    np.testing.assert_array_equal(perm.cpu().numpy(), order)
    np.testing.assert_array_equal(snd.cpu().numpy(), ei[order, 0])
