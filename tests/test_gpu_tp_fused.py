"""The tensor-product backward fused with the radial-MLP output layer's input gradient
(molix::tp_scatter_backward_gh, csrc/tp_fused.hip): grad_x, grad_Y and grad_h = gw W, with the
per-edge weight gradient gw staged in LDS and multiplied on the matrix cores, never written.

Against the fp64 oracle (oracle.equivariant.ChannelwiseTP: its weight gradient multiplied by W in
fp64), norm-wise relative error and max-abs error against the reference's RMS both <= 1e-5, on
the products the configs use (config 3: l <= 3, 128 channels, K 64; the literal config-5 layers:
K 128) and on graphs that exercise the persistent walk: receivers without edges, more waves than
edges, edges whose weight rows are shared (undirected pairs), unsorted edge lists.  At the config-3
graph (2.6 M edges) against the unfused tensor-product backward, its weight gradient multiplied by
W in fp64."""

import numpy as np
import pytest
import torch

import molnex_amd.kernels as K
from oracle import equivariant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _irr(ls, C=None):
    return "+".join((f"{C}x" if C else "") + f"{l}{'e' if l % 2 == 0 else 'o'}" for l in ls)


def _stats(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    return np.linalg.norm(got - ref) / np.linalg.norm(ref), np.abs(got - ref).max() / rms


def _t(a):
    return torch.tensor(a, dtype=torch.float32, device=DEV)


def _run(cfg, C, ei, x, Y, w, W, g, wrow=None, need_x=True, need_Y=True):
    N = x.shape[0]
    eit = torch.tensor(ei, device=DEV)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(eit, N)
    wr = None if wrow is None else torch.tensor(wrow, dtype=torch.int32, device=DEV)
    return K.tp_scatter_backward_gh(_t(g), _t(x), _t(Y), _t(w), row_ptr, perm, snd, wr, _t(W), cfg, C, need_x,
                                    need_Y)


def _system(in_ls, sh_ls, out_ls, C, Kh, N, E, seed, sort=True, empty_every=0):
    rng = np.random.default_rng(seed)
    cfg = K.tp_config_id(in_ls, sh_ls, out_ls)
    P, NX, NY, NO = K.tp_config_info(cfg)
    recv = rng.integers(0, N, E)
    if empty_every:  # receivers without edges
        recv = recv - recv % empty_every
    if sort:
        recv = np.sort(recv)
    ei = np.stack([rng.integers(0, N, E), recv], 1).astype(np.int64)
    x = rng.normal(size=(N, NX * C))
    Y = O.sh(sh_ls, rng.normal(size=(E, 3)))
    W = rng.normal(size=(P * C, Kh)) / np.sqrt(Kh)
    w = rng.normal(size=(E, P * C))
    g = rng.normal(size=(N, NO * C))
    tp = O.ChannelwiseTP(_irr(in_ls, C), _irr(sh_ls), _irr(out_ls), C)
    return cfg, tp, ei, x, Y, w, W, g


CASES = [([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3], 128, 64),  # config 3
         ([0], [0, 1, 2, 3], [0, 1], 128, 128),  # config 5 literal, layer 1
         ([0, 1], [0, 1, 2, 3], [0, 1], 128, 128),  # config 5 literal, layer 2
         ([0, 1, 2], [0, 1, 2], [0, 1, 2], 64, 64),
         ([0, 1], [0, 1], [0, 1], 192, 64)]


def _check(cfg, tp, C, ei, x, Y, w, W, g, wrow=None, what=""):
    gx, gY, gh = _run(cfg, C, ei, x, Y, w, W, g, wrow)
    we = w if wrow is None else w[wrow]
    rgx, rgY, rgw = tp.backward(x, Y, we, ei, g)
    for name, a, r in (("grad_x", gx, rgx), ("grad_Y", gY, rgY), ("grad_h", gh, rgw @ W)):
        rel, mx = _stats(a.cpu().numpy().reshape(r.shape), r)
        print(f"fused backward {what} {name}: rel {rel:.2e}, max-abs {mx:.2e} RMS")
        assert rel <= 1e-5 and mx <= 1e-5, (what, name, rel, mx)


@pytest.mark.parametrize("in_ls,sh_ls,out_ls,C,Kh", CASES)
def test_fused_backward_vs_fp64(in_ls, sh_ls, out_ls, C, Kh):
    cfg = K.tp_config_id(in_ls, sh_ls, out_ls)
    assert K.tp_backward_gh_supported(cfg, C, Kh)
    cfg, tp, ei, x, Y, w, W, g = _system(in_ls, sh_ls, out_ls, C, Kh, N=300, E=9000, seed=C + Kh)
    _check(cfg, tp, C, ei, x, Y, w, W, g, what=f"in={in_ls} C={C} K={Kh}")


def test_fused_backward_walk_edge_cases():
    """Receivers without edges (runs of empty CSR segments inside a wavefront's range), an
    unsorted edge list, fewer edges than wavefronts (most ranges empty), one edge."""
    ls = [0, 1, 2, 3]
    for N, E, seed, sort, empty in ((400, 5000, 1, True, 7), (250, 4000, 2, False, 0), (40, 300, 3, True, 5),
                                    (5, 1, 4, True, 0)):
        cfg, tp, ei, x, Y, w, W, g = _system(ls, ls, ls, 128, 64, N=N, E=E, seed=seed, sort=sort, empty_every=empty)
        _check(cfg, tp, 128, ei, x, Y, w, W, g, what=f"N={N} E={E} sorted={sort} empty={empty}")


def test_fused_backward_shared_weight_rows():
    """Edges reading their weights from shared rows (the two directions of an undirected pair):
    grad_h stays per directed edge."""
    rng = np.random.default_rng(9)
    ls = [0, 1, 2, 3]
    cfg, tp, ei, x, Y, w, W, g = _system(ls, ls, ls, 128, 64, N=200, E=4000, seed=9)
    wrow = rng.integers(0, 1500, ei.shape[0]).astype(np.int32)
    _check(cfg, tp, 128, ei, x, Y, w[:1500], W, g, wrow=wrow, what="shared rows")


def test_fused_backward_gradients_subsets_and_opcheck():
    """Without grad_x / grad_Y requested, grad_h is unchanged; torch.library.opcheck on the op."""
    ls = [0, 1]
    cfg, tp, ei, x, Y, w, W, g = _system(ls, [0, 1, 2, 3], ls, 128, 128, N=100, E=2000, seed=11)
    gx, gY, gh = _run(cfg, 128, ei, x, Y, w, W, g)
    gx2, gY2, gh2 = _run(cfg, 128, ei, x, Y, w, W, g, need_x=False, need_Y=False)
    assert gx2.numel() == 0 and gY2.numel() == 0
    assert torch.equal(gh, gh2)
    eit = torch.tensor(ei, device=DEV)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(eit, 100)
    args = (_t(g), _t(x), _t(Y), _t(w), row_ptr, perm, snd, None, _t(W), cfg, 128, True, True)
    torch.library.opcheck(torch.ops.molix.tp_scatter_backward_gh.default, args,
                          test_utils=("test_schema", "test_faketensor"))


def test_radial_tp_pairs_takes_fused_backward():
    """molix::radial_tp_pairs in edge and pair mode: the fused backward (config.tp_bwd_fused = True)
    against the unfused one (the default) on the same inputs."""
    from molnex_amd.config import config

    rng = np.random.default_rng(12)
    ls = [0, 1, 2, 3]
    cfg = K.tp_config_id(ls, ls, ls)
    N, C, Kh = 300, 128, 64
    pos = rng.uniform(0, 14.0, (N, 3)).astype(np.float32)
    box = torch.eye(3, device=DEV) * 14.0
    i, j, sh, d, dist = torch.ops.molix.neighbor_list(torch.tensor(pos, device=DEV), 5.0, box, True)
    ei = torch.stack([j.long(), i.long()], 1)
    E = ei.shape[0]
    row_ptr, perm, snd = torch.ops.molix.edge_csr(ei, N)
    feats = dist.reshape(-1, 1).repeat(1, 8).contiguous()
    pairs = K.EdgePairs.build(ei, N, row_ptr, perm, snd, feats)
    assert pairs is not None
    P, NX, NY, NO = K.tp_config_info(cfg)
    x = torch.randn(N, NX * C, device=DEV, requires_grad=True)
    Y = torch.ops.molix.spherical_harmonics(d, 3).detach().requires_grad_(True)
    W = torch.randn(P * C, Kh, device=DEV) / Kh ** 0.5
    b = torch.randn(P * C, device=DEV) * 0.1
    g = torch.randn(N, NO * C, device=DEV)
    for mode, rows in (("pair", pairs.pairs.shape[0]), ("edge", E)):
        h = torch.randn(rows, Kh, device=DEV, requires_grad=True)
        res = []
        for fused in (True, False):
            prev = config.tp_bwd_fused
            config.tp_bwd_fused = fused
            try:
                out, _ = torch.ops.molix.radial_tp_pairs(x, Y, h, W, b, row_ptr, perm, snd, pairs.wrow, pairs.pairs,
                                                         cfg, C)
                res.append(torch.autograd.grad(out, (x, Y, h), g))
            finally:
                config.tp_bwd_fused = prev
        for name, a, r in zip(("grad_x", "grad_Y", "grad_h"), res[0], res[1]):
            rel, mx = _stats(a.cpu(), r.cpu())
            print(f"radial_tp_pairs {mode} mode {name}: fused vs unfused rel {rel:.2e}, max-abs {mx:.2e}")
            assert rel <= 1e-5 and mx <= 1e-5, (mode, name)


def test_fused_backward_config3_scale():
    """The config-3 graph (50,000 atoms at 0.1 / A^3, rc 5 A, 2.6 M edges, 128 channels, K 64):
    the fused backward against the unfused tensor-product kernel (tp_scatter_backward writing gw;
    grad_h = gw W then formed in fp64), every output over the whole graph."""
    import bench

    torch.manual_seed(0)
    pos, box, edge_index, vec, L = bench.make_system(50_000, 0, True, torch.device(DEV))
    N, E, C, Kh = pos.shape[0], edge_index.shape[0], 128, 64
    ls = [0, 1, 2, 3]
    cfg = K.tp_config_id(ls, ls, ls)
    P, NX, NY, NO = K.tp_config_info(cfg)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(edge_index, N)
    Y = torch.ops.molix.spherical_harmonics(vec, 3)
    x = torch.randn(N, NX * C, device=DEV)
    w = torch.randn(E, P * C, device=DEV)
    W = torch.randn(P * C, Kh, device=DEV) / Kh ** 0.5
    g = torch.randn(N, NO * C, device=DEV)
    gx, gY, gh = K.tp_scatter_backward_gh(g, x, Y, w, row_ptr, perm, snd, None, W, cfg, C, True, True)
    rx, rY, rw = K.tp_scatter_backward(g, x, Y, w, row_ptr, perm, snd, cfg, C, True, True, True)
    # grad_h from the unfused per-edge weight gradient, multiplied by W in fp64 in row chunks
    Wd = W.double()
    rh = torch.cat([rw[i:i + 262144].double() @ Wd for i in range(0, E, 262144)])
    del rw
    for name, a, r in (("grad_x", gx, rx), ("grad_Y", gY, rY), ("grad_h", gh, rh)):
        a64, r64 = a.double(), r.double()
        rel = float((a64 - r64).norm() / r64.norm())
        mx = float((a64 - r64).abs().max() / (r64.norm() / r64.numel() ** 0.5))
        print(f"config 3 scale {name}: fused vs unfused rel {rel:.2e}, max-abs {mx:.2e} RMS")
        assert rel <= 1e-5 and mx <= 1e-5, name
