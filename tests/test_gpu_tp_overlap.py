"""The tensor-product backward run one path group at a time with each group's columns of the
per-edge weight gradient multiplied into the output layer's input gradient on a second stream
(kernels.tp_backward_overlapped, molix::radial_tp_pairs' backward with config.tp_bwd_overlap): against the fp64
oracle (norm-wise relative and max-abs / RMS error <= 1e-5), per edge and per undirected pair, and
at the config-3 graph size against the single-stream backward."""

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


@pytest.mark.parametrize("in_ls,sh_ls,out_ls,C,Kh", [([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3], 128, 64),
                                                     ([0, 1], [0, 1, 2, 3], [0, 1, 2, 3], 128, 128),
                                                     ([0], [0, 1, 2, 3], [0, 1, 2, 3], 128, 128),
                                                     ([0, 1, 2], [0, 1, 2], [0, 1, 2], 32, 32)])
@pytest.mark.parametrize("paired", [False, True])
def test_overlapped_backward_vs_fp64(in_ls, sh_ls, out_ls, C, Kh, paired):
    rng = np.random.default_rng(C + Kh + paired)
    cfg = K.tp_config_id(in_ls, sh_ls, out_ls)
    P, NX, NY, NO = K.tp_config_info(cfg)
    N, half = 200, 3000
    # undirected pairs: each edge and its reverse, shuffled
    a, b = rng.integers(0, N, half), rng.integers(0, N, half)
    ei = np.concatenate([np.stack([a, b], 1), np.stack([b, a], 1)]).astype(np.int64)
    order = rng.permutation(2 * half)
    ei = ei[order]
    pair_of = np.concatenate([np.arange(half), np.arange(half)])[order]
    pairs = np.zeros((half, 2), np.int32)
    for e, p in enumerate(pair_of):
        pairs[p, 0 if (pairs[p] == 0).all() and e == np.nonzero(pair_of == p)[0][0] else 1] = e
    x = rng.normal(size=(N, NX * C))
    Y = O.sh(sh_ls, rng.normal(size=(2 * half, 3)))
    wp = rng.normal(size=(half, P * C))
    W = rng.normal(size=(P * C, Kh)) / np.sqrt(Kh)
    g = rng.normal(size=(N, NO * C))
    tp = O.ChannelwiseTP(_irr(in_ls, C), _irr(sh_ls), _irr(out_ls), C)
    rgx, rgY, rgw = tp.backward(x, Y, wp[pair_of], ei, g)
    rgh = rgw @ W
    if paired:
        rgh = rgh[pairs[:, 0]] + rgh[pairs[:, 1]]
    eit = torch.tensor(ei, device=DEV)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(eit, N)
    wrow = torch.tensor(pair_of, dtype=torch.int32, device=DEV)
    gx, gY, gh = K.tp_backward_overlapped(_t(g), _t(x), _t(Y), _t(wp), row_ptr, perm, snd, wrow, _t(W),
                                          torch.tensor(pairs, device=DEV) if paired else None, cfg, C, True, True)
    torch.cuda.synchronize()
    for name, got, ref in (("grad_x", gx, rgx), ("grad_Y", gY, rgY), ("grad_h", gh, rgh)):
        rel, mx = _stats(got.cpu().numpy().reshape(ref.shape), ref)
        print(f"overlapped backward in={in_ls} paired={paired} {name}: rel {rel:.2e}, max-abs {mx:.2e} RMS")
        assert rel <= 1e-5 and mx <= 1e-5, (name, rel, mx)


def test_overlapped_backward_config3_scale():
    """The config-3 graph (2.6 M edges, 128 channels, K 64), per pair and per edge: grad_x and grad_Y
    against the single-stream tensor-product backward, grad_h against that backward's per-edge
    weight gradient multiplied by W in fp64."""
    import bench

    pos, box, ei, vec, L = bench.make_system(50_000, 0, True, torch.device(DEV))
    N, E, C, Kh = pos.shape[0], ei.shape[0], 128, 64
    ls = [0, 1, 2, 3]
    cfg = K.tp_config_id(ls, ls, ls)
    P, NX, NY, NO = K.tp_config_info(cfg)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(ei, N, False)
    r = torch.linalg.vector_norm(vec, dim=-1)
    pairs = K.EdgePairs.build(ei, N, row_ptr, perm, snd, r.reshape(-1, 1).repeat(1, 8).contiguous())
    assert pairs is not None
    torch.manual_seed(1)
    x = torch.randn(N, NX * C, device=DEV)
    Y = torch.ops.molix.spherical_harmonics(vec, 3)
    wp = torch.randn(pairs.pairs.shape[0], P * C, device=DEV)
    W = torch.randn(P * C, Kh, device=DEV) / Kh ** 0.5
    g = torch.randn(N, NO * C, device=DEV)
    rx, rY, rw = K.tp_scatter_backward(g, x, Y, wp, row_ptr, perm, snd, cfg, C, True, True, True, wrow=pairs.wrow)
    Wd = W.double()
    rh = torch.cat([rw[i:i + 262144].double() @ Wd for i in range(0, E, 262144)])
    del rw
    lead, part = pairs.pairs[:, 0].long(), pairs.pairs[:, 1].long()
    for mode, pr, ref_h in (("pair", pairs.pairs, rh[lead] + rh[part]), ("edge", None, rh)):
        gx, gY, gh = K.tp_backward_overlapped(g, x, Y, wp, row_ptr, perm, snd, pairs.wrow, W, pr, cfg, C, True, True)
        for name, a, ref in (("grad_x", gx, rx), ("grad_Y", gY, rY), ("grad_h", gh, ref_h)):
            a64, r64 = a.double(), ref.double()
            rel = float((a64 - r64).norm() / r64.norm())
            mx = float((a64 - r64).abs().max() / (r64.norm() / r64.numel() ** 0.5))
            print(f"config 3 {mode} mode {name}: rel {rel:.2e}, max-abs {mx:.2e} RMS")
            assert rel <= 1e-5 and mx <= 1e-5, (mode, name)
