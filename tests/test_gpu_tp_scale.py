"""Tensor product + scatter at BASELINE config-3 scale: 50,000 atoms in a periodic 79.37 A cube
(0.1 per A^3), the directed 5 A cell list (about 2.6 M edges), 128 channels, l <= 3 (23 paths).

Checked on samples against the fp64 oracle evaluated on exactly the edges each value depends on:
the outputs of sampled receivers and the weight / harmonic gradients of their edges, and the
feature gradient of sampled senders (all their outgoing edges).  Over the whole graph, the
receiver-walked backward (grad_x by atomics) must agree with the sender-walked one (no atomics).
Tolerance as in test_gpu_tp.py: norm-wise relative 1e-5, max-abs 1e-5 x RMS.
"""

import numpy as np
import pytest
import torch

from oracle import equivariant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
C = 128
IRR = "0e + 1o + 2e + 3o"


def _close(got, ref, what, rtol=1e-5):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    nref = np.linalg.norm(ref)
    err = np.linalg.norm(got - ref) / nref
    mx = np.abs(got - ref).max()
    rms = nref / np.sqrt(ref.size)
    assert err <= rtol and mx <= rtol * rms, f"{what}: rel {err:.2e}, max-abs {mx:.2e} (rms {rms:.2e})"


@pytest.fixture(scope="module")
def system():
    import molnex_amd.kernels as K

    ops = torch.ops.molix
    n, L = 50_000, (50_000 / 0.1) ** (1 / 3)
    g = torch.Generator().manual_seed(11)
    pos = (torch.rand(n, 3, generator=g, dtype=torch.float64) * L).float().to(DEV)
    box = torch.eye(3, device=DEV) * L
    i, j, _, deltas, _ = ops.neighbor_list(pos, 5.0, box, True)
    ei = torch.stack([j.long(), i.long()], 1)  # sender j -> receiver i, grouped by receiver
    E = ei.shape[0]
    assert E > 2_400_000
    config = K.tp_config_id([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3])
    P, NX, NY, NO = K.tp_config_info(config)
    gd = torch.Generator(device=DEV).manual_seed(12)
    x = torch.randn(n, NX * C, device=DEV, generator=gd)
    Y = ops.spherical_harmonics(deltas, 3)
    w = torch.randn(E, P * C, device=DEV, generator=gd)
    gout = torch.randn(n, NO * C, device=DEV, generator=gd)
    return dict(ops=ops, K=K, n=n, E=E, ei=ei, x=x, Y=Y, w=w, gout=gout, config=config)


def test_config3_sampled_receivers_and_senders_vs_oracle(system):
    s = system
    ops, K, ei = s["ops"], s["K"], s["ei"]
    row_ptr, perm, snd = ops.edge_csr(ei, s["n"])
    out = ops.tp_scatter(s["x"], s["Y"], s["w"], row_ptr, perm, snd, s["config"], C)
    gx, gY, gw = K.tp_scatter_backward(s["gout"], s["x"], s["Y"], s["w"], row_ptr, perm, snd, s["config"], C,
                                       True, True, True)
    tp = O.ChannelwiseTP(" + ".join(f"{C}x{t}" for t in IRR.split(" + ")), IRR, IRR, C)
    rng = np.random.default_rng(13)
    ei_cpu = ei.cpu().numpy()
    recv = rng.choice(s["n"], 12, replace=False)
    # receivers: their outputs, and grad_w / grad_Y of their edges
    eidx = np.concatenate([np.nonzero(ei_cpu[:, 1] == r)[0] for r in recv])
    sub = ei_cpu[eidx].copy()
    senders, sub[:, 0] = np.unique(sub[:, 0], return_inverse=True)
    _, sub[:, 1] = np.unique(sub[:, 1], return_inverse=True)
    order = np.sort(recv)
    xs = s["x"][torch.from_numpy(senders).to(DEV)].cpu().numpy()
    Ys = s["Y"][torch.from_numpy(eidx).to(DEV)].cpu().numpy()
    ws = s["w"][torch.from_numpy(eidx).to(DEV)].cpu().numpy()
    gs = s["gout"][torch.from_numpy(order).to(DEV)].cpu().numpy()
    ref = tp.forward(xs, Ys, ws, sub, len(order))
    _close(out[torch.from_numpy(order).to(DEV)].cpu().numpy(), ref, "out of sampled receivers")
    _, rY, rw = tp.backward(xs, Ys, ws, sub, gs)
    _close(gw[torch.from_numpy(eidx).to(DEV)].cpu().numpy(), rw, "grad_w of their edges")
    _close(gY[torch.from_numpy(eidx).to(DEV)].cpu().numpy(), rY, "grad_Y of their edges")
    # senders: grad_x over all of their outgoing edges
    send = rng.choice(s["n"], 12, replace=False)
    eidx = np.concatenate([np.nonzero(ei_cpu[:, 0] == v)[0] for v in send])
    sub = ei_cpu[eidx].copy()
    senders, sub[:, 0] = np.unique(sub[:, 0], return_inverse=True)
    receivers, sub[:, 1] = np.unique(sub[:, 1], return_inverse=True)
    xs = s["x"][torch.from_numpy(senders).to(DEV)].cpu().numpy()
    Ys = s["Y"][torch.from_numpy(eidx).to(DEV)].cpu().numpy()
    ws = s["w"][torch.from_numpy(eidx).to(DEV)].cpu().numpy()
    gs = s["gout"][torch.from_numpy(receivers).to(DEV)].cpu().numpy()
    rx, _, _ = tp.backward(xs, Ys, ws, sub, gs)
    _close(gx[torch.from_numpy(senders).to(DEV)].cpu().numpy(), rx, "grad_x of sampled senders")


def test_config3_receiver_and_sender_walked_backward_agree(system):
    s = system
    ops, K, ei = s["ops"], s["K"], s["ei"]
    row_ptr, perm, snd = ops.edge_csr(ei, s["n"])
    s_row, s_perm, s_recv = ops.edge_csr(ei.flip(1), s["n"])
    args = (s["gout"], s["x"], s["Y"], s["w"], row_ptr, perm, snd, s["config"], C, True, True, True)
    a = K.tp_scatter_backward(*args)
    b = K.tp_scatter_backward(*args, s_row, s_perm, s_recv)
    for name, u, v in zip(("grad_x", "grad_Y", "grad_w"), a, b):
        rel = float((u - v).norm() / v.norm())
        assert rel <= 1e-5, f"{name}: receiver- vs sender-walked rel {rel:.2e}"
        del u, v
    torch.cuda.empty_cache()
