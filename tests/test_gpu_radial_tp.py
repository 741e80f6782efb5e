"""The radial-MLP output layer fused with the tensor product (molix::radial_tp) and its fused
weight gradient (molix::tp_weight_grad): grad_h = gw W with the per-edge weight gradient gw formed
in registers, against the fp64 oracle (oracle.equivariant.ChannelwiseTP applied to the output
layer's result, its weight gradient multiplied by W in fp64); forward and all input gradients of
radial_tp against the fp64 oracle; MACE in eval mode (the fused path) against the oracle."""

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


def _case(in_ls, sh_ls, out_ls, C, Kh, N=60, E=900, seed=0, sort=True):
    rng = np.random.default_rng(seed)
    cfg = K.tp_config_id(in_ls, sh_ls, out_ls)
    P, NX, NY, NO = K.tp_config_info(cfg)
    recv = rng.integers(0, N, E)
    if sort:
        recv = np.sort(recv)
    ei = np.stack([rng.integers(0, N, E), recv], 1).astype(np.int64)
    x = rng.normal(size=(N, NX * C))
    v = rng.normal(size=(E, 3))
    Y = O.sh(sh_ls, v)
    h = rng.normal(size=(E, Kh))
    W = rng.normal(size=(P * C, Kh)) / np.sqrt(Kh)
    b = rng.normal(size=P * C) * 0.1
    g = rng.normal(size=(N, NO * C))
    tp = O.ChannelwiseTP(_irr(in_ls, C), _irr(sh_ls), _irr(out_ls), C)
    return cfg, tp, ei, x, Y, h, W, b, g


CASES = [([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3], 128, 64),  # config 3 shape
         ([0], [0, 1, 2, 3], [0, 1, 2, 3], 128, 128),  # config 5 literal, layer 1
         ([0, 1], [0, 1, 2, 3], [0, 1], 128, 128),  # config 5 literal, layer 2
         ([0, 1, 2], [0, 1, 2], [0, 1, 2], 32, 32),
         ([0, 1], [0, 1], [0, 1], 16, 16),
         ([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3], 48, 64)]


@pytest.mark.parametrize("in_ls,sh_ls,out_ls,C,Kh", CASES)
def test_tp_weight_grad_vs_fp64(in_ls, sh_ls, out_ls, C, Kh):
    cfg, tp, ei, x, Y, h, W, b, g = _case(in_ls, sh_ls, out_ls, C, Kh, seed=C + Kh)
    w = h @ W.T + b
    _, _, gw = tp.backward(x, Y, w, ei, g)
    ref = gw @ W
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)  # noqa: E731
    gh = K.tp_weight_grad(t(x), t(Y), t(g), torch.tensor(ei, device=DEV), t(W), cfg, C)
    rel, mx = _stats(gh.cpu(), ref)
    print(f"tp_weight_grad in={in_ls} C={C} K={Kh}: rel {rel:.2e}, max-abs {mx:.2e} RMS")
    assert rel <= 1e-5 and mx <= 1e-5


def test_tp_weight_grad_unsorted_and_invalid_edges():
    """Edges in random order, and edges with an index outside [0, N) (zero rows, as the
    receiver-walked backward leaves them out)."""
    cfg, tp, ei, x, Y, h, W, b, g = _case([0, 1, 2], [0, 1, 2], [0, 1, 2], 32, 64, seed=5, sort=False)
    ei[:3, 0] = [-1, 60, 1000]
    ok = (ei >= 0).all(1) & (ei < 60).all(1)
    w = h @ W.T + b
    _, _, gw = tp.backward(x, Y[ok], w[ok], ei[ok], g)
    ref = np.zeros((len(ei), W.shape[1]))
    ref[ok] = gw @ W
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)  # noqa: E731
    gh = K.tp_weight_grad(t(x), t(Y), t(g), torch.tensor(ei, device=DEV), t(W), cfg, 32)
    assert torch.equal(gh[:3].cpu(), torch.zeros(3, W.shape[1]))
    rel, mx = _stats(gh.cpu(), ref)
    assert rel <= 1e-5 and mx <= 1e-5


@pytest.mark.parametrize("in_ls,sh_ls,out_ls,C,Kh", CASES[:3])
def test_radial_tp_forward_and_gradients_vs_fp64(in_ls, sh_ls, out_ls, C, Kh):
    cfg, tp, ei, x, Y, h, W, b, g = _case(in_ls, sh_ls, out_ls, C, Kh, seed=7 + C)
    N = x.shape[0]
    w = h @ W.T + b
    ref = tp.forward(x, Y, w, ei, N)
    rgx, rgY, rgw = tp.backward(x, Y, w, ei, g)
    t = lambda a, rg=False: torch.tensor(a, dtype=torch.float32, device=DEV, requires_grad=rg)  # noqa: E731
    xt, Yt, ht = t(x, True), t(Y, True), t(h, True)
    eit = torch.tensor(ei, device=DEV)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(eit, N)
    out, wk = torch.ops.molix.radial_tp(xt, Yt, ht, t(W), t(b), row_ptr, perm, snd, eit, cfg, C)
    gx, gY, gh = torch.autograd.grad(out, (xt, Yt, ht), t(g))
    for name, a, r in (("out", out, ref), ("w", wk, w), ("grad_x", gx, rgx), ("grad_Y", gY, rgY),
                       ("grad_h", gh, rgw @ W)):
        rel, mx = _stats(a.detach().cpu(), r)
        print(f"radial_tp in={in_ls}: {name} rel {rel:.2e}, max-abs {mx:.2e} RMS")
        assert rel <= 1e-5 and mx <= 1e-5, name


def test_mace_eval_mode_uses_fused_path_and_matches_oracle():
    """A frozen MACE in eval mode runs radial_tp (its backward never writes the per-edge weight
    gradient); energy and forces against the fp64 oracle (config-1 sizes)."""
    from oracle import mace_ref
    from oracle import nlist as NL
    from tests.test_gpu_mace import CFG1, CFG1_LITERAL, build, molecules

    from molnex_amd.config import config

    prev = config.fused_weight_grad, config.paired_radial
    config.fused_weight_grad, config.paired_radial = True, False  # the per-pair path takes precedence
    try:
        _mace_eval_fused(CFG1, CFG1_LITERAL, build, molecules, mace_ref, NL)
    finally:
        config.fused_weight_grad, config.paired_radial = prev


def _mace_eval_fused(CFG1, CFG1_LITERAL, build, molecules, mace_ref, NL):
    for cfg in (CFG1, CFG1_LITERAL):
        pos, Z, batch = molecules()
        ii, jj, _, _ = NL.directed_pairs(pos.astype(np.float32), 5.0, None)
        edge_index = np.stack([jj, ii], 1).astype(np.int64)
        model = build(cfg).eval()
        for p in model.parameters():
            p.requires_grad_(False)
        calls = []
        real = K.tp_weight_grad

        def counting(*a, **k):  # the radial_tp backward looks the op up in molnex_amd.kernels
            calls.append(1)
            return real(*a, **k)

        K.tp_weight_grad = counting
        try:
            e, f = model(torch.tensor(Z, device=DEV), torch.tensor(pos, dtype=torch.float32, device=DEV),
                         torch.tensor(edge_index, device=DEV), torch.tensor(batch, device=DEV), 16)
        finally:
            K.tp_weight_grad = real
        assert calls, "the eval-mode forces did not go through molix::tp_weight_grad"
        sd = {k.removeprefix("encoder."): v for k, v in model.state_dict().items()}
        re, rf = mace_ref.energy_forces(sd, cfg, torch.tensor(Z), torch.tensor(pos.astype(np.float32),
                                                                             dtype=torch.float64),
                                        torch.tensor(edge_index), torch.tensor(batch), 16)
        rel_e = ((e.detach().cpu().double() - re).abs() / re.abs()).max().item()
        rel_f, mx_f = _stats(f.detach().cpu(), rf)
        print(f"MACE eval ({'literal' if cfg.get('hidden_ls') else 'as coded'}): energy {rel_e:.2e}, forces "
              f"{rel_f:.2e} (max {mx_f:.2e} RMS)")
        assert rel_e <= 1e-5 and rel_f <= 1e-5 and mx_f <= 1e-5
