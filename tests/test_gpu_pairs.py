"""Undirected pairs of a directed neighbor list (molix::edge_reverse, kernels.EdgePairs) and the
radial MLP's output layer applied once per pair (molix::radial_tp_pairs).

The pairing is checked against a numpy brute force (opposite sender / receiver, bit-identical
features); its use is checked two ways: the paired op against the per-edge composition on the GPU
(the weights are the same rows, so the product and grad_Y are bit-identical, grad_x equal up to
the order of its atomic additions; the output layer's input gradient adds the two directions in
another order) and against the fp64
oracle (oracle.equivariant.ChannelwiseTP of h W^T + b, the input gradient of each pair the sum of
its two edges' gw W).  MACE energies and forces in eval mode with the pairing against the same
model without it, and against the fp64 oracle."""

import numpy as np
import pytest
import torch

import molnex_amd.kernels as K
from molnex_amd.config import config
from oracle import equivariant as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
RC = 5.0


def _system(n, L, seed):
    rng = np.random.default_rng(seed)
    p = torch.tensor(rng.uniform(0, L, (n, 3)).astype(np.float32), device=DEV)
    box = torch.eye(3, device=DEV) * L
    i, j, sh, _, _ = torch.ops.molix.neighbor_list(p, RC, box, True)
    ei = torch.stack([j.long(), i.long()], 1)  # [sender, receiver]
    bond = torch.ops.molix.bond_vectors(p, ei, sh)
    return p, ei, bond


def _pairs(ei, n, feats):
    row_ptr, perm, snd = torch.ops.molix.edge_csr(ei, n)
    return K.EdgePairs.build(ei, n, row_ptr, perm, snd, feats), (row_ptr, perm, snd)


def _brute_reverse(ei, feats):
    """rev[e] by brute force over all edges: opposite direction, identical feature bits."""
    ei = ei.cpu().numpy()
    bits = feats.cpu().numpy().view(np.uint32).reshape(len(ei), -1)
    key = {}
    for e, (s, r) in enumerate(ei):
        key.setdefault((int(s), int(r), bits[e].tobytes()), []).append(e)
    rev = np.full(len(ei), -1)
    for e, (s, r) in enumerate(ei):
        cand = [c for c in key.get((int(r), int(s), bits[e].tobytes()), []) if c != e]
        if len(cand) == 1:
            rev[e] = cand[0]
    return rev


def test_edge_reverse_matches_brute_force_and_pairs_are_consistent():
    n, L = 700, (700 / 0.1) ** (1 / 3)
    p, ei, bond = _system(n, L, seed=3)
    feats = bond.norm(dim=-1, keepdim=True)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(ei, n)
    rev, bad = torch.ops.molix.edge_reverse(ei, n, row_ptr, perm, snd, feats)
    ref = _brute_reverse(ei, feats)
    assert int(bad.item()) == 0 and (ref >= 0).all()
    assert np.array_equal(rev.cpu().numpy(), ref)
    pr = K.EdgePairs.build(ei, n, row_ptr, perm, snd, feats)
    assert pr is not None
    E = ei.shape[0]
    P = pr.pairs.long()
    assert P.shape == (E // 2, 2) and bool((P[:, 0] < P[:, 1]).all())
    assert torch.equal(torch.sort(P.reshape(-1)).values, torch.arange(E, device=DEV))
    assert torch.equal(ei[P[:, 0]], ei[P[:, 1]].flip(1))
    # opposite bond vectors are exact negations (neighbor-list geometry)
    assert torch.equal(bond[P[:, 0]], -bond[P[:, 1]])
    ar = torch.arange(E // 2, device=DEV, dtype=torch.int32)
    assert torch.equal(pr.wrow[P[:, 0]], ar) and torch.equal(pr.wrow[P[:, 1]], ar)
    assert torch.equal(pr.lead, P[:, 0])


def test_no_pairing_when_partners_are_ambiguous_or_missing():
    p, ei, bond = _system(300, (300 / 0.1) ** (1 / 3), seed=5)
    feats = bond.norm(dim=-1, keepdim=True)
    # one pair listed twice: each of its edges has two equal candidates -- no unique partner
    row_ptr, perm, snd = torch.ops.molix.edge_csr(ei, 300)
    rev, _ = torch.ops.molix.edge_reverse(ei, 300, row_ptr, perm, snd, feats)
    dup = torch.tensor([0, int(rev[0])], device=DEV)
    pr, _ = _pairs(torch.cat([ei, ei[dup]]), 300, torch.cat([feats, feats[dup]]))
    assert pr is None
    # a neighbor list with two edges removed (and one with an odd edge count)
    keep = torch.ones(ei.shape[0], dtype=torch.bool, device=DEV)
    keep[7] = False
    keep[9] = False
    pr, _ = _pairs(ei[keep], 300, feats[keep])
    assert pr is None
    pr, _ = _pairs(ei[1:], 300, feats[1:])
    assert pr is None
    # features that differ between the two directions
    f2 = feats.clone()
    f2[11] = f2[11] * 1.0000001
    pr, _ = _pairs(ei, 300, f2)
    assert pr is None


def test_pairing_reused_for_new_positions():
    """The pairing depends only on the edge list: new positions on the same edges keep it (checked on
    the device), features that break a pair make the graph fall back to per-edge work."""
    from molnex_amd.molrep.interaction.tensor_product import EdgeGraph

    n, L = 300, (300 / 0.1) ** (1 / 3)
    p, ei, bond = _system(n, L, seed=8)
    box = torch.eye(3, device=DEV) * L
    i, j, sh, _, _ = torch.ops.molix.neighbor_list(p, RC, box, True)
    g = EdgeGraph(ei, n)
    f1 = bond.norm(dim=-1, keepdim=True)
    pr1 = g.pairs(f1)
    assert pr1 is not None
    p2 = p + 0.01 * torch.randn_like(p)  # same edge list, new positions
    f2 = torch.ops.molix.bond_vectors(p2, ei, sh).norm(dim=-1, keepdim=True)
    assert pr1.holds_for(f2)
    assert g.pairs(f2) is pr1
    f3 = f2.clone()
    f3[5] += 1e-3
    assert not pr1.holds_for(f3)
    assert g.pairs(f3) is None


def _irr(ls, C=None):
    return "+".join((f"{C}x" if C else "") + f"{l}{'e' if l % 2 == 0 else 'o'}" for l in ls)


def _stats(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref))
    return np.linalg.norm(got - ref) / np.linalg.norm(ref), np.abs(got - ref).max() / rms


CASES = [([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3], 64, 64),  # config 3 products
         ([0], [0, 1, 2, 3], [0, 1, 2, 3], 64, 128),  # config 5 literal, layer 1
         ([0, 1], [0, 1, 2, 3], [0, 1], 32, 128)]  # config 5 literal, layer 2


@pytest.mark.parametrize("in_ls,sh_ls,out_ls,C,Kh", CASES)
def test_radial_tp_pairs_vs_per_edge_and_fp64(in_ls, sh_ls, out_ls, C, Kh):
    n, L = 300, (300 / 0.1) ** (1 / 3)
    p, ei, bond = _system(n, L, seed=C + Kh)
    pr, (row_ptr, perm, snd) = _pairs(ei, n, bond.norm(dim=-1, keepdim=True))
    assert pr is not None
    E = ei.shape[0]
    cfg = K.tp_config_id(in_ls, sh_ls, out_ls)
    P, NX, NY, NO = K.tp_config_info(cfg)
    rng = np.random.default_rng(C)
    x = rng.normal(size=(n, NX * C)).astype(np.float32)
    Y = torch.ops.molix.spherical_harmonics(bond, max(sh_ls))
    hp = rng.normal(size=(E // 2, Kh)).astype(np.float32)
    W = (rng.normal(size=(P * C, Kh)) / np.sqrt(Kh)).astype(np.float32)
    b = (rng.normal(size=P * C) * 0.1).astype(np.float32)
    g = rng.normal(size=(n, NO * C)).astype(np.float32)
    t = lambda a, rg=False: torch.tensor(a, device=DEV, requires_grad=rg)  # noqa: E731
    wrow = pr.wrow.long()

    # paired op
    xt, Yt, ht, Wt, bt = t(x, True), Y.detach().clone().requires_grad_(True), t(hp, True), t(W, True), t(b, True)
    out, _ = torch.ops.molix.radial_tp_pairs(xt, Yt, ht, Wt, bt, row_ptr, perm, snd, pr.wrow, pr.pairs, cfg, C)
    gx, gY, gh, gW, gb = torch.autograd.grad(out, (xt, Yt, ht, Wt, bt), t(g))
    # per-edge composition on the GPU: every edge gets its pair's activations
    x2, Y2, h2, W2, b2 = t(x, True), Y.detach().clone().requires_grad_(True), t(hp, True), t(W, True), t(b, True)
    w2 = K.edge_weights(h2[wrow], W2, b2)
    out2 = torch.ops.molix.tp_scatter(x2, Y2, w2, row_ptr, perm, snd, cfg, C)
    gx2, gY2, gh2, gW2, gb2 = torch.autograd.grad(out2, (x2, Y2, h2, W2, b2), t(g))
    assert torch.equal(out, out2) and torch.equal(gY, gY2)
    # grad_x: the same terms, added by atomics in either order; grad_h: the two directions added
    # before the product instead of after; grad_W / grad_b: fp32 GEMM sums over the pairs instead
    # of the edges (each within the fp32 rounding of a sum over thousands of terms)
    for name, a, r in (("grad_x", gx, gx2), ("grad_h", gh, gh2), ("grad_W", gW, gW2), ("grad_b", gb, gb2)):
        rel, mx = _stats(a.cpu(), r.cpu())
        print(f"radial_tp_pairs in={in_ls} C={C}: {name} vs per edge rel {rel:.2e}, max-abs {mx:.2e} RMS")
    for name, a, r in (("grad_x", gx, gx2), ("grad_h", gh, gh2)):
        rel, mx = _stats(a.cpu(), r.cpu())
        assert rel <= 1e-5 and mx <= 1e-5, (name, rel, mx)

    # edge mode: activations per edge (both rows of a pair equal), per-edge input gradients --
    # bit-identical to the per-edge composition
    hf = t(hp[wrow.cpu().numpy()], True)
    out3, _ = torch.ops.molix.radial_tp_pairs(t(x), Y.detach(), hf, t(W), t(b), row_ptr, perm, snd, pr.wrow,
                                              pr.pairs, cfg, C)
    (gh3,) = torch.autograd.grad(out3, (hf,), t(g))
    hf2 = t(hp[wrow.cpu().numpy()], True)
    out4 = torch.ops.molix.tp_scatter(t(x), Y.detach(), K.edge_weights(hf2, t(W), t(b)), row_ptr, perm, snd, cfg, C)
    (gh4,) = torch.autograd.grad(out4, (hf2,), t(g))
    assert torch.equal(out3, out) and torch.equal(out4, out) and torch.equal(gh3, gh4)

    # fp64 oracle
    tp = O.ChannelwiseTP(_irr(in_ls, C), _irr(sh_ls), _irr(out_ls), C)
    ei_np, Y64 = ei.cpu().numpy(), Y.detach().cpu().double().numpy()
    wr = wrow.cpu().numpy()
    w64 = (hp.astype(np.float64) @ W.T.astype(np.float64) + b)[wr]
    ref = tp.forward(x.astype(np.float64), Y64, w64, ei_np, n)
    rgx, rgY, rgw = tp.backward(x.astype(np.float64), Y64, w64, ei_np, g.astype(np.float64))
    gwp = np.zeros((E // 2, P * C))
    np.add.at(gwp, wr, rgw)
    for name, a, r in (("out", out, ref), ("grad_x", gx, rgx), ("grad_Y", gY, rgY), ("grad_h", gh, gwp @ W),
                       ("grad_W", gW, gwp.T @ hp), ("grad_b", gb, gwp.sum(0))):
        rel, mx = _stats(a.detach().cpu(), r)
        print(f"radial_tp_pairs in={in_ls} C={C}: {name} vs fp64 rel {rel:.2e}, max-abs {mx:.2e} RMS")
    for name, a, r in (("out", out, ref), ("grad_x", gx, rgx), ("grad_Y", gY, rgY), ("grad_h", gh, gwp @ W)):
        rel, mx = _stats(a.detach().cpu(), r)
        assert rel <= 1e-5 and mx <= 1e-5, name
    # the output layer's parameter gradients (training only) are fp32 GEMMs summing over the
    # E/2 pairs (hipBLASLt, as for the per-edge layer): norm-wise within 1e-5, single entries
    # within the rounding of a sum of ~2,000 terms
    for name, a, r in (("grad_W", gW, gwp.T @ hp), ("grad_b", gb, gwp.sum(0))):
        rel, mx = _stats(a.detach().cpu(), r)
        assert rel <= 1e-5 and mx <= 1e-4, name


FUSED_CASES = [([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3], 64, 64),  # config 3 products
               ([0], [0, 1, 2, 3], [0, 1, 2, 3], 128, 128),  # config 5 literal, layer 1
               ([0, 1], [0, 1, 2, 3], [0, 1, 2, 3], 128, 128),  # config 5 literal, layer 2
               ([0, 1], [0, 1, 2, 3], [0, 1], 32, 32)]


@pytest.mark.parametrize("in_ls,sh_ls,out_ls,C,Kh", FUSED_CASES)
def test_radial_tp_pairs_fused_input_gradient(in_ls, sh_ls, out_ls, C, Kh):
    """The backward without the per-edge weight gradient in memory (work list of receiver batches,
    molix::tp_weight_grad_batched) against the one that writes and re-reads it: the forward, grad_Y
    bit-identical, grad_x within its atomic order, grad_h within 1e-5 (the same products summed in
    another order); and against the fp64 oracle, pair and edge mode.  Receivers of degree above and
    below 32 (batches that end inside a segment) and an atom without neighbours."""
    n, L = 300, (300 / 0.1) ** (1 / 3)
    p, ei, bond = _system(n, L, seed=7 * C + Kh)
    n += 1  # one more node without edges (no batch)
    pr, (row_ptr, perm, snd) = _pairs(ei, n, bond.norm(dim=-1, keepdim=True))
    assert pr is not None
    deg = (row_ptr[1:] - row_ptr[:-1]).cpu()
    assert deg.max() > 32 and bool((deg % 32 != 0).any()) and deg[-1] == 0
    batches = K.tp_gh_batches(row_ptr)
    E = ei.shape[0]
    cfg = K.tp_config_id(in_ls, sh_ls, out_ls)
    P, NX, NY, NO = K.tp_config_info(cfg)
    rng = np.random.default_rng(C + 3)
    x = rng.normal(size=(n, NX * C)).astype(np.float32)
    Y = torch.ops.molix.spherical_harmonics(bond, max(sh_ls))
    hp = rng.normal(size=(E // 2, Kh)).astype(np.float32)
    W = (rng.normal(size=(P * C, Kh)) / np.sqrt(Kh)).astype(np.float32)
    b = (rng.normal(size=P * C) * 0.1).astype(np.float32)
    g = rng.normal(size=(n, NO * C)).astype(np.float32)
    t = lambda a, rg=False: torch.tensor(a, device=DEV, requires_grad=rg)  # noqa: E731
    wrow = pr.wrow.long()
    res = []
    for bt in (None, batches):
        xt, Yt, ht = t(x, True), Y.detach().clone().requires_grad_(True), t(hp, True)
        out, _ = torch.ops.molix.radial_tp_pairs(xt, Yt, ht, t(W), t(b), row_ptr, perm, snd, pr.wrow, pr.pairs,
                                                 cfg, C, bt)
        res.append((out.detach(),) + torch.autograd.grad(out, (xt, Yt, ht), t(g)))
    (out0, gx0, gY0, gh0), (out1, gx1, gY1, gh1) = res
    assert torch.equal(out0, out1) and torch.equal(gY0, gY1)
    for name, a, r in (("grad_x", gx1, gx0), ("grad_h", gh1, gh0)):
        rel, mx = _stats(a.cpu(), r.cpu())
        print(f"fused grad_h in={in_ls} C={C} K={Kh}: {name} vs unfused rel {rel:.2e}, max-abs {mx:.2e} RMS")
        assert rel <= 1e-5 and mx <= 1e-5, (name, rel, mx)
    # edge mode
    hf = t(hp[wrow.cpu().numpy()], True)
    out3, _ = torch.ops.molix.radial_tp_pairs(t(x), Y.detach(), hf, t(W), t(b), row_ptr, perm, snd, pr.wrow,
                                              pr.pairs, cfg, C, batches)
    (gh3,) = torch.autograd.grad(out3, (hf,), t(g))
    # fp64 oracle (the isolated atom has no edges)
    tp = O.ChannelwiseTP(_irr(in_ls, C), _irr(sh_ls), _irr(out_ls), C)
    ei_np, Y64 = ei.cpu().numpy(), Y.detach().cpu().double().numpy()
    wr = wrow.cpu().numpy()
    w64 = (hp.astype(np.float64) @ W.T.astype(np.float64) + b)[wr]
    _, _, rgw = tp.backward(x.astype(np.float64), Y64, w64, ei_np, g.astype(np.float64))
    gwp = np.zeros((E // 2, P * C))
    np.add.at(gwp, wr, rgw)
    for name, a, r in (("grad_h pair", gh1, gwp @ W), ("grad_h edge", gh3, rgw @ W)):
        rel, mx = _stats(a.detach().cpu(), r)
        print(f"fused grad_h in={in_ls} C={C} K={Kh}: {name} vs fp64 rel {rel:.2e}, max-abs {mx:.2e} RMS")
        assert rel <= 1e-5 and mx <= 1e-5, name


def test_mace_eval_pairs_vs_per_edge_and_oracle(monkeypatch):
    """A frozen MACE (both variants, config-1 sizes) in eval mode takes the paired path; energies
    and forces against the same model per edge and against the fp64 oracle."""
    from oracle import mace_ref
    from oracle import nlist as NL
    from tests.test_gpu_mace import CFG1, CFG1_LITERAL, build, molecules

    real = torch.ops.molix.radial_tp_pairs
    calls = []

    def counting(*a, **k):
        calls.append(1)
        return real(*a, **k)

    monkeypatch.setattr(torch.ops.molix, "radial_tp_pairs", counting)
    for cfg in (CFG1, CFG1_LITERAL):
        pos, Z, batch = molecules()
        ii, jj, _, _ = NL.directed_pairs(pos.astype(np.float32), 5.0, None)
        edge_index = np.stack([jj, ii], 1).astype(np.int64)
        model = build(cfg).eval()
        for prm in model.parameters():
            prm.requires_grad_(False)
        args = (torch.tensor(Z, device=DEV), torch.tensor(pos, dtype=torch.float32, device=DEV),
                torch.tensor(edge_index, device=DEV), torch.tensor(batch, device=DEV), 16)
        calls.clear()
        e, f = model(*args)
        assert len(calls) == cfg["num_interactions"], "the paired path was not taken"
        monkeypatch.setattr(config, "paired_radial", False)
        e2, f2 = model(*args)
        monkeypatch.setattr(config, "paired_radial", True)
        rel_e = ((e - e2).abs().max() / e2.abs().max()).item()
        rel_f, mx_f = _stats(f.detach().cpu(), f2.detach().cpu())
        assert rel_e <= 1e-6 and rel_f <= 1e-6 and mx_f <= 1e-5, (rel_e, rel_f, mx_f)
        # the same with the fused output-layer input gradient (no per-edge weight gradient in memory)
        monkeypatch.setattr(config, "fused_weight_grad", True)
        e3, f3 = model(*args)
        monkeypatch.setattr(config, "fused_weight_grad", False)
        rel_e = ((e3 - e).abs().max() / e.abs().max()).item()
        rel_f, mx_f = _stats(f3.detach().cpu(), f.detach().cpu())
        assert rel_e == 0 and rel_f <= 1e-6 and mx_f <= 1e-5, (rel_e, rel_f, mx_f)
        sd = {k.removeprefix("encoder."): v for k, v in model.state_dict().items()}
        re, rf = mace_ref.energy_forces(sd, cfg, torch.tensor(Z), torch.tensor(pos.astype(np.float32),
                                                                                dtype=torch.float64),
                                        torch.tensor(edge_index), torch.tensor(batch), 16)
        e, f = e.detach().cpu().double(), f.detach().cpu().double()
        rel_e = ((e - re).abs() / re.abs()).max().item()
        rel_f, mx_f = _stats(f, rf)
        print(f"MACE paired ({'literal' if cfg.get('hidden_ls') else 'as coded'}): energy {rel_e:.2e}, "
              f"forces rel {rel_f:.2e} max-abs {mx_f:.2e} RMS")
        assert rel_e <= 1e-5 and rel_f <= 1e-5 and mx_f <= 1e-5
