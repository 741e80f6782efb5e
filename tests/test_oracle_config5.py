"""Pins of the fp64 config-5 composition (oracle.config5_ref) and of the as-coded MACE oracle,
on the CPU: forces are the exact negative gradient of the energy (central differences),
energies are invariant under translations, atom relabelling and wrapping an atom into another
periodic image (which checks the sign of the image shifts), and a planted sign mistake in the
shifts breaks that last invariance."""

import numpy as np
import pytest
import torch

from oracle import config5_ref, mace_ref
from oracle import nlist as NL

RC = 5.0


def _sd(cfg, seed=0):
    from molnex_amd.molpot import ChargeHead
    from molnex_amd.molpot.heads import AtomicEnergyMLP
    from molnex_amd.molrep.embedding import DiscreteEmbeddingSpec
    from molnex_amd.molzoo import MACE

    torch.manual_seed(seed)
    F = cfg["num_features"]
    literal = cfg.get("hidden_ls") is not None
    enc = MACE(node_attr_specs=[DiscreteEmbeddingSpec(input_key="Z", num_classes=3, emb_dim=F)], num_elements=3,
               num_features=F, r_max=RC, num_bessel=8, l_max=cfg["l_max"], num_interactions=2, correlation=3,
               avg_num_neighbors=cfg["avg_num_neighbors"], cutoff=cfg.get("cutoff", "cosine"),
               hidden_irreps=f"{F}x0e+{F}x1o" if literal else None)
    sd = dict(enc.state_dict())
    sd.update({f"energy.{k}": v for k, v in AtomicEnergyMLP(hidden_dim=F).state_dict().items()})
    return sd, ChargeHead(F, hidden_dim=8).state_dict()


AS_CODED = dict(num_features=4, num_interactions=2, l_max=2, correlation=3, r_max=RC, num_bessel=8,
                avg_num_neighbors=6.0)
LITERAL = dict(AS_CODED, l_max=3, cutoff="polynomial", hidden_ls=[0, 1])


def _periodic(n=24, L=11.0, seed=0):
    rng = np.random.default_rng(seed)
    while True:
        pos = rng.uniform(0, L, (n, 3))
        d = pos[:, None] - pos[None]
        d -= L * np.rint(d / L)
        r = np.linalg.norm(d, axis=-1) + np.eye(n) * 10
        if r.min() > 1.2:
            return pos, L


def _lists(pos, L):
    """Directed edges [source, target] + shifts and the half list + shifts, from the NL oracle."""
    box = np.eye(3) * L
    i, j, d, _ = NL.directed_pairs(pos, RC, box)
    sh = L * np.rint((pos[i] - pos[j] - d) / L)
    r, c, hd, _ = NL.half_pairs(pos, RC, box)
    hsh = L * np.rint((pos[r] - pos[c] - hd) / L)
    return np.stack([j, i], 1).astype(np.int64), sh, (r, c, hsh)


def _energy_forces(sd, sdq, cfg, Z, pos, L, lists=None):
    ei, sh, half = lists if lists is not None else _lists(pos, L)
    n = len(Z)
    return config5_ref.energy_forces(sd, sdq, cfg, torch.tensor(Z), torch.tensor(pos), torch.tensor(ei), sh,
                                     torch.zeros(n, dtype=torch.long), 1, np.eye(3) * L, half, (16, 16, 16), 6,
                                     0.3, 14.399645478425668)


@pytest.mark.parametrize("cfg", [AS_CODED, LITERAL], ids=["as_coded", "literal"])
def test_config5_oracle_forces_are_energy_gradient(cfg):
    pos, L = _periodic()
    Z = np.random.default_rng(1).integers(0, 3, len(pos))
    sd, sdq = _sd(cfg)
    lists = _lists(pos, L)
    e, f, q, e_mace, e_pme = _energy_forces(sd, sdq, cfg, Z, pos, L, lists)
    assert abs(q.sum().item()) < 1e-12 and abs(e_pme.item()) > 1e-6 and f.abs().max() > 1e-4
    h = 1e-5
    rng = np.random.default_rng(2)
    for a in rng.choice(len(pos), 4, replace=False):
        for ax in range(3):
            vals = []
            for s in (1, -1):
                p = pos.copy()
                p[a, ax] += s * h
                vals.append(_energy_forces(sd, sdq, cfg, Z, p, L, lists)[0].sum().item())
            fd = -(vals[0] - vals[1]) / (2 * h)
            assert abs(fd - f[a, ax].item()) <= 1e-6 * max(1.0, f.abs().max().item()), (a, ax, fd, f[a, ax].item())


@pytest.mark.parametrize("cfg", [AS_CODED, LITERAL], ids=["as_coded", "literal"])
def test_config5_oracle_translation_permutation_and_image_invariance(cfg):
    pos, L = _periodic(seed=3)
    Z = np.random.default_rng(4).integers(0, 3, len(pos))
    sd, sdq = _sd(cfg, seed=1)
    e0, f0, *_ = _energy_forces(sd, sdq, cfg, Z, pos, L)
    # translation by a vector that is not a lattice or mesh vector (PME's mesh breaks exact
    # translation invariance at its discretisation error: compare the MACE part tightly)
    t = np.array([0.31, -0.77, 1.13])
    e1, f1, _, em1, _ = _energy_forces(sd, sdq, cfg, Z, pos + t, L)
    _, _, _, em0, _ = _energy_forces(sd, sdq, cfg, Z, pos, L)
    assert abs(em1.item() - em0.item()) <= 1e-10 * abs(em0.item())
    assert abs(e1.item() - e0.item()) <= 1e-4 * abs(e0.item())
    # relabelling atoms
    perm = np.random.default_rng(5).permutation(len(Z))
    e2, f2, *_ = _energy_forces(sd, sdq, cfg, Z[perm], pos[perm], L)
    assert abs(e2.item() - e0.item()) <= 1e-10 * abs(e0.item())
    np.testing.assert_allclose(f2.numpy(), f0.numpy()[perm], atol=1e-9)
    # wrapping atom 0 into the next periodic image: a new list with shifts of the opposite image
    p3 = pos.copy()
    p3[0] += np.array([L, 0.0, -L])
    e3, f3, *_ = _energy_forces(sd, sdq, cfg, Z, p3, L)
    assert abs(e3.item() - e0.item()) <= 1e-9 * abs(e0.item())
    np.testing.assert_allclose(f3.numpy(), f0.numpy(), atol=1e-8)


def test_planted_shift_sign_breaks_image_invariance():
    """bond = pos[target] - pos[source] + shift (a sign mistake) must change the energy of a
    wrapped configuration: the image check above can fail."""
    cfg = AS_CODED
    pos, L = _periodic(seed=3)
    Z = np.random.default_rng(4).integers(0, 3, len(pos))
    sd, _ = _sd(cfg, seed=1)
    t = mace_ref._f64(sd)
    batch = torch.zeros(len(Z), dtype=torch.long)

    def energy(p, flip):
        ei, sh, _ = _lists(p, L)
        sh = -sh if flip else sh
        return mace_ref._readout(t, mace_ref.mace_layers(t, cfg, torch.tensor(Z), torch.tensor(p), torch.tensor(ei),
                                                         torch.tensor(sh)), batch, 1).item()

    p3 = pos.copy()
    p3[0] += np.array([L, 0.0, -L])
    assert abs(energy(p3, False) - energy(pos, False)) <= 1e-9 * abs(energy(pos, False))
    assert abs(energy(p3, True) - energy(pos, True)) > 1e-5 * abs(energy(pos, True))
