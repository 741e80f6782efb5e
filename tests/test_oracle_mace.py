"""The MACE oracle's own pieces are pinned to the numpy oracle (CPU)."""

import numpy as np
import torch

from oracle import equivariant as EQ
from oracle import mace_ref


def test_torch_harmonics_match_scipy_oracle():
    v = np.random.default_rng(0).normal(size=(100, 3))
    np.testing.assert_allclose(mace_ref.sh_torch(3, torch.tensor(v)).numpy(), EQ.sh(range(4), v), atol=1e-13)


def test_conv_tp_matches_numpy_oracle():
    rng = np.random.default_rng(1)
    C, N, E = 4, 7, 30
    irr = "+".join(f"{C}x{t}" for t in ["0e", "1o", "2e", "3o"])
    tp = EQ.ChannelwiseTP(irr, "0e+1o+2e+3o", "0e+1o+2e+3o", C)
    x, Y, w = rng.normal(size=(N, 16 * C)), rng.normal(size=(E, 16)), rng.normal(size=(E, 23 * C))
    ei = rng.integers(0, N, (E, 2))
    out, _ = mace_ref.conv_tp(torch.tensor(x), torch.tensor(Y), torch.tensor(w), torch.tensor(ei), N, 3, C)
    np.testing.assert_allclose(out.numpy(), tp.forward(x, Y, w, ei, N), atol=1e-11)


def test_linear_block_structure():
    rng = np.random.default_rng(2)
    x = torch.tensor(rng.normal(size=(5, 3 * 1 + 2 * 3)))  # 3x0e + 2x1o
    w = torch.tensor(rng.normal(size=3 * 4 + 2 * 5))
    out = mace_ref.linear(x, w, [(3, 0, 1), (2, 1, -1)], [(4, 0, 1), (5, 1, -1)])
    W0 = w[:12].reshape(3, 4)
    np.testing.assert_allclose(out[:, :4].numpy(), (x[:, :3] @ W0 / np.sqrt(3)).numpy(), atol=1e-12)
    x1 = x[:, 3:].reshape(5, 3, 2)
    W1 = w[12:].reshape(2, 5)
    np.testing.assert_allclose(out[:, 4:].reshape(5, 3, 5).numpy(), (x1 @ W1 / np.sqrt(2)).numpy(), atol=1e-12)


LITERAL = dict(num_elements=3, num_features=4, r_max=5.0, num_bessel=8, l_max=3, num_interactions=2,
               correlation=3, avg_num_neighbors=5.0, cutoff="polynomial", hidden_ls=[0, 1])


def _literal_state_dict(cfg, seed=0):
    from molnex_amd.molrep.embedding import DiscreteEmbeddingSpec
    from molnex_amd.molpot.heads import AtomicEnergyMLP
    from molnex_amd.molzoo import MACE

    torch.manual_seed(seed)
    F = cfg["num_features"]
    enc = MACE(node_attr_specs=[DiscreteEmbeddingSpec(input_key="Z", num_classes=cfg["num_elements"], emb_dim=F)],
               num_elements=cfg["num_elements"], num_features=F, r_max=cfg["r_max"], num_bessel=cfg["num_bessel"],
               l_max=cfg["l_max"], num_interactions=cfg["num_interactions"], correlation=cfg["correlation"],
               avg_num_neighbors=cfg["avg_num_neighbors"], cutoff="polynomial", hidden_irreps=f"{F}x0e+{F}x1o")
    sd = dict(enc.state_dict())
    sd.update({f"energy.{k}": v for k, v in AtomicEnergyMLP(hidden_dim=F).state_dict().items()})
    return sd


def test_literal_mace_oracle_is_rotation_and_inversion_invariant():
    """The literal configuration is O(3)-invariant by construction: the fp64 oracle's
    energies must not change under a rotation or an inversion of the positions, and its
    forces must rotate with them."""
    rng = np.random.default_rng(3)
    sd = _literal_state_dict(LITERAL)
    pos = rng.uniform(0, 4.0, (7, 3))
    Z = torch.tensor(rng.integers(0, 3, 7))
    ii, jj = np.nonzero((np.linalg.norm(pos[:, None] - pos[None], axis=-1) < 5.0) & ~np.eye(7, dtype=bool))
    ei = torch.tensor(np.stack([jj, ii], 1))
    batch = torch.zeros(7, dtype=torch.int64)
    e0, f0 = mace_ref.energy_forces(sd, LITERAL, Z, torch.tensor(pos), ei, batch, 1)
    R = EQ.random_rotation(np.random.default_rng(4))
    for Rg in (R, -R):
        e1, f1 = mace_ref.energy_forces(sd, LITERAL, Z, torch.tensor(pos @ Rg.T), ei, batch, 1)
        assert abs(e1.item() - e0.item()) <= 1e-10 * max(1.0, abs(e0.item()))
        np.testing.assert_allclose(f1.numpy(), f0.numpy() @ Rg.T, atol=1e-9)
    assert f0.abs().max() > 1e-6
