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
