"""The equivariant symmetric-contraction oracle and the product basis, on the CPU.

Pins (none of them retypes the construction): basis sizes against O(3)
character multiplicities; orthonormality and slot symmetry; rotation and
inversion equivariance of the dense contraction with the oracle's Wigner-D;
a planted parity mistake must fail the inversion check; the product's
monomial tables (what the HIP kernels are generated from) reproduce the dense
oracle on random inputs.
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import equivariant as EQ
from oracle import symcon as O

CONFIGS = [(li, lo, nu) for li in (1, 2, 3) for lo in (0, 1) for nu in (1, 2, 3)]


@pytest.mark.parametrize("l_in,L,nu", [(li, L, nu) for li in (1, 2, 3) for L in (0, 1) for nu in (1, 2, 3)])
def test_basis_size_matches_characters(l_in, L, nu):
    B = O.basis(tuple(range(l_in + 1)), L, nu)
    assert len(B) == round(O.character_multiplicity(l_in, L, nu))
    assert abs(O.character_multiplicity(l_in, L, nu) - len(B)) < 1e-6


def test_known_multiplicities():
    # Sym^2(0e+1o) -> 0e: x0^2 and |x1|^2; Sym^3 -> 0e: x0^3, x0 |x1|^2; Sym^2 -> 1o: x0 x1
    assert len(O.basis((0, 1), 0, 2)) == 2
    assert len(O.basis((0, 1), 0, 3)) == 2
    assert len(O.basis((0, 1), 1, 2)) == 1
    assert len(O.basis((0, 1), 1, 3)) == 2  # x0^2 x1, |x1|^2 x1


@pytest.mark.parametrize("l_in,L,nu", [(3, 0, 3), (3, 1, 3), (2, 1, 2)])
def test_basis_orthonormal_and_symmetric(l_in, L, nu):
    B = O.basis(tuple(range(l_in + 1)), L, nu)
    F = B.reshape(len(B), -1)
    assert np.abs(F @ F.T - np.eye(len(B))).max() < 1e-12
    for p in itertools.permutations(range(2, 2 + nu)):
        assert np.abs(B.transpose(0, 1, *p) - B).max() < 1e-12


def _case(l_in, l_out, nu, N=6, C=3, S=3, seed=0):
    rng = np.random.default_rng(seed)
    A = torch.from_numpy(rng.normal(size=(N, (l_in + 1) ** 2 * C)))
    z = torch.from_numpy(rng.integers(0, S, N))
    W = torch.from_numpy(rng.normal(size=(S, O.num_paths(l_in, l_out, nu), C)))
    return A, z, W


@pytest.mark.parametrize("l_in,l_out,nu", [(3, 1, 3), (2, 1, 2), (1, 1, 3)])
@pytest.mark.parametrize("improper", [False, True])
def test_contraction_equivariance(l_in, l_out, nu, improper):
    A, z, W = _case(l_in, l_out, nu)
    R = EQ.random_rotation(np.random.default_rng(5))
    if improper:
        R = -R
    C = W.shape[-1]
    out = O.contract(A, z, W, l_in, l_out, nu)
    out_rot = O.contract(O.rotate(A, R, l_in, C), z, W, l_in, l_out, nu)
    assert torch.allclose(out_rot, O.rotate(out, R, l_out, C), atol=1e-10)
    assert out.abs().max() > 1e-3


def test_planted_parity_mistake_fails_inversion():
    # dropping the parity rule admits pseudo-vector maps (e.g. (1 x 1 -> 2) x 2 -> 1): still
    # rotation-equivariant, but wrong under inversion -- the check above must see it
    l_in, l_out, nu = 2, 1, 3
    ls = (0, 1, 2)
    assert len(O.basis(ls, 1, 3, parity_rule=False)) > len(O.basis(ls, 1, 3))
    rng = np.random.default_rng(1)
    C, S = 2, 1
    P = sum(len(U) for _, _, U in O.paths(l_in, l_out, nu, parity_rule=False))
    A = torch.from_numpy(rng.normal(size=(4, 9 * C)))
    z = torch.zeros(4, dtype=torch.int64)
    W = torch.from_numpy(rng.normal(size=(S, P, C)))
    Rp = EQ.random_rotation(np.random.default_rng(2))
    for R, should_hold in ((Rp, True), (-Rp, False)):
        out = O.contract(A, z, W, l_in, l_out, nu, parity_rule=False)
        out_rot = O.contract(O.rotate(A, R, l_in, C), z, W, l_in, l_out, nu, parity_rule=False)
        ok = torch.allclose(out_rot, O.rotate(out, R, l_out, C), atol=1e-8)
        assert ok == should_hold


def test_invalid_types_give_zero():
    A, z, W = _case(2, 1, 2)
    z[1] = -1
    z[3] = W.shape[0]
    out = O.contract(A, z, W, 2, 1, 2)
    assert out[1].abs().max() == 0 and out[3].abs().max() == 0 and out[0].abs().max() > 0


@pytest.mark.parametrize("l_in,l_out,nu", CONFIGS)
def test_product_basis_and_monomial_tables_match_oracle(l_in, l_out, nu):
    """The product's basis equals the oracle's, and its monomial tables (the generator's
    input) evaluate to the dense oracle contraction."""
    from molnex_amd.symmetric import ProductBasisDescriptor, product_basis

    ls = tuple(range(l_in + 1))
    for L in range(l_out + 1):
        for k in range(1, nu + 1):
            assert np.abs(product_basis(ls, L, k) - O.basis(ls, L, k)).max() < 1e-10
    desc = ProductBasisDescriptor(ls, tuple(range(l_out + 1)), nu)
    assert desc.num_paths == O.num_paths(l_in, l_out, nu)
    A, z, W = _case(l_in, l_out, nu, N=5, C=2, S=2, seed=3)
    N, C = A.shape[0], W.shape[-1]
    a = A.reshape(N, -1, C).numpy()
    w = W.numpy()[z.numpy()]
    out = np.zeros((N, (l_out + 1) ** 2, C))
    p = 0
    for L, _, r, monos, coef in desc.parts:
        for qi, mono in enumerate(monos):
            m = np.prod([a[:, i, :] for i in mono], axis=0)  # (N, C)
            out[:, L * L:(L + 1) ** 2, :] += np.einsum("kM,nkc,nc->nMc", coef[:, :, qi], w[:, p:p + r, :], m)
        p += r
    ref = O.contract(A, z, W, l_in, l_out, nu).numpy().reshape(N, -1, C)
    assert np.abs(out - ref).max() < 1e-10 * max(1.0, np.abs(ref).max())
