"""Symmetric product basis of the MACE contraction (general equivariant case).

For node features A with irreps V = 0e + 1o + ... (one block per l, natural
parity, ``C`` channels) the contraction of correlation order nu maps, per
channel, the symmetric power Sym^nu(V) to an output irrep L:

    B[L, M] = sum_k W[z, L, nu, k] sum_{i1..inu} U_{L,nu,k}[M, i1..inu] A[i1] ... A[inu]

(MACE's product basis, Batatia et al. 2022, eq. 10; the reference reaches it
through cuequivariance's SymmetricContraction, which it only ever configures for
scalar channels, src/molrep/interaction/symmetric_contraction.py:90-109).
Here the basis U_{L,nu,k} is constructed as follows: every coupling chain
(l1 (x) l2 -> l12) (x) l3 -> L over all intermediate l12 (both parities) is
written out as a tensor over V^{(x)nu}, symmetrised over the nu slots and
sign-canonicalised, and the chains are orthonormalised by Gram-Schmidt in a
fixed order (``candidates``), which makes the basis unique; parity restricts the
chains to l1 + ... + l_nu = L mod 2.  Each U_k is then stored on sorted index
tuples (monomials) with the permutation multiplicity folded in.
"""

from __future__ import annotations

import itertools
import math
from functools import lru_cache

import numpy as np

from .irreps import coupling, sh_block

_EPS = 1e-10


def _real_sh_any(l: int, u: np.ndarray) -> np.ndarray:
    """Real harmonics of any degree (component normalisation) for unit vectors; l <= 3
    uses the closed forms of ``irreps.sh_block`` so the bases agree."""
    if l <= 3:
        return sh_block(l, u)
    x, y, z = u[..., 0], u[..., 1], u[..., 2]
    phi = np.arctan2(y, x)
    ct = np.clip(z, -1.0, 1.0)
    st = np.sqrt(np.maximum(0.0, 1 - ct * ct))
    # associated Legendre P_l^m (no Condon-Shortley phase) by the standard recursions
    P = {}
    for m in range(l + 1):
        pmm = np.ones_like(ct)
        for k in range(1, m + 1):
            pmm = pmm * (2 * k - 1) * st
        P[(m, m)] = pmm
        if m + 1 <= l:
            P[(m + 1, m)] = (2 * m + 1) * ct * pmm
        for ll in range(m + 2, l + 1):
            P[(ll, m)] = ((2 * ll - 1) * ct * P[(ll - 1, m)] - (ll + m - 1) * P[(ll - 2, m)]) / (ll - m)
    cols = []
    for m in range(-l, l + 1):
        am = abs(m)
        norm = math.sqrt((2 * l + 1) * math.factorial(l - am) / math.factorial(l + am))
        if m == 0:
            cols.append(norm * P[(l, 0)])
        elif m > 0:
            cols.append(math.sqrt(2) * norm * P[(l, am)] * np.cos(am * phi))
        else:
            cols.append(math.sqrt(2) * norm * P[(l, am)] * np.sin(am * phi))
    return np.stack(cols, axis=-1)


def _rotation(rng) -> np.ndarray:
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([[a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
                     [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
                     [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d]])


@lru_cache(maxsize=None)
def wigner_d(l: int, key: int) -> np.ndarray:
    """D^l of the key-th fixed pseudo-random rotation (Y^l(R u) = D Y^l(u))."""
    R = _rotation(np.random.default_rng(1000 + key))
    U = np.random.default_rng(77).normal(size=(4 * (2 * l + 1) + 8, 3))
    U /= np.linalg.norm(U, axis=1, keepdims=True)
    Dt, *_ = np.linalg.lstsq(_real_sh_any(l, U), _real_sh_any(l, U @ R.T), rcond=None)
    return Dt.T


@lru_cache(maxsize=None)
def coupling_any(l1: int, l2: int, l3: int) -> np.ndarray:
    """Unit-norm SO(3)-invariant tensor of l1 (x) l2 (x) l3 for any l (odd sums included)."""
    if max(l1, l2, l3) <= 3 and (l1 + l2 + l3) % 2 == 0:
        return coupling(l1, l2, l3)
    if not abs(l1 - l2) <= l3 <= l1 + l2:
        return np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    blocks = []
    for key in range(3):
        K = np.kron(np.kron(wigner_d(l1, key), wigner_d(l2, key)), wigner_d(l3, key))
        blocks.append(K - np.eye(K.shape[0]))
    _, s, vt = np.linalg.svd(np.concatenate(blocks))
    c = vt[-1].reshape(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1)
    c /= np.linalg.norm(c)
    flat = c.ravel()
    return c * np.sign(flat[np.argmax(np.abs(flat) > 1e-8)])


def _sym(T: np.ndarray) -> np.ndarray:
    nu = T.ndim - 1
    perms = list(itertools.permutations(range(1, nu + 1)))
    return sum(T.transpose(0, *p) for p in perms) / len(perms)


def _canonical_sign(v: np.ndarray) -> np.ndarray:
    """Flip ``v`` so that its first entry (C order) above 1e-9 x max |v| is positive."""
    flat = v.ravel()
    big = np.flatnonzero(np.abs(flat) > 1e-9 * np.abs(flat).max())
    return v if flat[big[0]] > 0 else -v


def candidates(in_ls: tuple, L: int, nu: int):
    """Coupling chains in construction order, each symmetrised over the nu slots and
    sign-canonicalised: for every multiset of input blocks b1 <= ... <= b_nu with
    l_b1 + ... + l_bnu = L (mod 2), and (nu = 3) every intermediate l12 ascending,
    the chain (l_b1 (x) l_b2 -> l12) (x) l_b3 -> L placed on slots (b1, b2, b3)."""
    off = np.cumsum([0] + [2 * l + 1 for l in in_ls])
    n = int(off[-1])
    out = []
    for tup in itertools.combinations_with_replacement(range(len(in_ls)), nu):
        lt = [in_ls[i] for i in tup]
        if (sum(lt) - L) % 2:
            continue
        sl = (slice(None),) + tuple(slice(off[i], off[i + 1]) for i in tup)
        blocks = []
        if nu == 1:
            if lt[0] == L:
                blocks.append(np.eye(2 * L + 1))
        elif nu == 2:
            if abs(lt[0] - lt[1]) <= L <= lt[0] + lt[1]:
                blocks.append(coupling_any(lt[0], lt[1], L).transpose(2, 0, 1))
        elif nu == 3:
            for l12 in range(abs(lt[0] - lt[1]), lt[0] + lt[1] + 1):
                if abs(l12 - lt[2]) <= L <= l12 + lt[2]:
                    blocks.append(np.einsum("abk,kcM->Mabc", coupling_any(lt[0], lt[1], l12),
                                            coupling_any(l12, lt[2], L)))
        else:
            raise ValueError("correlation order must be 1, 2 or 3")
        for blk in blocks:
            T = np.zeros((2 * L + 1,) + (n,) * nu)
            T[sl] = blk
            T = _sym(T)
            nrm = np.linalg.norm(T)
            if nrm > 1e-9:
                out.append(_canonical_sign(T / nrm))
    return out


@lru_cache(maxsize=None)
def product_basis(in_ls: tuple, L: int, nu: int) -> np.ndarray:
    """Orthonormal basis (r, 2L+1, n, ..., n) of the symmetric equivariant maps
    Sym^nu(V) -> V_L: Gram-Schmidt over ``candidates`` in order, a candidate whose
    residual norm is below 1e-6 being dependent and skipped; each basis vector keeps
    the orientation of its candidate (positive overlap)."""
    n = sum(2 * l + 1 for l in in_ls)
    basis = []
    for c in candidates(tuple(in_ls), L, nu):
        v = c.ravel().copy()
        for b in basis:
            v -= (b @ v) * b
        for b in basis:  # second pass (classical Gram-Schmidt twice is orthogonal to fp64)
            v -= (b @ v) * b
        r = np.linalg.norm(v)
        if r > 1e-6:
            basis.append(v / r)
    if not basis:
        return np.zeros((0, 2 * L + 1) + (n,) * nu)
    B = np.stack(basis).reshape((len(basis), 2 * L + 1) + (n,) * nu)
    B[np.abs(B) < _EPS] = 0.0
    return B


@lru_cache(maxsize=None)
def monomial_table(in_ls: tuple, L: int, nu: int):
    """(monomials, coef): sorted index tuples in the support and coef[k, M, q] =
    U_k[M, tuple_q] x (number of distinct orderings of tuple_q)."""
    B = product_basis(in_ls, L, nu)
    n = sum(2 * l + 1 for l in in_ls)
    monos, cols = [], []
    for tup in itertools.combinations_with_replacement(range(n), nu):
        v = B[(slice(None), slice(None)) + tup]
        if np.abs(v).max(initial=0.0) > _EPS:
            mult = math.factorial(nu)
            for c in set(tup):
                mult //= math.factorial(tup.count(c))
            monos.append(tup)
            cols.append(v * mult)
    coef = np.stack(cols, axis=-1) if cols else np.zeros((B.shape[0], 2 * L + 1, 0))
    return monos, coef


class ProductBasisDescriptor:
    """Everything a contraction of correlation <= nu_max from V = in_ls to out_Ls needs."""

    def __init__(self, in_ls, out_ls, nu_max: int):
        self.in_ls, self.out_ls, self.nu_max = tuple(in_ls), tuple(out_ls), nu_max
        self.n = sum(2 * l + 1 for l in self.in_ls)
        self.parts = []  # (L, nu, num_paths, monomials, coef)
        for L in self.out_ls:
            for nu in range(1, nu_max + 1):
                monos, coef = monomial_table(self.in_ls, L, nu)
                if coef.shape[0]:
                    self.parts.append((L, nu, coef.shape[0], monos, coef))
        self.num_paths = sum(p[2] for p in self.parts)
        self.out_dim = sum(2 * L + 1 for L in self.out_ls)
