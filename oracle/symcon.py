"""fp64 restatement of the equivariant symmetric contraction -- TEST INFRASTRUCTURE ONLY.

The reference reaches the MACE product basis through
``cuet.SymmetricContraction`` (src/molrep/interaction/symmetric_contraction.py:94-109,
configured there for scalar channels only; cuequivariance is absent here and its
basis is not reachable).  The product library defines its basis by a documented
recipe; this module rebuilds it from the oracle's own pieces and evaluates the
contraction densely:

* coupling tensors: ``oracle.equivariant.coupling`` (null space of
  D1 (x) D2 (x) D3 - I with Wigner-D fitted from scipy harmonics), any l;
* candidates: for each multiset of input blocks b1 <= .. <= b_nu (sorted) whose
  l's sum to L mod 2 and (nu = 3) each intermediate l12 ascending, the chain
  (l1 (x) l2 -> l12) (x) l3 -> L on slots (b1, b2, b3), averaged over the nu!
  slot permutations, normalised, and signed so that its first entry above
  1e-9 x max is positive;
* basis: Gram-Schmidt over the candidates in that order (residual below 1e-6
  dropped), each vector keeping its candidate's orientation;
* contraction: B[n, L, M, c] = sum_{nu,k} W[z_n, p, c] U_{L,nu,k}[M, i..] A[n, i, c]...
  in torch fp64, per (node, channel) row as the dense products A^{(x) nu} times the
  flattened U (autograd gives the reference gradients).

Pinned by (tests/test_oracle_symcon.py): the number of basis vectors equals the
multiplicity of V_L in Sym^nu(V) from O(3) characters; orthonormality; slot
symmetry; rotation and inversion equivariance of the contraction with the
oracle's Wigner-D; a planted parity mistake fails the inversion check.
"""

from __future__ import annotations

import itertools
from functools import lru_cache

import numpy as np
import torch

from . import equivariant as EQ


def _sym(T):
    nu = T.ndim - 1
    perms = list(itertools.permutations(range(1, nu + 1)))
    return sum(T.transpose(0, *p) for p in perms) / len(perms)


def _sign(v):
    f = v.ravel()
    k = np.flatnonzero(np.abs(f) > 1e-9 * np.abs(f).max())[0]
    return v if f[k] > 0 else -v


@lru_cache(maxsize=None)
def _cpl(l1, l2, l3):
    return EQ.coupling(l1, l2, l3)


def candidates(in_ls, L, nu, parity_rule=True):
    off = np.concatenate([[0], np.cumsum([2 * l + 1 for l in in_ls])]).astype(int)
    n = int(off[-1])
    out = []
    for tup in itertools.combinations_with_replacement(range(len(in_ls)), nu):
        lt = [in_ls[i] for i in tup]
        if parity_rule and (sum(lt) - L) % 2:
            continue
        sl = (slice(None),) + tuple(slice(off[i], off[i + 1]) for i in tup)
        blks = []
        if nu == 1:
            if lt[0] == L:
                blks.append(np.eye(2 * L + 1))
        elif nu == 2:
            if abs(lt[0] - lt[1]) <= L <= lt[0] + lt[1]:
                blks.append(np.moveaxis(_cpl(lt[0], lt[1], L), 2, 0))
        else:
            for l12 in range(abs(lt[0] - lt[1]), lt[0] + lt[1] + 1):
                if abs(l12 - lt[2]) <= L <= l12 + lt[2]:
                    c1, c2 = _cpl(lt[0], lt[1], l12), _cpl(l12, lt[2], L)
                    blk = np.zeros((2 * L + 1, 2 * lt[0] + 1, 2 * lt[1] + 1, 2 * lt[2] + 1))
                    for k in range(2 * l12 + 1):
                        blk += np.moveaxis(c2[k], 1, 0)[:, None, None, :] * c1[:, :, k][None, :, :, None]
                    blks.append(blk)
        for blk in blks:
            T = np.zeros((2 * L + 1,) + (n,) * nu)
            T[sl] = blk
            T = _sym(T)
            nrm = np.linalg.norm(T)
            if nrm > 1e-9:
                out.append(_sign(T / nrm))
    return out


@lru_cache(maxsize=None)
def basis(in_ls: tuple, L: int, nu: int, parity_rule: bool = True) -> np.ndarray:
    n = sum(2 * l + 1 for l in in_ls)
    vecs = []
    for c in candidates(in_ls, L, nu, parity_rule):
        v = c.ravel().copy()
        for _ in range(2):
            for b in vecs:
                v -= (b @ v) * b
        r = np.linalg.norm(v)
        if r > 1e-6:
            vecs.append(v / r)
    if not vecs:
        return np.zeros((0, 2 * L + 1) + (n,) * nu)
    return np.stack(vecs).reshape((len(vecs), 2 * L + 1) + (n,) * nu)


def paths(l_in, l_out, nu_max, parity_rule=True):
    """[(L, nu, U)] in weight order (L asc, nu asc)."""
    ls = tuple(range(l_in + 1))
    out = []
    for L in range(l_out + 1):
        for nu in range(1, nu_max + 1):
            U = basis(ls, L, nu, parity_rule)
            if len(U):
                out.append((L, nu, U))
    return out


def num_paths(l_in, l_out, nu_max):
    return sum(len(U) for _, _, U in paths(l_in, l_out, nu_max))


def contract(A, types, W, l_in, l_out, nu_max, parity_rule=True, chunk=128):
    """A (N, (l_in+1)^2 * C) ir_mul, types (N,), W (S, paths, C) -> (N, (l_out+1)^2 * C) fp64 torch.
    Nodes with types outside [0, S) give zeros.  Evaluated per row (node, channel) as the
    dense products A^{(x) nu} (flattened) times the flattened basis, in node chunks."""
    N = A.shape[0]
    ni = (l_in + 1) ** 2
    C = A.shape[1] // ni
    S = W.shape[0]
    valid = (types >= 0) & (types < S)
    z = torch.where(valid, types, torch.zeros_like(types))
    w_all = W.to(torch.float64)[z] * valid[:, None, None].to(torch.float64)  # (N, P, C)
    parts = paths(l_in, l_out, nu_max, parity_rule)
    mats = [(L, nu, len(U), torch.from_numpy(np.ascontiguousarray(U.reshape(len(U) * (2 * L + 1), -1))))
            for L, nu, U in parts]
    chunks = []
    for n0 in range(0, N, chunk):
        n1 = min(N, n0 + chunk)
        a = A[n0:n1].reshape(n1 - n0, ni, C).to(torch.float64).permute(0, 2, 1).reshape(-1, ni)  # rows (n, c)
        w = w_all[n0:n1]
        feats = {1: a}
        if nu_max >= 2:
            feats[2] = (a[:, :, None] * a[:, None, :]).reshape(a.shape[0], -1)
        if nu_max >= 3:
            feats[3] = (feats[2][:, :, None] * a[:, None, :]).reshape(a.shape[0], -1)
        outs = [a.new_zeros(n1 - n0, C, 2 * L + 1) for L in range(l_out + 1)]
        p = 0
        for L, nu, r, Um in mats:
            t = (feats[nu] @ Um.T).reshape(n1 - n0, C, r, 2 * L + 1)
            outs[L] = outs[L] + (w[:, p:p + r, :].permute(0, 2, 1)[..., None] * t).sum(2)
            p += r
        chunks.append(torch.cat([o.permute(0, 2, 1).reshape(n1 - n0, -1) for o in outs], dim=1))
    if not chunks:
        return A.new_zeros(0, (l_out + 1) ** 2 * C, dtype=torch.float64)
    return torch.cat(chunks, dim=0)


def rotate(A, R, l_max, C):
    """Rotate ir_mul features with blocks 0..l_max (natural parity; det R = -1 adds (-1)^l)."""
    N = A.shape[0]
    det = np.linalg.det(R)
    Rp = R * det
    blocks, off = [], 0
    for l in range(l_max + 1):
        d = 2 * l + 1
        D = torch.from_numpy(EQ.wigner_d(l, Rp) * (det ** l))
        blocks.append(torch.einsum("ab,nbc->nac", D, A[:, off:off + d * C].reshape(N, d, C).to(torch.float64)))
        off += d * C
    return torch.cat([b.reshape(N, -1) for b in blocks], dim=1)


def character_multiplicity(l_in, L, nu, nq=4000):
    """Multiplicity of V_L (parity (-1)^L) in Sym^nu(V), V = sum_{l <= l_in} V_l (parity (-1)^l),
    from O(3) characters: average over SO(3) (class function of the angle theta, weight
    (1 - cos theta) / pi) and over the inversion coset."""
    th = (np.arange(nq) + 0.5) * np.pi / nq

    def chi_l(l, t):
        return sum(np.cos(m * t) for m in range(-l, l + 1))

    def chi_V(t, inv, k=1):
        # character of g^k; inversion^k = inversion^(k mod 2)
        s = -1.0 if (inv and k % 2) else 1.0
        return sum((s ** l) * chi_l(l, k * t) for l in range(l_in + 1))

    def chi_sym(t, inv):
        c1 = chi_V(t, inv, 1)
        if nu == 1:
            return c1
        c2 = chi_V(t, inv, 2)
        if nu == 2:
            return (c1 * c1 + c2) / 2
        c3 = chi_V(t, inv, 3)
        return (c1 ** 3 + 3 * c2 * c1 + 2 * c3) / 6

    wgt = (1 - np.cos(th)) / np.pi * (np.pi / nq)
    tot = 0.0
    for inv in (False, True):
        pL = (-1.0) ** L if inv else 1.0
        tot += 0.5 * np.sum(wgt * chi_sym(th, inv) * pL * chi_l(L, th))
    return tot
