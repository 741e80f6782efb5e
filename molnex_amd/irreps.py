"""Irreps bookkeeping, real spherical-harmonic basis and real Clebsch-Gordan tables.

The reference delegates these conventions to the third-party ``cuequivariance``
package (``src/molrep/embedding/angular.py:89``,
``src/molrep/interaction/tensor_product.py:72-79``), which is not vendored.  This
module fixes one self-consistent set of conventions, computed in float64 NumPy
at import time:

* Irreps strings follow the O3 syntax used by the reference
  (``"32x0e + 32x1o"``); feature vectors use the ``ir_mul`` layout, i.e. every
  ``mul x ir`` block is stored ``[m][channel]``
  (``src/molrep/utils/equivariance.py:124-135``).
* Real spherical harmonics use "component" normalisation
  (``Y^0 = 1``, ``|Y^l|^2 = 2l+1`` on the unit sphere).  The ``l = 1`` block is
  ``sqrt(3) * (x, y, z)`` so that it rotates with the rotation matrix itself,
  as the reference tests assume
  (``tests/test_molrep/test_interaction/test_tensor_product.py:124-176``).
  Blocks ``l = 2, 3`` use the textbook real harmonics ordered ``m = -l..l``.
* The real coupling tensor for ``(l1, l2, l3)`` is the Gaunt integral
  ``G[m1,m2,m3] = ∫ Y1 Y2 Y3 dΩ`` rescaled to unit Frobenius norm.  It is the
  unique (up to sign) invariant tensor of the triple; the Gaunt form fixes the
  sign so that ``Σ G Y1(u) Y2(u) Y3(u) > 0``.
* A channelwise tensor-product path ``(l1, l2 -> l3)`` uses the coefficient
  ``sqrt(2 l3 + 1) * C`` ("component" path normalisation: unit-variance inputs
  give unit-variance outputs per path).
"""

from __future__ import annotations

import math
import re
from dataclasses import dataclass
from functools import lru_cache

import numpy as np

L_MAX_SUPPORTED = 3


# ---------------------------------------------------------------------------
# Irreps strings
# ---------------------------------------------------------------------------


@dataclass(frozen=True, order=True)
class Irrep:
    """One O3 irrep: angular momentum ``l`` and parity ``p`` (+1 even, -1 odd)."""

    l: int
    p: int

    @property
    def dim(self) -> int:
        return 2 * self.l + 1

    def __str__(self) -> str:
        return f"{self.l}{'e' if self.p == 1 else 'o'}"

    def sort_key(self) -> tuple[int, int]:
        # natural parity (-1)^l first, as O3 irreps are conventionally ordered
        return (self.l, 0 if self.p == (-1) ** self.l else 1)


@dataclass(frozen=True)
class MulIrrep:
    mul: int
    ir: Irrep

    @property
    def dim(self) -> int:
        return self.mul * self.ir.dim

    def __str__(self) -> str:
        return f"{self.mul}x{self.ir}"


_TOKEN = re.compile(r"^\s*(?:(\d+)\s*x\s*)?(\d+)\s*([eo])\s*$")


class Irreps(tuple):
    """Ordered direct sum of ``MulIrrep`` blocks, parsed from an O3 string."""

    def __new__(cls, spec="") -> "Irreps":
        if isinstance(spec, Irreps):
            return spec
        items: list[MulIrrep] = []
        if isinstance(spec, str):
            for tok in (t for t in spec.split("+") if t.strip()):
                m = _TOKEN.match(tok)
                if m is None:
                    raise ValueError(f"invalid irreps token {tok!r} in {spec!r}")
                mul = int(m.group(1)) if m.group(1) is not None else 1
                items.append(MulIrrep(mul, Irrep(int(m.group(2)), 1 if m.group(3) == "e" else -1)))
        else:
            for it in spec:
                if isinstance(it, MulIrrep):
                    items.append(it)
                else:
                    mul, ir = it
                    items.append(MulIrrep(int(mul), ir))
        return super().__new__(cls, items)

    @property
    def dim(self) -> int:
        return sum(b.dim for b in self)

    @property
    def num_irreps(self) -> int:
        return sum(b.mul for b in self)

    def offsets(self) -> list[int]:
        out, o = [], 0
        for b in self:
            out.append(o)
            o += b.dim
        return out

    def __str__(self) -> str:
        return " + ".join(str(b) for b in self)

    def __repr__(self) -> str:
        return f"Irreps({str(self)!r})"


# ---------------------------------------------------------------------------
# Real spherical harmonics (component normalisation), l <= 3
# ---------------------------------------------------------------------------

_S3 = math.sqrt(3.0)
_S5 = math.sqrt(5.0)
_S7 = math.sqrt(7.0)
_S15 = math.sqrt(15.0)
_S105 = math.sqrt(105.0)
_S35_8 = math.sqrt(35.0 / 8.0)
_S21_8 = math.sqrt(21.0 / 8.0)


def sh_block(l: int, u: np.ndarray) -> np.ndarray:
    """Real harmonics of degree ``l`` for unit vectors ``u`` (..., 3) -> (..., 2l+1).

    Written as homogeneous polynomials, so a zero vector maps to zero for l >= 1.
    """
    x, y, z = u[..., 0], u[..., 1], u[..., 2]
    if l == 0:
        return np.ones(u.shape[:-1] + (1,))
    if l == 1:
        return np.stack([_S3 * x, _S3 * y, _S3 * z], axis=-1)
    if l == 2:
        return np.stack(
            [
                _S15 * x * y,
                _S15 * y * z,
                0.5 * _S5 * (2 * z * z - x * x - y * y),
                _S15 * x * z,
                0.5 * _S15 * (x * x - y * y),
            ],
            axis=-1,
        )
    if l == 3:
        r2 = x * x + y * y + z * z
        return np.stack(
            [
                _S35_8 * y * (3 * x * x - y * y),
                _S105 * x * y * z,
                _S21_8 * y * (5 * z * z - r2),
                0.5 * _S7 * z * (5 * z * z - 3 * r2),
                _S21_8 * x * (5 * z * z - r2),
                0.5 * _S105 * z * (x * x - y * y),
                _S35_8 * x * (x * x - 3 * y * y),
            ],
            axis=-1,
        )
    raise ValueError(f"l={l} not supported (l <= {L_MAX_SUPPORTED})")


def spherical_harmonics(ls, vec: np.ndarray, normalize: bool = True) -> np.ndarray:
    """Concatenated real harmonics ``[Y^l for l in ls]`` of vectors (..., 3)."""
    v = np.asarray(vec, dtype=np.float64)
    if normalize:
        r = np.linalg.norm(v, axis=-1, keepdims=True)
        v = np.where(r > 0, v / np.where(r > 0, r, 1.0), 0.0)
    return np.concatenate([sh_block(l, v) for l in ls], axis=-1)


# ---------------------------------------------------------------------------
# Real coupling tensors from the Gaunt integral
# ---------------------------------------------------------------------------


@lru_cache(maxsize=None)
def _sphere_quadrature():
    # Gauss-Legendre in cos(theta) x uniform phi; exact for polynomial degree <= 11
    t, wt = np.polynomial.legendre.leggauss(8)
    nphi = 24
    phi = 2 * np.pi * np.arange(nphi) / nphi
    st = np.sqrt(1 - t * t)
    pts = np.stack(
        [
            (st[:, None] * np.cos(phi)[None, :]).ravel(),
            (st[:, None] * np.sin(phi)[None, :]).ravel(),
            np.repeat(t, nphi),
        ],
        axis=-1,
    )
    w = np.repeat(wt, nphi) * (2 * np.pi / nphi)
    return pts, w


@lru_cache(maxsize=None)
def _so3_quadrature():
    """Rotations and weights (summing to 1) integrating polynomials of degree <= 9 in the entries
    of R over SO(3) with the Haar measure: R = Rz(a) Ry(b) Rz(c), a and c on uniform 20-point
    grids (exact for trigonometric degree < 20), b by 24-point Gauss-Legendre on [0, pi] with the
    sin(b) density (an entire integrand of trigonometric degree <= 10: error at round-off)."""
    n = 20
    ang = 2 * np.pi * np.arange(n) / n
    t, wt = np.polynomial.legendre.leggauss(24)
    b = 0.5 * np.pi * (t + 1)
    wb = wt * 0.25 * np.pi * np.sin(b)  # sums to 1 over [0, pi]
    A, B, Cg = (g.ravel() for g in np.meshgrid(ang, b, ang, indexing="ij"))
    W = np.repeat(wb[None, :, None], n, 0).repeat(n, 2).ravel() / (n * n)

    def rz(a):
        c, s = np.cos(a), np.sin(a)
        o, z = np.ones_like(a), np.zeros_like(a)
        return np.stack([np.stack([c, -s, z], -1), np.stack([s, c, z], -1), np.stack([z, z, o], -1)], -2)

    def ry(a):
        c, s = np.cos(a), np.sin(a)
        o, z = np.ones_like(a), np.zeros_like(a)
        return np.stack([np.stack([c, z, s], -1), np.stack([z, o, z], -1), np.stack([-s, z, c], -1)], -2)

    return rz(A) @ ry(B) @ rz(Cg), W


# probe directions of the odd-triple construction (any three non-coplanar unit vectors)
_ODD_PROBES = (np.array([0.3, -0.5, 0.8]), np.array([-0.7, 0.2, 0.4]), np.array([0.1, 0.9, -0.3]))


def _odd_coupling(l1: int, l2: int, l3: int) -> np.ndarray:
    """Invariant tensor of a triple with odd ``l1 + l2 + l3`` (where the Gaunt integral vanishes,
    e.g. the cross product of 1 x 1 -> 1): the Haar average of ``Y1(R u) Y2(R v) Y3(R w)`` over
    SO(3) for three fixed directions, i.e. the projection of ``Y1(u) Y2(v) Y3(w)`` onto the
    one-dimensional invariant subspace, rescaled to unit norm, with the sign that makes its first
    entry (C order) above 1e-9 x max positive."""
    R, W = _so3_quadrature()
    u, v, w = (d / np.linalg.norm(d) for d in _ODD_PROBES)
    g = np.einsum("k,ka,kb,kc->abc", W, sh_block(l1, R @ u), sh_block(l2, R @ v), sh_block(l3, R @ w))
    nrm = np.linalg.norm(g)
    if nrm < 1e-8:
        raise RuntimeError(f"no invariant found for ({l1}, {l2}, {l3})")
    g /= nrm
    g[np.abs(g) < 1e-13] = 0.0
    flat = g.ravel()
    first = flat[np.flatnonzero(np.abs(flat) > 1e-9 * np.abs(flat).max())[0]]
    return g if first > 0 else -g


@lru_cache(maxsize=None)
def coupling(l1: int, l2: int, l3: int) -> np.ndarray:
    """Unit-norm real coupling tensor ``(2l1+1, 2l2+1, 2l3+1)``; zero if forbidden.

    Even ``l1 + l2 + l3``: the normalised Gaunt integral (sign: ``Σ G Y1(u) Y2(u) Y3(u) > 0``).
    Odd sums (paths such as ``1o x 1o -> 1e`` that appear with non-natural parities): the
    invariant of ``_odd_coupling`` (first non-zero entry positive)."""
    shape = (2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1)
    if not (abs(l1 - l2) <= l3 <= l1 + l2):
        return np.zeros(shape)
    if (l1 + l2 + l3) % 2:
        g = _odd_coupling(l1, l2, l3)
        g.setflags(write=False)
        return g
    pts, w = _sphere_quadrature()
    y1, y2, y3 = sh_block(l1, pts), sh_block(l2, pts), sh_block(l3, pts)
    g = np.einsum("q,qa,qb,qc->abc", w, y1, y2, y3)
    g /= np.linalg.norm(g)
    g[np.abs(g) < 1e-13] = 0.0
    g.setflags(write=False)
    return g


# ---------------------------------------------------------------------------
# Channelwise tensor-product descriptor
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class TPPath:
    i1: int  # block index in irreps_in1
    i2: int  # block index in irreps_in2
    l1: int
    l2: int
    l3: int
    p3: int
    out_block: int  # block index in the (sorted) output irreps


class ChannelwiseTPDescriptor:
    """Paths of ``x (mul x ir1) ⊗ Y (1 x ir2) -> mul x ir3`` with ir3 in a filter.

    Paths are enumerated in the order (block of in1, block of in2, l3 ascending);
    the per-edge weight tensor holds one segment of ``mul`` channels per path in
    that order (``[path][channel]`` for a uniform multiplicity).  Output blocks
    are the path outputs stably sorted by irrep (one block per path, with the
    multiplicity of the path's in1 block).
    Mirrors the construction used by ``ConvTP`` (``tensor_product.py:72-79``).
    """

    def __init__(self, irreps_in1, irreps_in2, irreps_out_filter):
        self.irreps_in1 = Irreps(irreps_in1)
        self.irreps_in2 = Irreps(irreps_in2)
        filt = {b.ir for b in Irreps(irreps_out_filter)}
        muls = {b.mul for b in self.irreps_in1}
        # the common multiplicity of irreps_in1, None when the blocks differ (each path then
        # carries its input block's multiplicity)
        self.mul = muls.pop() if len(muls) == 1 else None
        for b in self.irreps_in2:
            if b.mul != 1:
                raise ValueError("irreps_in2 must have multiplicity 1 per block")
        raw = []
        for i1, b1 in enumerate(self.irreps_in1):
            for i2, b2 in enumerate(self.irreps_in2):
                p3 = b1.ir.p * b2.ir.p
                for l3 in range(abs(b1.ir.l - b2.ir.l), b1.ir.l + b2.ir.l + 1):
                    if Irrep(l3, p3) in filt:
                        raw.append((i1, i2, b1.ir.l, b2.ir.l, l3, p3))
        order = sorted(range(len(raw)), key=lambda k: (Irrep(raw[k][4], raw[k][5]).sort_key(), k))
        out_block_of = {k: pos for pos, k in enumerate(order)}
        self.paths = [TPPath(*r, out_block=out_block_of[k]) for k, r in enumerate(raw)]
        self.irreps_out = Irreps([(self.irreps_in1[raw[k][0]].mul, Irrep(raw[k][4], raw[k][5])) for k in order])
        self.weight_numel = sum(self.irreps_in1[r[0]].mul for r in raw)
        for p in self.paths:
            if max(p.l1, p.l2, p.l3) > L_MAX_SUPPORTED:
                raise ValueError(f"l > {L_MAX_SUPPORTED} is not supported")

    @property
    def num_paths(self) -> int:
        return len(self.paths)

    def path_coefficient(self, path: TPPath) -> np.ndarray:
        return math.sqrt(2 * path.l3 + 1) * coupling(path.l1, path.l2, path.l3)

    def dense_operator(self) -> np.ndarray:
        """Per-channel operator ``T[path, k1, k2, k3]`` over component indices.

        ``k1`` indexes the ``num_irreps``-per-channel components of in1 (block
        offsets divided by ``mul``), ``k2`` the components of in2, ``k3`` those of
        the output.  out[k3, c] = Σ w[path, c] T[path, k1, k2, k3] x[k1, c] Y[k2].
        """
        n1 = sum(b.ir.dim for b in self.irreps_in1)
        n2 = self.irreps_in2.dim
        n3 = sum(b.ir.dim for b in self.irreps_out)
        off1 = np.cumsum([0] + [b.ir.dim for b in self.irreps_in1])
        off2 = np.cumsum([0] + [b.ir.dim for b in self.irreps_in2])
        off3 = np.cumsum([0] + [b.ir.dim for b in self.irreps_out])
        t = np.zeros((self.num_paths, n1, n2, n3))
        for k, p in enumerate(self.paths):
            c = self.path_coefficient(p)
            t[k, off1[p.i1]:off1[p.i1 + 1], off2[p.i2]:off2[p.i2 + 1], off3[p.out_block]:off3[p.out_block + 1]] = c
        return t


def irreps_from_l_max(l_max: int, hidden_dim: int) -> str:
    """``hidden_dim x (0e + 1o + ... )`` up to ``l_max`` (``tensor_product.py:116-133``)."""
    return " + ".join(f"{hidden_dim}x{l}{'e' if l % 2 == 0 else 'o'}" for l in range(l_max + 1))


def sh_irreps_from_l_max(l_max: int) -> str:
    """``1x0e + 1x1o + ...`` up to ``l_max`` (``tensor_product.py:136-149``)."""
    return " + ".join(f"1x{l}{'e' if l % 2 == 0 else 'o'}" for l in range(l_max + 1))
