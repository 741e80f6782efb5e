"""fp64 NumPy oracle for harmonics, coupling tables and the channelwise tensor
product + scatter -- TEST INFRASTRUCTURE ONLY.

The reference computes these through cuequivariance (absent here; see
``src/molrep/embedding/angular.py:89,104`` and
``src/molrep/interaction/tensor_product.py:72-79,101-111``).  This module
restates the mathematics with methods independent of the product code in
``molnex_amd/irreps.py``:

* harmonics from ``scipy.special.sph_harm_y`` (complex, Condon-Shortley) turned
  into the real basis ``sqrt(2)(-1)^m Re/Im``, scaled by ``sqrt(4 pi)``, with the
  l = 1 block reordered to (x, y, z);
* coupling tensors as the null space of ``D1 (x) D2 (x) D3 - I`` over random
  rotations, with ``D^l`` fitted from rotated harmonics (no Gaunt integral);
* the tensor product as a dense per-path contraction followed by a scatter-add;
  gradients by explicit transposed contractions.

Pinned by: closed forms (l=1 = sqrt3 u, orthonormality by quadrature), the
Wigner-D equivariance of every table, agreement between this null-space
construction and the product's Gaunt construction, finite differences of the
forward for every gradient, rotation equivariance of the full TP + scatter.
"""

from __future__ import annotations

import math
from functools import lru_cache

import numpy as np
import scipy.sparse as sp
from scipy.special import sph_harm_y


def scatter_add(index, values, num):
    """out[index[e]] += values[e] (fp64, via a sparse incidence matrix)."""
    E = values.shape[0]
    inc = sp.csr_matrix((np.ones(E), (np.asarray(index), np.arange(E))), shape=(num, E))
    F = int(np.prod(values.shape[1:], dtype=np.int64))
    return (inc @ values.reshape(E, F)).reshape((num,) + values.shape[1:])


def _irrep_list(ls_or_str):
    if isinstance(ls_or_str, str):
        out = []
        for tok in ls_or_str.split("+"):
            tok = tok.strip()
            mul, ir = tok.split("x") if "x" in tok else ("1", tok)
            out.append((int(mul), int(ir[:-1]), 1 if ir[-1] == "e" else -1))
        return out
    return [(1, l, (-1) ** l) for l in ls_or_str]


def real_sh(l: int, vec: np.ndarray) -> np.ndarray:
    """Real harmonics of degree l (component normalisation) of vectors (..., 3)."""
    v = np.asarray(vec, dtype=np.float64)
    r = np.linalg.norm(v, axis=-1)
    safe = np.where(r > 0, r, 1.0)
    u = v / safe[..., None]
    theta = np.arccos(np.clip(u[..., 2], -1, 1))
    phi = np.arctan2(u[..., 1], u[..., 0])
    cols = []
    for m in range(-l, l + 1):
        if m == 0:
            y = sph_harm_y(l, 0, theta, phi).real
        elif m > 0:
            y = math.sqrt(2) * (-1) ** m * sph_harm_y(l, m, theta, phi).real
        else:
            y = math.sqrt(2) * (-1) ** m * sph_harm_y(l, -m, theta, phi).imag
        cols.append(y * math.sqrt(4 * math.pi))
    Y = np.stack(cols, axis=-1)
    if l == 1:  # (m=-1, 0, +1) = (y, z, x) -> (x, y, z)
        Y = Y[..., [2, 0, 1]]
    if l > 0:
        Y = np.where((r > 0)[..., None], Y, 0.0)
    return Y


def sh(ls, vec):
    return np.concatenate([real_sh(l, vec) for l in ls], axis=-1)


def sh_grad_fd(ls, vec, grad_out, h=1e-6):
    """d<grad_out, sh(vec)>/d vec by central differences (fp64)."""
    vec = np.asarray(vec, np.float64)
    g = np.zeros_like(vec)
    for k in range(3):
        dv = np.zeros_like(vec)
        dv[..., k] = h
        g[..., k] = ((sh(ls, vec + dv) - sh(ls, vec - dv)) * grad_out).sum(-1) / (2 * h)
    return g


def random_rotation(rng) -> np.ndarray:
    q = rng.normal(size=4)
    q /= np.linalg.norm(q)
    a, b, c, d = q
    return np.array([
        [a * a + b * b - c * c - d * d, 2 * (b * c - a * d), 2 * (b * d + a * c)],
        [2 * (b * c + a * d), a * a - b * b + c * c - d * d, 2 * (c * d - a * b)],
        [2 * (b * d - a * c), 2 * (c * d + a * b), a * a - b * b - c * c + d * d],
    ])


def wigner_d(l: int, R: np.ndarray) -> np.ndarray:
    """D^l(R) with Y^l(R u) = D^l(R) Y^l(u), fitted on random points."""
    rng = np.random.default_rng(7 + l)
    U = rng.normal(size=(64, 3))
    A = real_sh(l, U)
    B = real_sh(l, U @ R.T)
    Dt, *_ = np.linalg.lstsq(A, B, rcond=None)
    return Dt.T


@lru_cache(maxsize=None)
def coupling(l1: int, l2: int, l3: int) -> np.ndarray:
    """Unit-norm invariant tensor of l1 (x) l2 (x) l3.  Sign: sum C Y1(u)Y2(u)Y3(u) > 0 for even
    l1 + l2 + l3; for odd sums (where that sum vanishes identically) the first entry in C order
    above 1e-9 x max is positive."""
    rng = np.random.default_rng(11)
    blocks = []
    for _ in range(3):
        R = random_rotation(rng)
        K = np.kron(np.kron(wigner_d(l1, R), wigner_d(l2, R)), wigner_d(l3, R))
        blocks.append(K - np.eye(K.shape[0]))
    M = np.concatenate(blocks, axis=0)
    _, s, vt = np.linalg.svd(M)
    c = vt[-1].reshape(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1)
    assert s[-1] < 1e-8 and (len(s) < 2 or s[-2] > 1e-3), "invariant space is not one-dimensional"
    c = c / np.linalg.norm(c)
    if (l1 + l2 + l3) % 2:
        flat = c.ravel()
        return c * np.sign(flat[np.flatnonzero(np.abs(flat) > 1e-9 * np.abs(flat).max())[0]])
    u = np.array([0.3, -0.5, 0.8])
    val = np.einsum("abc,a,b,c->", c, real_sh(l1, u), real_sh(l2, u), real_sh(l3, u))
    return c * np.sign(val)


def tp_paths(irreps_in1, irreps_in2, irreps_filter):
    """Paths (l1, l2, l3) of the channelwise product in weight order, output blocks
    sorted by (l, natural parity first), stable.  Returns (paths, out_order)."""
    in1, in2 = _irrep_list(irreps_in1), _irrep_list(irreps_in2)
    filt = {(l, p) for _, l, p in _irrep_list(irreps_filter)}
    paths = []
    for b1, (_, l1, p1) in enumerate(in1):
        for b2, (_, l2, p2) in enumerate(in2):
            for l3 in range(abs(l1 - l2), l1 + l2 + 1):
                if (l3, p1 * p2) in filt:
                    paths.append((b1, b2, l1, l2, l3, p1 * p2))
    order = sorted(range(len(paths)), key=lambda k: (paths[k][4], 0 if paths[k][5] == (-1) ** paths[k][4] else 1, k))
    return paths, order


def _offsets(dims):
    return np.concatenate([[0], np.cumsum(dims)]).astype(int)


class ChannelwiseTP:
    """out[r] = sum_{e: recv(e)=r} sum_p w[e,p,:] * (C_p x[send(e)] Y[e]) (ir_mul layout)."""

    def __init__(self, irreps_in1, irreps_in2, irreps_filter, channels):
        self.C = channels
        self.in1 = _irrep_list(irreps_in1)
        self.in2 = _irrep_list(irreps_in2)
        self.paths, order = tp_paths(irreps_in1, irreps_in2, irreps_filter)
        self.off1 = _offsets([2 * l + 1 for _, l, _ in self.in1])
        self.off2 = _offsets([2 * l + 1 for _, l, _ in self.in2])
        out_dims = [2 * self.paths[k][4] + 1 for k in order]
        self.off3_sorted = _offsets(out_dims)
        self.out_pos = {k: pos for pos, k in enumerate(order)}
        self.nx, self.ny, self.no = self.off1[-1], self.off2[-1], self.off3_sorted[-1]

    def _coef(self, p):
        l1, l2, l3 = p[2], p[3], p[4]
        return math.sqrt(2 * l3 + 1) * coupling(l1, l2, l3)

    def _blocks(self, k):
        b1, b2, l1, l2, l3, _ = self.paths[k]
        pos = self.out_pos[k]
        return (slice(self.off1[b1], self.off1[b1 + 1]), slice(self.off2[b2], self.off2[b2 + 1]),
                slice(self.off3_sorted[pos], self.off3_sorted[pos + 1]))

    def forward(self, x, Y, w, edge_index, num_nodes):
        C = self.C
        E = Y.shape[0]
        xs = np.asarray(x, np.float64).reshape(-1, self.nx, C)
        w3 = np.asarray(w, np.float64).reshape(E, len(self.paths), C)
        Y = np.asarray(Y, np.float64)
        s, r = edge_index[:, 0], edge_index[:, 1]
        out = np.zeros((num_nodes, self.no, C))
        for k, p in enumerate(self.paths):
            s1, s2, s3 = self._blocks(k)
            M = np.einsum("abc,eb->eca", self._coef(p), Y[:, s2])  # (E, m3, m1)
            msg = np.matmul(M, xs[:, s1][s]) * w3[:, k][:, None, :]  # (E, m3, C)
            out[:, s3] += scatter_add(r, msg, num_nodes)
        return out.reshape(num_nodes, -1)

    def backward(self, x, Y, w, edge_index, grad_out):
        C = self.C
        E = Y.shape[0]
        xs = np.asarray(x, np.float64).reshape(-1, self.nx, C)
        w3 = np.asarray(w, np.float64).reshape(E, len(self.paths), C)
        Y = np.asarray(Y, np.float64)
        g = np.asarray(grad_out, np.float64).reshape(-1, self.no, C)
        s, r = edge_index[:, 0], edge_index[:, 1]
        gx = np.zeros_like(xs)
        gY = np.zeros_like(Y)
        gw = np.zeros_like(w3)
        for k, p in enumerate(self.paths):
            s1, s2, s3 = self._blocks(k)
            cf = self._coef(p)
            gr, xe, we = g[:, s3][r], xs[:, s1][s], w3[:, k][:, None, :]
            M = np.einsum("abc,eb->eca", cf, Y[:, s2])  # (E, m3, m1)
            u = np.matmul(M.transpose(0, 2, 1), gr)  # (E, m1, C) = M^T g
            gw[:, k] = (xe * u).sum(1)
            gx[:, s1] += scatter_add(s, u * we, gx.shape[0])
            q = np.matmul(xe * we, gr.transpose(0, 2, 1))  # (E, m1, m3) = sum_C x w g
            gY[:, s2] += np.einsum("abc,eac->eb", cf, q)
        return gx.reshape(x.shape), gY, gw.reshape(E, -1)


class ChannelwiseTPMul:
    """The channelwise product + scatter for any irreps: a multiplicity per block of in1 (path k of
    in1 block b1 with multiplicity u takes the weights w[e, woff_k : woff_k + u] and writes an output
    block of (2 l3 + 1) x u in ir_mul layout), any parities (paths 1o x 1o -> 1e included), several
    blocks of one l.  Paths and the output order are those of ``tp_paths``; weight segments follow
    the path order.  Restated per path with dense contractions, independently of the product's
    path tables."""

    def __init__(self, irreps_in1, irreps_in2, irreps_filter):
        self.in1 = _irrep_list(irreps_in1)
        self.in2 = _irrep_list(irreps_in2)
        assert all(m == 1 for m, _, _ in self.in2)
        self.paths, order = tp_paths(irreps_in1, irreps_in2, irreps_filter)
        self.muls = [self.in1[p[0]][0] for p in self.paths]
        self.off1 = _offsets([m * (2 * l + 1) for m, l, _ in self.in1])
        self.off2 = _offsets([2 * l + 1 for _, l, _ in self.in2])
        self.off3 = _offsets([(2 * self.paths[k][4] + 1) * self.muls[k] for k in order])
        self.out_pos = {k: pos for pos, k in enumerate(order)}
        self.offw = _offsets(self.muls)
        self.nx, self.ny, self.no, self.nw = self.off1[-1], self.off2[-1], self.off3[-1], self.offw[-1]

    def _parts(self, k, x, Y, w, N, E):
        b1, b2, l1, l2, l3, _ = self.paths[k]
        u = self.muls[k]
        pos = self.out_pos[k]
        xb = x[:, self.off1[b1]:self.off1[b1 + 1]].reshape(N, 2 * l1 + 1, u)
        wk = w[:, self.offw[k]:self.offw[k + 1]]
        cf = math.sqrt(2 * l3 + 1) * coupling(l1, l2, l3)
        M = np.einsum("abc,eb->eca", cf, Y[:, self.off2[b2]:self.off2[b2 + 1]])  # (E, m3, m1)
        return xb, wk, cf, M, slice(self.off3[pos], self.off3[pos + 1]), (2 * l3 + 1, u)

    def forward(self, x, Y, w, edge_index, num_nodes):
        x, Y, w = (np.asarray(a, np.float64) for a in (x, Y, w))
        E = Y.shape[0]
        s, r = edge_index[:, 0], edge_index[:, 1]
        out = np.zeros((num_nodes, self.no))
        for k in range(len(self.paths)):
            xb, wk, _, M, s3, shp = self._parts(k, x, Y, w, x.shape[0], E)
            msg = np.matmul(M, xb[s]) * wk[:, None, :]  # (E, m3, u)
            out[:, s3] += scatter_add(r, msg, num_nodes).reshape(num_nodes, -1)
        return out

    def backward(self, x, Y, w, edge_index, grad_out):
        x, Y, w, g = (np.asarray(a, np.float64) for a in (x, Y, w, grad_out))
        N, E = x.shape[0], Y.shape[0]
        s, r = edge_index[:, 0], edge_index[:, 1]
        gx, gY, gw = np.zeros_like(x), np.zeros_like(Y), np.zeros_like(w)
        for k in range(len(self.paths)):
            b1, b2 = self.paths[k][:2]
            xb, wk, cf, M, s3, shp = self._parts(k, x, Y, w, N, E)
            gr = g[:, s3].reshape(-1, *shp)[r]  # (E, m3, u)
            xe = xb[s]
            uu = np.matmul(M.transpose(0, 2, 1), gr)  # (E, m1, u)
            gw[:, self.offw[k]:self.offw[k + 1]] = (xe * uu).sum(1)
            gx[:, self.off1[b1]:self.off1[b1 + 1]] += scatter_add(s, uu * wk[:, None, :], N).reshape(N, -1)
            q = np.matmul(xe * wk[:, None, :], gr.transpose(0, 2, 1))  # (E, m1, m3)
            gY[:, self.off2[b2]:self.off2[b2 + 1]] += np.einsum("abc,eac->eb", cf, q)
        return gx, gY, gw


def rotate_irreps(feat, R, irreps, channels, layout="ir_mul"):
    """Apply D(R) blockwise to ir_mul features (..., dim)."""
    out = np.array(feat, dtype=np.float64, copy=True)
    off = 0
    for mul, l, p in _irrep_list(irreps):
        d = 2 * l + 1
        blk = out[..., off:off + d * mul].reshape(*out.shape[:-1], d, mul)
        out[..., off:off + d * mul] = np.einsum("ab,...bm->...am", wigner_d(l, R), blk).reshape(*out.shape[:-1], -1)
        off += d * mul
    return out
