"""PME oracle (TEST INFRASTRUCTURE ONLY): fp64 NumPy restatement of the reference's
CPU ops molix::pme_direct and molix::pme_reciprocal
(/root/reference/src/molix/op/src/pme/pme_cpu.cpp).

Pinned by: tests/golden/pme_golden.npz (outputs and gradients of the reference op
itself, compiled from its sources by oracle/Makefile), the Madelung constant of
NaCl from direct + reciprocal - self, alpha-independence of that sum, and finite
differences of the energies.
"""

from __future__ import annotations

import math

import numpy as np


def invert_box(box: np.ndarray) -> np.ndarray:
    """Reciprocal vectors of a lower-triangular cell (pme_cpu.cpp:22-35)."""
    b = box
    s = 1.0 / (b[0, 0] * b[1, 1] * b[2, 2])
    r = np.zeros((3, 3))
    r[0, 0] = b[1, 1] * b[2, 2] * s
    r[1, 0] = -b[1, 0] * b[2, 2] * s
    r[1, 1] = b[0, 0] * b[2, 2] * s
    r[2, 0] = (b[1, 0] * b[2, 1] - b[1, 1] * b[2, 0]) * s
    r[2, 1] = -b[0, 0] * b[2, 1] * s
    r[2, 2] = b[0, 0] * b[1, 1] * s
    return r


def splines(pos: np.ndarray, box: np.ndarray, recip: np.ndarray, grid, order: int):
    """Per-atom grid origin and B-spline weights/derivatives (pme_cpu.cpp:37-91).

    Returns (gridIndex (N,3) int, data (N, order, 3), ddata (N, order, 3)).
    """
    p = np.array(pos, dtype=np.float64, copy=True)
    for i in (2, 1, 0):
        scale = np.floor(p[:, i] * recip[i, i])
        p -= scale[:, None] * box[i][None, :]
    t = p @ recip  # t[i] = sum_j p[j] recip[j][i]
    g = np.asarray(grid, dtype=np.float64)
    t = (t - np.floor(t)) * g
    ti = t.astype(np.int64)
    dr = t - ti
    gidx = ti % np.asarray(grid, dtype=np.int64)
    n = pos.shape[0]
    data = np.zeros((n, order, 3))
    ddata = np.zeros((n, order, 3))
    data[:, 1] = dr
    data[:, 0] = 1 - dr
    for j in range(3, order):
        div = 1.0 / (j - 1)
        data[:, j - 1] = div * dr * data[:, j - 2]
        for k in range(1, j - 1):
            data[:, j - k - 1] = div * ((dr + k) * data[:, j - k - 2] + (j - k - dr) * data[:, j - k - 1])
        data[:, 0] = div * (1 - dr) * data[:, 0]
    ddata[:, 0] = -data[:, 0]
    for j in range(1, order):
        ddata[:, j] = data[:, j - 1] - data[:, j]
    scale = 1.0 / (order - 1)
    data[:, order - 1] = scale * dr * data[:, order - 2]
    for j in range(1, order - 1):
        data[:, order - j - 1] = scale * ((dr + j) * data[:, order - j - 2] + (order - j - dr) * data[:, order - j - 1])
    data[:, 0] = scale * (1 - dr) * data[:, 0]
    return gidx, data, ddata


def _stencil(gidx, grid, order):
    ix = (gidx[:, 0, None] + np.arange(order)[None]) % grid[0]
    iy = (gidx[:, 1, None] + np.arange(order)[None]) % grid[1]
    iz = (gidx[:, 2, None] + np.arange(order)[None]) % grid[2]
    return ix, iy, iz


def reciprocal(pos, charges, box, grid, order, alpha, coulomb, moduli):
    """Energy and (d/dpos, d/dq) of the reciprocal-space sum (pme_cpu.cpp:220-431)."""
    pos = np.asarray(pos, np.float64)
    q = np.asarray(charges, np.float64)
    box = np.asarray(box, np.float64)
    grid = tuple(int(g) for g in grid)
    recip = invert_box(box)
    sqrt_k = math.sqrt(coulomb)
    gidx, data, ddata = splines(pos, box, recip, grid, order)
    ix, iy, iz = _stencil(gidx, grid, order)
    w = (q * sqrt_k)[:, None, None, None] * data[:, :, None, None, 0] * data[:, None, :, None, 1] * \
        data[:, None, None, :, 2]
    real = np.zeros(grid)
    np.add.at(real, (ix[:, :, None, None], iy[:, None, :, None], iz[:, None, None, :]), w)
    G = np.fft.rfftn(real)
    kx = np.arange(grid[0])
    ky = np.arange(grid[1])
    kz = np.arange(grid[2] // 2 + 1)
    mx = np.where(kx < (grid[0] + 1) // 2, kx, kx - grid[0])
    my = np.where(ky < (grid[1] + 1) // 2, ky, ky - grid[1])
    mz = np.where(kz < (grid[2] + 1) // 2, kz, kz - grid[2])
    MX, MY, MZ = np.meshgrid(mx, my, mz, indexing="ij")
    mhx = MX * recip[0, 0]
    mhy = MX * recip[1, 0] + MY * recip[1, 1]
    mhz = MX * recip[2, 0] + MY * recip[2, 1] + MZ * recip[2, 2]
    m2 = mhx ** 2 + mhy ** 2 + mhz ** 2
    xm, ym, zm = (np.asarray(m, np.float64) for m in moduli)
    denom = m2 * (math.pi * box[0, 0] * box[1, 1] * box[2, 2]) * xm[:, None, None] * ym[None, :, None] * \
        zm[None, None, kz]
    with np.errstate(divide="ignore", invalid="ignore"):
        eterm = np.exp(-(math.pi ** 2 / alpha ** 2) * m2) / denom
    eterm[0, 0, 0] = 0.0
    scale = np.where((kz > 0) & (kz <= (grid[2] - 1) // 2), 2.0, 1.0)[None, None, :]
    energy = 0.5 * np.sum(scale * eterm * (G.real ** 2 + G.imag ** 2))
    G = G * eterm
    real2 = np.fft.irfftn(G, s=grid, axes=(0, 1, 2), norm="forward")
    gvals = real2[ix[:, :, None, None], iy[:, None, :, None], iz[:, None, None, :]]  # (N, p, p, p)
    dx, dy, dz = data[:, :, 0], data[:, :, 1], data[:, :, 2]
    ddx, ddy, ddz = ddata[:, :, 0], ddata[:, :, 1], ddata[:, :, 2]
    d0 = np.einsum("na,nb,nc,nabc->n", ddx, dy, dz, gvals)
    d1 = np.einsum("na,nb,nc,nabc->n", dx, ddy, dz, gvals)
    d2 = np.einsum("na,nb,nc,nabc->n", dx, dy, ddz, gvals)
    dq = np.einsum("na,nb,nc,nabc->n", dx, dy, dz, gvals)
    s = q * sqrt_k
    dpos = np.stack([
        s * (d0 * grid[0] * recip[0, 0]),
        s * (d0 * grid[0] * recip[1, 0] + d1 * grid[1] * recip[1, 1]),
        s * (d0 * grid[0] * recip[2, 0] + d1 * grid[1] * recip[2, 1] + d2 * grid[2] * recip[2, 2]),
    ], axis=1)
    return energy, dpos, dq * sqrt_k


def direct(pos, charges, neighbors, deltas, distances, exclusions, alpha, coulomb):
    """Energy and (d/dpos, d/dq) of the real-space sum over a pair list minus the
    excluded pairs' erf term (pme_cpu.cpp:95-164)."""
    pos = np.asarray(pos, np.float64)
    q = np.asarray(charges, np.float64)
    nb = np.asarray(neighbors)
    d = np.asarray(deltas, np.float64)
    r = np.asarray(distances, np.float64)
    excl = np.asarray(exclusions)
    n = q.shape[0]
    a1, a2 = nb[0].astype(np.int64), nb[1].astype(np.int64)
    include = a1 > -1
    # a pair is skipped when atom2 appears in atom1's exclusion list (descending, -1 padded);
    # the reference scans while excl[atom1][j] >= atom2
    if excl.size:
        hit = np.zeros_like(include)
        rows = excl[np.where(include, a1, 0)]
        run = np.ones_like(include)
        for j in range(excl.shape[1]):
            run &= rows[:, j] >= a2
            hit |= run & (rows[:, j] == a2)
        include &= ~hit
    a1, a2, d, r = a1[include], a2[include], d[include], r[include]
    from scipy.special import erfc, erf

    inv = 1.0 / r
    ar = alpha * r
    ex = np.exp(-ar * ar)
    ec = erfc(ar)
    pref = coulomb * inv
    energy = np.sum(pref * ec * q[a1] * q[a2])
    dq = np.zeros(n)
    np.add.at(dq, a1, pref * ec * q[a2])
    np.add.at(dq, a2, pref * ec * q[a1])
    dedr = pref * q[a1] * q[a2] * (ec + ar * ex * (2 / math.sqrt(math.pi))) * inv * inv
    dpos = np.zeros((n, 3))
    np.add.at(dpos, a1, -dedr[:, None] * d)
    np.add.at(dpos, a2, dedr[:, None] * d)
    if excl.size:
        for i in range(n):
            for j in range(excl.shape[1]):
                k = excl[i, j]
                if not k > i:
                    break
                dr = pos[i] - pos[k]
                rr = math.sqrt(dr @ dr)
                ar2 = alpha * rr
                pf = coulomb / rr
                e = math.erf(ar2)
                energy -= pf * e * q[i] * q[k]
                dq[i] -= pf * e * q[k]
                dq[k] -= pf * e * q[i]
                de = pf * q[i] * q[k] * (e - ar2 * math.exp(-ar2 * ar2) * 2 / math.sqrt(math.pi)) / (rr * rr)
                dpos[i] += de * dr
                dpos[k] -= de * dr
    _ = erf
    return energy, dpos, dq


def bspline_moduli(K: int, order: int) -> np.ndarray:
    """|b(m)|^-2 denominators used by smooth PME (Essmann et al. 1995, eq. 4.4):
    moduli[m] = |sum_{k=0}^{order-2} M_order(k+1) exp(2 pi i m k / K)|^2, zeros
    replaced by the mean of their neighbours."""
    # cardinal B-spline values at integer knots via the recursion
    def M(n, x):
        if n == 2:
            return max(0.0, 1.0 - abs(x - 1.0))
        return (x * M(n - 1, x) + (n - x) * M(n - 1, x - 1.0)) / (n - 1)

    w = np.array([M(order, k + 1.0) for k in range(order - 1)])
    m = np.arange(K)
    ph = 2 * np.pi * np.outer(m, np.arange(order - 1)) / K
    mod = (w * np.cos(ph)).sum(1) ** 2 + (w * np.sin(ph)).sum(1) ** 2
    for i in range(K):
        if mod[i] < 1e-7:
            mod[i] = 0.5 * (mod[(i - 1) % K] + mod[(i + 1) % K])
    return mod
