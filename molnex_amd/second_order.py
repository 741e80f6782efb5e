"""Second derivatives of the ``molix`` ops: autograd formulas for their backward ops.

Force-matching training differentiates the forces (themselves an autograd gradient, taken with
``create_graph=True`` by ``ForceDerivation`` in training mode, src/molpot/derivation/
force_derivation.py:38-43) once more with respect to the parameters.  That runs the backward of
each backward op; this module registers those formulas.

* Multilinear ops reuse the HIP kernels.  ``tp_scatter`` is linear in each of x, Y and w, so with
  L1 = <g, T(x, Y, w)> and the second-order seed L2 = <ggx, dL1/dx> + <ggY, dL1/dY> + <ggw, dL1/dw>
  = <g, T(ggx, Y, w) + T(x, ggY, w) + T(x, Y, ggw)>:
      dL2/dg = T(ggx, Y, w) + T(x, ggY, w) + T(x, Y, ggw)          (three forward launches)
      dL2/dx = gx(g; Y := ggY) + gx(g; w := ggw)                    (backward launches with one
      dL2/dY = gY(g; x := ggx) + gY(g; w := ggw)                     argument substituted)
      dL2/dw = gw(g; x := ggx) + gw(g; Y := ggY)
  ``bond_vectors`` (its gradient is a signed scatter whose adjoint is the gather itself) and the
  radial MLP's output layer (``edge_weights``: gh = g W, whose adjoints are h W^T and g^T h) work
  the same way.
* The equivariant symmetric contraction has a generated second-order kernel
  (``mnx_sc_bwd2_f32``: monomial values, directional derivatives along the seed and their
  gradients, straight-line per configuration).  The harmonics and the scalar contraction, cheap
  pointwise polynomials, differentiate torch restatements of the same formulas on the GPU;
  ``sc_torch`` restates the equivariant contraction for the tests.

The PME ops keep the reference's first-order-only autograd (pme_cpu.cpp:208-215).
"""

from __future__ import annotations

import math
from functools import lru_cache

import torch
from torch import Tensor

from . import kernels as K

_S3, _S5, _S7, _S15 = 3 ** 0.5, 5 ** 0.5, 7 ** 0.5, 15 ** 0.5
_A3, _B3, _C3 = (35 / 8) ** 0.5, 105 ** 0.5, (21 / 8) ** 0.5


def sh_torch(v: Tensor, l_max: int) -> Tensor:
    """The harmonics of ``molix::spherical_harmonics`` (csrc/sh.hip: component normalisation,
    u = v/|v|, u = 0 for the zero vector) as differentiable torch polynomials."""
    r2 = (v * v).sum(dim=-1, keepdim=True)
    pos = r2 > 0
    inv = torch.where(pos, torch.rsqrt(torch.where(pos, r2, torch.ones_like(r2))), torch.zeros_like(r2))
    u = v * inv
    x, y, z = u[..., 0], u[..., 1], u[..., 2]
    out = [torch.ones_like(x)]
    if l_max >= 1:
        out += [_S3 * x, _S3 * y, _S3 * z]
    if l_max >= 2:
        out += [_S15 * x * y, _S15 * y * z, 0.5 * _S5 * (2 * z * z - x * x - y * y), _S15 * x * z,
                0.5 * _S15 * (x * x - y * y)]
    if l_max >= 3:
        x2, y2, z2 = x * x, y * y, z * z
        out += [_A3 * y * (3 * x2 - y2), _B3 * x * y * z, _C3 * y * (4 * z2 - x2 - y2),
                0.5 * _S7 * z * (2 * z2 - 3 * x2 - 3 * y2), _C3 * x * (4 * z2 - x2 - y2),
                0.5 * _B3 * z * (x2 - y2), _A3 * x * (x2 - 3 * y2)]
    return torch.stack(out, dim=-1)


def _seed(t, needed):
    return t if (needed and t is not None and t.numel() > 0) else None


def _vjp_second(fn, primals, cotangent, seeds, needs):
    """Derivatives of <seeds, d<cotangent, fn(primals)>/d primals> with respect to
    (cotangent, *primals), through torch autograd of the restatement ``fn``."""
    with torch.enable_grad():
        ps = [p.detach().requires_grad_(True) for p in primals]
        ct = cotangent.detach().requires_grad_(True)
        first = torch.autograd.grad(fn(*ps), ps, ct, create_graph=True)
        pairs = [(f, s) for f, s in zip(first, seeds) if s is not None]
        if not pairs:
            return [None] * (1 + len(ps))
        wrt = [ct, *ps]
        outs = torch.autograd.grad([f for f, _ in pairs], wrt, [s for _, s in pairs], allow_unused=True)
    return [o if (o is not None and n) else None for o, n in zip(outs, needs)]


# ---------------------------------------------------------------------------
# harmonics
# ---------------------------------------------------------------------------

def _sh2_setup(ctx, inputs, output):
    vectors, grad, l_max = inputs
    ctx.save_for_backward(vectors, grad)
    ctx.l_max = l_max


def _sh2_bwd(ctx, ggv):
    v, g = ctx.saved_tensors
    nv, ng = ctx.needs_input_grad[:2]
    dg, dv = _vjp_second(lambda vv: sh_torch(vv, ctx.l_max), [v.float()], g.float(), [ggv], [ng, nv])
    return dv, dg, None


K.spherical_harmonics_backward.register_autograd(_sh2_bwd, setup_context=_sh2_setup)


# ---------------------------------------------------------------------------
# radial edge embedding
# ---------------------------------------------------------------------------

def bessel_cutoff_torch(r: Tensor, num_radial: int, r_cut: float, eps: float, mu: Tensor | None,
                        sigma: Tensor | None, cutoff: int, exponent: int) -> Tensor:
    """The formula of ``molix::bessel_cutoff`` in torch (differentiable twice)."""
    freqs = torch.arange(1, num_radial + 1, dtype=r.dtype, device=r.device) * (math.pi / r_cut)
    rr = r.unsqueeze(-1)
    phi = math.sqrt(2.0 / r_cut) * torch.sin(rr * freqs) / (rr + eps)
    if mu is not None:
        phi = (phi - mu.to(r.dtype)) / sigma.to(r.dtype)
    if cutoff == 0:
        return phi
    if cutoff == 1:
        c = 0.5 * (torch.cos(math.pi * (r / r_cut)) + 1.0)
    else:
        x = r / r_cut
        g = torch.full_like(x, float((exponent + 1) * exponent // 2))
        for k in range(exponent - 2, -1, -1):
            g = g * x + float((k + 2) * (k + 1) // 2)
        c = (1.0 - x) ** 3 * g
    c = torch.where(r < r_cut, c, torch.zeros_like(c))
    return phi * c.unsqueeze(-1)


def _bc2_setup(ctx, inputs, output):
    grad, r, num_radial, r_cut, eps, mu, sigma, cutoff, exponent = inputs
    ctx.save_for_backward(grad, r, mu, sigma)
    ctx.args = (num_radial, r_cut, eps, cutoff, exponent)


def _bc2_bwd(ctx, ggr):
    g, r, mu, sigma = ctx.saved_tensors
    n, r_cut, eps, cutoff, exponent = ctx.args
    ng, nr = ctx.needs_input_grad[:2]
    # in fp64: the basis' derivatives cancel for small f r (the first-order kernel does the same)
    seed = None if ggr is None else ggr.double()
    dg, dr = _vjp_second(lambda rr: bessel_cutoff_torch(rr, n, r_cut, eps, mu, sigma, cutoff, exponent),
                         [r.double()], g.double(), [seed], [ng, nr])
    dg = None if dg is None else dg.to(g.dtype)
    dr = None if dr is None else dr.to(r.dtype)
    return dg, dr, None, None, None, None, None, None, None


K.bessel_cutoff_backward.register_autograd(_bc2_bwd, setup_context=_bc2_setup)


# ---------------------------------------------------------------------------
# bond vectors
# ---------------------------------------------------------------------------

def _bond2_setup(ctx, inputs, output):
    grad, edge_index, num_atoms = inputs
    ctx.save_for_backward(edge_index)


def _bond2_bwd(ctx, ggpos):
    (edge_index,) = ctx.saved_tensors
    dg = K.bond_vectors(ggpos.contiguous(), edge_index) if ctx.needs_input_grad[0] else None
    return dg, None, None


K.bond_vectors_backward.register_autograd(_bond2_bwd, setup_context=_bond2_setup)


# ---------------------------------------------------------------------------
# radial MLP output layer
# ---------------------------------------------------------------------------

def _ew2_setup(ctx, inputs, output):
    grad, weight = inputs
    ctx.save_for_backward(grad, weight)


def _ew2_bwd(ctx, ggh):
    grad, weight = ctx.saved_tensors
    ng, nw = ctx.needs_input_grad[:2]
    dg = K.edge_weights(ggh.contiguous(), weight) if ng else None
    dw = None
    if nw:  # d/dW <ggh, grad W> = grad^T ggh over all rows
        dw = K.tall_tn(grad, ggh)
    return dg, dw


K.edge_weights_backward.register_autograd(_ew2_bwd, setup_context=_ew2_setup)


# ---------------------------------------------------------------------------
# tensor product + scatter
# ---------------------------------------------------------------------------

def _tp2_setup(ctx, inputs, output):
    (g, x, Y, w, row_ptr, perm, senders, config, channels, need_x, need_Y, need_w, s_row_ptr, s_perm,
     s_receivers, wrow) = inputs
    ctx.shared_rows = wrow is not None
    ctx.save_for_backward(g, x, Y, w, row_ptr, perm, senders)
    ctx.sender_csr = (s_row_ptr, s_perm, s_receivers) if s_row_ptr is not None else ()
    ctx.cfg = (config, channels)
    ctx.need = (need_x, need_Y, need_w)


def _tp2_bwd(ctx, ggx, ggY, ggw):
    if ctx.shared_rows:
        raise NotImplementedError("second derivatives of tp_scatter with shared weight rows (wrow) are not "
                                  "implemented; use one weight row per edge when differentiating twice")
    g, x, Y, w, row_ptr, perm, senders = ctx.saved_tensors
    csr = (row_ptr, perm, senders)
    cfg, extra = ctx.cfg, ctx.sender_csr
    live = lambda t, need: t if (need and t is not None and t.numel() > 0) else None  # noqa: E731
    ggx, ggY, ggw = live(ggx, ctx.need[0]), live(ggY, ctx.need[1]), live(ggw, ctx.need[2])
    want_g, want_x, want_Y, want_w = ctx.needs_input_grad[:4]
    dg = dx = dY = dw = None
    if want_g:
        terms = [K.tp_scatter(a, b, c, *csr, *cfg)
                 for a, b, c, seed in ((ggx, Y, w, ggx), (x, ggY, w, ggY), (x, Y, ggw, ggw)) if seed is not None]
        if terms:
            dg = terms[0]
            for t in terms[1:]:
                dg = dg + t

    def acc(a, b):
        return b if a is None else (a if b is None else a + b)

    if ggx is not None and (want_Y or want_w):
        _, bY, bw = K.tp_scatter_backward(g, ggx, Y, w, *csr, *cfg, False, want_Y, want_w, *extra)
        dY, dw = acc(dY, bY if want_Y else None), acc(dw, bw if want_w else None)
    if ggY is not None and (want_x or want_w):
        bx, _, bw = K.tp_scatter_backward(g, x, ggY, w, *csr, *cfg, want_x, False, want_w, *extra)
        dx, dw = acc(dx, bx if want_x else None), acc(dw, bw if want_w else None)
    if ggw is not None and (want_x or want_Y):
        bx, bY, _ = K.tp_scatter_backward(g, x, Y, ggw, *csr, *cfg, want_x, want_Y, False, *extra)
        dx, dY = acc(dx, bx if want_x else None), acc(dY, bY if want_Y else None)
    shape = lambda t, ref: None if t is None else t.reshape(ref.shape)  # noqa: E731
    return (shape(dg, g), shape(dx, x), shape(dY, Y), shape(dw, w)) + (None,) * 12


K.tp_scatter_backward.register_autograd(_tp2_bwd, setup_context=_tp2_setup)


def _tpa2_setup(ctx, inputs, output):
    g, x, Y, w, row_ptr, perm, senders, table, need_x, need_Y, need_w = inputs
    ctx.save_for_backward(g, x, Y, w, row_ptr, perm, senders)
    ctx.table = table
    ctx.need = (need_x, need_Y, need_w)


def _tpa2_bwd(ctx, ggx, ggY, ggw):
    """The table-driven product is trilinear too: the same three forward and three backward terms."""
    g, x, Y, w, row_ptr, perm, senders = ctx.saved_tensors
    csr, tb = (row_ptr, perm, senders), ctx.table
    live = lambda t, need: t if (need and t is not None and t.numel() > 0) else None  # noqa: E731
    ggx, ggY, ggw = live(ggx, ctx.need[0]), live(ggY, ctx.need[1]), live(ggw, ctx.need[2])
    want_g, want_x, want_Y, want_w = ctx.needs_input_grad[:4]
    dg = dx = dY = dw = None
    if want_g:
        for a, b, c, seed in ((ggx, Y, w, ggx), (x, ggY, w, ggY), (x, Y, ggw, ggw)):
            if seed is not None:
                t = K.tp_any(a, b, c, *csr, tb)
                dg = t if dg is None else dg + t

    def acc(a, b):
        return b if a is None else (a if b is None else a + b)

    if ggx is not None and (want_Y or want_w):
        _, bY, bw = K.tp_any_backward(g, ggx, Y, w, *csr, tb, False, want_Y, want_w)
        dY, dw = acc(dY, bY if want_Y else None), acc(dw, bw if want_w else None)
    if ggY is not None and (want_x or want_w):
        bx, _, bw = K.tp_any_backward(g, x, ggY, w, *csr, tb, want_x, False, want_w)
        dx, dw = acc(dx, bx if want_x else None), acc(dw, bw if want_w else None)
    if ggw is not None and (want_x or want_Y):
        bx, bY, _ = K.tp_any_backward(g, x, Y, ggw, *csr, tb, want_x, want_Y, False)
        dx, dY = acc(dx, bx if want_x else None), acc(dY, bY if want_Y else None)
    shape = lambda t, ref: None if t is None else t.reshape(ref.shape)  # noqa: E731
    return (shape(dg, g), shape(dx, x), shape(dY, Y), shape(dw, w)) + (None,) * 7


K.tp_any_backward.register_autograd(_tpa2_bwd, setup_context=_tpa2_setup)


# per-edge product with shared weights (Allegro): out = TP(s x, Y; w) is multilinear in
# (x, Y, w, s), so each second-order term is the forward or the backward with one factor replaced
# by its incoming cotangent (as for the scatter product above)

def _etp2_setup(ctx, inputs, output):
    g, x, Y, w, config, channels, need_x, need_Y, need_w, x_scale, need_scale = inputs
    ctx.save_for_backward(g, x, Y, w, x_scale)
    ctx.cfg = (config, channels)
    ctx.need = (need_x, need_Y, need_w, bool(need_scale and x_scale is not None))


def _etp2_bwd(ctx, ggx, ggY, ggw, ggs):
    g, x, Y, w, s = ctx.saved_tensors
    cfg = ctx.cfg
    live = lambda t, need: t if (need and t is not None and t.numel() > 0) else None  # noqa: E731
    ggx, ggY, ggw = live(ggx, ctx.need[0]), live(ggY, ctx.need[1]), live(ggw, ctx.need[2])
    ggs = live(ggs, ctx.need[3])
    want_g, want_x, want_Y, want_w = ctx.needs_input_grad[:4]
    want_s = s is not None and ctx.needs_input_grad[9]
    xf = x.reshape(ggx.shape) if ggx is not None else x
    dg = dx = dY = dw = ds = None

    def acc(a, b):
        return b if a is None else (a if b is None else a + b)

    if want_g:
        terms = []
        if ggx is not None:
            terms.append((ggx, Y, w, s))
        if ggY is not None:
            terms.append((x, ggY, w, s))
        if ggw is not None:
            terms.append((x, Y, ggw, s))
        if ggs is not None:
            terms.append((x, Y, w, ggs))
        for xa, Ya, wa, sa in terms:
            dg = acc(dg, K.edge_tp(xa, Ya, wa, *cfg, sa))
    if ggx is not None and (want_Y or want_w or want_s):
        _, bY, bw, bs = K.edge_tp_backward(g, ggx, Y, w, *cfg, False, want_Y, want_w, s, want_s)
        dY, dw, ds = acc(dY, bY if want_Y else None), acc(dw, bw if want_w else None), acc(ds, bs if want_s else None)
    if ggY is not None and (want_x or want_w or want_s):
        bx, _, bw, bs = K.edge_tp_backward(g, xf, ggY, w, *cfg, want_x, False, want_w, s, want_s)
        dx, dw, ds = acc(dx, bx if want_x else None), acc(dw, bw if want_w else None), acc(ds, bs if want_s else None)
    if ggw is not None and (want_x or want_Y or want_s):
        bx, bY, _, bs = K.edge_tp_backward(g, xf, Y, ggw, *cfg, want_x, want_Y, False, s, want_s)
        dx, dY, ds = acc(dx, bx if want_x else None), acc(dY, bY if want_Y else None), acc(ds, bs if want_s else None)
    if ggs is not None and (want_x or want_Y or want_w):
        bx, bY, bw, _ = K.edge_tp_backward(g, xf, Y, w, *cfg, want_x, want_Y, want_w, ggs, False)
        dx, dY, dw = acc(dx, bx if want_x else None), acc(dY, bY if want_Y else None), acc(dw, bw if want_w else None)
    shape = lambda t, ref: None if t is None or ref is None else t.reshape(ref.shape)  # noqa: E731
    return (shape(dg, g), shape(dx, x), shape(dY, Y), shape(dw, w), None, None, None, None, None,
            shape(ds, s), None)


K.edge_tp_backward.register_autograd(_etp2_bwd, setup_context=_etp2_setup)


# ---------------------------------------------------------------------------
# symmetric contractions
# ---------------------------------------------------------------------------

def sc_scalar_torch(x: Tensor, z: Tensor, w: Tensor) -> Tensor:
    """``out[n, c] = sum_k w[z_n, k, c] x[n, c]^(k+1)`` (molix::symmetric_contraction_scalar)."""
    wz = w.index_select(0, z.reshape(-1))
    xs = x.reshape(-1, w.shape[-1])
    out, p = torch.zeros_like(xs), xs
    for k in range(w.shape[1]):
        out = out + wz[:, k] * p
        p = p * xs
    return out.reshape(x.shape)


def _scs2_setup(ctx, inputs, output):
    grad, x, z, w, need_x, need_w = inputs
    ctx.save_for_backward(grad, x, z, w)
    ctx.need = (need_x, need_w)


def _scs2_bwd(ctx, ggx, ggw):
    g, x, z, w = ctx.saved_tensors
    seeds = [_seed(ggx, ctx.need[0]), _seed(ggw, ctx.need[1])]
    ng, nx, _, nw = ctx.needs_input_grad[:4]
    dg, dx, dw = _vjp_second(lambda xx, ww: sc_scalar_torch(xx, z, ww), [x, w], g, seeds, [ng, nx, nw])
    return dg, dx, None, dw, None, None


K.symmetric_contraction_scalar_backward.register_autograd(_scs2_bwd, setup_context=_scs2_setup)


@lru_cache(maxsize=None)
def _sc_tables(l_in: int, l_out: int, nu: int, device: str, dtype: torch.dtype):
    """Per product-basis part: (first path, L, monomial index tensor (Q, nu), coef (r, 2L+1, Q)), in
    the kernels' path order (by output L, then correlation, then basis index)."""
    from .symmetric import ProductBasisDescriptor

    desc = ProductBasisDescriptor(tuple(range(l_in + 1)), tuple(range(l_out + 1)), nu)
    parts, p0 = [], 0
    for L, nu_, r, monos, coef in desc.parts:
        idx = torch.tensor(monos, dtype=torch.long, device=device).reshape(-1, nu_)
        parts.append((p0, L, idx, torch.tensor(coef, dtype=dtype, device=device)))
        p0 += r
    return parts


def sc_torch(x: Tensor, z: Tensor, w: Tensor, l_in: int, l_out: int, nu: int, rows: int = 8192) -> Tensor:
    """``B[n, L, M, c] = sum_{nu, k} w[z_n, p, c] sum_q coef_k[M, q] prod_j A[n, q_j, c]``
    (molix::symmetric_contraction), in row chunks."""
    C = w.shape[-1]
    ni, no = (l_in + 1) ** 2, (l_out + 1) ** 2
    A = x.reshape(-1, ni, C)
    zz = z.reshape(-1)
    parts = _sc_tables(l_in, l_out, nu, str(x.device), x.dtype)
    chunks = []
    for i in range(0, A.shape[0], rows):
        a, wz = A[i:i + rows], w.index_select(0, zz[i:i + rows])
        blocks = [a.new_zeros(a.shape[0], 2 * L + 1, C) for L in range(l_out + 1)]
        for p0, L, idx, coef in parts:
            # index_select: its backward is an index_add, not a sort-based index_put
            m = a.index_select(1, idx[:, 0])
            for j in range(1, idx.shape[1]):
                m = m * a.index_select(1, idx[:, j])
            P = torch.einsum("kmq,nqc->nkmc", coef, m)
            blocks[L] = blocks[L] + (wz[:, p0:p0 + coef.shape[0], None, :] * P).sum(1)
        chunks.append(torch.cat(blocks, dim=1))
    return torch.cat(chunks, dim=0).reshape(*x.shape[:-1], no * C)


def _sc2_setup(ctx, inputs, output):
    grad, x, z, w, l_in, l_out, nu, need_x, need_w = inputs
    ctx.save_for_backward(grad, x, z, w)
    ctx.cfg = (l_in, l_out, nu)
    ctx.need = (need_x, need_w)


def _sc2_bwd(ctx, ggx, ggw):
    g, x, z, w = ctx.saved_tensors
    sx, sw = _seed(ggx, ctx.need[0]), _seed(ggw, ctx.need[1])
    ng, nx, _, nw = ctx.needs_input_grad[:4]
    if (sx is None and sw is None) or not (ng or nx or nw):
        return (None,) * 9
    dg, dx, dw = K.symmetric_contraction_backward2(g.contiguous(), x, z, w, sx, sw, *ctx.cfg, ng, nx, nw)
    return (dg.reshape(g.shape) if ng else None, dx.reshape(x.shape) if nx else None, None,
            dw if nw else None, None, None, None, None, None)


K.symmetric_contraction_backward.register_autograd(_sc2_bwd, setup_context=_sc2_setup)


# ---------------------------------------------------------------------------
# segment sums (per-graph energies, message aggregation)
# ---------------------------------------------------------------------------
# segment_sum_backward: gv[r] = w[r] g[idx[r]], gw[r] = <g[idx[r]], v[r]>; both linear in g, so
# with the seeds (ggv, ggw):
#   dL2/dg[s] = sum_{idx[r] = s} (w[r] ggv[r] + ggw[r] v[r])   (two segment sums)
#   dL2/dv[r] = ggw[r] g[idx[r]]                               (the gather with weights ggw)
#   dL2/dw[r] = <ggv[r], g[idx[r]]>                            (the per-row dot with values ggv)

def _seg2_setup(ctx, inputs, output):
    grad, index, values, weights, need_values, need_weights = inputs
    ctx.save_for_backward(grad, index, values, weights)
    ctx.num_segments = grad.shape[0]


def _seg2_bwd(ctx, ggv, ggw):
    grad, index, values, weights = ctx.saved_tensors
    ng, _, nv, nw = (list(ctx.needs_input_grad) + [False] * 4)[:4]
    has_v = ggv is not None and ggv.numel() > 0
    has_w = ggw is not None and ggw.numel() > 0
    dg = dv = dw = None
    if ng:
        dg = grad.new_zeros(grad.shape)
        if has_v:
            dg = dg + K.segment_sum(ggv.reshape(values.shape).contiguous(), index, ctx.num_segments, weights, False)
        if has_w:
            dg = dg + K.segment_sum(values, index, ctx.num_segments, ggw.reshape(-1).contiguous(), False)
    if nv and has_w:
        dv = K.segment_sum_backward(grad, index, values, ggw.reshape(-1).contiguous(), True, False)[0]
    if nw and weights is not None and has_v:
        dw = K.segment_sum_backward(grad, index, ggv.reshape(values.shape).contiguous(), weights, False, True)[1]
    return dg, None, dv, dw, None, None


K.segment_sum_backward.register_autograd(_seg2_bwd, setup_context=_seg2_setup)
