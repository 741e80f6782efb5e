"""Equivariant linear layers (src/molrep/interaction/linear.py:43-105 and the
cuet.Linear calls of mace.py:270-291, element_update.py:101-109, node.py:153-159).

``Linear`` mixes channels within each irrep type: for an output block
``mul_o x ir`` and every input block ``mul_b x ir`` of the same irrep,
``out[m, o] += sum_c W_bo[c, o] x_b[m, c] / sqrt(fan_in)`` with ``fan_in`` the
total input multiplicity of that irrep (ir_mul layout, weights ~ N(0, 1)).
With ``weight_classes`` the weights are external, one set per class, selected
per row by ``weight_indices`` (cuet's indexed_linear).  Each output block is one
GEMM (rows = (node, m), K = the concatenated channels of its source blocks) on
the GPU through torch.mm (hipBLASLt); forward and backward are written out so
every gradient slice is produced once.

On the GPU (float32, multiplicities that are multiples of 8) the blocks run in
the HIP kernel ``mnx_block_linear_f32`` instead (fp32-accurate split-bf16 matrix-core products): rows (node, m) are read in
place from the ir_mul input (no gather copy), the 1/sqrt(fan_in) scale is folded
into the stacked weights and each output block is written directly; the input
gradient is the same kernel on the output-gradient blocks with transposed
weights.  Weight gradients (training) use the torch path below.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
from pydantic import BaseModel

from ... import kernels as K
from ...config import config
from ...irreps import Irreps


class Linear(nn.Module):
    def __init__(self, irreps_in, irreps_out, *, layout=None, internal_weights: bool = True,
                 weight_classes: int | None = None, method: str | None = None, dtype=None):
        super().__init__()
        self.irreps_in = Irreps(irreps_in)
        self.irreps_out = Irreps(irreps_out)
        self.weight_classes = weight_classes
        self.method = method
        in_off, out_off = self.irreps_in.offsets(), self.irreps_out.offsets()
        # one entry per output block: (out offset, out mul, dim, [(in offset, in mul, weight offset)], fan_in)
        self.plan = []
        woff = 0
        for ob, o in enumerate(self.irreps_out):
            srcs = []
            for ib, b in enumerate(self.irreps_in):
                if b.ir == o.ir:
                    srcs.append((in_off[ib], b.mul, woff))
                    woff += b.mul * o.mul
            fan_in = sum(s[1] for s in srcs)
            self.plan.append((out_off[ob], o.mul, o.ir.dim, srcs, fan_in))
        self.weight_numel = woff
        # a constant factor on the output, applied to the weights (F(x, w) s = F(x, s w): no extra
        # pass over the output, gradients by autograd); not part of the state_dict
        self.output_scale = 1.0
        dt = dtype if dtype is not None else config.ftype
        if internal_weights and weight_classes is None:
            self.weight = nn.Parameter(torch.randn(1, self.weight_numel, dtype=dt))
        else:
            self.register_parameter("weight", None)
        self._setup_hip()

    def _mix(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """x (R, dim_in), w (weight_numel,) -> (R, dim_out)."""
        if x.is_cuda and x.dtype == torch.float32 and w.dtype == torch.float32 and self._hip_ok():
            return _HipBlockLinear.apply(x, w, self)
        return _BlockLinear.apply(x, w, self.plan, self.irreps_out.dim)

    def _hip_ok(self) -> bool:
        return self._hip_plan is not None

    def _setup_hip(self) -> None:
        """Launch lists and fragment-order weight tables of the HIP block kernel, for shapes it
        takes: every multiplicity a multiple of 8, at most 8 source blocks per output block and 8
        consumers per input block.  The tables are non-persistent buffers, so they follow the
        module's device and appear as constants when the module is traced."""
        ok = all(b.mul % 8 == 0 for b in self.irreps_in) and all(o.mul % 8 == 0 for o in self.irreps_out)
        users = {}
        for _, _, _, srcs, _ in self.plan:
            ok = ok and len(srcs) <= 8
            for o, _, _ in srcs:
                users[o] = users.get(o, 0) + 1
        ok = ok and all(c <= 8 for c in users.values())
        self._hip_plan = _hip_plan(self) if ok else None
        for name in ("idx_f", "sc_f", "idx_b", "sc_b"):
            self.register_buffer("_hip_" + name, self._hip_plan.pop(name) if ok else None, persistent=False)

    def forward(self, x: torch.Tensor, weight: torch.Tensor | None = None,
                weight_indices: torch.Tensor | None = None) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.irreps_in.dim)
        if self.weight_classes is None:
            w = self.weight if weight is None else weight
            if self.output_scale != 1.0:
                w = w * self.output_scale
            out = self._mix(x2, w.reshape(-1))
        else:
            if weight is None or weight_indices is None:
                raise ValueError("indexed linear needs weight and weight_indices")
            if self.output_scale != 1.0:
                weight = weight * self.output_scale
            idx = weight_indices.reshape(-1)
            if x2.is_cuda and x2.dtype == torch.float32 and weight.dtype == torch.float32 and self._hip_ok():
                out = _HipIndexedLinear.apply(x2, weight, K.class_groups(idx, self.weight_classes), idx, self)
            else:
                out = _IndexedLinear.apply(x2, weight, idx, self)
        return out.reshape(*shape[:-1], self.irreps_out.dim)


def _tn_mm(a, b):
    """``a^T @ b`` for tall ``a``, ``b`` (rows >> columns).  hipBLASLt handles the single long
    reduction poorly (456 us for 200k x 128 x 128 on MI355X); 32 batched slabs summed
    afterwards run in 71 us."""
    R = a.shape[0]
    if R < (1 << 13) or not a.is_cuda:
        return a.t() @ b
    nc = 32
    rows = R // nc
    main = nc * rows
    out = torch.bmm(a[:main].reshape(nc, rows, a.shape[1]).transpose(1, 2),
                    b[:main].reshape(nc, rows, b.shape[1])).sum(0)
    if main < R:
        out += a[main:].t() @ b[main:]
    return out


def _gather_rows(x, srcs, d):
    """(R*d, K) rows (node, m), columns = the channels of every source block of one irrep."""
    R = x.shape[0]
    if len(srcs) == 1:
        o, m, _ = srcs[0]
        return x[:, o:o + d * m].reshape(R * d, m)
    return torch.cat([x[:, o:o + d * m].reshape(R, d, m) for o, m, _ in srcs], dim=2).reshape(R * d, -1)


def _block_forward(x, w, plan, dim_out):
    R = x.shape[0]
    out = x.new_empty(R, dim_out)
    for off_o, mul_o, d, srcs, fan_in in plan:
        if not srcs:
            out[:, off_o:off_o + d * mul_o] = 0
            continue
        ws = torch.cat([w[wo:wo + m * mul_o].view(m, mul_o) for _, m, wo in srcs], dim=0)
        y = torch.mm(_gather_rows(x, srcs, d), ws) * (1.0 / math.sqrt(fan_in))
        out[:, off_o:off_o + d * mul_o] = y.view(R, d * mul_o)
    return out


def _block_backward(x, w, g, plan, need_x, need_w):
    R = x.shape[0]
    gx = x.new_empty(x.shape) if need_x else None
    gw = torch.zeros_like(w) if need_w else None
    written = set()  # input blocks whose grad_x slice already holds a contribution
    for off_o, mul_o, d, srcs, fan_in in plan:
        if not srcs:
            continue
        s = 1.0 / math.sqrt(fan_in)
        go = g[:, off_o:off_o + d * mul_o].reshape(R * d, mul_o)
        if need_x:
            ws = torch.cat([w[wo:wo + m * mul_o].view(m, mul_o) for _, m, wo in srcs], dim=0)
            gxs = torch.mm(go, ws.t()) * s  # (R*d, K)
            k0 = 0
            for o, m, _ in srcs:
                part = gxs[:, k0:k0 + m].reshape(R, d * m)
                if o in written:
                    gx[:, o:o + d * m] += part
                else:
                    gx[:, o:o + d * m] = part
                    written.add(o)
                k0 += m
        if need_w:
            gws = _tn_mm(_gather_rows(x, srcs, d), go) * s  # (K, mul_o)
            k0 = 0
            for _, m, wo in srcs:
                gw[wo:wo + m * mul_o] += gws[k0:k0 + m].reshape(-1)
                k0 += m
    if need_x:
        in_off = {}
        for _, _, d, srcs, _ in plan:
            for o, m, _ in srcs:
                in_off[o] = d * m
        # input blocks that feed no output get zero gradient
        covered = sorted(written)
        pos = 0
        for o in covered:
            if o > pos:
                gx[:, pos:o] = 0
            pos = o + in_off[o]
        if pos < x.shape[1]:
            gx[:, pos:] = 0
    return gx, gw


def _lin_tiles(N: int) -> int:
    """Output tiles of 32 columns per wavefront (``lin_tiles`` in csrc/linear.hip)."""
    return 4 if N >= 128 else -(-N // 32)


def _frag_order(K: int, N: int):
    """(k, c, valid) of every element of the kernel's weight layout
    [column group][64-row chunk][k/16][tile][lane][8] (csrc/linear.hip): lane l of k-step q
    holds W[16q + 8(l/32) + j][32t + l%32], the bf16 MFMA B operand."""
    nt = _lin_tiles(N)
    Y, C = -(-N // (nt * 32)), -(-K // 64)
    ar = torch.arange
    y = ar(Y).view(-1, 1, 1, 1, 1, 1)
    ch = ar(C).view(1, -1, 1, 1, 1, 1)
    q = ar(4).view(1, 1, -1, 1, 1, 1)
    t = ar(nt).view(1, 1, 1, -1, 1, 1)
    ln = ar(64).view(1, 1, 1, 1, -1, 1)
    i = ar(8).view(1, 1, 1, 1, 1, -1)
    k, c = torch.broadcast_tensors(ch * 64 + 16 * q + 8 * (ln // 32) + i, y * nt * 32 + 32 * t + ln % 32)
    k, c = k.reshape(-1), c.reshape(-1)
    return k, c, (k < K) & (c < N)


def _frag_block(rows, N):
    """Gather indices and scales of one block's fragment-ordered weights.  ``rows`` lists the
    stacked row segments (length, first flat index, step between rows, step between columns,
    scale): W[k][c] = w[first + (k - k_seg) * row_step + c * col_step] * scale."""
    K = sum(r[0] for r in rows)
    k, c, valid = _frag_order(K, N)
    base = torch.zeros(max(K, 1), dtype=torch.long)
    cstep = torch.zeros(max(K, 1), dtype=torch.long)
    scale = torch.zeros(max(K, 1))
    k0 = 0
    for length, first, row_step, col_step, sc in rows:
        kk = torch.arange(length)
        base[k0:k0 + length] = first + kk * row_step
        cstep[k0:k0 + length] = col_step
        scale[k0:k0 + length] = sc
        k0 += length
    kc = k.clamp(max=max(K - 1, 0))
    idx = torch.where(valid, base[kc] + c * cstep[kc], torch.zeros_like(k))
    sc = torch.where(valid, scale[kc], torch.zeros(()))
    return idx, sc


def _hip_plan(lin: "Linear"):
    """Launch descriptors and fragment-ordered weight indices for the HIP block kernel.

    fwd: per output block (out offset, mul_o, d, segments [(col, comp, len)], float offset of its
    weights); the weights are w[idx_f] * scale_f with the stacked source weights (sum of source
    muls) x mul_o in the kernel's fragment order.
    bwd: per input block (in offset, mul, d, segments over the output-gradient blocks, offset);
    weights w[idx_b] * scale_b: the transposed blocks, (sum of consumer mul_o) x mul."""
    fwd, idx_f, sc_f, off = [], [], [], 0
    consumers = {}
    for off_o, mul_o, d, srcs, fan_in in lin.plan:
        s = 1.0 / math.sqrt(fan_in) if srcs else 0.0
        segs, rows = [], []
        for o, m, wo in srcs:
            segs.append((o, m, m))
            rows.append((m, wo, mul_o, 1, s))  # W_src[c][p] = w[wo + c * mul_o + p]
            consumers.setdefault(o, []).append((off_o, mul_o, wo, s))
        fwd.append((off_o, mul_o, d, segs, off))
        if segs:
            i_, s_ = _frag_block(rows, mul_o)
            idx_f.append(i_)
            sc_f.append(s_)
            off += i_.numel()
    bwd, idx_b, sc_b, off = [], [], [], 0
    in_off = lin.irreps_in.offsets()
    for ib, b in enumerate(lin.irreps_in):
        o, m, d = in_off[ib], b.mul, b.ir.dim
        segs, rows = [], []
        for off_o, mul_o, wo, s in consumers.get(o, []):
            segs.append((off_o, mul_o, mul_o))
            rows.append((mul_o, wo, 1, mul_o, s))  # W^T[p][c] = w[wo + c * mul_o + p]
        bwd.append((o, m, d, segs, off))
        if segs:
            i_, s_ = _frag_block(rows, m)
            idx_b.append(i_)
            sc_b.append(s_)
            off += i_.numel()
    cat = lambda xs, dt: torch.cat(xs).to(dt) if xs else torch.zeros(0, dtype=dt)
    return {"fwd": K.block_linear_desc(fwd), "bwd": K.block_linear_desc(bwd), "idx_f": cat(idx_f, torch.long),
            "sc_f": cat(sc_f, torch.float32), "idx_b": cat(idx_b, torch.long), "sc_b": cat(sc_b, torch.float32)}


class _HipBlockLinear(torch.autograd.Function):
    """out = F(x, w): the blocks of ``lin`` on the HIP kernel."""

    @staticmethod
    def forward(ctx, x, w, lin):
        ws = w.index_select(0, lin._hip_idx_f.to(w.device)) * lin._hip_sc_f.to(w.device)
        out = torch.ops.molix.block_linear(x, ws, lin._hip_plan["fwd"], lin.irreps_out.dim)
        ctx.save_for_backward(x, w)
        ctx.lin = lin
        return out

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        lin = ctx.lin
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        gx = gw = None
        g = g.contiguous()
        if need_x:
            gx = _HipBlockLinearT.apply(g, w, lin)
        if need_w:
            _, gw = _block_backward(x, w, g, lin.plan, False, True)
        return gx, gw, None


class _HipBlockLinearT(torch.autograd.Function):
    """gx = F^T(g, w), the input gradient of ``_HipBlockLinear`` (the same kernel with the
    output-gradient blocks as segments and the transposed weights).  Its own backward (second
    order) is F(ggx, w) for g and, since <ggx, F^T(g, w)> = <F(ggx, w), g>, the weight gradient
    with x := ggx for w."""

    @staticmethod
    def forward(ctx, g, w, lin):
        wb = w.index_select(0, lin._hip_idx_b.to(w.device)) * lin._hip_sc_b.to(w.device)
        gx = torch.ops.molix.block_linear(g, wb, lin._hip_plan["bwd"], lin.irreps_in.dim)
        ctx.save_for_backward(g, w)
        ctx.lin = lin
        return gx

    @staticmethod
    def backward(ctx, ggx):
        g, w = ctx.saved_tensors
        lin = ctx.lin
        need_g, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        ggx = ggx.contiguous()
        dg = _HipBlockLinear.apply(ggx, w, lin) if need_g else None
        dw = _block_backward(ggx, w, g, lin.plan, False, True)[1] if need_w else None
        return dg, dw, None


class _BlockLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, plan, dim_out):
        ctx.save_for_backward(x, w)
        ctx.plan = plan
        return _block_forward(x, w, plan, dim_out)

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        gx, gw = _block_backward(x, w, g, ctx.plan, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return gx, gw, None, None


def _indexed_weight_grad(x, g, weight, idx, lin):
    """d<g, indexed linear(x)>/d weight, one block backward per class present (one host
    synchronisation: training only); nodes of an out-of-range class contribute nothing."""
    gw = torch.zeros_like(weight)
    for cls, rows in _class_rows(idx, lin.weight_classes, strict=False):
        gw[cls] = _block_backward(x[rows], weight[cls].reshape(-1), g[rows], lin.plan, False, True)[1].view_as(gw[cls])
    return gw


class _HipIndexedLinear(torch.autograd.Function):
    """out = F_z(x, W): each node's rows through its class's weights on the HIP indexed block
    kernel (nodes grouped by class on the device, no host synchronisation); the input gradient is
    the same kernel with the transposed weights.  Weight gradients (training) take the per-class
    torch path."""

    @staticmethod
    def forward(ctx, x, weight, groups, idx, lin):
        ws = weight.index_select(1, lin._hip_idx_f.to(weight.device)) * lin._hip_sc_f.to(weight.device)
        out = torch.ops.molix.indexed_block_linear(x, ws.contiguous(), *groups, lin._hip_plan["fwd"],
                                                   lin.irreps_out.dim)
        ctx.save_for_backward(x, weight, idx)
        ctx.groups, ctx.lin = groups, lin
        return out

    @staticmethod
    def backward(ctx, g):
        x, weight, idx = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        g = g.contiguous()
        gx = _HipIndexedLinearT.apply(g, weight, ctx.groups, idx, ctx.lin) if need_x else None
        gw = _indexed_weight_grad(x, g, weight, idx, ctx.lin) if need_w else None
        return gx, gw, None, None, None


class _HipIndexedLinearT(torch.autograd.Function):
    """gx = F_z^T(g, W), the input gradient of ``_HipIndexedLinear``; its own backward (second
    order) is F_z(ggx, W) for g and the weight gradient with x := ggx for W."""

    @staticmethod
    def forward(ctx, g, weight, groups, idx, lin):
        wb = weight.index_select(1, lin._hip_idx_b.to(weight.device)) * lin._hip_sc_b.to(weight.device)
        gx = torch.ops.molix.indexed_block_linear(g, wb.contiguous(), *groups, lin._hip_plan["bwd"],
                                                  lin.irreps_in.dim)
        ctx.save_for_backward(g, weight, idx)
        ctx.groups, ctx.lin = groups, lin
        return gx

    @staticmethod
    def backward(ctx, ggx):
        g, weight, idx = ctx.saved_tensors
        need_g, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        ggx = ggx.contiguous()
        dg = _HipIndexedLinear.apply(ggx, weight, ctx.groups, idx, ctx.lin) if need_g else None
        dw = _indexed_weight_grad(ggx, g, weight, idx, ctx.lin) if need_w else None
        return dg, dw, None, None, None


class _IndexedLinear(torch.autograd.Function):
    """Rows grouped by class, one block linear per class; gradients written per class rows."""

    @staticmethod
    def forward(ctx, x, weight, idx, lin):
        groups = list(_class_rows(idx, lin.weight_classes))
        if sum(len(r) for _, r in groups) != x.shape[0]:
            raise ValueError("weight_indices must lie in [0, weight_classes)")
        out = x.new_empty(x.shape[0], lin.irreps_out.dim)
        for cls, rows in groups:
            out[rows] = _block_forward(x[rows], weight[cls].reshape(-1), lin.plan, lin.irreps_out.dim)
        ctx.save_for_backward(x, weight)
        ctx.groups, ctx.lin = groups, lin
        return out

    @staticmethod
    def backward(ctx, g):
        x, weight = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        gx = torch.empty_like(x) if need_x else None
        gw = torch.zeros_like(weight) if need_w else None
        for cls, rows in ctx.groups:
            gxr, gwr = _block_backward(x[rows], weight[cls].reshape(-1), g[rows], ctx.lin.plan, need_x, need_w)
            if need_x:
                gx[rows] = gxr
            if need_w:
                gw[cls] = gwr.view_as(gw[cls])
        return gx, gw, None, None


def _class_rows(idx: torch.Tensor, num_classes: int, strict: bool = True):
    """Row indices of each class present (one host sync per call).  ``strict``: an index outside
    [0, num_classes) raises; otherwise such rows are left out."""
    if strict and idx.numel() and (int(idx.min()) < 0 or int(idx.max()) >= num_classes):
        raise ValueError(f"weight_indices must lie in [0, {num_classes})")
    if not strict:
        idx = torch.where((idx >= 0) & (idx < num_classes), idx, torch.full_like(idx, num_classes))
    order = torch.argsort(idx, stable=True)
    counts = torch.bincount(idx, minlength=num_classes).tolist()[:num_classes]
    start = 0
    for cls, c in enumerate(counts):
        if c:
            yield cls, order[start:start + c]
        start += c


class EquivariantLinearSpec(BaseModel):
    irreps_in: str
    irreps_out: str


class EquivariantLinear(nn.Module):
    def __init__(self, *, irreps_in: str, irreps_out: str):
        super().__init__()
        self.config = EquivariantLinearSpec(irreps_in=irreps_in, irreps_out=irreps_out)
        self.irreps_in = Irreps(self.config.irreps_in)
        self.irreps_out = Irreps(self.config.irreps_out)
        self.linear = Linear(self.irreps_in, self.irreps_out, dtype=config.ftype)

    def forward(self, features: torch.Tensor) -> torch.Tensor:
        return self.linear(features)
