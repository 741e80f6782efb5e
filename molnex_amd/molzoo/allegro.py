"""Allegro edge encoder (src/molzoo/allegro.py:1-642) on the HIP kernels.

Same classes, constructor arguments, attribute names (``embedding.{radial_basis, cutoff_fn,
spherical_harmonics, type_embedding, scalar_mlp, tensor_env}``, ``layers.i.{tp, tp_linear,
env_embed, latent_mlp, tensor_env}``), in/out keys and output ``(n_edges, num_layers,
num_scalar_features)`` as the reference.

The layer product ``TP(env_w . V_ij, Y_agg(src))`` (allegro.py:352-359,457-458, a
``cuet.ChannelWiseTensorProduct`` with shared internal weights) runs as ``molix::edge_tp``: one
HIP kernel per direction, lanes holding (edge, channel) pairs so that the 8-16 channels Allegro
uses still fill a 64-wide wavefront.  Its projection (allegro.py:363-367,
``cuet.Linear(tp.irreps_out, irreps_in)``) connects only output blocks whose irrep is an input
irrep, so only those paths are computed; the weight keeps one entry per path of the full product,
in the reference's order, and the unused entries receive zero gradient as they do there.  The
layer's env scaling of the tensor track before the product is fused into the same kernel.  With
16 channels and projection weights that take no gradient, the product and the projection run as
one ``molix::edge_tp_proj`` pass per direction (the product's rows stay in registers); otherwise
the projection runs in the HIP block-linear kernel over the edges.  Because every irrep block of the
tensor track has the same multiplicity, the ir_mul features are ``[sum_l (2l+1)][channel]`` and the
per-channel scalings are one broadcast multiply.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn
from pydantic import BaseModel, ConfigDict, Field

from .. import kernels as K
from ..config import config
from ..irreps import Irreps
from ..molrep.embedding.angular import SphericalHarmonics
from ..molrep.embedding.cutoff import PolynomialCutoff
from ..molrep.embedding.radial import BesselRBF
from ..molrep.interaction.linear import Linear
from ..molrep.interaction.tensor_product import irreps_from_l_max, sh_irreps_from_l_max
from .mace import _get, _set


def _env_weight_harmonics(edge_angular, env_weights, l_max, num_tensor_features, irreps_dim):
    """``Y_lm(e) * env(e, c)`` in ir_mul order (allegro.py:55-97): with uniform multiplicity the
    layout is ``[m over all l][c]``, an outer product per edge (``molix::channel_outer`` on float32
    GPU tensors: both gradients in one pass)."""
    E, D = edge_angular.shape
    F = env_weights.shape[1]
    if (edge_angular.is_cuda and edge_angular.dtype == torch.float32 and env_weights.dtype == torch.float32
            and D in K.CHANNEL_PRODUCT_COMPONENTS and F % 4 == 0 and (F // 4) & (F // 4 - 1) == 0 and F <= 256):
        return K.channel_outer(edge_angular, env_weights)
    out = edge_angular.unsqueeze(-1) * env_weights.unsqueeze(-2)
    return out.reshape(E, irreps_dim)


def _silu_stack(mlp: nn.Sequential, x: torch.Tensor) -> torch.Tensor:
    """``mlp(x)`` for a stack of [Linear -> SiLU] layers of one width: one fused HIP kernel each way
    (``molix::radial_hidden``, gradient w.r.t. x only) when the parameters need no gradient and the
    shape is compiled (the pair embedding's scalar MLP, 40 -> 64 -> 64 -> 64 at the defaults: six
    passes over (E, 64) activations in the torch form), else the modules themselves."""
    lins, acts = list(mlp)[0::2], list(mlp)[1::2]
    ok = (config.fused_radial and x.is_cuda and x.dim() == 2 and x.dtype == torch.float32 and len(lins) == len(acts)
          and all(isinstance(m, nn.Linear) and m.bias is not None and m.weight.dtype == torch.float32 for m in lins)
          and all(isinstance(m, nn.SiLU) for m in acts)
          and len({m.out_features for m in lins}) == 1 and lins[0].in_features == x.shape[1]
          and all(m.in_features == lins[0].out_features for m in lins[1:])
          and not (torch.is_grad_enabled() and any(p.requires_grad for p in mlp.parameters())))
    if ok and K.radial_supported(lins[0].in_features, lins[0].out_features, len(lins)):
        raw = torch.cat([t.detach().reshape(-1) for m in lins for t in (m.weight, m.bias)])
        return K.radial_hidden(x, raw, lins[0].in_features, lins[0].out_features, len(lins))
    return mlp(x)


def _scale_by_channel(tensor, scale, l_max, num_tensor_features):
    """Scale every component of channel ``c`` by ``scale[e, c]`` (allegro.py:100-130): the
    ``molix::channel_scale`` kernel (both gradients in one pass) for float32 GPU tensors."""
    E, F = tensor.shape[0], num_tensor_features
    if (tensor.is_cuda and tensor.dtype == torch.float32 and scale.dtype == torch.float32 and F % 4 == 0
            and tensor.dim() == 2 and tensor.shape[1] % F == 0
            and tensor.shape[1] // F in K.CHANNEL_PRODUCT_COMPONENTS):
        return K.channel_scale(tensor, scale, tensor.shape[1] // F)
    return (tensor.reshape(E, -1, F) * scale.unsqueeze(-2)).reshape(E, -1)


def _times_envelope(scalars: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """``scalars * u`` for an (E, F) ``scalars`` and the (E, 1) cutoff envelope ``u``: the outer
    product kernel with one component (``molix::channel_outer``: the envelope's gradient, a sum
    over the F channels, formed in the same pass as the scalars') for float32 GPU tensors."""
    F = scalars.shape[-1]
    if (scalars.is_cuda and scalars.dtype == torch.float32 and u.dtype == torch.float32 and scalars.dim() == 2
            and u.shape == (scalars.shape[0], 1) and F % 4 == 0 and (F // 4) & (F // 4 - 1) == 0 and F <= 256):
        return K.channel_outer(u, scalars)
    return scalars * u


class _EnvelopeStack(torch.autograd.Function):
    """``stack([s_l * u for s_l in xs], 1)`` (allegro.py:628-641) as one pass each way
    (``molix::channel_outer_stack``: the stack is never formed on its own, and the envelope's
    gradient, a sum over layers and channels, comes in the same pass as the features').
    Differentiated again (create_graph), the backward runs in tracked ops."""

    @staticmethod
    def forward(ctx, u, *xs):
        ctx.save_for_backward(u, *xs)
        return K.channel_outer_stack(u, list(xs))

    @staticmethod
    def backward(ctx, g):
        u, *xs = ctx.saved_tensors
        need_u, need_x = ctx.needs_input_grad[0], any(ctx.needs_input_grad[1:])
        if torch.is_grad_enabled():
            gx = [g[:, l] * u for l in range(len(xs))]
            gu = sum((g[:, l] * x).sum(-1, keepdim=True) for l, x in enumerate(xs)) if need_u else None
        else:
            res = K.channel_outer_stack_backward(g.contiguous(), u, list(xs), need_u, need_x)
            gu, gx = res[0], res[1:]
        return (gu if need_u else None, *[gx[l] if ctx.needs_input_grad[1 + l] else None for l in range(len(xs))])


def _envelope_stack(per_layer, u):
    """``stack(per_layer, 1) * u[..., None]`` for (E, F) features and the (E, 1) envelope: one
    pass with ``_EnvelopeStack`` for float32 GPU tensors, else the stack and ``_times_envelope``."""
    F = per_layer[0].shape[-1]
    if (u.is_cuda and u.dtype == torch.float32 and u.shape == (per_layer[0].shape[0], 1) and len(per_layer) <= 8
            and F % 4 == 0 and (F // 4) & (F // 4 - 1) == 0 and F <= 256
            and all(x.dtype == torch.float32 and x.dim() == 2 and x.shape == per_layer[0].shape for x in per_layer)):
        return _EnvelopeStack.apply(u, *per_layer)
    stacked = torch.stack(per_layer, dim=1)
    return _times_envelope(stacked.reshape(stacked.shape[0], -1), u).reshape(stacked.shape)


def _type_pair_embedding(emb: nn.Embedding, zs: torch.Tensor, zd: torch.Tensor) -> torch.Tensor:
    """``cat([emb(zs), emb(zd)], -1)``: with the table frozen (no gradient to it), one row gather
    from the (types^2, 2 dim) table of all ordered type pairs (``molix::gather_rows``) instead of two
    embedding lookups and a concatenation over the edges."""
    w = emb.weight
    if (w.is_cuda and w.dtype == torch.float32 and not (torch.is_grad_enabled() and w.requires_grad)
            and emb.padding_idx is None and emb.max_norm is None):
        S = w.shape[0]
        table = torch.cat([w.repeat_interleave(S, 0), w.repeat(S, 1)], dim=1)
        return K.gather_rows(table, zs.long() * S + zd.long())
    return torch.cat([emb(zs), emb(zd)], dim=-1)


def _tail_torch(s, nt, lat, tenv, a, b, F):
    """The layer tail in autograd-tracked ops: ``updated = a s + b latent([s, nt[:, :F]])`` and
    the output env scaling of ``nt`` by ``tensor_env(updated)``."""
    combined = torch.cat([s, nt[:, :F]], dim=-1)
    mlp = nn.functional.linear(combined, lat.weight * b, lat.bias * b if lat.bias is not None else None)
    updated = torch.add(mlp, s, alpha=a)
    return updated, _scale_by_channel(nt, tenv(updated), None, F)


def _tail_weights(layer, S):
    """(W_s, W_t, b c) of the frozen tail: ``updated = s W_s^T + nt[:, :F] W_t^T + b c`` with the
    residual folded into the square block (``W_s = b W[:, :S] + a I``: ``a s`` needs no pass of its
    own, forward or backward)."""
    lat = layer.latent_mlp[0]
    a, b = layer.residual_a, layer.residual_b
    ws = torch.eye(S, dtype=lat.weight.dtype, device=lat.weight.device).mul_(a).add_(lat.weight[:, :S], alpha=b)
    return ws, lat.weight[:, S:] * b, lat.bias * b


def _row_linear(h, weight, bias=None):
    """``h @ weight.T + bias`` on the split-fp16 row kernel (``molix::edge_weights``, fp32-accurate,
    faster than hipBLASLt on these tall, narrow shapes) where it takes the shape, else ``addmm``."""
    N, Kd = weight.shape
    if h.is_contiguous() and K.edge_weights_supported(Kd, N):
        return K.edge_weights(h, weight, bias)
    return torch.addmm(bias, h, weight.t()) if bias is not None else h @ weight.t()


def _row_grad(g, weight, out=None):
    """``g @ weight`` (the input gradient of ``_row_linear``), or ``out += g @ weight`` in the same
    pass when ``out`` is given (a column block of a wider tensor too)."""
    N, Kd = weight.shape
    if K.edge_weights_supported(Kd, N) and (out is None or (out.data_ptr() % 16 == 0 and out.stride(1) == 1
                                                            and out.stride(0) % 4 == 0)):
        if out is None:
            return K.edge_weights_backward(g, weight)
        K.edge_weights_backward_acc(g, weight, out)
        return out
    return g @ weight if out is None else out.addmm_(g, weight)


def _tail_grads_tracked(layer, s, nt, g_upd, g_out, need_s, need_nt):
    """(grad s, grad nt) of the layer tail in tracked ops (for a backward that is differentiated
    again), the env scale recomputed from s and nt so that second derivatives reach them.  Not
    autograd.grad on a recomputed tail: nt itself depends on s through the layer's product."""
    lat, tenv = layer.latent_mlp[0], layer.tensor_env
    a, b, F = layer.residual_a, layer.residual_b, layer.num_tensor_features
    ws = lat.weight[:, :s.shape[1]] * b
    wt = lat.weight[:, s.shape[1]:] * b
    with torch.enable_grad():
        upd = torch.add(torch.addmm(lat.bias * b, torch.cat([s, nt[:, :F]], dim=1), lat.weight.t() * b), s, alpha=a)
        tv_t = torch.addmm(tenv.bias, upd, tenv.weight.t())
        if g_out is not None:
            g_nt, g_tv = K.channel_scale_backward(g_out.contiguous(), nt, tv_t, nt.shape[1] // F, True, True)
            g_lat = g_tv @ tenv.weight if g_upd is None else g_upd + g_tv @ tenv.weight
        else:
            g_nt, g_lat = torch.zeros_like(nt), g_upd
        if g_lat is None:
            return None, (g_nt if need_nt else None)
        g_s = a * g_lat + g_lat @ ws if need_s else None
        if need_nt:
            g_nt = torch.cat([g_nt[:, :F] + g_lat @ wt, g_nt[:, F:]], dim=1)
    return g_s, (g_nt if need_nt else None)


class _LayerTail(torch.autograd.Function):
    """The layer tail with frozen parameters (the energy + forces path) as GEMMs on row blocks:
    ``updated = s W_s^T + nt[:, :F] W_t^T + b c`` (``_tail_weights``: the residual a s folded into
    W_s) without the concatenation, and a backward that never forms the latent gradient: with
    ``g_lat = g_upd + g_tv T`` (T the env layer's weight), ``g_s = g_upd W_s + g_tv (T W_s)`` and the
    scalar columns of nt get ``g_upd W_t + g_tv (T W_t)``, two products each, the second accumulated
    in the same pass.  The env scaling's backward gives nt's gradient in one pass for both
    gradients; there is no zero-filled slice gradient and no accumulation pass.  Differentiated
    again (create_graph), the backward runs the same formulas in tracked ops, with the env scale
    recomputed from the inputs."""

    @staticmethod
    def forward(ctx, s, nt, layer):
        tenv = layer.tensor_env
        F = layer.num_tensor_features
        ws, wt, bc = _tail_weights(layer, s.shape[1])
        upd = _row_linear(s, ws, bc)
        upd.addmm_(nt[:, :F], wt.t())
        tv = torch.addmm(tenv.bias, upd, tenv.weight.t())
        out = K.channel_scale(nt, tv, nt.shape[1] // F)
        ctx.save_for_backward(s, nt, tv)
        ctx.layer = layer
        # an output nothing uses (the last layer's tensor track) arrives as None, not as zeros
        ctx.set_materialize_grads(False)
        return upd, out

    @staticmethod
    def backward(ctx, g_upd, g_out):
        s, nt, tv = ctx.saved_tensors
        layer = ctx.layer
        lat, tenv = layer.latent_mlp[0], layer.tensor_env
        a, b, F = layer.residual_a, layer.residual_b, layer.num_tensor_features
        need_s, need_nt = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if torch.is_grad_enabled():
            # differentiated again (create_graph): the same gradient formulas in tracked ops
            g_s, g_nt = _tail_grads_tracked(layer, s, nt, g_upd, g_out, need_s, need_nt)
            return g_s, g_nt, None
        g_s, g_nt = _tail_grads(layer, s, nt, tv, g_upd, g_out, need_s, need_nt)
        return g_s, g_nt, None


def _tail_grads(layer, s, nt, tv, g_upd, g_out, need_s, need_nt):
    """(grad s, grad nt) of the frozen tail: with ``g_lat = g_upd + g_tv T`` (T the env layer's
    weight), ``g_s = g_upd W_s + g_tv (T W_s)`` and the scalar columns of nt get
    ``g_upd W_t + g_tv (T W_t)``: two products each, the second accumulated in the same pass, and the
    latent gradient never formed."""
    tenv, F = layer.tensor_env, layer.num_tensor_features
    g_tv = None
    if g_out is not None:
        g_nt, g_tv = K.channel_scale_backward(g_out.contiguous(), nt, tv, nt.shape[1] // F, need_nt, True)
    else:
        g_nt = torch.zeros_like(nt) if need_nt else None
    if g_upd is None and g_tv is None:
        return None, (g_nt if need_nt else None)
    ws, wt, _ = _tail_weights(layer, s.shape[1])
    g_upd = g_upd.contiguous() if g_upd is not None else None

    def through(w):
        tw = tenv.weight @ w
        if g_upd is None:
            return _row_grad(g_tv, tw)
        out = _row_grad(g_upd, w)
        return _row_grad(g_tv, tw, out) if g_tv is not None else out

    g_s = through(ws) if need_s else None
    if need_nt:
        g_nt[:, :F] += through(wt)
    return g_s, (g_nt if need_nt else None)


class _LayerChain(torch.autograd.Function):
    """A whole layer with frozen parameters and the fused product + projection, its output env
    scaling left to the next layer (the first layer's tensor track, harmonics times the embedding's
    env weights, comes in the same way: V the (E, D) harmonics shared by the channels, tvp the env
    weights): env weights ``x_scale = env_embed(s)`` (times the previous
    layer's output env weights ``tvp``, which scale the tensor track channel by channel and so fold
    into the product's x_scale: TP(s (t x)) = (s t) TP(x)), ``nt = edge_tp_proj(V, Y_src, w, proj,
    x_scale)``, the tail's ``updated`` and this layer's env weights ``tv = tensor_env(updated)``.
    Returns (updated, nt, tv); the layer's tensor output is ``nt`` scaled by ``tv``, formed only
    where a caller needs it.  One Function, so that the env layer's input gradient is accumulated
    into the scalars' gradient in the same pass and the latent gradient is never formed.
    Differentiated again (create_graph), the backward runs the same formulas in tracked ops (the
    tail is linear in its inputs; the product's backward is ``molix::edge_tp``'s, which has second
    derivatives).  With ``tvp_lin`` (the embedding's frozen env layer, for the first layer) the
    env weights ``tvp = tvp_lin(s)`` of the same scalars are formed here, and their input gradient
    joins the scalars' gradient in the same accumulating product.  The fourth output is ``s`` itself:
    a caller that routes its other use of ``s`` through it (the encoder's stack of per-layer
    features) hands that gradient to this backward, which accumulates its own products into it
    instead of leaving autograd an extra pass to add the two."""

    @staticmethod
    def forward(ctx, s, V, tvp, eY, layer, w, proj, tvp_lin=None, need_tv=True):
        ee, tenv, F = layer.env_embed, layer.tensor_env, layer.num_tensor_features
        if tvp_lin is not None:
            tvp = torch.addmm(tvp_lin.bias, s, tvp_lin.weight.t())
        xs = _row_linear(s, ee.weight, ee.bias)
        nt = K.edge_tp_proj(V, eY, w, layer.tp.config_id, proj, xs, tvp)  # the product scales by xs tvp
        ws, wt, bc = _tail_weights(layer, s.shape[1])
        upd = _row_grad(nt[:, :F], wt.t().contiguous(), _row_linear(s, ws, bc))
        # the last layer's env weights scale only its tensor output, which an encoder does not return
        tv = torch.addmm(tenv.bias, upd, tenv.weight.t()) if need_tv else None
        ctx.save_for_backward(s, V, tvp, eY, w, proj, xs)
        ctx.layer, ctx.tvp_lin = layer, tvp_lin
        ctx.set_materialize_grads(False)
        return upd, nt, tv, s

    @staticmethod
    def backward(ctx, g_upd, g_nt, g_tv, g_pass):
        s, V, tvp, eY, w, proj, xs = ctx.saved_tensors
        layer, tl = ctx.layer, ctx.tvp_lin
        ee, tenv, cfg = layer.env_embed, layer.tensor_env, layer.tp.config_id
        a, b, F = layer.residual_a, layer.residual_b, layer.num_tensor_features
        need_s, need_V, need_tvp, need_eY = ctx.needs_input_grad[:4]
        need_tvp = need_tvp and tvp is not None and tl is None
        inner = tl is not None and need_s  # tvp formed here from s: its gradient joins g_s
        nout = 9
        if g_upd is None and g_nt is None and g_tv is None:
            return (g_pass,) + (None,) * (nout - 1)
        if torch.is_grad_enabled():
            lat = layer.latent_mlp[0]
            with torch.enable_grad():
                xs_t = nn.functional.linear(s, ee.weight, ee.bias)
                tvp_t = nn.functional.linear(s, tl.weight, tl.bias) if tl is not None else tvp
                xe_t = xs_t * tvp_t if tvp_t is not None else xs_t
                g_lat = None
                if g_upd is not None:
                    g_lat = g_upd
                if g_tv is not None:
                    g_lat = g_tv @ tenv.weight if g_lat is None else g_lat + g_tv @ tenv.weight
                g_s = None
                if g_lat is not None:
                    if need_s:
                        g_s = a * g_lat + g_lat @ (lat.weight[:, :s.shape[1]] * b)
                    cols = g_lat @ (lat.weight[:, s.shape[1]:] * b)
                    base = g_nt if g_nt is not None else V.new_zeros(V.shape[0], layer.irreps_dim)
                    g_nt = torch.cat([base[:, :F] + cols, base[:, F:]], dim=1)
                g_tp = K.edge_tp_proj_adjoint(g_nt, proj, K.edge_tp_proj_blocks(cfg))
                Vf = K._expand_shared_x(V, cfg)
                gV, geY, _, g_xe = K.edge_tp_backward(g_tp.contiguous(), Vf, eY, w, cfg, 16, need_V, need_eY, False,
                                                      xe_t, need_s or need_tvp)
                if need_V and Vf is not V:
                    gV = gV.reshape(V.shape[0], -1, 16).sum(-1)
                g_tvp = g_xe * xs_t if need_tvp or inner else None
                if need_s:
                    g_x = (g_xe * tvp_t if tvp_t is not None else g_xe) @ ee.weight
                    if inner:
                        g_x = g_x + g_tvp @ tl.weight
                    g_s = g_x if g_s is None else g_s + g_x
                    if g_pass is not None:
                        g_s = g_s + g_pass
            return (g_s, gV.reshape(V.shape) if need_V else None, g_tvp if need_tvp else None,
                    geY.reshape(eY.shape) if need_eY else None, None, None, None, None, None)
        ws = None
        if g_upd is not None or g_tv is not None:
            ws, wt, _ = _tail_weights(layer, s.shape[1])
            # g_upd may be a strided slice of the stacked features' gradient: the row kernel reads it
            # in place
            g_tv = g_tv.contiguous() if g_tv is not None else None

            def through(wm, out):
                # out += (g_upd + g_tv T) wm as g_upd wm + g_tv (T wm): the latent gradient is never
                # formed
                if g_upd is not None:
                    _row_grad(g_upd, wm, out)
                if g_tv is not None:
                    _row_grad(g_tv, tenv.weight @ wm, out)

            # the incoming gradient of nt is this Function's to consume (the next layer's backward
            # made it): its scalar columns take the latent part in place, in the products' own pass
            g_nt = g_nt.contiguous() if g_nt is not None else V.new_zeros(V.shape[0], layer.irreps_dim)
            through(wt, g_nt[:, :F])
        gV, geY, _, g_x, g_tvp = K.edge_tp_proj_backward(g_nt, V, eY, w, cfg, proj, need_V, need_eY, False, xs,
                                                         need_s, tvp, need_tvp or inner)
        g_s = None
        if need_s:
            # g_s = g_upd W_s + [g_tv | g_x | g_tvp] [T W_s ; W_env ; W_tvp]: the 16-wide gradients in
            # one product accumulated into the first (one pass over the (E, S) result instead of
            # one per gradient)
            heads, mats = [g_x], [ee.weight]
            if g_tv is not None:
                heads, mats = [g_tv] + heads, [tenv.weight @ ws] + mats
            if inner:
                heads, mats = heads + [g_tvp], mats + [tl.weight]
            # the pass-through output's gradient (the same scalars' other use) is this Function's
            # to consume: the products accumulate into it
            acc = g_pass.contiguous() if g_pass is not None else None
            if g_upd is not None:
                acc = _row_grad(g_upd, ws, acc)
            g_s = _row_grad(torch.cat(heads, dim=1) if len(heads) > 1 else heads[0],
                            torch.cat(mats, dim=0) if len(mats) > 1 else mats[0], acc)
        return (g_s, gV.reshape(V.shape) if need_V else None, g_tvp if need_tvp else None,
                geY.reshape(eY.shape) if need_eY else None, None, None, None, None, None)


def _tail_ok(layer, s, nt_dim):
    mods = list(layer.latent_mlp)
    F = layer.num_tensor_features
    params = [p for m in (layer.latent_mlp, layer.tensor_env) for p in m.parameters()]
    return (len(mods) == 1 and isinstance(mods[0], nn.Linear) and mods[0].bias is not None
            and layer.tensor_env.bias is not None and s.is_cuda and s.dtype == torch.float32 and s.dim() == 2
            and F % 4 == 0 and nt_dim % F == 0 and nt_dim // F in K.CHANNEL_PRODUCT_COMPONENTS
            and all(p.dtype == torch.float32 for p in params)
            and not (torch.is_grad_enabled() and any(p.requires_grad for p in params)))


def _env_lin_ok(lin, s):
    """Whether ``lin`` (an env layer of the scalars ``s``) can run inside ``_LayerChain``."""
    return (isinstance(lin, nn.Linear) and lin.bias is not None and lin.weight.dtype == torch.float32
            and lin.bias.dtype == torch.float32 and lin.in_features == s.shape[1]
            and not (torch.is_grad_enabled() and (lin.weight.requires_grad or lin.bias.requires_grad)))


def _layer_chain(layer, s, V, tvp, eY, tvp_lin=None, need_tv=True):
    """(updated, nt, tv, s) of ``_LayerChain`` when every parameter the layer reads is frozen and the
    fused product + projection applies; None otherwise.  ``tvp_lin``, given in place of ``tvp``,
    is the env layer whose output on ``s`` is ``tvp`` (formed inside the Function when frozen);
    with ``need_tv`` false, tv is None (not formed)."""
    tp, lin, ee = layer.tp, layer.tp_linear, layer.env_embed
    params = [tp.weight, lin.weight, ee.weight] + ([ee.bias] if ee.bias is not None else [])
    if (layer._proj_scale is None or ee.bias is None or not V.is_cuda or V.dtype != torch.float32
            or any(p.dtype != torch.float32 for p in params)
            or (torch.is_grad_enabled() and any(p.requires_grad for p in params))
            or not _tail_ok(layer, s, layer.irreps_dim)):
        return None
    w = tp.weight.reshape(tp.num_paths_full, tp.channels).index_select(0, tp.kept_paths)
    proj = lin.weight.reshape(-1, 16) * (layer._proj_scale * lin.output_scale if lin.output_scale != 1.0
                                         else layer._proj_scale)
    if tvp_lin is not None and not _env_lin_ok(tvp_lin, s):
        tvp, tvp_lin = tvp_lin(s), None
    return _LayerChain.apply(s.contiguous(), V.contiguous(), tvp.contiguous() if tvp is not None else None,
                             eY.contiguous(), layer, w, proj, tvp_lin, need_tv)


def _layer_tail(layer, s, nt):
    """``(updated, env-scaled nt)`` of an Allegro layer: ``_LayerTail`` when its parameters are
    frozen and the shapes fit the kernels (float32 on the GPU, one latent layer), else the tracked
    module form."""
    mods = list(layer.latent_mlp)
    F = layer.num_tensor_features
    if nt.dtype == torch.float32 and nt.dim() == 2 and _tail_ok(layer, s, nt.shape[1]):
        return _LayerTail.apply(s.contiguous(), nt.contiguous(), layer)
    return _tail_torch(s, nt, mods[0] if len(mods) == 1 else None, layer.tensor_env, layer.residual_a,
                       layer.residual_b, F) if len(mods) == 1 else _tail_modules(layer, s, nt)


def _tail_modules(layer, s, nt):
    """The tail with a latent MLP of hidden layers: the modules, b folded into the last layer."""
    F = layer.num_tensor_features
    mods = list(layer.latent_mlp)
    h = torch.cat([s, nt[:, :F]], dim=-1)
    for m in mods[:-1]:
        h = m(h)
    last = mods[-1]
    mlp = nn.functional.linear(h, last.weight * layer.residual_b,
                               last.bias * layer.residual_b if last.bias is not None else None)
    updated = torch.add(mlp, s, alpha=layer.residual_a)
    return updated, _scale_by_channel(nt, layer.tensor_env(updated), None, F)


def _full_paths(in_irreps: Irreps, sh_irreps: Irreps):
    """(l1, l2, l3, parity) of every path of the unfiltered channelwise product, in the weight
    order of cuet.ChannelWiseTensorProduct (input block, harmonics block, l3 ascending)."""
    paths = []
    for b1 in in_irreps:
        for b2 in sh_irreps:
            for l3 in range(abs(b1.ir.l - b2.ir.l), b1.ir.l + b2.ir.l + 1):
                paths.append((b1.ir.l, b2.ir.l, l3, b1.ir.p * b2.ir.p))
    return paths


class EdgeChannelWiseTensorProduct(nn.Module):
    """Per-edge channelwise product ``F x (0..l_max) (x) (0..l_max)`` with one weight per path and
    channel shared by all edges (``shared_weights=True, internal_weights=True``).  ``irreps_out``
    lists the blocks the Allegro projection reads: the paths whose output irrep is an input irrep,
    merged into one block per irrep (paths x C channels, in path order)."""

    def __init__(self, irreps_in, irreps_sh, *, dtype=None):
        super().__init__()
        self.irreps_in1 = Irreps(irreps_in)
        self.irreps_in2 = Irreps(irreps_sh)
        muls = {b.mul for b in self.irreps_in1}
        if len(muls) != 1:
            raise ValueError("EdgeChannelWiseTensorProduct needs one multiplicity for every input block")
        self.channels = muls.pop()
        ls = [b.ir.l for b in self.irreps_in1]
        if ls != list(range(len(ls))) or [b.ir.l for b in self.irreps_in2] != ls:
            raise ValueError("EdgeChannelWiseTensorProduct: input and harmonics must be l = 0..l_max, in order")
        full = _full_paths(self.irreps_in1, self.irreps_in2)
        kept_irreps = {(b.ir.l, b.ir.p) for b in self.irreps_in1}
        kept = [k for k, (l1, l2, l3, p) in enumerate(full) if (l3, p) in kept_irreps]
        self.num_paths_full = len(full)
        self.weight_numel = len(full) * self.channels
        self.register_buffer("kept_paths", torch.tensor(kept, dtype=torch.long), persistent=False)
        self.config_id = K.tp_config_id(ls, ls, ls)
        if self.config_id < 0 or not K.edge_tp_supported(self.config_id, self.channels):
            raise ValueError(f"no per-edge tensor-product kernel for l_max={ls[-1]}, {self.channels} channels")
        num_paths, nx, ny, no = K.tp_config_info(self.config_id)
        if num_paths != len(kept):
            raise RuntimeError("compiled per-edge product does not match the path enumeration")
        # one block per output irrep, (paths of that irrep) x C channels, path-major in path order
        # (molix::edge_tp's layout): the same numbers as per-path blocks sorted by irrep, with the
        # projection's weights in the same flat order, and one projection segment per irrep
        counts = {}
        for k in kept:
            l3, par = full[k][2], full[k][3]
            counts[(l3, par)] = counts.get((l3, par), 0) + 1
        self.irreps_out = Irreps(" + ".join(
            f"{n * self.channels}x{l3}{'e' if par == 1 else 'o'}" for (l3, par), n in sorted(counts.items())))
        if self.irreps_out.dim != no * self.channels:
            raise RuntimeError("compiled per-edge product output size mismatch")
        dt = dtype if dtype is not None else config.ftype
        self.weight = nn.Parameter(torch.randn(1, self.weight_numel, dtype=dt))

    def forward(self, x: torch.Tensor, y: torch.Tensor, x_scale: torch.Tensor | None = None) -> torch.Tensor:
        """``TP(x, y)``; with ``x_scale`` (E, C), ``TP(x_scale * x, y)`` channel by channel (fused)."""
        w = self.weight.reshape(self.num_paths_full, self.channels).index_select(0, self.kept_paths)
        return K.edge_tp(x, y, w, self.config_id, self.channels, x_scale)


class PairEmbedding(nn.Module):
    """Two-body embedding on edges (allegro.py:137-249): Bessel x polynomial-cutoff radial
    features, harmonics, concatenated source / destination type embeddings -> scalar MLP ->
    per-channel environment weights -> initial tensor features."""

    def __init__(self, *, num_elements: int, num_scalar_features: int, num_tensor_features: int, r_max: float,
                 num_bessel: int = 8, l_max: int = 2, type_emb_dim: int = 16,
                 scalar_mlp_hiddens: list[int] | None = None, poly_p: int = 6):
        super().__init__()
        self.num_scalar_features = num_scalar_features
        self.num_tensor_features = num_tensor_features
        self.l_max = l_max
        self.radial_basis = BesselRBF(r_cut=r_max, num_radial=num_bessel)
        self.cutoff_fn = PolynomialCutoff(r_cut=r_max, exponent=poly_p)
        self.spherical_harmonics = SphericalHarmonics(l_max=l_max)
        self.type_embedding = nn.Embedding(num_elements, type_emb_dim, dtype=config.ftype)
        widths = [num_bessel + 2 * type_emb_dim]
        widths += list(scalar_mlp_hiddens) if scalar_mlp_hiddens is not None else [num_scalar_features] * 2
        widths.append(num_scalar_features)
        layers: list[nn.Module] = []
        for a, b in zip(widths[:-1], widths[1:]):
            layers += [nn.Linear(a, b, dtype=config.ftype), nn.SiLU()]
        self.scalar_mlp = nn.Sequential(*layers)
        self.irreps_dim = Irreps(irreps_from_l_max(l_max, num_tensor_features)).dim
        self.tensor_env = nn.Linear(num_scalar_features, num_tensor_features, dtype=config.ftype)

    def parts(self, Z, bond_dist, bond_diff, edge_index, env=True):
        """(scalar features, env weights, harmonics, cutoff envelope): the embedding before the
        tensor track ``harmonics x env weights`` is formed (env weights None with ``env=False``:
        ``tensor_env`` of the scalar features, left to the caller)."""
        src, dst = edge_index[:, 0], edge_index[:, 1]
        edge_cutoff = self.cutoff_fn(bond_dist)
        edge_radial = self.radial_basis(bond_dist) * edge_cutoff.unsqueeze(-1)
        edge_angular = self.spherical_harmonics(bond_diff / (bond_dist.unsqueeze(-1) + 1e-8))
        type_embed = _type_pair_embedding(self.type_embedding, Z[src], Z[dst])
        scalar_features = _silu_stack(self.scalar_mlp, torch.cat([edge_radial, type_embed], dim=-1))
        return scalar_features, self.tensor_env(scalar_features) if env else None, edge_angular, edge_cutoff

    def forward(self, Z, bond_dist, bond_diff, edge_index):
        scalar_features, env_weights, edge_angular, edge_cutoff = self.parts(Z, bond_dist, bond_diff, edge_index)
        tensor_features = _env_weight_harmonics(edge_angular, env_weights, self.l_max, self.num_tensor_features,
                                                self.irreps_dim)
        return scalar_features, tensor_features, edge_angular, edge_cutoff


def _fused_projection_scale(tp: EdgeChannelWiseTensorProduct, lin: Linear) -> torch.Tensor | None:
    """Per-row scale (1/sqrt(fan_in) of each projected irrep) that turns the projection's weight
    vector, viewed as (paths*16, 16), into ``molix::edge_tp_proj``'s ``proj``; None when the fused
    kernel does not apply (channels other than 16, or a projection whose weight blocks are not one
    per product irrep, in the product's row order)."""
    if tp.channels != 16 or lin.weight is None or lin.weight_classes is not None:
        return None
    blocks = K.edge_tp_proj_blocks(tp.config_id)
    if not blocks or len(blocks) != len(lin.plan) or lin.weight_numel != tp.kept_paths.numel() * 256:
        return None
    scale, row = [], 0
    for (l, nb, J, I), (off_o, mul_o, d, srcs, fan_in) in zip(blocks, lin.plan):
        M = 2 * l + 1
        if (mul_o != 16 or d != M or off_o != I * 16 or len(srcs) != 1
                or srcs[0] != (row * 16, nb * 16, J * 256)):
            return None
        scale += [1.0 / math.sqrt(fan_in)] * (nb * 16)
        row += M * nb
    return torch.tensor(scale, dtype=lin.weight.dtype).unsqueeze(1)


def _product_and_projection(layer, x, y, s):
    """``tp_linear(tp(x, y, x_scale=s))`` (allegro.py:465-466).  With 16 channels, float32 on the
    GPU and projection weights that take no gradient, one ``molix::edge_tp_proj`` pass: the
    product's (E, paths x 16) rows per irrep are projected in registers and never reach memory."""
    tp, lin = layer.tp, layer.tp_linear
    sc = layer._proj_scale
    if (sc is not None and x.is_cuda and x.dtype == torch.float32 and lin.weight.dtype == torch.float32
            and not (torch.is_grad_enabled() and lin.weight.requires_grad)):
        w = tp.weight.reshape(tp.num_paths_full, tp.channels).index_select(0, tp.kept_paths)
        proj = lin.weight.reshape(-1, 16) * (sc * lin.output_scale if lin.output_scale != 1.0 else sc)
        return K.edge_tp_proj(x, y, w, tp.config_id, proj, s)
    return lin(tp(x, y, x_scale=s))


class AllegroLayer(nn.Module):
    """One Allegro layer (allegro.py:252-480): env-scaled tensor track (x) neighbourhood-aggregated
    harmonics of the edge's source, projection back to the tensor irreps, latent MLP on
    ``[scalars, fresh invariants]`` with the residual ``a x + b MLP``, output env scaling."""

    def __init__(self, *, num_scalar_features: int, num_tensor_features: int, l_max: int = 2,
                 latent_mlp_hiddens: list[int] | None = None, latent_activation: type[nn.Module] | None = nn.SiLU,
                 avg_num_neighbors: float | None = None, residual_alpha: float = 0.5):
        super().__init__()
        self.num_scalar_features = num_scalar_features
        self.num_tensor_features = num_tensor_features
        self.l_max = l_max
        self.avg_num_neighbors = float(avg_num_neighbors) if avg_num_neighbors is not None else None
        irreps = irreps_from_l_max(l_max, num_tensor_features)
        sh_irreps = sh_irreps_from_l_max(l_max)
        self.tp = EdgeChannelWiseTensorProduct(irreps, sh_irreps, dtype=config.ftype)
        self.tp_linear = Linear(self.tp.irreps_out, irreps, dtype=config.ftype)
        self.env_embed = nn.Linear(num_scalar_features, num_tensor_features, dtype=config.ftype)
        widths = [num_scalar_features + num_tensor_features] + (list(latent_mlp_hiddens) if latent_mlp_hiddens else [])
        layers: list[nn.Module] = []
        for a, b in zip(widths[:-1], widths[1:]):
            layers.append(nn.Linear(a, b, dtype=config.ftype))
            if latent_activation is not None:
                layers.append(latent_activation())
        layers.append(nn.Linear(widths[-1], num_scalar_features, dtype=config.ftype))
        self.latent_mlp = nn.Sequential(*layers)
        self.tensor_env = nn.Linear(num_scalar_features, num_tensor_features, dtype=config.ftype)
        norm = math.sqrt(1.0 + float(residual_alpha) ** 2)
        self.residual_a = 1.0 / norm
        self.residual_b = float(residual_alpha) / norm
        self.irreps_dim = Irreps(irreps).dim
        self._sh_dim = Irreps(sh_irreps).dim
        self.register_buffer("_proj_scale", _fused_projection_scale(self.tp, self.tp_linear), persistent=False)

    def source_harmonics(self, edge_angular, edge_index, n_nodes: int):
        """The harmonics of every edge summed onto its source node and normalised (1/sqrt of the
        constant average neighbour count, or of the node's out-degree), gathered back per edge
        (allegro.py:436-446); index_select (backward: one index_add) rather than node_Y[src]
        (sort-based accumulating backward)."""
        src = edge_index[:, 0]
        dt, dev = edge_angular.dtype, edge_angular.device
        node_Y = torch.zeros(n_nodes, self._sh_dim, dtype=dt, device=dev).index_add(0, src, edge_angular)
        if self.avg_num_neighbors is not None:
            node_Y = node_Y / math.sqrt(self.avg_num_neighbors)
        else:
            count = torch.zeros(n_nodes, dtype=dt, device=dev).index_add(0, src, torch.ones_like(src, dtype=dt))
            node_Y = node_Y / count.clamp(min=1.0).sqrt().unsqueeze(-1)
        return node_Y.index_select(0, src)

    def forward(self, scalar_features, tensor_features, edge_angular, edge_index, n_nodes: int):
        F = self.num_tensor_features
        edge_node_Y = self.source_harmonics(edge_angular, edge_index, n_nodes)
        chained = _layer_chain(self, scalar_features, tensor_features, None, edge_node_Y)
        if chained is not None:
            upd, nt, tv, _ = chained
            return upd, _scale_by_channel(nt, tv, self.l_max, F)
        # TP(env_w . V, Y_agg(src)): the per-channel env scaling (allegro.py:447-450) runs inside the
        # product kernel, as TP(s x) = s TP(x) channel by channel
        new_tensor = _product_and_projection(self, tensor_features, edge_node_Y, self.env_embed(scalar_features))
        # a x + b MLP([x, scalar part of the new tensor]) and the output env scaling
        return _layer_tail(self, scalar_features, new_tensor)


class AllegroSpec(BaseModel):
    """Configuration of the Allegro encoder (allegro.py:487-503)."""

    model_config = ConfigDict(arbitrary_types_allowed=True)

    num_elements: int = Field(..., gt=0)
    num_scalar_features: int = Field(64, gt=0)
    num_tensor_features: int = Field(16, gt=0)
    r_max: float = Field(..., gt=0.0)
    num_bessel: int = Field(8, gt=0)
    l_max: int = Field(2, ge=0)
    num_layers: int = Field(2, gt=0)
    poly_p: int = Field(6, ge=1)
    scalar_mlp_hiddens: list[int] | None = None
    latent_mlp_hiddens: list[int] | None = None
    avg_num_neighbors: float | None = None
    residual_alpha: float = 0.5


class Allegro(nn.Module):
    """Allegro equivariant edge encoder (allegro.py:506-642): pair embedding, ``num_layers``
    Allegro layers, per-layer scalars times the cutoff envelope stacked into
    ``edges.edge_features (n_edges, num_layers, num_scalar_features)``.  ``forward`` takes the
    reference's GraphBatch (any mapping answering ``td["edges", "bond_dist"]`` or
    ``td["edges"]["bond_dist"]``) or keyword tensors (then returns the features)."""

    in_keys = [("atoms", "Z"), ("edges", "edge_index"), ("edges", "bond_diff"), ("edges", "bond_dist")]
    out_keys = [("edges", "edge_features")]

    def __init__(self, *, num_elements: int, num_scalar_features: int = 64, num_tensor_features: int = 16,
                 r_max: float, num_bessel: int = 8, l_max: int = 2, num_layers: int = 2, poly_p: int = 6,
                 scalar_mlp_hiddens: list[int] | None = None, latent_mlp_hiddens: list[int] | None = None,
                 latent_activation: type[nn.Module] | None = nn.SiLU, avg_num_neighbors: float | None = None,
                 residual_alpha: float = 0.5):
        super().__init__()
        self.config = AllegroSpec(num_elements=num_elements, num_scalar_features=num_scalar_features,
                                  num_tensor_features=num_tensor_features, r_max=r_max, num_bessel=num_bessel,
                                  l_max=l_max, num_layers=num_layers, poly_p=poly_p,
                                  scalar_mlp_hiddens=scalar_mlp_hiddens, latent_mlp_hiddens=latent_mlp_hiddens,
                                  avg_num_neighbors=avg_num_neighbors, residual_alpha=residual_alpha)
        self.embedding = PairEmbedding(num_elements=num_elements, num_scalar_features=num_scalar_features,
                                       num_tensor_features=num_tensor_features, r_max=r_max, num_bessel=num_bessel,
                                       l_max=l_max, scalar_mlp_hiddens=scalar_mlp_hiddens, poly_p=poly_p)
        self.layers = nn.ModuleList([
            AllegroLayer(num_scalar_features=num_scalar_features, num_tensor_features=num_tensor_features,
                         l_max=l_max, latent_mlp_hiddens=latent_mlp_hiddens, latent_activation=latent_activation,
                         avg_num_neighbors=avg_num_neighbors, residual_alpha=residual_alpha)
            for _ in range(num_layers)
        ])

    def encode(self, Z, bond_dist, bond_diff, edge_index):
        emb = self.embedding
        scalars, _, edge_angular, edge_cutoff = emb.parts(Z, bond_dist, bond_diff, edge_index, env=False)
        # the tensor track enters the first layer as the harmonics shared by the channels with the
        # env weights as its channel scale (folded into the layer's product), when the layer takes
        # it; the env weights are then formed inside the layer's Function (``env_lin``)
        tensors, tv, env_lin = edge_angular, None, emb.tensor_env
        u = edge_cutoff.unsqueeze(-1)
        per_layer = []
        n = int(Z.shape[0])
        src_Y = {}  # the source harmonics depend on the layer only through its normalisation
        for k, layer in enumerate(self.layers):
            key = layer.avg_num_neighbors
            if key not in src_Y:
                src_Y[key] = layer.source_harmonics(edge_angular, edge_index, n)
            chained = _layer_chain(layer, scalars, tensors, tv, src_Y[key], env_lin, k + 1 < len(self.layers))
            if chained is not None:
                scalars_in = scalars
                scalars, tensors, tv, passed = chained
                if per_layer and per_layer[-1] is scalars_in:
                    per_layer[-1] = passed  # the previous layer's features, routed through this Function
            else:
                if env_lin is not None:
                    tv = env_lin(scalars)
                if tensors is edge_angular:  # first layer: form the tensor track
                    tensors = _env_weight_harmonics(edge_angular, tv, emb.l_max, emb.num_tensor_features,
                                                    emb.irreps_dim)
                elif tv is not None:
                    tensors = _scale_by_channel(tensors, tv, layer.l_max, layer.num_tensor_features)
                tv = None
                scalars, tensors = layer(scalars, tensors, edge_angular, edge_index, n)
            env_lin = None
            per_layer.append(scalars)
        # every layer's scalars times the cutoff envelope, written into the stack in one pass
        return _envelope_stack(per_layer, u)

    def forward(self, td=None, *, Z=None, bond_dist=None, bond_diff=None, edge_index=None):
        if td is None:
            return self.encode(Z, bond_dist, bond_diff, edge_index)
        feats = self.encode(_get(td, "atoms", "Z"), _get(td, "edges", "bond_dist"), _get(td, "edges", "bond_diff"),
                            _get(td, "edges", "edge_index"))
        _set(td, "edges", "edge_features", feats)
        return td


__all__ = ["Allegro", "AllegroLayer", "AllegroSpec", "EdgeChannelWiseTensorProduct", "PairEmbedding"]
