"""Torch custom ops (namespace ``molix``) over the molnex C ABI.

Every op here runs the HIP kernels of ``lib/libmolnex_hip.so`` on the current
stream; there are no CPU implementations (a CPU tensor raises).  Fake (meta)
implementations and autograd formulas are registered so the ops trace under
``torch.compile`` / ``torch.export`` like the reference's ops
(``src/molix/op/src/molix_meta.cpp:19-70``).

Ops
---
``molix::get_neighbor_pairs``   reference schema, verbatim (``molix_library.cpp:22-26``)
``molix::neighbor_list``        directed / half cell list, exact size, sorted (i, j)
``molix::spherical_harmonics``  real SH l <= 3 (``cuet.SphericalHarmonics``)
``molix::edge_csr``             receiver CSR of an (E, 2) edge list
``molix::tp_scatter``           channelwise TP + scatter-sum (``cuet.ChannelWiseTensorProduct``)
``molix::tp_any``               the same for any irreps (l <= 3), driven by a path table
``molix::edge_tp``              per-edge channelwise TP with shared weights, no scatter (Allegro's layer product)
``molix::edge_tp_proj``         ``edge_tp`` (16 channels) and the projection after it in one pass (Allegro)
``molix::radial_hidden``        fused hidden stack of the radial weight MLP (gradient w.r.t. its input)
``molix::edge_weights``         output layer of the radial weight MLP (per-edge TP weights), near-fp32 split-fp16 MFMA
``molix::bond_vectors``         pos[receiver] - pos[sender] - shift per edge, with its position gradient
``molix::block_linear``         equivariant (ir_mul) block linear with pre-ordered weights (``cuet.Linear``)
``molix::indexed_block_linear`` the block linear with one weight set per node class (ElementUpdate)
``molix::radial_tp``            radial-MLP output layer + tp_scatter, backward through ``molix::tp_weight_grad``
``molix::edge_reverse``         the opposite edge of each edge (undirected pairs with identical radial inputs)
``molix::radial_tp_pairs``      radial-MLP output layer once per undirected pair + tp_scatter over both directions
``molix::segment_sum``          weighted segment sum of rows by segment id (scatter_sum / MessageAggregation)
"""

from __future__ import annotations

import ctypes as C
import warnings

C_int32_5 = C.c_int32 * 5

import torch
from torch import Tensor

from . import _lib
from ._lib import check, ptr
from .config import config as _settings

MNX_NLIST_HALF, MNX_NLIST_FULL = 0, 1
MNX_NLIST_COMPACT, MNX_NLIST_TRIANGULAR = 0, 1


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_gpu(name: str, *ts: Tensor) -> None:
    for t in ts:
        if t is not None and t.numel() > 0 and t.device.type != "cuda":
            raise RuntimeError(f"molix::{name} runs on the GPU only (got a {t.device} tensor)")


def _ws(nbytes: int, device) -> Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# Neighbor list
# ---------------------------------------------------------------------------


def _nlist_run(positions: Tensor, cutoff: float, box: Tensor | None, mode: int):
    """Stage 1 of the cell list; returns (workspace, total pair count on host)."""
    lib = _lib.load()
    n = positions.shape[0]
    f64 = positions.dtype == torch.float64
    ws = _ws(lib.mnx_nlist_workspace_bytes(n), positions.device)
    total = torch.empty(1, dtype=torch.int64, device=positions.device)
    fn = lib.mnx_nlist_count_f64 if f64 else lib.mnx_nlist_count_f32
    check(fn(ptr(positions), n, float(cutoff), ptr(box), mode, ptr(ws), ws.numel(), ptr(total),
             _stream(positions)), "neighbor list count")
    t = int(total.item())
    if t < 0:
        raise _lib.MolnexError("neighbor list: an atom has more than 4096 neighbours within the cutoff")
    return ws, t


def _nlist_emit(positions, cutoff, box, mode, layout, ws, capacity, idx_i, idx_j, deltas, dist, shifts):
    lib = _lib.load()
    f64 = positions.dtype == torch.float64
    fn = lib.mnx_nlist_emit_f64 if f64 else lib.mnx_nlist_emit_f32
    check(fn(ptr(positions), positions.shape[0], float(cutoff), ptr(box), mode, layout, ptr(ws), ws.numel(),
             capacity, ptr(idx_i), ptr(idx_j), ptr(deltas), ptr(dist), ptr(shifts), _stream(positions)),
          "neighbor list emit")


def _prep_positions(positions: Tensor, box_vectors: Tensor):
    if positions.dtype not in (torch.float32, torch.float64):
        raise TypeError("positions must be float32 or float64")
    pos = positions.detach().contiguous()
    box = None
    if box_vectors is not None and box_vectors.numel() != 0:
        if tuple(box_vectors.shape) != (3, 3):
            raise ValueError("box_vectors must be (3, 3) or empty")
        box = box_vectors.detach().to(device=pos.device, dtype=pos.dtype).contiguous()
    return pos, box


@torch.library.custom_op(
    "molix::get_neighbor_pairs",
    mutates_args=(),
    device_types="cuda",
    schema="(Tensor positions, Scalar cutoff, Scalar max_num_pairs, Tensor box_vectors) -> "
    "(Tensor neighbors, Tensor deltas, Tensor distances, Tensor num_pairs)",
)
def get_neighbor_pairs(positions, cutoff, max_num_pairs, box_vectors):
    """Half pair list within ``cutoff`` (reference ``get_neighbor_pairs.cpp:28-77``).

    ``max_num_pairs == -1``: width ``N(N-1)/2``, pair (i, j) at slot
    ``i(i-1)/2 + j``; otherwise width ``max_num_pairs`` with the pairs sorted by
    (i, j) first (the first ``max_num_pairs`` of them when there are more,
    like the CUDA/meta widths, ``molix_meta.cpp:25-27``).  Padding is -1 / NaN.
    """
    _require_gpu("get_neighbor_pairs", positions, box_vectors)
    pos, box = _prep_positions(positions, box_vectors)
    n = pos.shape[0]
    mnp = int(max_num_pairs)
    width = n * (n - 1) // 2 if mnp == -1 else mnp
    layout = MNX_NLIST_TRIANGULAR if mnp == -1 else MNX_NLIST_COMPACT
    neighbors = torch.empty((2, width), dtype=torch.int32, device=pos.device)
    deltas = torch.empty((width, 3), dtype=pos.dtype, device=pos.device)
    distances = torch.empty((width,), dtype=pos.dtype, device=pos.device)
    ws, total = _nlist_run(pos, float(cutoff), box, MNX_NLIST_HALF)
    if total > width:
        # the reference's CPU path widens its outputs to every pair here; this op keeps the
        # schema width as its CUDA path does, so say so once per call site
        warnings.warn(f"get_neighbor_pairs: {total} pairs within the cutoff, max_num_pairs={width}: "
                      "the outputs hold the first max_num_pairs pairs in (i, j) order, num_pairs the full "
                      "count", RuntimeWarning, stacklevel=2)
    _nlist_emit(pos, float(cutoff), box, MNX_NLIST_HALF, layout, ws, width, neighbors[0], neighbors[1], deltas,
                distances, None)
    num_pairs = torch.full((1,), total, dtype=torch.int32, device=pos.device)
    return neighbors, deltas, distances, num_pairs


@get_neighbor_pairs.register_fake
def _(positions, cutoff, max_num_pairs, box_vectors):
    n = positions.shape[0]
    mnp = int(max_num_pairs)
    width = n * (n - 1) // 2 if mnp == -1 else mnp
    return (
        positions.new_empty((2, width), dtype=torch.int32),
        positions.new_empty((width, 3)),
        positions.new_empty((width,)),
        positions.new_empty((1,), dtype=torch.int32),
    )


@torch.library.custom_op("molix::get_neighbor_pairs_backward", mutates_args=(), device_types="cuda")
def get_neighbor_pairs_backward(neighbors: Tensor, deltas: Tensor, distances: Tensor, grad_deltas: Tensor,
                                grad_distances: Tensor, num_atoms: int) -> Tensor:
    """d/d positions of <g_deltas, deltas> + <g_dist, distances> (``get_neighbor_pairs.cu:81-102``)."""
    lib = _lib.load()
    gpos = torch.zeros((num_atoms, 3), dtype=deltas.dtype, device=deltas.device)
    width = neighbors.shape[1]
    nb = neighbors.contiguous()
    fn = lib.mnx_nlist_backward_f64 if deltas.dtype == torch.float64 else lib.mnx_nlist_backward_f32
    check(fn(ptr(nb[0]), ptr(nb[1]), ptr(deltas.contiguous()), ptr(distances.contiguous()),
             ptr(grad_deltas.contiguous()), ptr(grad_distances.contiguous()), width, num_atoms, ptr(gpos),
             _stream(deltas)), "get_neighbor_pairs backward")
    return gpos


@get_neighbor_pairs_backward.register_fake
def _(neighbors, deltas, distances, grad_deltas, grad_distances, num_atoms):
    return deltas.new_empty((num_atoms, 3))


def _gnp_setup(ctx, inputs, output):
    positions = inputs[0]
    neighbors, deltas, distances, _ = output
    ctx.save_for_backward(neighbors, deltas, distances)
    ctx.num_atoms = positions.shape[0]


def _gnp_backward(ctx, g_neighbors, g_deltas, g_distances, g_num):
    neighbors, deltas, distances = ctx.saved_tensors
    if g_deltas is None:
        g_deltas = torch.zeros_like(deltas)
    if g_distances is None:
        g_distances = torch.zeros_like(distances)
    gpos = get_neighbor_pairs_backward(neighbors, deltas, distances, g_deltas, g_distances, ctx.num_atoms)
    return gpos, None, None, None


get_neighbor_pairs.register_autograd(_gnp_backward, setup_context=_gnp_setup)


@torch.library.custom_op("molix::neighbor_list", mutates_args=(), device_types="cuda")
def neighbor_list(positions: Tensor, cutoff: float, box_vectors: Tensor, full: bool) -> tuple[
        Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Exact-size cell list sorted by (i, j): ``full`` gives all ordered pairs i != j,
    otherwise the reference half list (i > j).

    Returns ``(i, j, shifts, deltas, distances)``: int32 ``i``/``j``; ``deltas``
    = the reference's minimum-image ``pos[i] - pos[j]`` (bit-exact), ``shifts``
    the image offset with ``deltas = pos[i] - (pos[j] + shifts)``.
    """
    _require_gpu("neighbor_list", positions, box_vectors)
    pos, box = _prep_positions(positions, box_vectors)
    mode = MNX_NLIST_FULL if full else MNX_NLIST_HALF
    ws, total = _nlist_run(pos, cutoff, box, mode)
    dev, dt = pos.device, pos.dtype
    ii = torch.empty(total, dtype=torch.int32, device=dev)
    jj = torch.empty(total, dtype=torch.int32, device=dev)
    sh = torch.empty((total, 3), dtype=dt, device=dev)
    dd = torch.empty((total, 3), dtype=dt, device=dev)
    dist = torch.empty(total, dtype=dt, device=dev)
    _nlist_emit(pos, cutoff, box, mode, MNX_NLIST_COMPACT, ws, total, ii, jj, dd, dist, sh)
    return ii, jj, sh, dd, dist


@neighbor_list.register_fake
def _(positions, cutoff, box_vectors, full):
    ctx = torch.library.get_ctx()
    e = ctx.new_dynamic_size()
    return (positions.new_empty((e,), dtype=torch.int32), positions.new_empty((e,), dtype=torch.int32),
            positions.new_empty((e, 3)), positions.new_empty((e, 3)), positions.new_empty((e,)))


# ---------------------------------------------------------------------------
# Spherical harmonics
# ---------------------------------------------------------------------------


def _f32_rows(t: Tensor, width: int, what: str) -> Tensor:
    if t.dtype != torch.float32:
        raise TypeError(f"{what} must be float32 (the HIP kernels compute in fp32), got {t.dtype}")
    return t.reshape(-1, width).contiguous()


@torch.library.custom_op("molix::spherical_harmonics", mutates_args=(), device_types="cuda")
def spherical_harmonics(vectors: Tensor, l_max: int) -> Tensor:
    """Real harmonics ``[Y^0 .. Y^l_max]`` of normalised ``vectors`` (..., 3)."""
    _require_gpu("spherical_harmonics", vectors)
    v = _f32_rows(vectors, 3, "vectors")
    d = (l_max + 1) ** 2
    out = torch.empty((v.shape[0], d), dtype=torch.float32, device=v.device)
    check(_lib.load().mnx_sh_fwd_f32(ptr(v), v.shape[0], l_max, ptr(out), _stream(v)), "spherical_harmonics")
    return out.reshape(*vectors.shape[:-1], d)


@spherical_harmonics.register_fake
def _(vectors, l_max):
    return vectors.new_empty((*vectors.shape[:-1], (l_max + 1) ** 2))


@torch.library.custom_op("molix::spherical_harmonics_backward", mutates_args=(), device_types="cuda")
def spherical_harmonics_backward(vectors: Tensor, grad: Tensor, l_max: int) -> Tensor:
    v = _f32_rows(vectors, 3, "vectors")
    d = (l_max + 1) ** 2
    g = _f32_rows(grad, d, "grad")
    gv = torch.empty_like(v)
    check(_lib.load().mnx_sh_bwd_f32(ptr(v), ptr(g), v.shape[0], l_max, ptr(gv), _stream(v)),
          "spherical_harmonics backward")
    return gv.reshape(vectors.shape)


@spherical_harmonics_backward.register_fake
def _(vectors, grad, l_max):
    return torch.empty_like(vectors)


def _sh_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0])
    ctx.l_max = inputs[1]


def _sh_backward(ctx, grad):
    (v,) = ctx.saved_tensors
    return spherical_harmonics_backward(v, grad, ctx.l_max), None


spherical_harmonics.register_autograd(_sh_backward, setup_context=_sh_setup)


# ---------------------------------------------------------------------------
# Receiver CSR and the channelwise tensor product
# ---------------------------------------------------------------------------


@torch.library.custom_op("molix::edge_csr", mutates_args=(), device_types="cuda")
def edge_csr(edge_index: Tensor, num_nodes: int, validate: bool = True) -> tuple[Tensor, Tensor, Tensor]:
    """Receiver CSR of ``edge_index`` (E, 2) = [sender, receiver]: ``(row_ptr, perm, senders)``.

    With ``validate`` (one host synchronisation) it raises if an index lies outside
    ``[0, num_nodes)``; without it such edges are left out of the CSR unchecked, the
    trusted-input convention of the reference's ops (``src/molix/F/locality.py:3-5``).
    """
    _require_gpu("edge_csr", edge_index)
    if edge_index.ndim != 2 or edge_index.shape[1] != 2:
        raise ValueError(f"edge_index must be (E, 2), got {tuple(edge_index.shape)}")
    lib = _lib.load()
    ei = edge_index.to(torch.int64).contiguous()
    E = ei.shape[0]
    dev = ei.device
    row_ptr = torch.empty(num_nodes + 1, dtype=torch.int32, device=dev)
    perm = torch.empty(E, dtype=torch.int32, device=dev)
    snd = torch.empty(E, dtype=torch.int32, device=dev)
    invalid = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = _ws(lib.mnx_csr_workspace_bytes(num_nodes, E), dev)
    check(lib.mnx_csr_build(ptr(ei), E, num_nodes, ptr(row_ptr), ptr(perm), ptr(snd), ptr(invalid), ptr(ws),
                            ws.numel(), _stream(ei)), "edge_csr")
    if validate and E > 0:
        bad = int(invalid.item())
        if bad != 0:
            raise ValueError(f"edge_index has {bad} edges with a node index outside [0, {num_nodes})")
    return row_ptr, perm, snd


@edge_csr.register_fake
def _(edge_index, num_nodes, validate=True):
    E = edge_index.shape[0]
    return (edge_index.new_empty((num_nodes + 1,), dtype=torch.int32),
            edge_index.new_empty((E,), dtype=torch.int32), edge_index.new_empty((E,), dtype=torch.int32))


def tp_config_id(in_ls, sh_ls, out_ls) -> int:
    mask = lambda ls: sum(1 << l for l in ls)  # noqa: E731
    return int(_lib.load().mnx_tp_config(mask(in_ls), mask(sh_ls), mask(out_ls)))


def tp_config_info(config: int) -> tuple[int, int, int, int]:
    info = (C.c_int32 * 4)()
    check(_lib.load().mnx_tp_config_info(config, info), "tp_config_info")
    return tuple(info)


def _check_wrow(wrow: Tensor | None, E: int, Ew: int, what: str) -> None:
    if wrow is None:
        if Ew != E:
            raise ValueError(f"{what}: w has {Ew} rows for {E} edges")
    elif wrow.dtype != torch.int32 or wrow.shape != (E,) or not wrow.is_contiguous():
        raise ValueError(f"{what}: wrow must be a contiguous int32 ({E},) tensor")


@torch.library.custom_op("molix::tp_scatter", mutates_args=(), device_types="cuda")
def tp_scatter(x: Tensor, Y: Tensor, w: Tensor, row_ptr: Tensor, perm: Tensor, senders: Tensor, config: int,
               channels: int, s_row_ptr: Tensor | None = None, s_perm: Tensor | None = None,
               s_receivers: Tensor | None = None, wrow: Tensor | None = None) -> Tensor:
    """``out[r] = sum_{e -> r} TP(x[send(e)], Y[e]; w[e])`` for a compiled configuration.

    ``(row_ptr, perm, senders)`` is the receiver CSR (``edge_csr``).  The optional sender CSR
    (``edge_csr`` of the column-swapped edge list) selects the atomic-free backward.  With ``wrow``
    (int32, one entry per edge) edge e takes its weights from row ``wrow[e]`` of ``w`` (rows shared
    by edges with equal weights, e.g. the two directions of an undirected pair)."""
    _require_gpu("tp_scatter", x, Y, w, row_ptr)
    num_paths, nx, ny, no = tp_config_info(config)
    N = row_ptr.shape[0] - 1
    E = Y.shape[0]
    xs = _f32_rows(x, nx * channels, "x")
    Ys = _f32_rows(Y, ny, "Y")
    ws_ = _f32_rows(w, num_paths * channels, "w")
    if xs.shape[0] != N or perm.shape[0] != E:
        raise ValueError("tp_scatter: inconsistent sizes of x / Y / CSR")
    _check_wrow(wrow, E, ws_.shape[0], "tp_scatter")
    if s_row_ptr is not None and (s_row_ptr.shape[0] != N + 1 or s_perm is None or s_receivers is None
                                  or s_perm.shape[0] != E or s_receivers.shape[0] != E):
        raise ValueError("tp_scatter: inconsistent sender CSR")
    out = torch.empty((N, no * channels), dtype=torch.float32, device=xs.device)
    check(_lib.load().mnx_tp_fwd_rows_f32(config, channels, ptr(xs), ptr(Ys), ptr(ws_), ptr(wrow), ptr(row_ptr),
                                          ptr(perm), ptr(senders), N, E, ptr(out), _stream(xs)), "tp_scatter")
    return out


@tp_scatter.register_fake
def _(x, Y, w, row_ptr, perm, senders, config, channels, s_row_ptr=None, s_perm=None, s_receivers=None, wrow=None):
    num_paths, nx, ny, no = tp_config_info(config)
    return x.new_empty((row_ptr.shape[0] - 1, no * channels))


@torch.library.custom_op("molix::tp_scatter_backward", mutates_args=(), device_types="cuda")
def tp_scatter_backward(grad_out: Tensor, x: Tensor, Y: Tensor, w: Tensor, row_ptr: Tensor, perm: Tensor,
                        senders: Tensor, config: int, channels: int, need_x: bool, need_Y: bool,
                        need_w: bool, s_row_ptr: Tensor | None = None, s_perm: Tensor | None = None,
                        s_receivers: Tensor | None = None, wrow: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """Gradients of ``<grad_out, tp_scatter(...)>`` w.r.t. x, Y, w (empty when not needed).
    With the sender CSR the gradients are walked by sender (grad_x without atomics).  With
    ``wrow`` the weight gradient is per edge, (E, num_paths * C), not yet summed over the edges
    that share a row of ``w``."""
    lib = _lib.load()
    num_paths, nx, ny, no = tp_config_info(config)
    N = row_ptr.shape[0] - 1
    E = Y.shape[0]
    xs = _f32_rows(x, nx * channels, "x")
    Ys = _f32_rows(Y, ny, "Y")
    wss = _f32_rows(w, num_paths * channels, "w")
    go = _f32_rows(grad_out, no * channels, "grad_out")
    _check_wrow(wrow, E, wss.shape[0], "tp_scatter_backward")
    dev = xs.device
    by_sender = s_row_ptr is not None
    if need_x:
        gx = torch.empty_like(xs) if by_sender else torch.zeros_like(xs)
    else:
        gx = xs.new_empty(0)
    gY = torch.empty_like(Ys) if need_Y else Ys.new_empty(0)
    gw = wss.new_empty(E, num_paths * channels) if need_w else wss.new_empty(0)
    if by_sender:
        check(lib.mnx_tp_bwd_sender_rows_f32(config, channels, ptr(xs), ptr(Ys), ptr(wss), ptr(wrow), ptr(go),
                                             ptr(s_row_ptr), ptr(s_perm), ptr(s_receivers), N, E, ptr(gx), ptr(gY),
                                             ptr(gw), _stream(xs)), "tp_scatter backward (by sender)")
    else:
        ws = _ws(lib.mnx_tp_bwd_workspace_bytes(config, channels, E) if need_Y else 1, dev)
        check(lib.mnx_tp_bwd_rows_f32(config, channels, ptr(xs), ptr(Ys), ptr(wss), ptr(wrow), ptr(go),
                                      ptr(row_ptr), ptr(perm), ptr(senders), N, E, ptr(gx), ptr(gY), ptr(gw),
                                      ptr(ws), ws.numel(), _stream(xs)), "tp_scatter backward")
    if E == 0:
        gY.zero_() if need_Y else None
    return gx, gY, gw


@tp_scatter_backward.register_fake
def _(grad_out, x, Y, w, row_ptr, perm, senders, config, channels, need_x, need_Y, need_w, s_row_ptr=None,
      s_perm=None, s_receivers=None, wrow=None):
    return (torch.empty_like(x) if need_x else x.new_empty(0), torch.empty_like(Y) if need_Y else Y.new_empty(0),
            w.new_empty(Y.shape[0], w.shape[1]) if need_w else w.new_empty(0))


def _tp_setup(ctx, inputs, output):
    x, Y, w, row_ptr, perm, senders, config, channels, s_row_ptr, s_perm, s_receivers, wrow = inputs
    ctx.save_for_backward(x, Y, w, row_ptr, perm, senders, wrow)
    ctx.sender_csr = (s_row_ptr, s_perm, s_receivers)
    ctx.config, ctx.channels = config, channels


def _tp_backward(ctx, grad_out):
    x, Y, w, row_ptr, perm, senders, wrow = ctx.saved_tensors
    nx, nY, nw = ctx.needs_input_grad[:3]
    gx, gY, gw = tp_scatter_backward(grad_out.contiguous(), x, Y, w, row_ptr, perm, senders, ctx.config,
                                     ctx.channels, nx, nY, nw, *ctx.sender_csr, wrow)
    if nw and wrow is not None:  # sum the per-edge gradients over the edges that share a row
        gw = torch.zeros(w.shape[0], gw.shape[1], dtype=gw.dtype, device=gw.device).index_add_(0, wrow.long(), gw)
    return (gx.reshape(x.shape) if nx else None, gY.reshape(Y.shape) if nY else None,
            gw.reshape(w.shape) if nw else None, None, None, None, None, None, None, None, None, None)


tp_scatter.register_autograd(_tp_backward, setup_context=_tp_setup)


def tp_any_table(desc) -> list[int]:
    """Path table of ``molix::tp_any`` for a ``ChannelwiseTPDescriptor``: ``[P, NX, NY, NO, NW]``
    then per path ``[triple, x offset, Y offset, output offset, weight offset, multiplicity]`` (offsets
    in floats within a row; ir_mul blocks; weight segments in path order; output blocks in the
    descriptor's sorted order)."""
    lib = _lib.load()
    in1, in2, out = desc.irreps_in1, desc.irreps_in2, desc.irreps_out
    off1, off2, off3 = in1.offsets(), in2.offsets(), out.offsets()
    table = [desc.num_paths, in1.dim, in2.dim, out.dim, desc.weight_numel]
    woff = 0
    for p in desc.paths:
        t = int(lib.mnx_tp_any_triple(p.l1, p.l2, p.l3))
        if t < 0:
            raise ValueError(f"tp_any: no coupling kernel for ({p.l1}, {p.l2} -> {p.l3})")
        mul = in1[p.i1].mul
        table += [t, off1[p.i1], off2[p.i2], off3[p.out_block], woff, mul]
        woff += mul
    return table


def _any_dims(table: list[int]) -> tuple[int, int, int, int]:
    return table[1], table[2], table[3], table[4]


def _any_ctable(table: list[int]):
    return (C.c_int32 * len(table))(*table), len(table)


@torch.library.custom_op("molix::tp_any", mutates_args=(), device_types="cuda")
def tp_any(x: Tensor, Y: Tensor, w: Tensor, row_ptr: Tensor, perm: Tensor, senders: Tensor,
           table: list[int]) -> Tensor:
    """``out[r] = sum_{e -> r} TP(x[send(e)], Y[e]; w[e])`` for any irreps with l <= 3, driven by the
    path table of ``tp_any_table`` (the compiled ``tp_scatter`` configurations cover uniform
    multiplicity, natural parity and one block per l)."""
    _require_gpu("tp_any", x, Y, w, row_ptr)
    nx, ny, no, nw = _any_dims(table)
    N = row_ptr.shape[0] - 1
    E = Y.shape[0]
    if no == 0:  # no path survives the output filter
        return torch.zeros((N, 0), dtype=torch.float32, device=x.device)
    xs = _f32_rows(x, nx, "x")
    Ys = _f32_rows(Y, ny, "Y")
    ws_ = _f32_rows(w, nw, "w")
    if xs.shape[0] != N or perm.shape[0] != E or senders.shape[0] != E or ws_.shape[0] != E:
        raise ValueError("tp_any: inconsistent sizes of x / Y / w / CSR")
    out = torch.empty((N, no), dtype=torch.float32, device=xs.device)
    tb, n = _any_ctable(table)
    check(_lib.load().mnx_tp_any_fwd_f32(tb, n, ptr(xs), ptr(Ys), ptr(ws_), ptr(row_ptr), ptr(perm), ptr(senders),
                                         N, E, ptr(out), _stream(xs)), "tp_any")
    return out


@tp_any.register_fake
def _(x, Y, w, row_ptr, perm, senders, table):
    return x.new_empty((row_ptr.shape[0] - 1, table[3]))


@torch.library.custom_op("molix::tp_any_backward", mutates_args=(), device_types="cuda")
def tp_any_backward(grad_out: Tensor, x: Tensor, Y: Tensor, w: Tensor, row_ptr: Tensor, perm: Tensor,
                    senders: Tensor, table: list[int], need_x: bool, need_Y: bool,
                    need_w: bool) -> tuple[Tensor, Tensor, Tensor]:
    """Gradients of ``<grad_out, tp_any(...)>`` w.r.t. x and Y (fp32 atomics) and w (empty when not
    needed)."""
    nx, ny, no, nw = _any_dims(table)
    N = row_ptr.shape[0] - 1
    E = Y.shape[0]
    if no == 0:
        return (torch.zeros_like(x) if need_x else x.new_empty(0), torch.zeros_like(Y) if need_Y else Y.new_empty(0),
                w.new_zeros(E, 0) if need_w else w.new_empty(0))
    xs = _f32_rows(x, nx, "x")
    Ys = _f32_rows(Y, ny, "Y")
    wss = _f32_rows(w, nw, "w")
    go = _f32_rows(grad_out, no, "grad_out")
    if (xs.shape[0] != N or go.shape[0] != N or wss.shape[0] != E or perm.shape[0] != E
            or senders.shape[0] != E):
        raise ValueError("tp_any_backward: inconsistent sizes of x / grad_out / w / CSR")
    gx = torch.zeros_like(xs) if need_x else xs.new_empty(0)
    gY = torch.zeros_like(Ys) if need_Y else Ys.new_empty(0)
    gw = wss.new_empty(E, nw) if need_w else wss.new_empty(0)
    tb, n = _any_ctable(table)
    check(_lib.load().mnx_tp_any_bwd_f32(tb, n, ptr(xs), ptr(Ys), ptr(wss), ptr(go), ptr(row_ptr), ptr(perm),
                                         ptr(senders), N, E, ptr(gx) if need_x else None,
                                         ptr(gY) if need_Y else None, ptr(gw) if need_w else None, _stream(xs)),
          "tp_any backward")
    return gx, gY, gw


@tp_any_backward.register_fake
def _(grad_out, x, Y, w, row_ptr, perm, senders, table, need_x, need_Y, need_w):
    return (torch.empty_like(x) if need_x else x.new_empty(0), torch.empty_like(Y) if need_Y else Y.new_empty(0),
            w.new_empty(Y.shape[0], w.shape[1]) if need_w else w.new_empty(0))


def _tp_any_setup(ctx, inputs, output):
    x, Y, w, row_ptr, perm, senders, table = inputs
    ctx.save_for_backward(x, Y, w, row_ptr, perm, senders)
    ctx.table = table


def _tp_any_bwd(ctx, grad_out):
    x, Y, w, row_ptr, perm, senders = ctx.saved_tensors
    nx, nY, nw = ctx.needs_input_grad[:3]
    gx, gY, gw = tp_any_backward(grad_out.contiguous(), x, Y, w, row_ptr, perm, senders, ctx.table, nx, nY, nw)
    return (gx.reshape(x.shape) if nx else None, gY.reshape(Y.shape) if nY else None,
            gw.reshape(w.shape) if nw else None, None, None, None, None)


tp_any.register_autograd(_tp_any_bwd, setup_context=_tp_any_setup)


def edge_tp_supported(config: int, channels: int) -> bool:
    """Whether ``molix::edge_tp`` has a kernel for this configuration and channel count."""
    return config >= 0 and _lib.load().mnx_edge_tp_bwd_workspace_bytes(config, channels, 1) > 0


def edge_tp_out_rows(ls: list[int]) -> list[int]:
    """Output layout of ``molix::edge_tp`` for input, harmonics and outputs l = ``ls``: entry i is the
    row (C channels each) that holds row i of the per-path layout (one block per path, blocks
    sorted by output irrep in path order, component-major within a block).  The kernel stores the
    paths that share an output irrep as one block of multiplicity (paths x C), component
    outermost: row = first row of the irrep + m3 * (its paths) + the path's rank among them."""
    from .irreps import ChannelwiseTPDescriptor, Irreps

    irr = Irreps(" + ".join(f"1x{l}{'e' if l % 2 == 0 else 'o'}" for l in ls))
    d = ChannelwiseTPDescriptor(irr, irr, irr)
    offs = [0]
    for b in d.irreps_out:
        offs.append(offs[-1] + b.ir.dim)
    by_l = {}
    for p in sorted(d.paths, key=lambda p: offs[p.out_block]):
        by_l.setdefault(p.l3, []).append(p)
    rows = [0] * offs[-1]
    for l3, ps in by_l.items():
        base = min(offs[p.out_block] for p in ps)
        for b, p in enumerate(ps):
            for m3 in range(2 * l3 + 1):
                rows[offs[p.out_block] + m3] = base + m3 * len(ps) + b
    return rows


@torch.library.custom_op("molix::edge_tp", mutates_args=(), device_types="cuda")
def edge_tp(x: Tensor, Y: Tensor, w: Tensor, config: int, channels: int, x_scale: Tensor | None = None) -> Tensor:
    """``out[e] = TP(s[e] * x[e], Y[e]; w)``: per-edge channelwise product with weights shared by
    all edges (``w`` is ``(num_paths, C)``), no scatter -- Allegro's layer product
    (src/molzoo/allegro.py:352-359,457-458); the optional ``x_scale`` ``(E, C)`` multiplies every
    component of channel c of x[e] first (the env weights of allegro.py:447-450).  The paths of
    one output irrep form one block of (paths x C) channels (``edge_tp_out_rows``), so the
    projection that follows reads one input segment per irrep."""
    _require_gpu("edge_tp", x, Y, w, x_scale)
    num_paths, nx, ny, no = tp_config_info(config)
    E = Y.shape[0]
    xs = _f32_rows(x, nx * channels, "x")
    Ys = _f32_rows(Y, ny, "Y")
    ws_ = _f32_rows(w, channels, "w")
    sc = None if x_scale is None else _f32_rows(x_scale, channels, "x_scale")
    if xs.shape[0] != E or ws_.shape[0] != num_paths or (sc is not None and sc.shape[0] != E):
        raise ValueError("edge_tp: x must be (E, NX*C), w (num_paths, C), x_scale (E, C)")
    out = torch.empty((E, no * channels), dtype=torch.float32, device=xs.device)
    check(_lib.load().mnx_edge_tp_fwd_f32(config, channels, ptr(xs), ptr(Ys), ptr(ws_),
                                          ptr(sc) if sc is not None else None, E, ptr(out), _stream(xs)),
          "edge_tp")
    return out


@edge_tp.register_fake
def _(x, Y, w, config, channels, x_scale=None):
    num_paths, nx, ny, no = tp_config_info(config)
    return x.new_empty((Y.shape[0], no * channels))


@torch.library.custom_op("molix::edge_tp_backward", mutates_args=(), device_types="cuda")
def edge_tp_backward(grad_out: Tensor, x: Tensor, Y: Tensor, w: Tensor, config: int, channels: int,
                     need_x: bool, need_Y: bool, need_w: bool, x_scale: Tensor | None = None,
                     need_scale: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """Gradients of ``<grad_out, edge_tp(...)>`` w.r.t. x, Y, the shared w and x_scale (empty when
    not needed); the weight gradient is summed over edges in a fixed order."""
    lib = _lib.load()
    num_paths, nx, ny, no = tp_config_info(config)
    E = Y.shape[0]
    xs = _f32_rows(x, nx * channels, "x")
    Ys = _f32_rows(Y, ny, "Y")
    wss = _f32_rows(w, channels, "w")
    sc = None if x_scale is None else _f32_rows(x_scale, channels, "x_scale")
    go = _f32_rows(grad_out, no * channels, "grad_out")
    gx = torch.empty_like(xs) if need_x else xs.new_empty(0)
    gY = torch.empty_like(Ys) if need_Y else Ys.new_empty(0)
    gw = torch.empty_like(wss) if need_w else wss.new_empty(0)
    need_scale = bool(need_scale and sc is not None)
    gs = torch.empty_like(sc) if need_scale else xs.new_empty(0)
    ws = _ws(max(int(lib.mnx_edge_tp_bwd_workspace_bytes(config, channels, E)), 1), xs.device)
    check(lib.mnx_edge_tp_bwd_f32(config, channels, ptr(xs), ptr(Ys), ptr(wss), ptr(sc) if sc is not None else None,
                                  ptr(go), E, ptr(gx) if need_x else None, ptr(gY) if need_Y else None,
                                  ptr(gw) if need_w else None, ptr(gs) if need_scale else None, ptr(ws), ws.numel(),
                                  _stream(xs)),
          "edge_tp backward")
    return gx, gY, gw, gs


@edge_tp_backward.register_fake
def _(grad_out, x, Y, w, config, channels, need_x, need_Y, need_w, x_scale=None, need_scale=False):
    return (torch.empty_like(x) if need_x else x.new_empty(0), torch.empty_like(Y) if need_Y else Y.new_empty(0),
            torch.empty_like(w) if need_w else w.new_empty(0),
            torch.empty_like(x_scale) if (need_scale and x_scale is not None) else x.new_empty(0))


def _etp_setup(ctx, inputs, output):
    x, Y, w, config, channels, x_scale = inputs
    ctx.save_for_backward(x, Y, w, x_scale)
    ctx.config, ctx.channels = config, channels


def _etp_backward(ctx, grad_out):
    x, Y, w, x_scale = ctx.saved_tensors
    nx, nY, nw = ctx.needs_input_grad[:3]
    ns = x_scale is not None and ctx.needs_input_grad[5]
    gx, gY, gw, gs = edge_tp_backward(grad_out.contiguous(), x, Y, w, ctx.config, ctx.channels, nx, nY, nw,
                                      x_scale, ns)
    return (gx.reshape(x.shape) if nx else None, gY.reshape(Y.shape) if nY else None,
            gw.reshape(w.shape) if nw else None, None, None, gs.reshape(x_scale.shape) if ns else None)


edge_tp.register_autograd(_etp_backward, setup_context=_etp_setup)


# the product fused with the projection after it (16 channels)

def edge_tp_proj_blocks(config: int) -> tuple[tuple[int, int, int, int], ...]:
    """Projected irreps of ``molix::edge_tp_proj`` for ``config``, in row order: (l, paths of output
    irrep l, their first row block J in ``proj``, first projected component I); empty when the
    configuration has no fused kernel."""
    buf = (C.c_int32 * 16)()
    n = int(_lib.load().mnx_edge_tp_proj_info(config, buf))
    return tuple(tuple(int(v) for v in buf[4 * i:4 * i + 4]) for i in range(max(n, 0)))


def edge_tp_proj_adjoint(g: Tensor, proj: Tensor, blocks) -> Tensor:
    """Gradient of the product's rows (``molix::edge_tp``'s layout, 16 channels) from the gradient
    of the projected rows: per irrep, ``G_l (E*M, 16) @ P_l^T`` with ``P_l`` its ``(paths*16, 16)``
    rows of ``proj`` (tracked torch ops: the differentiable form of the fused backward)."""
    E = g.shape[0]
    parts = []
    for l, nb, J, I in blocks:
        M = 2 * l + 1
        gb = g[:, I * 16:(I + M) * 16].reshape(E * M, 16)
        parts.append((gb @ proj[J * 16:(J + nb) * 16].t()).reshape(E, M * nb * 16))
    return torch.cat(parts, dim=1)


def edge_tp_project(t: Tensor, proj: Tensor, blocks) -> Tensor:
    """The projection alone on ``molix::edge_tp``'s output (16 channels): per irrep,
    ``T_l (E*M, paths*16) @ P_l`` written at its projected rows.  ``edge_tp_proj`` computes
    ``edge_tp_project(edge_tp(...), proj, blocks)`` in one pass."""
    E = t.shape[0]
    parts, row = [], 0
    for l, nb, J, I in blocks:
        M = 2 * l + 1
        tb = t[:, row * 16:(row + M * nb) * 16].reshape(E * M, nb * 16)
        parts.append((tb @ proj[J * 16:(J + nb) * 16]).reshape(E, M * 16))
        row += M * nb
    return torch.cat(parts, dim=1)


def _proj_args(x, Y, w, config, proj, x_scale, x_scale2=None):
    blocks = edge_tp_proj_blocks(config)
    if not blocks:
        raise ValueError(f"edge_tp_proj: no fused kernel for config {config}")
    num_paths, nx, ny, no = tp_config_info(config)
    E = Y.shape[0]
    shared = x.dim() == 2 and x.shape[1] == nx  # one value per component for all channels
    xs = _f32_rows(x, nx if shared else nx * 16, "x")
    Ys = _f32_rows(Y, ny, "Y")
    ws_ = _f32_rows(w, 16, "w")
    pj = _f32_rows(proj, 16, "proj")
    sc = None if x_scale is None else _f32_rows(x_scale, 16, "x_scale")
    sc2 = None if x_scale2 is None else _f32_rows(x_scale2, 16, "x_scale2")
    if (xs.shape[0] != E or ws_.shape[0] != num_paths or pj.shape[0] != num_paths * 16
            or (sc is not None and sc.shape[0] != E) or (sc2 is not None and sc2.shape[0] != E)):
        raise ValueError("edge_tp_proj: x must be (E, NX*16) or (E, NX), w (num_paths, 16), "
                         "proj (num_paths*16, 16), x_scale and x_scale2 (E, 16)")
    ni = sum(2 * l + 1 for l, _, _, _ in blocks)
    return blocks, xs, int(shared), Ys, ws_, pj, sc, sc2, ni


@torch.library.custom_op("molix::edge_tp_proj", mutates_args=(), device_types="cuda")
def edge_tp_proj(x: Tensor, Y: Tensor, w: Tensor, config: int, proj: Tensor,
                 x_scale: Tensor | None = None, x_scale2: Tensor | None = None) -> Tensor:
    """``molix::edge_tp`` with 16 channels followed by the projection back to the input irreps
    (src/molzoo/allegro.py:363-367,465-466: cuet.Linear(tp.irreps_out, irreps_in) on the product),
    in one pass that never writes the product's rows: ``out`` (E, NI*16), irreps l = 0..l_max in
    ir_mul.  ``proj`` (num_paths*16, 16) holds the projection's weights by row block
    (``edge_tp_proj_blocks``: the paths of output irrep l are blocks J_l .. J_l + paths - 1, rows
    J*16 + c for input channel c), scaled as applied.  ``x`` may also be (E, NX): one value per
    component shared by all 16 channels (channel weights then come in through ``x_scale``).  An
    optional ``x_scale2`` (E, 16) multiplies ``x_scale`` (the scale is their product, formed in the
    kernel)."""
    _require_gpu("edge_tp_proj", x, Y, w, proj, x_scale, x_scale2)
    blocks, xs, shared, Ys, ws_, pj, sc, sc2, ni = _proj_args(x, Y, w, config, proj, x_scale, x_scale2)
    E = Ys.shape[0]
    out = torch.empty((E, ni * 16), dtype=torch.float32, device=xs.device)
    check(_lib.load().mnx_edge_tp_proj_fwd_f32(config, ptr(xs), shared, ptr(Ys), ptr(ws_),
                                               ptr(sc) if sc is not None else None,
                                               ptr(sc2) if sc2 is not None else None, ptr(pj), E, ptr(out),
                                               _stream(xs)),
          "edge_tp_proj")
    return out


@edge_tp_proj.register_fake
def _(x, Y, w, config, proj, x_scale=None, x_scale2=None):
    ni = sum(2 * l + 1 for l, _, _, _ in edge_tp_proj_blocks(config))
    return x.new_empty((Y.shape[0], ni * 16))


@torch.library.custom_op("molix::edge_tp_proj_backward", mutates_args=(), device_types="cuda")
def edge_tp_proj_backward(grad_out: Tensor, x: Tensor, Y: Tensor, w: Tensor, config: int, proj: Tensor,
                          need_x: bool, need_Y: bool, need_w: bool, x_scale: Tensor | None = None,
                          need_scale: bool = False, x_scale2: Tensor | None = None,
                          need_scale2: bool = False) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients of ``<grad_out, edge_tp_proj(...)>`` w.r.t. x, Y, w, x_scale and x_scale2 (empty
    when not needed) in one pass: the projected gradient is taken back through the projection in
    registers, then the product's backward; the weight gradient is summed over edges in a fixed
    order."""
    lib = _lib.load()
    blocks, xs, shared, Ys, wss, pj, sc, sc2, ni = _proj_args(x, Y, w, config, proj, x_scale, x_scale2)
    E = Ys.shape[0]
    go = _f32_rows(grad_out, ni * 16, "grad_out")
    gx = torch.empty_like(xs) if need_x else xs.new_empty(0)
    gY = torch.empty_like(Ys) if need_Y else Ys.new_empty(0)
    gw = torch.empty_like(wss) if need_w else wss.new_empty(0)
    need_scale = bool(need_scale and sc is not None)
    gs = torch.empty_like(sc) if need_scale else xs.new_empty(0)
    need_scale2 = bool(need_scale2 and sc2 is not None)
    gs2 = torch.empty_like(sc2) if need_scale2 else xs.new_empty(0)
    ws = _ws(max(int(lib.mnx_edge_tp_proj_bwd_workspace_bytes(config, E)), 1), xs.device)
    check(lib.mnx_edge_tp_proj_bwd_f32(config, ptr(xs), shared, ptr(Ys), ptr(wss),
                                       ptr(sc) if sc is not None else None, ptr(sc2) if sc2 is not None else None,
                                       ptr(pj), ptr(go), E, ptr(gx) if need_x else None,
                                       ptr(gY) if need_Y else None, ptr(gw) if need_w else None,
                                       ptr(gs) if need_scale else None, ptr(gs2) if need_scale2 else None,
                                       ptr(ws), ws.numel(), _stream(xs)),
          "edge_tp_proj backward")
    return gx, gY, gw, gs, gs2


@edge_tp_proj_backward.register_fake
def _(grad_out, x, Y, w, config, proj, need_x, need_Y, need_w, x_scale=None, need_scale=False, x_scale2=None,
      need_scale2=False):
    return (torch.empty_like(x) if need_x else x.new_empty(0), torch.empty_like(Y) if need_Y else Y.new_empty(0),
            torch.empty_like(w) if need_w else w.new_empty(0),
            torch.empty_like(x_scale) if (need_scale and x_scale is not None) else x.new_empty(0),
            torch.empty_like(x_scale2) if (need_scale2 and x_scale2 is not None) else x.new_empty(0))


def _expand_shared_x(x: Tensor, config: int) -> Tensor:
    """x (E, NX) shared by the 16 channels as the (E, NX*16) rows ``molix::edge_tp`` reads (tracked:
    its gradient is the channel sum); other x unchanged."""
    nx = tp_config_info(config)[1]
    if x.dim() == 2 and x.shape[1] == nx:
        return x.unsqueeze(-1).expand(x.shape[0], nx, 16).reshape(x.shape[0], nx * 16)
    return x


def _etpp_setup(ctx, inputs, output):
    x, Y, w, config, proj, x_scale, x_scale2 = inputs
    ctx.save_for_backward(x, Y, w, proj, x_scale, x_scale2)
    ctx.config = config


def _etpp_backward(ctx, grad_out):
    x, Y, w, proj, x_scale, x_scale2 = ctx.saved_tensors
    config = ctx.config
    nx, nY, nw = ctx.needs_input_grad[:3]
    npj = ctx.needs_input_grad[4]
    ns = x_scale is not None and ctx.needs_input_grad[5]
    ns2 = x_scale2 is not None and ctx.needs_input_grad[6]
    gp = gs2 = None
    if npj or torch.is_grad_enabled():
        # the projection's weight gradient, or differentiated again (create_graph): the projection's
        # adjoint in tracked ops, then molix::edge_tp's backward (which has second derivatives)
        blocks = edge_tp_proj_blocks(config)
        g_tp = edge_tp_proj_adjoint(grad_out, proj, blocks)
        xf = _expand_shared_x(x, config)
        sc = x_scale if x_scale2 is None else (x_scale2 if x_scale is None else x_scale * x_scale2)
        gx, gY, gw, gsc = edge_tp_backward(g_tp.contiguous(), xf, Y, w, config, 16, nx, nY, nw, sc,
                                           sc is not None and (ns or ns2))
        gs = gsc * x_scale2 if (ns and x_scale2 is not None) else gsc
        if ns2:
            gs2 = gsc * x_scale if x_scale is not None else gsc
        if nx and xf is not x:
            gx = gx.reshape(x.shape[0], -1, 16).sum(-1)
        if npj:
            t = edge_tp(xf, Y, w, config, 16, sc)
            E, parts, row = t.shape[0], [], 0
            for l, nb, J, I in blocks:
                M = 2 * l + 1
                tb = t[:, row * 16:(row + M * nb) * 16].reshape(E * M, nb * 16)
                parts.append(tb.t() @ grad_out[:, I * 16:(I + M) * 16].reshape(E * M, 16))
                row += M * nb
            gp = torch.cat(parts, dim=0).reshape(proj.shape)
    else:
        gx, gY, gw, gs, gs2 = edge_tp_proj_backward(grad_out.contiguous(), x, Y, w, config, proj, nx, nY, nw,
                                                    x_scale, ns, x_scale2, ns2)
    return (gx.reshape(x.shape) if nx else None, gY.reshape(Y.shape) if nY else None,
            gw.reshape(w.shape) if nw else None, None, gp, gs.reshape(x_scale.shape) if ns else None,
            gs2.reshape(x_scale2.shape) if ns2 else None)


edge_tp_proj.register_autograd(_etpp_backward, setup_context=_etpp_setup)


# ---------------------------------------------------------------------------
# Particle-mesh Ewald (reference schemas, molix_library.cpp:29-41)
# ---------------------------------------------------------------------------

_PME_RECIP_SCHEMA = ("(Tensor positions, Tensor charges, Tensor box_vectors, Scalar gridx, Scalar gridy, "
                     "Scalar gridz, Scalar order, Scalar alpha, Scalar coulomb, Tensor xmoduli, Tensor ymoduli, "
                     "Tensor zmoduli) -> Tensor")
_PME_DIRECT_SCHEMA = ("(Tensor positions, Tensor charges, Tensor neighbors, Tensor deltas, Tensor distances, "
                      "Tensor exclusions, Scalar alpha, Scalar coulomb) -> Tensor")


def _fsuffix(t: Tensor) -> str:
    if t.dtype == torch.float64:
        return "f64"
    if t.dtype == torch.float32:
        return "f32"
    raise TypeError(f"PME needs float32 or float64 tensors, got {t.dtype}")


def _pme_recip_energy(positions, charges, box, gx, gy, gz, order, alpha, coulomb, xm, ym, zm):
    """spread -> rfftn (rocFFT) -> convolve; returns (energy, convolved half spectrum)."""
    lib = _lib.load()
    sfx = _fsuffix(positions)
    dt, dev = positions.dtype, positions.device
    pos = positions.detach().contiguous()
    q = charges.detach().to(dt).contiguous()
    b = box.detach().to(device=dev, dtype=dt).contiguous()
    mods = [m.detach().to(device=dev, dtype=dt).contiguous() for m in (xm, ym, zm)]
    for m, g in zip(mods, (gx, gy, gz)):
        if m.numel() < g:
            raise ValueError("moduli shorter than the grid")
    grid = torch.empty((gx, gy, gz), dtype=dt, device=dev)
    sws = _ws(lib.mnx_pme_spread_workspace_bytes(pos.shape[0], gx, gy, gz), dev)
    check(getattr(lib, f"mnx_pme_spread_{sfx}")(ptr(pos), ptr(q), ptr(b), pos.shape[0], gx, gy, gz, order,
                                                float(coulomb), ptr(grid), ptr(sws), sws.numel(), _stream(pos)),
          "pme spread")
    spec = torch.fft.rfftn(grid).contiguous()
    energy = torch.empty((), dtype=dt, device=dev)
    ws = _ws(lib.mnx_pme_convolve_workspace_bytes(gx, gy, gz), dev)
    check(getattr(lib, f"mnx_pme_convolve_{sfx}")(ptr(torch.view_as_real(spec)), ptr(b), gx, gy, gz, float(alpha),
                                                  ptr(mods[0]), ptr(mods[1]), ptr(mods[2]), ptr(energy), ptr(ws),
                                                  ws.numel(), _stream(pos)), "pme convolve")
    return energy, spec, pos, q, b


@torch.library.custom_op("molix::pme_reciprocal", mutates_args=(), device_types="cuda", schema=_PME_RECIP_SCHEMA)
def pme_reciprocal(positions, charges, box_vectors, gridx, gridy, gridz, order, alpha, coulomb, xmoduli, ymoduli,
                   zmoduli):
    """Reciprocal-space PME energy (reference ``pme_cpu.cpp:220-296,378``): B-spline spread on the GPU,
    rocFFT real-to-complex transform, influence-function convolution with the energy sum."""
    _require_gpu("pme_reciprocal", positions, charges, box_vectors)
    e, *_ = _pme_recip_energy(positions, charges, box_vectors, int(gridx), int(gridy), int(gridz), int(order),
                              alpha, coulomb, xmoduli, ymoduli, zmoduli)
    return e


@pme_reciprocal.register_fake
def _(positions, charges, box_vectors, gridx, gridy, gridz, order, alpha, coulomb, xmoduli, ymoduli, zmoduli):
    return positions.new_empty(())


@torch.library.custom_op("molix::pme_reciprocal_backward", mutates_args=(), device_types="cuda")
def pme_reciprocal_backward(positions: Tensor, charges: Tensor, box_vectors: Tensor, gridx: int, gridy: int,
                            gridz: int, order: int, alpha: float, coulomb: float, xmoduli: Tensor, ymoduli: Tensor,
                            zmoduli: Tensor) -> tuple[Tensor, Tensor]:
    """(dE/dpos, dE/dq): recompute the convolved spectrum, irfftn(norm='forward'), gather
    (reference backward ``pme_cpu.cpp:392-430``)."""
    lib = _lib.load()
    _, spec, pos, q, b = _pme_recip_energy(positions, charges, box_vectors, gridx, gridy, gridz, order, alpha,
                                           coulomb, xmoduli, ymoduli, zmoduli)
    return _pme_recip_gather(spec, pos, q, b, gridx, gridy, gridz, order, coulomb)


def _pme_recip_gather(spec, pos, q, b, gx, gy, gz, order, coulomb):
    """irfftn(norm='forward') of the convolved half spectrum, then the B-spline gather of
    (dE/dpos, dE/dq)."""
    lib = _lib.load()
    real = torch.fft.irfftn(spec, s=(gx, gy, gz), norm="forward").contiguous()
    dpos = torch.empty_like(pos)
    dq = torch.empty_like(q)
    check(getattr(lib, f"mnx_pme_gather_{_fsuffix(pos)}")(ptr(pos), ptr(q), ptr(b), pos.shape[0], ptr(real), gx, gy,
                                                          gz, order, float(coulomb), ptr(dpos), ptr(dq),
                                                          _stream(pos)), "pme gather")
    return dpos, dq


@pme_reciprocal_backward.register_fake
def _(positions, charges, box_vectors, gridx, gridy, gridz, order, alpha, coulomb, xmoduli, ymoduli, zmoduli):
    return torch.empty_like(positions), torch.empty_like(charges)


def _pme_recip_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], inputs[1], inputs[2], inputs[9], inputs[10], inputs[11])
    ctx.args = tuple(inputs[3:9])


def _pme_recip_bwd(ctx, grad):
    pos, q, box, xm, ym, zm = ctx.saved_tensors
    gx, gy, gz, order, alpha, coulomb = ctx.args
    dpos, dq = pme_reciprocal_backward(pos, q, box, int(gx), int(gy), int(gz), int(order), float(alpha),
                                       float(coulomb), xm, ym, zm)
    return (dpos * grad, (dq * grad).to(q.dtype)) + (None,) * 10


pme_reciprocal.register_autograd(_pme_recip_bwd, setup_context=_pme_recip_setup)


@torch.library.custom_op("molix::pme_reciprocal_spectrum", mutates_args=(), device_types="cuda")
def pme_reciprocal_spectrum(positions: Tensor, charges: Tensor, box_vectors: Tensor, gridx: int, gridy: int,
                            gridz: int, order: int, alpha: float, coulomb: float, xmoduli: Tensor, ymoduli: Tensor,
                            zmoduli: Tensor) -> tuple[Tensor, Tensor]:
    """``molix::pme_reciprocal`` that also returns the convolved half spectrum (gridx, gridy,
    gridz // 2 + 1), complex: its backward transforms that spectrum back and gathers, instead of
    spreading and transforming the charges a second time (the reference's backward recomputes,
    ``pme_cpu.cpp:392-430``).  The spectrum output carries no gradient."""
    _require_gpu("pme_reciprocal_spectrum", positions, charges, box_vectors)
    e, spec, *_ = _pme_recip_energy(positions, charges, box_vectors, int(gridx), int(gridy), int(gridz), int(order),
                                    alpha, coulomb, xmoduli, ymoduli, zmoduli)
    return e, spec


@pme_reciprocal_spectrum.register_fake
def _(positions, charges, box_vectors, gridx, gridy, gridz, order, alpha, coulomb, xmoduli, ymoduli, zmoduli):
    cdt = torch.complex128 if positions.dtype == torch.float64 else torch.complex64
    return positions.new_empty(()), positions.new_empty((gridx, gridy, gridz // 2 + 1), dtype=cdt)


@torch.library.custom_op("molix::pme_reciprocal_gather", mutates_args=(), device_types="cuda")
def pme_reciprocal_gather(positions: Tensor, charges: Tensor, box_vectors: Tensor, spectrum: Tensor, gridx: int,
                          gridy: int, gridz: int, order: int, coulomb: float) -> tuple[Tensor, Tensor]:
    """(dE/dpos, dE/dq) of ``molix::pme_reciprocal_spectrum`` from its spectrum output."""
    _require_gpu("pme_reciprocal_gather", positions, charges, box_vectors, spectrum)
    dt = positions.dtype
    if spectrum.shape != (gridx, gridy, gridz // 2 + 1) or not spectrum.is_complex():
        raise ValueError("pme_reciprocal_gather: spectrum must be complex (gridx, gridy, gridz // 2 + 1)")
    pos = positions.detach().contiguous()
    q = charges.detach().to(dt).contiguous()
    b = box_vectors.detach().to(device=pos.device, dtype=dt).contiguous()
    return _pme_recip_gather(spectrum, pos, q, b, int(gridx), int(gridy), int(gridz), int(order), coulomb)


@pme_reciprocal_gather.register_fake
def _(positions, charges, box_vectors, spectrum, gridx, gridy, gridz, order, coulomb):
    return torch.empty_like(positions), torch.empty_like(charges)


def _pme_spec_setup(ctx, inputs, output):
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(output[1])
    ctx.save_for_backward(inputs[0], inputs[1], inputs[2], output[1])
    ctx.args = (int(inputs[3]), int(inputs[4]), int(inputs[5]), int(inputs[6]), float(inputs[8]))


def _pme_spec_bwd(ctx, grad, _grad_spec):
    if grad is None:
        return (None,) * 12
    pos, q, box, spec = ctx.saved_tensors
    dpos, dq = pme_reciprocal_gather(pos, q, box, spec, *ctx.args)
    return (dpos * grad, (dq * grad).to(q.dtype)) + (None,) * 10


pme_reciprocal_spectrum.register_autograd(_pme_spec_bwd, setup_context=_pme_spec_setup)


def _pme_direct_run(positions, charges, neighbors, deltas, distances, exclusions, alpha, coulomb, grads=True):
    """Energy, and (dE/dpos, dE/dq) when ``grads`` (else None, None: no derivative atomics)."""
    lib = _lib.load()
    sfx = _fsuffix(positions)
    dt, dev = positions.dtype, positions.device
    pos = positions.detach().contiguous()
    q = charges.detach().to(dt).contiguous()
    nb = neighbors.to(torch.int32).contiguous()
    dl = deltas.detach().to(dt).contiguous()
    ds = distances.detach().to(dt).contiguous()
    ex = exclusions.to(device=dev, dtype=torch.int32).contiguous()
    n, P = pos.shape[0], nb.shape[1]
    if ex.ndim != 2 or (ex.numel() and ex.shape[0] != n):
        raise ValueError("exclusions must be (num_atoms, max_exclusions)")
    max_excl = ex.shape[1] if ex.numel() else 0
    energy = torch.empty((), dtype=dt, device=dev)
    dpos = torch.empty_like(pos) if grads else None
    dq = torch.empty_like(q) if grads else None
    ws = _ws(lib.mnx_pme_direct_workspace_bytes(n, P), dev)
    check(getattr(lib, f"mnx_pme_direct_{sfx}")(ptr(pos), ptr(q), n, ptr(nb), P, ptr(dl), ptr(ds), ptr(ex), max_excl,
                                                float(alpha), float(coulomb), ptr(energy),
                                                ptr(dpos), ptr(dq), ptr(ws),
                                                ws.numel(), _stream(pos)), "pme direct")
    return energy, dpos, dq


@torch.library.custom_op("molix::pme_direct", mutates_args=(), device_types="cuda", schema=_PME_DIRECT_SCHEMA)
def pme_direct(positions, charges, neighbors, deltas, distances, exclusions, alpha, coulomb):
    """Real-space PME energy over a pair list minus excluded pairs (reference ``pme_cpu.cpp:95-216``).
    Like the reference, the gradient w.r.t. positions is the analytic one through the pair
    geometry (deltas / distances are treated as functions of positions, ``pme_cpu.cpp:208-215``)."""
    _require_gpu("pme_direct", positions, charges, neighbors)
    e, _, _ = _pme_direct_run(positions, charges, neighbors, deltas, distances, exclusions, alpha, coulomb,
                              grads=False)
    return e


@pme_direct.register_fake
def _(positions, charges, neighbors, deltas, distances, exclusions, alpha, coulomb):
    return positions.new_empty(())


@torch.library.custom_op("molix::pme_direct_backward", mutates_args=(), device_types="cuda")
def pme_direct_backward(positions: Tensor, charges: Tensor, neighbors: Tensor, deltas: Tensor, distances: Tensor,
                        exclusions: Tensor, alpha: float, coulomb: float) -> tuple[Tensor, Tensor]:
    _, dpos, dq = _pme_direct_run(positions, charges, neighbors, deltas, distances, exclusions, alpha, coulomb)
    return dpos, dq


@pme_direct_backward.register_fake
def _(positions, charges, neighbors, deltas, distances, exclusions, alpha, coulomb):
    return torch.empty_like(positions), torch.empty_like(charges)


def _pme_direct_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs[:6])
    ctx.args = (float(inputs[6]), float(inputs[7]))


def _pme_direct_bwd(ctx, grad):
    dpos, dq = pme_direct_backward(*ctx.saved_tensors, *ctx.args)
    q = ctx.saved_tensors[1]
    return (dpos * grad, (dq * grad).to(q.dtype)) + (None,) * 6


pme_direct.register_autograd(_pme_direct_bwd, setup_context=_pme_direct_setup)


# ---------------------------------------------------------------------------
# Symmetric contraction of scalar channels (symmetric_contraction.py:90-109)
# ---------------------------------------------------------------------------


@torch.library.custom_op("molix::symmetric_contraction_scalar", mutates_args=(), device_types="cuda")
def symmetric_contraction_scalar(x: Tensor, atom_types: Tensor, weight: Tensor) -> Tensor:
    """``out[n, c] = sum_k weight[z_n, k, c] x[n, c]^(k+1)``; weight ``(S, degree, D)``."""
    _require_gpu("symmetric_contraction_scalar", x, atom_types, weight)
    S, nu, D = weight.shape
    xs = _f32_rows(x, D, "x")
    z = atom_types.to(torch.int64).contiguous()
    w = weight.contiguous()
    out = torch.empty_like(xs)
    check(_lib.load().mnx_sc_scalar_fwd_f32(ptr(xs), ptr(z), ptr(w), xs.shape[0], D, S, nu, ptr(out), _stream(xs)),
          "symmetric_contraction_scalar")
    return out.reshape(x.shape)


@symmetric_contraction_scalar.register_fake
def _(x, atom_types, weight):
    return torch.empty_like(x)


@torch.library.custom_op("molix::symmetric_contraction_scalar_backward", mutates_args=(), device_types="cuda")
def symmetric_contraction_scalar_backward(grad: Tensor, x: Tensor, atom_types: Tensor, weight: Tensor,
                                          need_x: bool, need_w: bool) -> tuple[Tensor, Tensor]:
    S, nu, D = weight.shape
    xs = _f32_rows(x, D, "x")
    g = _f32_rows(grad, D, "grad")
    z = atom_types.to(torch.int64).contiguous()
    w = weight.contiguous()
    gx = torch.empty_like(xs) if need_x else xs.new_empty(0)
    gw = torch.zeros_like(w) if need_w else w.new_empty(0)
    check(_lib.load().mnx_sc_scalar_bwd_f32(ptr(xs), ptr(z), ptr(w), ptr(g), xs.shape[0], D, S, nu, ptr(gx), ptr(gw),
                                            _stream(xs)), "symmetric_contraction_scalar backward")
    return gx.reshape(x.shape) if need_x else gx, gw


@symmetric_contraction_scalar_backward.register_fake
def _(grad, x, atom_types, weight, need_x, need_w):
    return (torch.empty_like(x) if need_x else x.new_empty(0), torch.empty_like(weight) if need_w else
            weight.new_empty(0))


def _sc_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _sc_bwd(ctx, grad):
    x, z, w = ctx.saved_tensors
    nx, _, nw = ctx.needs_input_grad
    gx, gw = symmetric_contraction_scalar_backward(grad.contiguous(), x, z, w, nx, nw)
    return (gx if nx else None), None, (gw if nw else None)


symmetric_contraction_scalar.register_autograd(_sc_bwd, setup_context=_sc_setup)


# ---------------------------------------------------------------------------
# Equivariant symmetric contraction (MACE product basis; the reference reaches it
# through cuet.SymmetricContraction, symmetric_contraction.py:94-109)
# ---------------------------------------------------------------------------


def sc_config_id(l_in: int, l_out: int, correlation: int) -> int:
    cfg = int(_lib.load().mnx_sc_config(l_in, l_out, correlation))
    if cfg < 0:
        raise ValueError(_lib.load().mnx_last_error().decode())
    return cfg


def sc_config_info(config: int) -> tuple[int, int, int, int]:
    """(dim_in, dim_out, paths, coefficients) per channel."""
    info = (C.c_int32 * 4)()
    check(_lib.load().mnx_sc_config_info(config, info), "sc_config_info")
    return tuple(info)


def _sc_shapes(x, weight, l_in, l_out, correlation):
    cfg = sc_config_id(l_in, l_out, correlation)
    ni, no, paths, _ = sc_config_info(cfg)
    if weight.dim() != 3 or weight.shape[1] != paths:
        raise ValueError(f"weight must be (num_elements, {paths}, channels), got {tuple(weight.shape)}")
    S, _, Cc = weight.shape
    if x.shape[-1] != ni * Cc:
        raise ValueError(f"x last dim {x.shape[-1]} != {ni} x {Cc}")
    return cfg, ni, no, S, Cc


@torch.library.custom_op("molix::symmetric_contraction", mutates_args=(), device_types="cuda")
def symmetric_contraction(x: Tensor, atom_types: Tensor, weight: Tensor, l_in: int, l_out: int,
                          correlation: int) -> Tensor:
    """B = sum_{nu<=correlation} U_nu . W[z] (x^{(x)nu}); x (N, (l_in+1)^2 C) ir_mul, weight
    (S, paths, C) -> (N, (l_out+1)^2 C)."""
    _require_gpu("symmetric_contraction", x, atom_types, weight)
    cfg, ni, no, S, Cc = _sc_shapes(x, weight, l_in, l_out, correlation)
    xs = _f32_rows(x, ni * Cc, "x")
    z = atom_types.to(torch.int64).reshape(-1).contiguous()
    w = weight.contiguous()
    out = torch.empty((xs.shape[0], no * Cc), dtype=torch.float32, device=xs.device)
    check(_lib.load().mnx_sc_fwd_f32(cfg, ptr(xs), ptr(z), ptr(w), xs.shape[0], Cc, S, ptr(out), _stream(xs)),
          "symmetric_contraction")
    return out.reshape(*x.shape[:-1], no * Cc)


@symmetric_contraction.register_fake
def _(x, atom_types, weight, l_in, l_out, correlation):
    return x.new_empty(*x.shape[:-1], (l_out + 1) ** 2 * weight.shape[-1])


@torch.library.custom_op("molix::symmetric_contraction_backward", mutates_args=(), device_types="cuda")
def symmetric_contraction_backward(grad: Tensor, x: Tensor, atom_types: Tensor, weight: Tensor, l_in: int,
                                   l_out: int, correlation: int, need_x: bool,
                                   need_w: bool) -> tuple[Tensor, Tensor]:
    cfg, ni, no, S, Cc = _sc_shapes(x, weight, l_in, l_out, correlation)
    xs = _f32_rows(x, ni * Cc, "x")
    g = _f32_rows(grad, no * Cc, "grad")
    z = atom_types.to(torch.int64).reshape(-1).contiguous()
    w = weight.contiguous()
    # nodes grouped by element: one weight-gradient flush per element run
    order = class_groups(z, S)[0] if need_w else None
    gx = torch.empty_like(xs) if need_x else xs.new_empty(0)
    gw = torch.zeros_like(w) if need_w else w.new_empty(0)
    check(_lib.load().mnx_sc_bwd_f32(cfg, ptr(xs), ptr(z), ptr(w), ptr(g), ptr(order), xs.shape[0], Cc, S,
                                     ptr(gx) if need_x else None, ptr(gw) if need_w else None, _stream(xs)),
          "symmetric_contraction backward")
    return (gx.reshape(x.shape) if need_x else gx), gw


@symmetric_contraction_backward.register_fake
def _(grad, x, atom_types, weight, l_in, l_out, correlation, need_x, need_w):
    return (torch.empty_like(x) if need_x else x.new_empty(0),
            torch.empty_like(weight) if need_w else weight.new_empty(0))


@torch.library.custom_op("molix::symmetric_contraction_backward2", mutates_args=(), device_types="cuda")
def symmetric_contraction_backward2(grad: Tensor, x: Tensor, atom_types: Tensor, weight: Tensor,
                                    seed_x: Tensor | None, seed_w: Tensor | None, l_in: int, l_out: int,
                                    correlation: int, need_grad: bool, need_x: bool,
                                    need_w: bool) -> tuple[Tensor, Tensor, Tensor]:
    """Second order of ``symmetric_contraction``: gradients of <seed_x, grad_x> + <seed_w, grad_w>
    (the first-order gradients of <grad, B>) with respect to grad, x and weight (empty when not
    needed)."""
    cfg, ni, no, S, Cc = _sc_shapes(x, weight, l_in, l_out, correlation)
    xs = _f32_rows(x, ni * Cc, "x")
    g = _f32_rows(grad, no * Cc, "grad")
    sx = None if seed_x is None else _f32_rows(seed_x, ni * Cc, "seed_x")
    sw = None if seed_w is None else seed_w.to(torch.float32).contiguous()
    z = atom_types.to(torch.int64).reshape(-1).contiguous()
    w = weight.contiguous()
    order = class_groups(z, S)[0] if need_w else None
    dg = torch.empty_like(g) if need_grad else g.new_empty(0)
    dx = torch.empty_like(xs) if need_x else xs.new_empty(0)
    dw = torch.zeros_like(w) if need_w else w.new_empty(0)
    check(_lib.load().mnx_sc_bwd2_f32(cfg, ptr(xs), ptr(z), ptr(w), ptr(g), ptr(sx), ptr(sw), ptr(order), xs.shape[0],
                                      Cc, S, ptr(dg), ptr(dx), ptr(dw), _stream(xs)),
          "symmetric_contraction second order")
    return dg, dx, dw


@symmetric_contraction_backward2.register_fake
def _(grad, x, atom_types, weight, seed_x, seed_w, l_in, l_out, correlation, need_grad, need_x, need_w):
    return (torch.empty_like(grad) if need_grad else grad.new_empty(0),
            torch.empty_like(x) if need_x else x.new_empty(0),
            torch.empty_like(weight) if need_w else weight.new_empty(0))


def _scg_setup(ctx, inputs, output):
    x, z, w, l_in, l_out, nu = inputs
    ctx.save_for_backward(x, z, w)
    ctx.cfg = (l_in, l_out, nu)


def _scg_bwd(ctx, grad):
    x, z, w = ctx.saved_tensors
    nx, _, nw = ctx.needs_input_grad[:3]
    gx, gw = symmetric_contraction_backward(grad.contiguous(), x, z, w, *ctx.cfg, nx, nw)
    return (gx if nx else None), None, (gw if nw else None), None, None, None


symmetric_contraction.register_autograd(_scg_bwd, setup_context=_scg_setup)


# ---------------------------------------------------------------------------
# Radial weight MLP hidden stack
# ---------------------------------------------------------------------------

def radial_supported(kin: int, hidden: int, layers: int) -> bool:
    """Whether the fused hidden-stack kernels are compiled for this shape."""
    return _lib.load().mnx_radial_frag_floats(int(kin), int(hidden), int(layers)) > 0


def _aligned16(t: Tensor) -> Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _radial_frag(params: Tensor, kin: int, hidden: int, layers: int) -> Tensor:
    lib = _lib.load()
    n = lib.mnx_radial_frag_floats(kin, hidden, layers)
    if n < 0:
        raise ValueError(f"radial_hidden: no kernel for in={kin}, hidden={hidden}, layers={layers}")
    raw = params.detach().to(torch.float32).contiguous()
    if raw.numel() != lib.mnx_radial_raw_floats(kin, hidden, layers):
        raise ValueError("radial_hidden: parameter vector has the wrong length")
    frag = torch.empty(n, dtype=torch.float32, device=raw.device)
    check(lib.mnx_radial_pack_f32(ptr(raw), kin, hidden, layers, ptr(frag), _stream(raw)), "radial_hidden pack")
    return frag


@torch.library.custom_op("molix::radial_hidden", mutates_args=(), device_types="cuda")
def radial_hidden(feats: Tensor, params: Tensor, kin: int, hidden: int, layers: int) -> Tensor:
    """``mlp[:-1](feats)`` of ``RadialWeightMLP`` (``radial_mlp.py:38-93``: [Linear -> SiLU] x layers)
    in one HIP kernel.  ``params`` = concatenated ``W_j.flatten(), b_j`` of the hidden Linears."""
    _require_gpu("radial_hidden", feats, params)
    if feats.dtype != torch.float32 or feats.dim() != 2 or feats.shape[1] != kin:
        raise ValueError("radial_hidden: feats must be float32 (E, kin)")
    f = feats.contiguous()
    frag = _radial_frag(params, kin, hidden, layers)
    out = f.new_empty(f.shape[0], hidden)
    check(_lib.load().mnx_radial_fwd_f32(ptr(f), f.shape[0], kin, hidden, layers, ptr(frag), ptr(out), _stream(f)),
          "radial_hidden")
    return out


@radial_hidden.register_fake
def _(feats, params, kin, hidden, layers):
    return feats.new_empty(feats.shape[0], hidden)


@torch.library.custom_op("molix::radial_hidden_backward", mutates_args=(), device_types="cuda")
def radial_hidden_backward(grad: Tensor, feats: Tensor, params: Tensor, kin: int, hidden: int,
                           layers: int) -> Tensor:
    """dL/dfeats of ``radial_hidden`` (forward recomputed in registers)."""
    f = feats.contiguous()
    g = _aligned16(grad.to(torch.float32))
    frag = _radial_frag(params, kin, hidden, layers)
    gf = torch.empty_like(f)
    check(_lib.load().mnx_radial_bwd_f32(ptr(f), f.shape[0], kin, hidden, layers, ptr(frag), ptr(g), ptr(gf),
                                         _stream(f)), "radial_hidden backward")
    return gf


@radial_hidden_backward.register_fake
def _(grad, feats, params, kin, hidden, layers):
    return torch.empty_like(feats)


def _radial_setup(ctx, inputs, output):
    feats, params, kin, hidden, layers = inputs
    ctx.save_for_backward(feats, params)
    ctx.cfg = (kin, hidden, layers)


def _radial_torch(feats: Tensor, params: Tensor, kin: int, hidden: int, layers: int) -> Tensor:
    """The hidden stack in tracked torch ops from the same flat parameters (W_j row-major, b_j)."""
    z, off, k = feats, 0, kin
    for _ in range(layers):
        w = params[off:off + hidden * k].reshape(hidden, k)
        b = params[off + hidden * k:off + hidden * k + hidden]
        off += hidden * k + hidden
        z = torch.nn.functional.silu(torch.nn.functional.linear(z, w, b))
        k = hidden
    return z


def _radial_bwd(ctx, grad):
    feats, params = ctx.saved_tensors
    if ctx.needs_input_grad[1]:
        raise RuntimeError("molix::radial_hidden computes no parameter gradient; use the Sequential path "
                           "when the radial MLP is trained")
    if not ctx.needs_input_grad[0]:
        return None, None, None, None, None
    if torch.is_grad_enabled() and feats.requires_grad:
        # differentiated again (create_graph): the input gradient of the stack recomputed in
        # tracked ops on the saved input, so that it stays a function of it
        with torch.enable_grad():
            (gf,) = torch.autograd.grad(_radial_torch(feats, params.detach(), *ctx.cfg), feats, grad,
                                        create_graph=True)
        return gf, None, None, None, None
    return radial_hidden_backward(grad, feats, params, *ctx.cfg), None, None, None, None


radial_hidden.register_autograd(_radial_bwd, setup_context=_radial_setup)


# ---------------------------------------------------------------------------
# Radial weight MLP output layer (per-edge tensor-product weights)
# ---------------------------------------------------------------------------


def edge_weights_supported(in_dim: int, out_dim: int) -> bool:
    """Whether ``molix::edge_weights`` (and its backward) take an in_dim -> out_dim Linear."""
    return _lib.load().mnx_edge_weights_frag_elems(int(in_dim), int(out_dim), 1) > 0 and out_dim % 8 == 0


def _ew_frag(weight: Tensor, backward: bool) -> Tensor:
    lib = _lib.load()
    N, K = weight.shape
    n = lib.mnx_edge_weights_frag_elems(K, N, int(backward))
    if n < 0:
        raise ValueError(f"edge_weights: no kernel for a {K} -> {N} layer")
    w = weight.detach().to(torch.float32).contiguous()
    frag = torch.empty(n, dtype=torch.int16, device=w.device)
    check(lib.mnx_edge_weights_pack_f32(ptr(w), K, N, int(backward), ptr(frag), _stream(w)), "edge_weights pack")
    return frag


@torch.library.custom_op("molix::edge_weights", mutates_args=(), device_types="cuda")
def edge_weights(h: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    """``h @ weight.T + bias``: the last Linear of ``RadialWeightMLP`` (``radial_mlp.py:38-93``) mapping
    the (E, K) hidden activations to the (E, N) per-edge tensor-product weights.  Near-fp32: rows of
    h and columns of the weight are scaled by powers of two into [1, 2), each value is split into
    two fp16 parts, and three partial products per pair are accumulated in fp32 on the matrix cores
    (the scales are undone exactly)."""
    _require_gpu("edge_weights", h, weight, bias)
    if h.dtype != torch.float32 or weight.dtype != torch.float32 or h.dim() != 2 or weight.dim() != 2:
        raise TypeError("edge_weights: h (E, K) and weight (N, K) must be float32")
    N, K = weight.shape
    if h.shape[1] != K:
        raise ValueError(f"edge_weights: h has {h.shape[1]} columns, weight expects {K}")
    if bias is not None and (bias.dtype != torch.float32 or bias.shape != (N,)):
        raise ValueError("edge_weights: bias must be float32 (N,)")
    x = _aligned16(h)
    frag = _ew_frag(weight, False)
    out = x.new_empty(x.shape[0], N)
    b = None if bias is None else bias.detach().contiguous()
    check(_lib.load().mnx_edge_weights_f32(ptr(x), x.shape[0], K, ptr(frag), ptr(b), N, ptr(out), _stream(x)),
          "edge_weights")
    return out


@edge_weights.register_fake
def _(h, weight, bias=None):
    return h.new_empty(h.shape[0], weight.shape[0])


def _edge_weights_rows(h: Tensor, rows: Tensor, weight: Tensor, bias: Tensor | None) -> Tensor:
    """``h[rows] @ weight.T + bias`` (rows int32), reading the selected rows of h in place."""
    N, K = weight.shape
    x = _aligned16(h.to(torch.float32))
    frag = _ew_frag(weight, False)
    out = x.new_empty(rows.shape[0], N)
    b = None if bias is None else bias.detach().contiguous()
    check(_lib.load().mnx_edge_weights_rows_f32(ptr(x), ptr(rows), rows.shape[0], K, ptr(frag), ptr(b), N,
                                                ptr(out), _stream(x)), "edge_weights (rows)")
    return out


@torch.library.custom_op("molix::edge_weights_backward", mutates_args=(), device_types="cuda")
def edge_weights_backward(grad: Tensor, weight: Tensor) -> Tensor:
    """``grad @ weight``: dL/dh of ``edge_weights`` (same split-fp16 arithmetic)."""
    N, K = weight.shape
    if grad.dim() != 2 or grad.shape[1] != N:
        raise ValueError("edge_weights_backward: grad must be (E, N)")
    g = grad.to(torch.float32)
    # rows may be strided (e.g. one layer's slice of a stacked gradient): read in place when the
    # row stride is a multiple of 4 floats and the rows are 16-byte aligned
    if not (g.stride(1) == 1 and g.stride(0) >= N and g.stride(0) % 4 == 0 and g.data_ptr() % 16 == 0):
        g = _aligned16(g)
    frag = _ew_frag(weight, True)
    gh = g.new_empty(g.shape[0], K)
    check(_lib.load().mnx_edge_weights_bwd_cols_f32(ptr(g), g.stride(0), None, g.shape[0], N, ptr(frag), K, ptr(gh),
                                                    0, _stream(g)),
          "edge_weights backward")
    return gh


@edge_weights_backward.register_fake
def _(grad, weight):
    return grad.new_empty(grad.shape[0], weight.shape[1])


@torch.library.custom_op("molix::edge_weights_backward_acc", mutates_args=("out",), device_types="cuda")
def edge_weights_backward_acc(grad: Tensor, weight: Tensor, out: Tensor) -> None:
    """``out += grad @ weight`` in place (``out`` a float32 (E, K) tensor with unit column stride,
    16-byte aligned rows a multiple of 4 floats apart, so a column block of a wider tensor too;
    ``grad`` may be a column block as well): the input-gradient product of ``edge_weights``
    accumulated into an existing result in the same pass (``mnx_edge_weights_bwd_into_f32`` with
    accumulation), instead of a product and an add."""
    N, K = weight.shape
    if grad.dim() != 2 or grad.shape[1] != N:
        raise ValueError("edge_weights_backward_acc: grad must be (E, N)")
    if (out.dtype != torch.float32 or out.shape != (grad.shape[0], K) or out.data_ptr() % 16 != 0
            or (out.shape[0] > 1 and (out.stride(1) != 1 or out.stride(0) < K or out.stride(0) % 4 != 0))):
        raise ValueError("edge_weights_backward_acc: out must be a float32 (E, K) with unit column stride and "
                         "16-byte aligned rows a multiple of 4 floats apart")
    g = grad.to(torch.float32)
    # rows may be strided (a column block of a wider tensor): unit column stride, a row stride that
    # is a multiple of 4 floats and 16-byte aligned rows are read in place
    if not (g.stride(1) == 1 and g.stride(0) >= N and g.stride(0) % 4 == 0 and g.data_ptr() % 16 == 0):
        g = _aligned16(g)
    frag = _ew_frag(weight, True)
    ldh = out.stride(0) if out.shape[0] > 1 else K
    check(_lib.load().mnx_edge_weights_bwd_into_f32(ptr(g), g.stride(0), None, g.shape[0], N, ptr(frag), K,
                                                    ptr(out), ldh, 1, _stream(g)),
          "edge_weights backward (accumulating)")


@edge_weights_backward_acc.register_fake
def _(grad, weight, out):
    return None


# mnx_tall_tn_f32 takes row strides below 2^25 floats (its 16-row step offsets stay in 31 bits)
_TALL_MAX_STRIDE = 1 << 25


def _rows_f32(t: Tensor, what: str) -> Tensor:
    """``t`` itself when its rows are unit-stride with a row stride the tall GEMM accepts, else a
    contiguous copy (e.g. a column slice of a very wide tensor)."""
    if t.dtype != torch.float32 or t.dim() != 2:
        raise TypeError(f"{what} must be a 2-D float32 tensor")
    ok = t.stride(1) == 1 and t.shape[1] <= t.stride(0) < _TALL_MAX_STRIDE
    return t if ok else t.contiguous()


@torch.library.custom_op("molix::tall_tn", mutates_args=(), device_types="cuda")
def tall_tn(a: Tensor, b: Tensor) -> Tensor:
    """``a.T @ b`` for tall float32 ``a`` (K, M) and ``b`` (K, N), K >> M, N: a layer's weight
    gradient summed over all edges, fp32-accurate on the bf16 matrix cores (split operands),
    deterministic; rows may be strided."""
    _require_gpu("tall_tn", a, b)
    a2, b2 = _rows_f32(a, "a"), _rows_f32(b, "b")
    if a2.shape[0] != b2.shape[0]:
        raise ValueError(f"tall_tn: {a2.shape[0]} rows against {b2.shape[0]}")
    K, M, N = a2.shape[0], a2.shape[1], b2.shape[1]
    out = torch.empty((M, N), dtype=torch.float32, device=a2.device)
    lib = _lib.load()
    ws = _ws(lib.mnx_tall_tn_workspace_bytes(K, M, N), a2.device)
    check(lib.mnx_tall_tn_f32(ptr(a2), a2.stride(0), ptr(b2), b2.stride(0), K, M, N, ptr(out), None, ptr(ws),
                              ws.numel(), _stream(a2)), "tall_tn")
    return out


@tall_tn.register_fake
def _(a, b):
    return a.new_empty((a.shape[1], b.shape[1]))


def _tall_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _tall_bwd(ctx, g):
    a, b = ctx.saved_tensors
    na, nb = ctx.needs_input_grad
    return (b @ g.t() if na else None, a @ g if nb else None)


tall_tn.register_autograd(_tall_bwd, setup_context=_tall_setup)


@torch.library.custom_op("molix::tall_tn_colsum", mutates_args=(), device_types="cuda")
def tall_tn_colsum(a: Tensor, b: Tensor) -> tuple[Tensor, Tensor]:
    """``(a.T @ b, a.sum(0))`` from one pass over ``a`` (``tall_tn`` with the column sums of ``a``:
    a layer's weight and bias gradients)."""
    _require_gpu("tall_tn_colsum", a, b)
    a2, b2 = _rows_f32(a, "a"), _rows_f32(b, "b")
    if a2.shape[0] != b2.shape[0]:
        raise ValueError(f"tall_tn_colsum: {a2.shape[0]} rows against {b2.shape[0]}")
    K, M, N = a2.shape[0], a2.shape[1], b2.shape[1]
    out = torch.empty((M, N), dtype=torch.float32, device=a2.device)
    cs = torch.empty((M,), dtype=torch.float32, device=a2.device)
    lib = _lib.load()
    ws = _ws(lib.mnx_tall_tn_workspace_bytes(K, M, N), a2.device)
    check(lib.mnx_tall_tn_f32(ptr(a2), a2.stride(0), ptr(b2), b2.stride(0), K, M, N, ptr(out), ptr(cs), ptr(ws),
                              ws.numel(), _stream(a2)), "tall_tn_colsum")
    return out, cs


@tall_tn_colsum.register_fake
def _(a, b):
    return a.new_empty((a.shape[1], b.shape[1])), a.new_empty((a.shape[1],))


def _tallc_bwd(ctx, g, gc):
    a, b = ctx.saved_tensors
    na, nb = ctx.needs_input_grad
    ga = gb = None
    if na:
        ga = b @ g.t() if g is not None else None
        if gc is not None:
            ga = gc.expand(a.shape[0], -1) if ga is None else ga + gc
    if nb and g is not None:
        gb = a @ g
    return ga, gb


tall_tn_colsum.register_autograd(_tallc_bwd, setup_context=_tall_setup)


def silu_bwd2(x: Tensor, g: Tensor, gg: Tensor) -> tuple[Tensor, Tensor]:
    """Adjoints of ``gx = g * silu'(x)`` for the seed ``gg``: ``(gg g silu''(x), gg silu'(x))``, one
    fused pass (float32 CUDA tensors of one shape)."""
    _require_gpu("silu_bwd2", x, g, gg)
    xs, gs, ggs = (t.contiguous() for t in (x, g, gg))
    if not (xs.dtype == gs.dtype == ggs.dtype == torch.float32) or not (xs.shape == gs.shape == ggs.shape):
        raise ValueError("silu_bwd2: x, g and gg must be float32 tensors of one shape")
    dx, dg = torch.empty_like(xs), torch.empty_like(xs)
    check(_lib.load().mnx_silu_bwd2_f32(ptr(xs), ptr(gs), ptr(ggs), xs.numel(), ptr(dx), ptr(dg), _stream(xs)),
          "silu_bwd2")
    return dx, dg


def _ew_setup(ctx, inputs, output):
    h, weight = inputs[0], inputs[1]
    ctx.save_for_backward(h, weight)
    ctx.has_bias = len(inputs) > 2 and inputs[2] is not None


def _ew_bwd(ctx, grad):
    h, weight = ctx.saved_tensors
    need_h, need_w = ctx.needs_input_grad[:2]
    need_b = len(ctx.needs_input_grad) > 2 and ctx.needs_input_grad[2]
    grad = grad.contiguous()
    gh = edge_weights_backward(grad, weight) if need_h else None
    gw = None
    gb = None
    if need_w:  # training: the (N, K) weight gradient summed over all rows (and the bias's)
        if need_b and ctx.has_bias:
            gw, gb = tall_tn_colsum(grad, h)
        else:
            gw = tall_tn(grad, h)
    elif need_b and ctx.has_bias:
        gb = grad.sum(0)
    return (gh, gw, gb)[:len(ctx.needs_input_grad)]


edge_weights.register_autograd(_ew_bwd, setup_context=_ew_setup)


# ---------------------------------------------------------------------------
# Radial-MLP output layer + tensor product, with the fused weight gradient
# ---------------------------------------------------------------------------


def tp_weight_grad_supported(config: int, channels: int, hidden: int) -> bool:
    """Whether ``molix::tp_weight_grad`` takes this configuration, channel count and hidden width."""
    return config >= 0 and channels % 16 == 0 and hidden in (16, 32, 64, 128)


@torch.library.custom_op("molix::tp_weight_grad", mutates_args=(), device_types="cuda")
def tp_weight_grad(x: Tensor, Y: Tensor, grad_out: Tensor, edge_index: Tensor, weight: Tensor, config: int,
                   channels: int) -> Tensor:
    """``grad_h = gw @ weight`` for the per-edge weights ``w = h @ weight.T + b`` of a
    ``tp_scatter``: the weight gradient ``gw = d<grad_out, tp_scatter(x, Y, w)>/dw`` is formed per
    edge in registers and multiplied on the matrix cores, never written (``weight`` is the output
    layer's (num_paths * C, K) matrix)."""
    _require_gpu("tp_weight_grad", x, Y, grad_out, edge_index, weight)
    num_paths, nx, ny, no = tp_config_info(config)
    Nw, K = weight.shape
    if Nw != num_paths * channels:
        raise ValueError(f"tp_weight_grad: weight has {Nw} rows, the product has {num_paths} x {channels}")
    xs = _aligned16(_f32_rows(x, nx * channels, "x"))
    Ys = _f32_rows(Y, ny, "Y")
    go = _aligned16(_f32_rows(grad_out, no * channels, "grad_out"))
    ei = edge_index.to(torch.int64).contiguous()
    if ei.dim() != 2 or ei.shape[1] != 2 or ei.shape[0] != Ys.shape[0] or go.shape[0] != xs.shape[0]:
        raise ValueError("tp_weight_grad: inconsistent sizes of x / Y / grad_out / edge_index")
    frag = _ew_frag(weight, True)
    gh = xs.new_empty(Ys.shape[0], K)
    check(_lib.load().mnx_tp_weight_grad_f32(config, channels, ptr(xs), ptr(Ys), ptr(go), ptr(ei), xs.shape[0],
                                             Ys.shape[0], ptr(frag), K, ptr(gh), _stream(xs)), "tp_weight_grad")
    return gh


@tp_weight_grad.register_fake
def _(x, Y, grad_out, edge_index, weight, config, channels):
    return x.new_empty(Y.shape[0], weight.shape[1])


@torch.library.custom_op("molix::radial_tp", mutates_args=(), device_types="cuda")
def radial_tp(x: Tensor, Y: Tensor, h: Tensor, weight: Tensor, bias: Tensor | None, row_ptr: Tensor, perm: Tensor,
              senders: Tensor, edge_index: Tensor, config: int, channels: int) -> tuple[Tensor, Tensor]:
    """``tp_scatter(x, Y, w)`` with ``w = h @ weight.T + bias`` (the radial MLP's output layer,
    ``radial_mlp.py:76-82``, feeding ConvTP, ``tensor_product.py:72-79,101-111``).  Returns
    ``(out, w)``; ``w`` is kept for the backward, whose gradient with respect to ``h`` comes from
    ``tp_weight_grad`` (the per-edge weight gradient is never materialised) and whose tensor-product
    backward skips the weight gradient.  The output layer's parameters get no gradient here."""
    w = edge_weights(h, weight, bias)
    out = tp_scatter(x, Y, w, row_ptr, perm, senders, config, channels)
    return out, w


@radial_tp.register_fake
def _(x, Y, h, weight, bias, row_ptr, perm, senders, edge_index, config, channels):
    num_paths, nx, ny, no = tp_config_info(config)
    return x.new_empty((row_ptr.shape[0] - 1, no * channels)), h.new_empty((h.shape[0], weight.shape[0]))


def _rtp_setup(ctx, inputs, output):
    x, Y, h, weight, bias, row_ptr, perm, senders, edge_index, config, channels = inputs
    ctx.save_for_backward(x, Y, h, weight, output[1], row_ptr, perm, senders, edge_index)
    ctx.config, ctx.channels = config, channels
    # the returned weights usually get no gradient: pass None rather than an (E, N) zero tensor
    ctx.set_materialize_grads(False)


def _rtp_backward(ctx, g_out, g_w):
    x, Y, h, weight, w, row_ptr, perm, senders, edge_index = ctx.saved_tensors
    nig = ctx.needs_input_grad
    if nig[3] or nig[4]:
        raise RuntimeError("molix::radial_tp gives no gradient for the output layer's weight and bias; use the "
                           "separate edge_weights + tp_scatter ops when they are trained")
    need_x, need_Y, need_h = nig[0], nig[1], nig[2]
    gx = gY = gh = None
    if g_out is not None and (need_x or need_Y):
        gx, gY, _ = tp_scatter_backward(g_out.contiguous(), x, Y, w, row_ptr, perm, senders, ctx.config,
                                        ctx.channels, need_x, need_Y, False)
        gx = gx.reshape(x.shape) if need_x else None
        gY = gY.reshape(Y.shape) if need_Y else None
    if need_h:
        gh = (tp_weight_grad(x, Y, g_out.contiguous(), edge_index, weight, ctx.config, ctx.channels)
              if g_out is not None else torch.zeros_like(h))
        if g_w is not None:  # a caller that used the returned weights as well
            gh = gh + edge_weights_backward(g_w.contiguous(), weight)
    return gx, gY, gh, None, None, None, None, None, None, None, None


radial_tp.register_autograd(_rtp_backward, setup_context=_rtp_setup)


# ---------------------------------------------------------------------------
# Undirected pairs: the radial MLP once per pair of opposite edges
# ---------------------------------------------------------------------------


@torch.library.custom_op("molix::edge_reverse", mutates_args=(), device_types="cuda")
def edge_reverse(edge_index: Tensor, num_nodes: int, row_ptr: Tensor, perm: Tensor, senders: Tensor,
                 feats: Tensor) -> tuple[Tensor, Tensor]:
    """``(rev, bad)``: ``rev[e]`` (int32) is the edge that runs opposite to e (sender and receiver
    swapped) with bit-identical features ``feats[e]`` (the radial inputs of the MLP), or -1 when there
    is not exactly one; ``bad`` (int32, one element) counts the edges without a partner."""
    _require_gpu("edge_reverse", edge_index, feats)
    E = edge_index.shape[0]
    f = feats.to(torch.float32).reshape(E, -1).contiguous()
    ei = edge_index.to(torch.int64).contiguous()
    rev = torch.empty(E, dtype=torch.int32, device=ei.device)
    bad = torch.zeros(2, dtype=torch.int32, device=ei.device)
    check(_lib.load().mnx_edge_reverse(ptr(ei), E, num_nodes, ptr(row_ptr), ptr(perm), ptr(senders), ptr(f),
                                       f.shape[1], ptr(rev), ptr(bad), _stream(ei)), "edge_reverse")
    return rev, bad[:1].clone()


@edge_reverse.register_fake
def _(edge_index, num_nodes, row_ptr, perm, senders, feats):
    return (edge_index.new_empty((edge_index.shape[0],), dtype=torch.int32),
            edge_index.new_empty((1,), dtype=torch.int32))


class EdgePairs:
    """The undirected pairs of a directed edge list whose two directions carry identical radial
    features (a neighbor list's pairs: opposite bond vectors are exact negations).  ``pairs``
    (int32, (E/2, 2)): the two edges of each pair, pair i led by its lower edge id, in ascending
    order of that id; ``wrow`` (int32, (E,)): the pair of each edge; ``lead`` (int64, (E/2,)): the
    lower edge of each pair.  ``build`` returns None unless every edge has exactly one partner
    (one host synchronisation)."""

    def __init__(self, pairs: Tensor, wrow: Tensor, lead: Tensor):
        self.pairs, self.wrow, self.lead = pairs, wrow, lead

    @staticmethod
    def build(edge_index: Tensor, num_nodes: int, row_ptr: Tensor, perm: Tensor, senders: Tensor,
              feats: Tensor) -> "EdgePairs | None":
        E = edge_index.shape[0]
        if E == 0 or E % 2:
            return None
        _require_gpu("EdgePairs", edge_index, feats)
        lib = _lib.load()
        dev = edge_index.device
        ei = edge_index.to(torch.int64).contiguous()
        f = feats.detach().to(torch.float32).reshape(E, -1).contiguous()
        wrow = torch.empty(E, dtype=torch.int32, device=dev)
        lead = torch.empty(E // 2, dtype=torch.int64, device=dev)
        pairs = torch.empty((E // 2, 2), dtype=torch.int32, device=dev)
        bad = torch.zeros(2, dtype=torch.int32, device=dev)
        ws = _ws(lib.mnx_edge_pairs_workspace_bytes(E), dev)
        check(lib.mnx_edge_pairs(ptr(ei), E, num_nodes, ptr(row_ptr), ptr(perm), ptr(senders), ptr(f), f.shape[1],
                                 ptr(wrow), ptr(lead), ptr(pairs), ptr(bad), ptr(ws), ws.numel(), _stream(ei)),
              "edge pairs")
        if int(bad[0].item()) != 0:
            return None
        return EdgePairs(pairs, wrow, lead)

    def holds_for(self, feats: Tensor) -> bool:
        """Whether the two edges of every pair still have bit-identical rows of ``feats`` (one host
        synchronisation; the pairing itself depends only on the edge list)."""
        lib = _lib.load()
        f = feats.detach().to(torch.float32).reshape(self.wrow.shape[0], -1).contiguous()
        bad = torch.zeros(1, dtype=torch.int32, device=f.device)
        check(lib.mnx_edge_pairs_verify(ptr(self.pairs), self.pairs.shape[0], ptr(f), f.shape[1], ptr(bad),
                                        _stream(f)), "edge pairs verify")
        return int(bad.item()) == 0


@torch.library.custom_op("molix::gather_rows", mutates_args=(), device_types="cuda")
def gather_rows(src: Tensor, idx: Tensor) -> Tensor:
    """``src[idx]`` for a float32 (R, F) ``src`` and int64 indices (the radial features of the lead
    edge of each undirected pair; Allegro's type-pair embedding rows).  Its backward scatters the
    gradient rows back without accumulation, so it needs distinct indices: callers with repeated
    indices use it where ``src`` takes no gradient."""
    _require_gpu("gather_rows", src, idx)
    if src.dtype != torch.float32 or src.dim() != 2 or idx.dtype != torch.int64 or idx.dim() != 1:
        raise ValueError("gather_rows: src must be float32 (R, F), idx int64 (n,)")
    s = src.contiguous()
    i = idx.contiguous()
    out = s.new_empty(i.shape[0], s.shape[1])
    check(_lib.load().mnx_gather_rows_f32(ptr(s), ptr(i), i.shape[0], s.shape[1], ptr(out), _stream(s)),
          "gather_rows")
    return out


@gather_rows.register_fake
def _(src, idx):
    return src.new_empty(idx.shape[0], src.shape[1])


@torch.library.custom_op("molix::scatter_rows", mutates_args=(), device_types="cuda")
def scatter_rows(grad: Tensor, idx: Tensor, num_rows: int) -> Tensor:
    """The adjoint of ``gather_rows``: a (num_rows, F) tensor with ``grad[i]`` at row ``idx[i]``, zero
    elsewhere (indices distinct)."""
    g = grad.to(torch.float32).contiguous()
    i = idx.contiguous()
    out = torch.zeros(num_rows, g.shape[1], dtype=torch.float32, device=g.device)
    check(_lib.load().mnx_scatter_rows_f32(ptr(g), ptr(i), i.shape[0], g.shape[1], ptr(out), _stream(g)),
          "scatter_rows")
    return out


@scatter_rows.register_fake
def _(grad, idx, num_rows):
    return grad.new_empty(num_rows, grad.shape[1])


def _gr_setup(ctx, inputs, output):
    src, idx = inputs
    ctx.save_for_backward(idx)
    ctx.rows = src.shape[0]


def _gr_backward(ctx, grad):
    (idx,) = ctx.saved_tensors
    return scatter_rows(grad, idx, ctx.rows), None


gather_rows.register_autograd(_gr_backward, setup_context=_gr_setup)


def _sr_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[1])


def _sr_backward(ctx, grad):
    (idx,) = ctx.saved_tensors
    return gather_rows(grad.contiguous(), idx), None, None


scatter_rows.register_autograd(_sr_backward, setup_context=_sr_setup)


@torch.library.custom_op("molix::edge_weights_backward_pairs", mutates_args=(), device_types="cuda")
def edge_weights_backward_pairs(grad: Tensor, pairs: Tensor, weight: Tensor) -> Tensor:
    """``(grad[pairs[:, 0]] + grad[pairs[:, 1]]) @ weight``: dL/dh of an output layer applied once per
    undirected pair, from the per-edge weight gradient (same split-fp16 arithmetic as
    ``edge_weights_backward``, the two rows added as they are loaded)."""
    N, K = weight.shape
    if grad.dim() != 2 or grad.shape[1] != N:
        raise ValueError("edge_weights_backward_pairs: grad must be (E, N)")
    if pairs.dtype != torch.int32 or pairs.dim() != 2 or pairs.shape[1] != 2 or not pairs.is_contiguous():
        raise ValueError("edge_weights_backward_pairs: pairs must be a contiguous int32 (P, 2) tensor")
    g = _aligned16(grad.to(torch.float32))
    frag = _ew_frag(weight, True)
    gh = g.new_empty(pairs.shape[0], K)
    check(_lib.load().mnx_edge_weights_bwd_pairs_f32(ptr(g), ptr(pairs), pairs.shape[0], N, ptr(frag), K, ptr(gh),
                                                     _stream(g)), "edge_weights backward (pairs)")
    return gh


@edge_weights_backward_pairs.register_fake
def _(grad, pairs, weight):
    return grad.new_empty(pairs.shape[0], weight.shape[1])


@torch.library.custom_op("molix::pair_sum_rows", mutates_args=(), device_types="cuda")
def pair_sum_rows(src: Tensor, pairs: Tensor) -> Tensor:
    """``src[pairs[:, 0]] + src[pairs[:, 1]]`` for int32 (P, 2) pairs and rows of a multiple of 4 floats
    (one kernel)."""
    _require_gpu("pair_sum_rows", src, pairs)
    if src.dtype != torch.float32 or src.dim() != 2 or src.shape[1] % 4:
        raise ValueError("pair_sum_rows: src must be float32 (n, F) with F a multiple of 4")
    s = _aligned16(src)
    p = pairs.to(torch.int32).contiguous()
    out = s.new_empty(p.shape[0], s.shape[1])
    check(_lib.load().mnx_pair_sum_rows_f32(ptr(s), ptr(p), p.shape[0], s.shape[1], ptr(out), _stream(s)),
          "pair_sum_rows")
    return out


@pair_sum_rows.register_fake
def _(src, pairs):
    return src.new_empty(pairs.shape[0], src.shape[1])


def tp_gh_batches(row_ptr: Tensor) -> Tensor:
    """The work list of ``tp_weight_grad_batched``: (receiver, first CSR slot) of every batch of up to 32
    consecutive edges of one receiver, int32 (B, 2).  One host synchronisation (the batch count):
    build it once per graph."""
    rp = row_ptr.to(torch.int64)
    n = rp.shape[0] - 1
    nb = (rp[1:] - rp[:-1] + 31) // 32
    total = int(nb.sum().item())
    r = torch.repeat_interleave(torch.arange(n, device=rp.device), nb, output_size=total)
    first = torch.cumsum(nb, 0) - nb
    t0 = rp[:-1].index_select(0, r) + 32 * (torch.arange(total, device=rp.device) - first.index_select(0, r))
    return torch.stack([r, t0], 1).to(torch.int32).contiguous()


_GH2_ROWS: dict = {}


def _gh2_frag(weight: Tensor, config: int, channels: int) -> Tensor:
    """The output layer's W with its rows in ``tp_weight_grad_batched``'s contraction order, packed
    as the backward fragment of ``edge_weights``."""
    key = (config, channels, weight.device)
    rows = _GH2_ROWS.get(key)
    if rows is None:
        num_paths = tp_config_info(config)[0]
        host = (C.c_int32 * (num_paths * channels))()
        check(_lib.load().mnx_tp_weight_grad_rows(config, channels, host), "tp_weight_grad rows")
        rows = torch.tensor(list(host), dtype=torch.int64).to(weight.device)
        _GH2_ROWS[key] = rows
    return _ew_frag(weight.detach().index_select(0, rows), True)


@torch.library.custom_op("molix::tp_weight_grad_batched", mutates_args=(), device_types="cuda")
def tp_weight_grad_batched(x: Tensor, Y: Tensor, grad_out: Tensor, row_ptr: Tensor, perm: Tensor, senders: Tensor,
                           batches: Tensor, weight: Tensor, config: int, channels: int) -> Tensor:
    """``grad_h = gw @ weight`` per directed edge (as ``tp_weight_grad``) over the receiver CSR, one
    wavefront per batch of ``tp_gh_batches``: the batch's receiver's output gradient is staged in LDS
    and the sender rows are read once per 16-channel chunk, so the per-edge weight gradient ``gw``
    is formed from registers and LDS and multiplied on the matrix cores without being written."""
    _require_gpu("tp_weight_grad_batched", x, Y, grad_out, row_ptr, perm, senders, batches, weight)
    num_paths, nx, ny, no = tp_config_info(config)
    Nw, K = weight.shape
    if Nw != num_paths * channels:
        raise ValueError(f"tp_weight_grad_batched: weight has {Nw} rows, the product has {num_paths} x {channels}")
    xs = _aligned16(_f32_rows(x, nx * channels, "x"))
    Ys = _f32_rows(Y, ny, "Y")
    go = _aligned16(_f32_rows(grad_out, no * channels, "grad_out"))
    N, E = xs.shape[0], Ys.shape[0]
    if (go.shape[0] != N or row_ptr.shape[0] != N + 1 or perm.shape[0] != E or senders.shape[0] != E
            or batches.dim() != 2 or batches.shape[1] != 2):
        raise ValueError("tp_weight_grad_batched: inconsistent sizes of x / Y / grad_out / CSR / batches")
    rp, pm, sd = (t.to(torch.int32).contiguous() for t in (row_ptr, perm, senders))
    bt = batches.to(torch.int32).contiguous()
    frag = _gh2_frag(weight, config, channels)
    gh = xs.new_empty(E, K)
    check(_lib.load().mnx_tp_weight_grad_batched_f32(config, channels, ptr(xs), ptr(Ys), ptr(go), ptr(rp), ptr(pm),
                                                     ptr(sd), ptr(bt), bt.shape[0], N, E, ptr(frag), K, ptr(gh),
                                                     _stream(xs)), "tp_weight_grad_batched")
    return gh


@tp_weight_grad_batched.register_fake
def _(x, Y, grad_out, row_ptr, perm, senders, batches, weight, config, channels):
    return x.new_empty(Y.shape[0], weight.shape[1])


_AUX_STREAMS: dict = {}


def _aux_stream(device: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for work that overlaps the current stream's."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    s = _AUX_STREAMS.get(idx)
    if s is None:
        s = _AUX_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return s


def tp_backward_overlapped(grad_out: Tensor, x: Tensor, Y: Tensor, w: Tensor, row_ptr: Tensor, perm: Tensor,
                           senders: Tensor, wrow: Tensor | None, weight: Tensor, pairs: Tensor | None, config: int,
                           channels: int, need_x: bool, need_Y: bool) -> tuple[Tensor, Tensor, Tensor]:
    """``(grad_x, grad_Y, grad_h)`` of ``<grad_out, tp_scatter(x, Y, w[wrow])>`` with ``w = h @ weight.T + b``:
    the tensor product's backward runs one path group at a time on the current stream
    (``mnx_tp_bwd_group_rows_f32``), and as each group's columns of the per-edge weight gradient are
    written, a second stream multiplies them into ``grad_h`` (``mnx_edge_weights_bwd_cols_f32``,
    accumulating over the groups in launch order) while the next group's backward runs: the
    atomic-bound tensor-product backward and the memory-bound output-layer product overlap.
    ``pairs``: ``grad_h`` per undirected pair (the two edges' rows added), else per edge."""
    lib = _lib.load()
    num_paths, nx, ny, no = tp_config_info(config)
    Ch = channels
    Nw, K = weight.shape
    if Nw != num_paths * Ch:
        raise ValueError(f"tp_backward_overlapped: weight has {Nw} rows, the product has {num_paths} x {Ch}")
    xs = _f32_rows(x, nx * Ch, "x")
    Ys = _f32_rows(Y, ny, "Y")
    wss = _f32_rows(w, num_paths * Ch, "w")
    go = _f32_rows(grad_out, no * Ch, "grad_out")
    N, E = row_ptr.shape[0] - 1, Ys.shape[0]
    _check_wrow(wrow, E, wss.shape[0], "tp_backward_overlapped")
    dev = xs.device
    gx = torch.zeros_like(xs) if need_x else xs.new_empty(0)
    gY = torch.empty_like(Ys) if need_Y else Ys.new_empty(0)
    gw = wss.new_empty(E, num_paths * Ch)
    rows = pairs.shape[0] if pairs is not None else E
    gh = xs.new_empty(rows, K)
    if E == 0:
        gY.zero_() if need_Y else None
        return gx, gY, gh.zero_()
    ws = _ws(lib.mnx_tp_bwd_workspace_bytes(config, Ch, E), dev) if need_Y else None
    bounds = (C_int32_5)()
    ng = lib.mnx_tp_group_paths(config, bounds)
    if ng <= 0:
        raise RuntimeError("tp_backward_overlapped: no path groups")
    Wf = weight.detach().to(torch.float32).contiguous()
    main, aux = torch.cuda.current_stream(dev), _aux_stream(dev)
    ms, ax = main.cuda_stream, aux.cuda_stream
    # largest groups first, so that the product left without overlap at the end is the smallest
    order = sorted(range(ng), key=lambda g: -(bounds[g + 1] - bounds[g]))
    frags = []
    for i, g in enumerate(order):
        p0, p1 = bounds[g], bounds[g + 1]
        check(lib.mnx_tp_bwd_group_rows_f32(config, Ch, g, ptr(xs), ptr(Ys), ptr(wss), ptr(wrow), ptr(go),
                                            ptr(row_ptr), ptr(perm), ptr(senders), N, E, ptr(gx) if need_x else None,
                                            ptr(gw), ptr(ws), ws.numel() if ws is not None else 0, ms),
              "tp_scatter backward (path group)")
        frag = _ew_frag(Wf[p0 * Ch:p1 * Ch], True)
        frags.append(frag)
        ev = torch.cuda.Event()
        ev.record(main)
        aux.wait_event(ev)
        check(lib.mnx_edge_weights_bwd_cols_f32(gw.data_ptr() + 4 * p0 * Ch, num_paths * Ch, ptr(pairs), rows,
                                                (p1 - p0) * Ch, ptr(frag), K, ptr(gh), int(i > 0), ax),
              "edge_weights backward (column slice)")
    if need_Y:
        check(lib.mnx_tp_bwd_reduce_gy_f32(config, Ch, E, ptr(ws), ws.numel(), ptr(gY), ms), "tp_scatter grad_Y")
    # the current stream waits for the second one before anything here is freed, so the caching
    # allocator (which reuses blocks in the current stream's order) cannot hand them out early
    main.wait_stream(aux)
    del frags
    return gx, gY, gh


def tp_backward_gh_supported(config: int, channels: int, K: int) -> bool:
    """Whether ``tp_scatter_backward_gh`` has a kernel for this product and hidden width."""
    return config >= 0 and bool(_lib.load().mnx_tp_bwd_gh_supported(config, channels, K))


@torch.library.custom_op("molix::tp_scatter_backward_gh", mutates_args=(), device_types="cuda")
def tp_scatter_backward_gh(grad_out: Tensor, x: Tensor, Y: Tensor, w: Tensor, row_ptr: Tensor, perm: Tensor,
                           senders: Tensor, wrow: Tensor | None, weight: Tensor, config: int, channels: int,
                           need_x: bool, need_Y: bool) -> tuple[Tensor, Tensor, Tensor]:
    """``(grad_x, grad_Y, grad_h)`` of ``<grad_out, tp_scatter(x, Y, w[wrow])>`` with ``w = h @ weight.T + b``:
    the tensor-product backward fused with the output layer's input gradient ``grad_h = gw @ weight``
    per directed edge, the per-edge weight gradient ``gw`` formed and multiplied on the matrix cores
    without being written (``mnx_tp_bwd_gh_rows_f32``).  First order only (eval mode)."""
    _require_gpu("tp_scatter_backward_gh", grad_out, x, Y, w, row_ptr, perm, senders, wrow, weight)
    lib = _lib.load()
    num_paths, nx, ny, no = tp_config_info(config)
    Nw, K = weight.shape
    if Nw != num_paths * channels:
        raise ValueError(f"tp_scatter_backward_gh: weight has {Nw} rows, the product has {num_paths} x {channels}")
    xs = _f32_rows(x, nx * channels, "x")
    Ys = _f32_rows(Y, ny, "Y")
    wss = _f32_rows(w, num_paths * channels, "w")
    go = _f32_rows(grad_out, no * channels, "grad_out")
    Wc = _f32_rows(weight, K, "weight")
    N, E = row_ptr.shape[0] - 1, Ys.shape[0]
    _check_wrow(wrow, E, wss.shape[0], "tp_scatter_backward_gh")
    gx = torch.zeros_like(xs) if need_x else xs.new_empty(0)
    gY = torch.empty_like(Ys) if need_Y else Ys.new_empty(0)
    gh = xs.new_empty(E, K)
    ws = _ws(lib.mnx_tp_bwd_gh_workspace_bytes(config, channels, E, K, ny), xs.device)
    check(lib.mnx_tp_bwd_gh_rows_f32(config, channels, ptr(xs), ptr(Ys), ptr(wss), ptr(wrow), ptr(go), ptr(row_ptr),
                                     ptr(perm), ptr(senders), N, E, ny, ptr(Wc), K, ptr(gx), ptr(gY), ptr(gh),
                                     ptr(ws), ws.numel(), _stream(xs)), "tp_scatter backward (fused grad h)")
    if E == 0:
        gh.zero_()
        gY.zero_() if need_Y else None
    return gx, gY, gh


@tp_scatter_backward_gh.register_fake
def _(grad_out, x, Y, w, row_ptr, perm, senders, wrow, weight, config, channels, need_x, need_Y):
    return (torch.empty_like(x) if need_x else x.new_empty(0), torch.empty_like(Y) if need_Y else Y.new_empty(0),
            x.new_empty(Y.shape[0], weight.shape[1]))


@torch.library.custom_op("molix::radial_tp_pairs", mutates_args=(), device_types="cuda")
def radial_tp_pairs(x: Tensor, Y: Tensor, h: Tensor, weight: Tensor, bias: Tensor | None, row_ptr: Tensor,
                    perm: Tensor, senders: Tensor, wrow: Tensor, pairs: Tensor, config: int,
                    channels: int, batches: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """``(tp_scatter(x, Y, w[wrow]), w)`` with ``w = h @ weight.T + bias`` computed once per undirected
    pair (``wrow`` maps every edge to its pair, ``pairs`` lists each pair's two edges, lead first:
    ``EdgePairs``).  Equal to the output layer applied per directed edge (the reference's
    composition, ``mace.py:321-329``, ``tensor_product.py:101-111``), since both directions of a pair
    have the same radial inputs.  ``w`` (one row per pair) is returned for the backward.

    ``h``, the radial MLP's hidden activations (``radial_mlp.py:76-82``), has one row per pair (its
    lead edge's; pair mode) or one row per edge (edge mode).  In pair mode the backward adds the two
    edges' weight gradients as it forms the output layer's input gradient
    (``edge_weights_backward_pairs``): the gradient reaching each pair's radial inputs is the sum
    of both directions', which leaves every function of the positions (energies, forces, virials)
    as per edge.  In edge mode the forward uses the lead rows of ``h`` and the backward gives every
    edge its own input gradient (``edge_weights_backward``), as the per-edge composition does.

    With ``batches`` (``tp_gh_batches(row_ptr)``) and no output-layer parameter gradient, the backward
    does not write the per-edge weight gradient: the tensor-product backward gives grad x and grad Y
    only and ``tp_weight_grad_batched`` forms grad h per directed edge (summed over each pair's two
    edges in pair mode)."""
    if h.shape[0] == pairs.shape[0]:
        w = edge_weights(h, weight, bias)
    else:  # the lead rows of h, read in place
        w = _edge_weights_rows(h, pairs[:, 0].contiguous(), weight, bias)
    return tp_scatter(x, Y, w, row_ptr, perm, senders, config, channels, wrow=wrow), w


@radial_tp_pairs.register_fake
def _(x, Y, h, weight, bias, row_ptr, perm, senders, wrow, pairs, config, channels, batches=None):
    num_paths, nx, ny, no = tp_config_info(config)
    return x.new_empty((row_ptr.shape[0] - 1, no * channels)), h.new_empty((pairs.shape[0], weight.shape[0]))


def _rtpp_setup(ctx, inputs, output):
    x, Y, h, weight, bias, row_ptr, perm, senders, wrow, pairs, config, channels = inputs[:12]
    batches = inputs[12] if len(inputs) > 12 else None
    ctx.save_for_backward(x, Y, h, weight, output[1], row_ptr, perm, senders, wrow, pairs, batches)
    ctx.config, ctx.channels, ctx.has_bias = config, channels, bias is not None
    # the returned weights usually get no gradient: pass None rather than a (pairs, N) zero tensor
    ctx.set_materialize_grads(False)


def _rtpp_backward(ctx, g_out, g_w):
    x, Y, h, weight, w, row_ptr, perm, senders, wrow, pairs, batches = ctx.saved_tensors
    nig = ctx.needs_input_grad
    need_x, need_Y, need_h, need_W = nig[0], nig[1], nig[2], nig[3]
    need_b = nig[4] and ctx.has_bias
    gx = gY = gh = gW = gb = None
    per_pair = h.shape[0] == pairs.shape[0]
    if batches is not None and g_out is not None and need_h and not (need_W or need_b):
        # grad h without the per-edge weight gradient in memory
        go = g_out.contiguous()
        if need_x or need_Y:
            gx, gY, _ = tp_scatter_backward(go, x, Y, w, row_ptr, perm, senders, ctx.config, ctx.channels,
                                            need_x, need_Y, False, wrow=wrow)
            gx = gx.reshape(x.shape) if need_x else None
            gY = gY.reshape(Y.shape) if need_Y else None
        ghe = tp_weight_grad_batched(x, Y, go, row_ptr, perm, senders, batches, weight, ctx.config, ctx.channels)
        gh = pair_sum_rows(ghe, pairs) if per_pair else ghe
        if g_w is not None:
            ghw = edge_weights_backward(g_w.contiguous(), weight)
            gh = gh + ghw if per_pair else gh.index_add(0, pairs[:, 0].long(), ghw)
        return gx, gY, gh, None, None, None, None, None, None, None, None, None, None
    if (batches is None and _settings.tp_bwd_fused and g_out is not None and need_h and not (need_W or need_b)
            and tp_backward_gh_supported(ctx.config, ctx.channels, weight.shape[1])):
        # the tensor-product backward and the output layer's input gradient in one pass: the
        # per-edge weight gradient is formed and consumed on chip
        gx, gY, ghe = tp_scatter_backward_gh(g_out.contiguous(), x, Y, w, row_ptr, perm, senders, wrow, weight,
                                             ctx.config, ctx.channels, need_x, need_Y)
        gx = gx.reshape(x.shape) if need_x else None
        gY = gY.reshape(Y.shape) if need_Y else None
        gh = pair_sum_rows(ghe, pairs) if per_pair else ghe
        if g_w is not None:
            ghw = edge_weights_backward(g_w.contiguous(), weight)
            gh = gh + ghw if per_pair else gh.index_add(0, pairs[:, 0].long(), ghw)
        return gx, gY, gh, None, None, None, None, None, None, None, None, None, None
    if (batches is None and _settings.tp_bwd_overlap and g_out is not None and need_h and not (need_W or need_b)
            and ctx.channels % 8 == 0 and weight.shape[1] in (16, 32, 64, 128)):
        # the tensor-product backward group by group, each group's weight-gradient columns
        # multiplied into grad h on a second stream while the next group runs
        gx, gY, gh = tp_backward_overlapped(g_out.contiguous(), x, Y, w, row_ptr, perm, senders, wrow, weight,
                                            pairs if per_pair else None, ctx.config, ctx.channels, need_x, need_Y)
        gx = gx.reshape(x.shape) if need_x else None
        gY = gY.reshape(Y.shape) if need_Y else None
        if g_w is not None:
            ghw = edge_weights_backward(g_w.contiguous(), weight)
            gh = gh + ghw if per_pair else gh.index_add(0, pairs[:, 0].long(), ghw)
        return gx, gY, gh, None, None, None, None, None, None, None, None, None, None
    gw = None  # per-edge weight gradient, (E, N)
    if g_out is not None and (need_x or need_Y or need_h or need_W or need_b):
        gx, gY, gw = tp_scatter_backward(g_out.contiguous(), x, Y, w, row_ptr, perm, senders, ctx.config,
                                         ctx.channels, need_x, need_Y, need_h or need_W or need_b, wrow=wrow)
        gx = gx.reshape(x.shape) if need_x else None
        gY = gY.reshape(Y.shape) if need_Y else None
        if not (need_h or need_W or need_b):
            gw = None
    lead = pairs[:, 0].long()
    if need_h:
        if gw is None:
            gh = torch.zeros_like(h)
        elif per_pair:
            gh = edge_weights_backward_pairs(gw, pairs, weight)
        else:
            gh = edge_weights_backward(gw, weight)
        if g_w is not None:  # a caller that used the returned per-pair weights as well
            ghw = edge_weights_backward(g_w.contiguous(), weight)
            gh = gh + ghw if per_pair else gh.index_add(0, lead, ghw)
    if need_W or need_b:  # training: the per-pair weight gradient, then hipBLASLt GEMMs
        gp = gw[lead] + gw[pairs[:, 1].long()] if gw is not None else torch.zeros_like(w)
        if g_w is not None:
            gp = gp + g_w
        if need_W:
            hl = h if per_pair else h.index_select(0, lead)
            gW = tall_tn(gp, hl)
        gb = gp.sum(0) if need_b else None
    return gx, gY, gh, gW, gb, None, None, None, None, None, None, None, None


radial_tp_pairs.register_autograd(_rtpp_backward, setup_context=_rtpp_setup)


# ---------------------------------------------------------------------------
# Equivariant block linear
# ---------------------------------------------------------------------------

def block_linear_desc(blocks) -> list[int]:
    """Flat launch list of ``molix::block_linear``: per output block
    ``out_off, mul, d, w_off, nseg`` followed by ``col, comp, len`` of each input segment."""
    flat = []
    for off, mul, d, segs, woff in blocks:
        flat += [int(off), int(mul), int(d), int(woff), len(segs)]
        for sg in segs:
            flat += [int(v) for v in sg]
    return flat


def _parse_blocks(blocks: list[int]):
    i = 0
    while i < len(blocks):
        if i + 5 > len(blocks):
            raise ValueError("block_linear: truncated block list")
        off, mul, d, woff, n = blocks[i:i + 5]
        segs = blocks[i + 5:i + 5 + 3 * n]
        if n < 0 or len(segs) != 3 * n:
            raise ValueError("block_linear: truncated block list")
        i += 5 + 3 * n
        yield off, mul, d, woff, [tuple(segs[3 * s:3 * s + 3]) for s in range(n)]


@torch.library.custom_op("molix::block_linear", mutates_args=(), device_types="cuda")
def block_linear(a: Tensor, weights: Tensor, blocks: list[int], out_dim: int) -> Tensor:
    """One ``mnx_block_linear_f32`` launch per output block of an ir_mul linear
    (``src/molrep/interaction/linear.py:43-105``): ``blocks`` as built by ``block_linear_desc``,
    ``weights`` the concatenated fragment-ordered (pre-scaled) weights of every block.  Every column
    of the (R, out_dim) result must belong to exactly one block."""
    _require_gpu("block_linear", a, weights)
    if a.dtype != torch.float32 or weights.dtype != torch.float32 or a.dim() != 2:
        raise TypeError("block_linear: a must be float32 (R, dim_in) and weights float32")
    lib = _lib.load()
    x = _aligned16(a)
    w = _aligned16(weights.reshape(-1))
    R, dim_in = x.shape
    out = x.new_empty(R, out_dim)
    covered = 0
    for off, mul, d, woff, segs in _parse_blocks(blocks):
        if off < 0 or off + d * mul > out_dim or mul <= 0 or d <= 0:
            raise ValueError("block_linear: output block outside the result")
        covered += d * mul
        if any(c < 0 or ln <= 0 or c + (d - 1) * cp + ln > dim_in for c, cp, ln in segs):
            raise ValueError("block_linear: input segment outside the input rows")
        k = sum(ln for _, _, ln in segs)
        if segs and (woff < 0 or woff + lib.mnx_block_linear_frag_floats(k, mul) > w.numel()):
            raise ValueError("block_linear: block weights outside the weight vector")
        n = len(segs)
        cols = (C.c_int64 * max(n, 1))(*[sg[0] for sg in segs])
        comps = (C.c_int32 * max(n, 1))(*[sg[1] for sg in segs])
        lens = (C.c_int32 * max(n, 1))(*[sg[2] for sg in segs])
        wp = w.data_ptr() + 4 * woff if segs else None
        check(lib.mnx_block_linear_f32(ptr(x), dim_in, n, cols, comps, lens, wp, mul, R, d, ptr(out), out_dim, off,
                                       mul, _stream(x)), "block_linear")
    if covered != out_dim:
        raise ValueError("block_linear: output blocks do not cover the result")
    return out


@block_linear.register_fake
def _(a, weights, blocks, out_dim):
    return a.new_empty(a.shape[0], out_dim)


@torch.library.custom_op("molix::class_groups", mutates_args=(), device_types="cuda")
def _class_groups_op(classes: Tensor, num_classes: int) -> tuple[Tensor, Tensor]:
    lib = _lib.load()
    c = classes.reshape(-1).to(torch.int64).contiguous()
    n = c.shape[0]
    order = torch.empty(n, dtype=torch.int32, device=c.device)
    class_start = torch.empty(num_classes + 2, dtype=torch.int32, device=c.device)
    ws = _ws(lib.mnx_class_groups_workspace_bytes(n, num_classes), c.device)
    check(lib.mnx_class_groups(ptr(c), n, num_classes, ptr(order), ptr(class_start), ptr(ws), ws.numel(),
                               _stream(c)), "class_groups")
    return order, class_start


@_class_groups_op.register_fake
def _(classes, num_classes):
    return (classes.new_empty(classes.numel(), dtype=torch.int32),
            classes.new_empty(num_classes + 2, dtype=torch.int32))


def class_groups(classes: Tensor, num_classes: int) -> tuple[Tensor, Tensor]:
    """Nodes grouped by class without a host synchronisation: ``order`` (int32, classes ascending,
    ascending node id within a class, out-of-range classes last) and ``class_start`` (int32,
    ``num_classes + 2`` entries: where class s begins in ``order``, s = num_classes being the
    out-of-range nodes)."""
    if classes.device.type != "cuda":
        raise RuntimeError(f"molix::class_groups runs on the GPU only (got a {classes.device} tensor)")
    return _class_groups_op(classes, int(num_classes))


@torch.library.custom_op("molix::indexed_block_linear", mutates_args=(), device_types="cuda")
def indexed_block_linear(a: Tensor, weights: Tensor, order: Tensor, class_start: Tensor, blocks: list[int],
                         out_dim: int) -> Tensor:
    """``block_linear`` with one weight set per node class (``cuet.Linear(weight_classes=S,
    method="indexed_linear")``, ``src/molrep/interaction/element_update.py:101-109``): ``weights``
    (S, F) holds every class's concatenated fragment-ordered weights, ``order`` / ``class_start``
    come from ``class_groups``.  Nodes of an out-of-range class get zeros."""
    _require_gpu("indexed_block_linear", a, weights, order, class_start)
    if a.dtype != torch.float32 or weights.dtype != torch.float32 or a.dim() != 2 or weights.dim() != 2:
        raise TypeError("indexed_block_linear: a must be float32 (R, dim_in) and weights float32 (S, F)")
    lib = _lib.load()
    x = _aligned16(a)
    S, F = weights.shape
    if F % 4:
        raise ValueError("indexed_block_linear: per-class weight length must be a multiple of 4")
    w = _aligned16(weights)
    R, dim_in = x.shape
    if order.shape[0] != R or class_start.shape[0] != S + 2:
        raise ValueError("indexed_block_linear: order must be (R,) and class_start (S + 2,)")
    od = order.to(torch.int32).contiguous()
    cs = class_start.to(torch.int32).contiguous()
    out = x.new_empty(R, out_dim)
    covered = 0
    for off, mul, d, woff, segs in _parse_blocks(blocks):
        if off < 0 or off + d * mul > out_dim or mul <= 0 or d <= 0:
            raise ValueError("indexed_block_linear: output block outside the result")
        covered += d * mul
        if any(c < 0 or ln <= 0 or c + (d - 1) * cp + ln > dim_in for c, cp, ln in segs):
            raise ValueError("indexed_block_linear: input segment outside the input rows")
        k = sum(ln for _, _, ln in segs)
        if segs and (woff < 0 or woff + lib.mnx_block_linear_frag_floats(k, mul) > F):
            raise ValueError("indexed_block_linear: block weights outside the per-class weights")
        n = len(segs)
        cols = (C.c_int64 * max(n, 1))(*[sg[0] for sg in segs])
        comps = (C.c_int32 * max(n, 1))(*[sg[1] for sg in segs])
        lens = (C.c_int32 * max(n, 1))(*[sg[2] for sg in segs])
        wp = w.data_ptr() + 4 * woff if segs else None
        check(lib.mnx_indexed_block_linear_f32(ptr(x), dim_in, n, cols, comps, lens, wp, F, S, ptr(od), ptr(cs),
                                               mul, R, d, ptr(out), out_dim, off, mul, _stream(x)),
              "indexed_block_linear")
    if covered != out_dim:
        raise ValueError("indexed_block_linear: output blocks do not cover the result")
    return out


@indexed_block_linear.register_fake
def _(a, weights, order, class_start, blocks, out_dim):
    return a.new_empty(a.shape[0], out_dim)


# ---------------------------------------------------------------------------
# Bond vectors
# ---------------------------------------------------------------------------

@torch.library.custom_op("molix::bond_vectors", mutates_args=(), device_types="cuda")
def bond_vectors(positions: Tensor, edge_index: Tensor, shifts: Tensor | None = None) -> Tensor:
    """``positions[edge_index[:, 1]] - positions[edge_index[:, 0]] - shifts`` for an (E, 2) edge list of
    [sender, receiver] rows: the reference's ``bond_diff = pos[target] - pos[source]``
    (``src/molix/data/tasks/neighbor_list.py:86-95``).  Backward: one kernel, receiver terms summed
    over each wavefront's runs of equal receivers (neighbor-list order), sender terms atomically."""
    _require_gpu("bond_vectors", positions, edge_index, shifts)
    if positions.dtype != torch.float32:
        raise TypeError("bond_vectors: positions must be float32")
    pos = positions.detach().contiguous()
    ei = edge_index.to(torch.int64).contiguous()
    if ei.dim() != 2 or ei.shape[1] != 2:
        raise ValueError("edge_index must be (E, 2)")
    sh = None if shifts is None else shifts.detach().to(torch.float32).reshape(-1, 3).contiguous()
    if sh is not None and sh.shape[0] != ei.shape[0]:
        raise ValueError("shifts must be (E, 3)")
    out = pos.new_empty(ei.shape[0], 3)
    check(_lib.load().mnx_bond_vectors_f32(ptr(pos), pos.shape[0], ptr(ei), ptr(sh), ei.shape[0], ptr(out),
                                           _stream(pos)), "bond_vectors")
    return out


@bond_vectors.register_fake
def _(positions, edge_index, shifts=None):
    return positions.new_empty(edge_index.shape[0], 3)


@torch.library.custom_op("molix::bond_vectors_backward", mutates_args=(), device_types="cuda")
def bond_vectors_backward(grad: Tensor, edge_index: Tensor, num_atoms: int) -> Tensor:
    ei = edge_index.to(torch.int64).contiguous()
    g = grad.to(torch.float32).contiguous()
    gpos = g.new_empty(num_atoms, 3)
    check(_lib.load().mnx_bond_vectors_bwd_f32(ptr(ei), ptr(g), ei.shape[0], num_atoms, ptr(gpos), _stream(g)),
          "bond_vectors backward")
    return gpos


@bond_vectors_backward.register_fake
def _(grad, edge_index, num_atoms):
    return grad.new_empty(num_atoms, 3)


def _bond_setup(ctx, inputs, output):
    positions, edge_index = inputs[0], inputs[1]
    ctx.save_for_backward(edge_index)
    ctx.num_atoms = positions.shape[0]


def _bond_bwd(ctx, grad):
    (edge_index,) = ctx.saved_tensors
    gpos = bond_vectors_backward(grad, edge_index, ctx.num_atoms) if ctx.needs_input_grad[0] else None
    gsh = -grad if (len(ctx.needs_input_grad) > 2 and ctx.needs_input_grad[2]) else None
    return gpos, None, gsh


bond_vectors.register_autograd(_bond_bwd, setup_context=_bond_setup)


# ---------------------------------------------------------------------------
# Per-channel scaling of an ir_mul edge tensor (Allegro's output env scaling)
# ---------------------------------------------------------------------------


def _cs_rows(t: Tensor, width: int, what: str) -> Tensor:
    if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != width:
        raise ValueError(f"channel_scale: {what} must be float32 (E, {width})")
    return _aligned16(t)


@torch.library.custom_op("molix::channel_scale", mutates_args=(), device_types="cuda")
def channel_scale(t: Tensor, s: Tensor, components: int) -> Tensor:
    """``out[e][d][c] = t[e][d][c] * s[e][c]`` for an (E, D*F) ir_mul tensor and (E, F) scales: the
    reference's ``_scale_by_channel`` (src/molzoo/allegro.py:95-128); one HIP pass each way (the
    backward forms both gradients in one pass, ``mnx_channel_scale_bwd_f32``)."""
    _require_gpu("channel_scale", t, s)
    F = s.shape[1]
    ts = _cs_rows(t, components * F, "t")
    ss = _cs_rows(s, F, "s")
    if ts.shape[0] != ss.shape[0]:
        raise ValueError("channel_scale: t and s must have the same number of rows")
    out = torch.empty_like(ts)
    check(_lib.load().mnx_channel_scale_f32(ptr(ts), ptr(ss), ts.shape[0], components, F, ptr(out), _stream(ts)),
          "channel_scale")
    return out


@channel_scale.register_fake
def _(t, s, components):
    return t.new_empty(t.shape)


@torch.library.custom_op("molix::channel_scale_backward", mutates_args=(), device_types="cuda")
def channel_scale_backward(grad: Tensor, t: Tensor, s: Tensor, components: int, need_t: bool,
                           need_s: bool) -> tuple[Tensor, Tensor]:
    """(grad * s, sum_d grad * t) of ``channel_scale`` in one pass; an empty tensor for a gradient
    not requested."""
    _require_gpu("channel_scale_backward", grad, t, s)
    F = s.shape[1]
    g = _cs_rows(grad, components * F, "grad")
    ts = _cs_rows(t, components * F, "t")
    ss = _cs_rows(s, F, "s")
    gt = torch.empty_like(g) if need_t else g.new_empty(0)
    gs = torch.empty_like(ss) if need_s else g.new_empty(0)
    check(_lib.load().mnx_channel_scale_bwd_f32(ptr(g), ptr(ts), ptr(ss), g.shape[0], components, F,
                                                ptr(gt) if need_t else None, ptr(gs) if need_s else None,
                                                _stream(g)), "channel_scale backward")
    return gt, gs


@channel_scale_backward.register_fake
def _(grad, t, s, components, need_t, need_s):
    return (grad.new_empty(grad.shape) if need_t else grad.new_empty(0),
            s.new_empty(s.shape) if need_s else s.new_empty(0))


def _cs_setup(ctx, inputs, output):
    t, s, components = inputs
    ctx.save_for_backward(t, s)
    ctx.components = components


def _cs_bwd(ctx, grad):
    t, s = ctx.saved_tensors
    need_t, need_s = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    if not (need_t or need_s):
        return None, None, None
    gt, gs = channel_scale_backward(grad.contiguous(), t, s, ctx.components, need_t, need_s)
    return (gt if need_t else None), (gs if need_s else None), None


channel_scale.register_autograd(_cs_bwd, setup_context=_cs_setup)


def _cs2_setup(ctx, inputs, output):
    grad, t, s, components, need_t, need_s = inputs
    ctx.save_for_backward(grad, t, s)
    ctx.components = components
    ctx.flags = (need_t, need_s)


def _cs2_bwd(ctx, ggt, ggs):
    """Second order: gt = g s and gs = sum_d g t are bilinear, so with cotangents (ggt, ggs)
    d/dg = ggt s + t ggs, d/dt = g ggs, d/ds = sum_d ggt g -- the same two kernels."""
    grad, t, s = ctx.saved_tensors
    D = ctx.components
    need_t, need_s = ctx.flags
    has_t = need_t and ggt is not None and ggt.numel() > 0
    has_s = need_s and ggs is not None and ggs.numel() > 0
    dg = dt = ds = None
    if ctx.needs_input_grad[0]:
        dg = torch.zeros_like(grad)
        if has_t:
            dg = dg + channel_scale(ggt.contiguous(), s, D)
        if has_s:
            dg = dg + channel_scale(t, ggs.contiguous(), D)
    if ctx.needs_input_grad[1] and has_s:
        dt = channel_scale(grad, ggs.contiguous(), D)
    if ctx.needs_input_grad[2] and has_t:
        ds = channel_scale_backward(ggt.contiguous(), grad, s, D, False, True)[1]
    return dg, dt, ds, None, None, None


channel_scale_backward.register_autograd(_cs2_bwd, setup_context=_cs2_setup)


CHANNEL_PRODUCT_COMPONENTS = (1, 4, 9, 16)


@torch.library.custom_op("molix::channel_outer", mutates_args=(), device_types="cuda")
def channel_outer(y: Tensor, s: Tensor) -> Tensor:
    """``out[e][d][c] = y[e][d] * s[e][c]`` as an (E, D*F) ir_mul tensor: the env-weighted harmonics
    of Allegro's pair embedding (src/molzoo/allegro.py:55-92); the backward forms both gradients in
    one pass (``mnx_channel_outer_bwd_f32``)."""
    _require_gpu("channel_outer", y, s)
    if y.dtype != torch.float32 or y.dim() != 2:
        raise ValueError("channel_outer: y must be float32 (E, D)")
    E, D = y.shape
    F = s.shape[1]
    ys = y.contiguous()
    ss = _cs_rows(s, F, "s")
    if ss.shape[0] != E:
        raise ValueError("channel_outer: y and s must have the same number of rows")
    out = ys.new_empty(E, D * F)
    check(_lib.load().mnx_channel_outer_f32(ptr(ys), ptr(ss), E, D, F, ptr(out), _stream(ys)), "channel_outer")
    return out


@channel_outer.register_fake
def _(y, s):
    return y.new_empty(y.shape[0], y.shape[1] * s.shape[1])


@torch.library.custom_op("molix::channel_outer_backward", mutates_args=(), device_types="cuda")
def channel_outer_backward(grad: Tensor, y: Tensor, s: Tensor, need_y: bool, need_s: bool) -> tuple[Tensor, Tensor]:
    """(sum_c grad * s, sum_d grad * y) of ``channel_outer`` in one pass; an empty tensor for a
    gradient not requested."""
    _require_gpu("channel_outer_backward", grad, y, s)
    E, D = y.shape
    F = s.shape[1]
    g = _cs_rows(grad, D * F, "grad")
    ys = y.contiguous()
    ss = _cs_rows(s, F, "s")
    gy = torch.empty_like(ys) if need_y else g.new_empty(0)
    gs = torch.empty_like(ss) if need_s else g.new_empty(0)
    check(_lib.load().mnx_channel_outer_bwd_f32(ptr(g), ptr(ys), ptr(ss), E, D, F, ptr(gy) if need_y else None,
                                                ptr(gs) if need_s else None, _stream(g)), "channel_outer backward")
    return gy, gs


@channel_outer_backward.register_fake
def _(grad, y, s, need_y, need_s):
    return (y.new_empty(y.shape) if need_y else y.new_empty(0), s.new_empty(s.shape) if need_s else s.new_empty(0))


def _co_setup(ctx, inputs, output):
    y, s = inputs
    ctx.save_for_backward(y, s)


def _co_bwd(ctx, grad):
    y, s = ctx.saved_tensors
    need_y, need_s = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    if not (need_y or need_s):
        return None, None
    gy, gs = channel_outer_backward(grad.contiguous(), y, s, need_y, need_s)
    return (gy if need_y else None), (gs if need_s else None)


channel_outer.register_autograd(_co_bwd, setup_context=_co_setup)


def _co2_setup(ctx, inputs, output):
    grad, y, s, need_y, need_s = inputs
    ctx.save_for_backward(grad, y, s)
    ctx.flags = (need_y, need_s)


def _co2_bwd(ctx, ggy, ggs):
    """Second order: gy = sum_c g s and gs = sum_d g y are bilinear, so with cotangents (ggy, ggs)
    d/dg = ggy (x) s + y (x) ggs, d/dy = sum_c g ggs, d/ds = sum_d g ggy -- the same two kernels."""
    grad, y, s = ctx.saved_tensors
    need_y, need_s = ctx.flags
    has_y = need_y and ggy is not None and ggy.numel() > 0
    has_s = need_s and ggs is not None and ggs.numel() > 0
    dg = dy = ds = None
    if ctx.needs_input_grad[0]:
        dg = torch.zeros_like(grad)
        if has_y:
            dg = dg + channel_outer(ggy.contiguous(), s)
        if has_s:
            dg = dg + channel_outer(y, ggs.contiguous())
    if ctx.needs_input_grad[1] and has_s:
        dy = channel_outer_backward(grad, y, ggs.contiguous(), True, False)[0]
    if ctx.needs_input_grad[2] and has_y:
        ds = channel_outer_backward(grad, ggy.contiguous(), s, False, True)[1]
    return dg, dy, ds, None, None


channel_outer_backward.register_autograd(_co2_bwd, setup_context=_co2_setup)


def _stack_args(y: Tensor, s, what: str):
    L = len(s)
    if not 1 <= L <= 8 or y.dtype != torch.float32 or y.numel() != (s[0].shape[0] if L else 0):
        raise ValueError(f"{what}: y must be float32 with one entry per row and 1 to 8 inputs")
    E, F = s[0].shape if s[0].dim() == 2 else (-1, -1)
    if F < 4 or F % 4 or (F // 4) & (F // 4 - 1) or F > 256:
        raise ValueError(f"{what}: inputs must be (E, F) with F / 4 a power of two <= 64")
    ss = [_cs_rows(t, F, "s") for t in s]
    if any(t.shape[0] != E for t in ss):
        raise ValueError(f"{what}: inputs must all have the same number of rows")
    return y.reshape(-1).contiguous(), ss, E, F


def _ptr_array(ts) -> C.c_void_p:
    return C.cast((C.c_void_p * len(ts))(*[t.data_ptr() for t in ts]), C.c_void_p)


@torch.library.custom_op("molix::channel_outer_stack", mutates_args=(), device_types="cuda")
def channel_outer_stack(y: Tensor, s: list[Tensor]) -> Tensor:
    """``stack([y * s_l for s_l in s], 1)`` for a per-edge factor ``y`` (E rows of one entry) and
    L (E, F) inputs, (E, L, F) in one pass: the cutoff envelope on Allegro's per-layer scalar
    features and their stack (src/molzoo/allegro.py:628-641).  No autograd of its own; the
    backward is ``channel_outer_stack_backward``."""
    _require_gpu("channel_outer_stack", y, *s)
    ys, ss, E, F = _stack_args(y, s, "channel_outer_stack")
    out = ys.new_empty(E, len(ss), F)
    check(_lib.load().mnx_channel_outer_stack_f32(ptr(ys), _ptr_array(ss), len(ss), E, F, ptr(out), _stream(ys)),
          "channel_outer_stack")
    return out


@channel_outer_stack.register_fake
def _(y, s):
    return y.new_empty(s[0].shape[0], len(s), s[0].shape[1])


@torch.library.custom_op("molix::channel_outer_stack_backward", mutates_args=(), device_types="cuda")
def channel_outer_stack_backward(grad: Tensor, y: Tensor, s: list[Tensor], need_y: bool,
                                 need_s: bool) -> list[Tensor]:
    """``[grad y, grad s_0, ..., grad s_{L-1}]`` of ``channel_outer_stack`` in one pass: grad y
    (shaped like ``y``) ``= sum_l sum_c grad[:, l, c] s_l[:, c]``, grad s_l ``= grad[:, l] y``;
    empty tensors for gradients not requested."""
    _require_gpu("channel_outer_stack_backward", grad, y, *s)
    ys, ss, E, F = _stack_args(y, s, "channel_outer_stack_backward")
    L = len(ss)
    if grad.dtype != torch.float32 or tuple(grad.shape) != (E, L, F):
        raise ValueError(f"channel_outer_stack_backward: grad must be float32 ({E}, {L}, {F})")
    g = _aligned16(grad)
    gy = torch.empty_like(ys) if need_y else g.new_empty(0)
    gs = [torch.empty_like(t) for t in ss] if need_s else [g.new_empty(0) for _ in ss]
    check(_lib.load().mnx_channel_outer_stack_bwd_f32(ptr(g), ptr(ys), _ptr_array(ss), L, E, F,
                                                      ptr(gy) if need_y else None,
                                                      _ptr_array(gs) if need_s else None, _stream(g)),
          "channel_outer_stack backward")
    return [gy.reshape(y.shape) if need_y else gy] + gs


@channel_outer_stack_backward.register_fake
def _(grad, y, s, need_y, need_s):
    return ([y.new_empty(y.shape) if need_y else y.new_empty(0)]
            + [t.new_empty(t.shape) if need_s else t.new_empty(0) for t in s])


# ---------------------------------------------------------------------------
# Radial edge embedding (Bessel basis x cutoff envelope)
# ---------------------------------------------------------------------------

CUTOFF_KINDS = {"none": 0, "cosine": 1, "polynomial": 2}


def _basis_args(r, mu, sigma, num_radial):
    rr = r.detach().to(torch.float32).reshape(-1).contiguous()
    m = None if mu is None else mu.detach().to(torch.float32).reshape(-1).contiguous()
    s = None if sigma is None else sigma.detach().to(torch.float32).reshape(-1).contiguous()
    if (m is None) != (s is None) or (m is not None and (m.numel() != num_radial or s.numel() != num_radial)):
        raise ValueError("bessel_cutoff: mu and sigma must both be None or both have num_radial entries")
    return rr, m, s


@torch.library.custom_op("molix::bessel_cutoff", mutates_args=(), device_types="cuda")
def bessel_cutoff(r: Tensor, num_radial: int, r_cut: float, eps: float, mu: Tensor | None, sigma: Tensor | None,
                  cutoff: int, exponent: int) -> Tensor:
    """``BesselRBF(r) * cutoff(r)[..., None]`` in one kernel (``radial.py:36-148``, ``cutoff.py:23-161``,
    ``mace.py:180-182``): ``(r.shape..., num_radial)``.  ``cutoff``: 0 none, 1 cosine, 2 polynomial
    (``exponent``); ``mu`` / ``sigma`` the basis normalisation or both None."""
    _require_gpu("bessel_cutoff", r, mu, sigma)
    rr, m, sg = _basis_args(r, mu, sigma, num_radial)
    out = rr.new_empty(rr.shape[0], num_radial)
    check(_lib.load().mnx_bessel_cutoff_f32(ptr(rr), rr.shape[0], num_radial, float(r_cut), float(eps), ptr(m),
                                            ptr(sg), cutoff, exponent, ptr(out), _stream(rr)), "bessel_cutoff")
    return out.reshape(*r.shape, num_radial)


@bessel_cutoff.register_fake
def _(r, num_radial, r_cut, eps, mu, sigma, cutoff, exponent):
    return r.new_empty(*r.shape, num_radial, dtype=torch.float32)


@torch.library.custom_op("molix::bessel_cutoff_backward", mutates_args=(), device_types="cuda")
def bessel_cutoff_backward(grad: Tensor, r: Tensor, num_radial: int, r_cut: float, eps: float, mu: Tensor | None,
                           sigma: Tensor | None, cutoff: int, exponent: int) -> Tensor:
    rr, m, sg = _basis_args(r, mu, sigma, num_radial)
    g = grad.to(torch.float32).reshape(-1, num_radial).contiguous()
    gr = rr.new_empty(rr.shape[0])
    check(_lib.load().mnx_bessel_cutoff_bwd_f32(ptr(rr), rr.shape[0], num_radial, float(r_cut), float(eps), ptr(m),
                                                ptr(sg), cutoff, exponent, ptr(g), ptr(gr), _stream(rr)),
          "bessel_cutoff backward")
    return gr.reshape(r.shape)


@bessel_cutoff_backward.register_fake
def _(grad, r, num_radial, r_cut, eps, mu, sigma, cutoff, exponent):
    return r.new_empty(r.shape, dtype=torch.float32)


def _bc_setup(ctx, inputs, output):
    r, num_radial, r_cut, eps, mu, sigma, cutoff, exponent = inputs
    ctx.save_for_backward(r, mu, sigma)
    ctx.args = (num_radial, r_cut, eps, cutoff, exponent)


def _bc_bwd(ctx, grad):
    r, mu, sigma = ctx.saved_tensors
    n, r_cut, eps, cutoff, exponent = ctx.args
    gr = None
    if ctx.needs_input_grad[0]:
        gr = bessel_cutoff_backward(grad.contiguous(), r, n, r_cut, eps, mu, sigma, cutoff, exponent).to(r.dtype)
    return gr, None, None, None, None, None, None, None


bessel_cutoff.register_autograd(_bc_bwd, setup_context=_bc_setup)




# ---------------------------------------------------------------------------
# Segment sums (molix.F.scatter_sum / batch_add, MessageAggregation)
# ---------------------------------------------------------------------------


def _segment_csr(index: Tensor, num_segments: int, validate: bool) -> tuple[Tensor, Tensor]:
    """Rows grouped by segment id, ascending row id within a segment: (row_ptr, perm)."""
    idx = index.to(torch.int64).reshape(-1)
    row_ptr, perm, _ = edge_csr(torch.stack([idx, idx], dim=1), num_segments, validate)
    return row_ptr, perm


@torch.library.custom_op("molix::segment_sum", mutates_args=(), device_types="cuda")
def segment_sum(values: Tensor, index: Tensor, num_segments: int, weights: Tensor | None = None,
                validate: bool = True) -> Tensor:
    """``out[n] = sum_{r: index[r] = n} weights[r] * values[r]`` for ``values`` (R, D), ``index`` (R,)
    and ``weights`` (R,) or None: a CSR walk with no atomics and a fixed summation order.  With
    ``validate`` (one host synchronisation) an index outside ``[0, num_segments)`` raises, as torch's
    ``scatter_add_`` does; without it such rows are left out."""
    _require_gpu("segment_sum", values, index, weights)
    if values.dim() != 2:
        raise ValueError(f"segment_sum: values must be (rows, D), got {tuple(values.shape)}")
    v = _f32_rows(values, values.shape[1], "values")
    if index.dim() != 1 or index.shape[0] != v.shape[0]:
        raise ValueError(f"segment_sum: index must be ({v.shape[0]},), got {tuple(index.shape)}")
    w = None if weights is None else _f32_rows(weights, 1, "weights").reshape(-1)
    if w is not None and w.shape[0] != v.shape[0]:
        raise ValueError("segment_sum: weights must have one entry per row")
    out = v.new_empty(num_segments, v.shape[1])
    row_ptr, perm = _segment_csr(index, num_segments, validate)
    check(_lib.load().mnx_segment_sum_f32(ptr(v), v.shape[0], v.shape[1], ptr(row_ptr), ptr(perm), ptr(w),
                                          num_segments, ptr(out), _stream(v)), "segment_sum")
    return out


@segment_sum.register_fake
def _(values, index, num_segments, weights=None, validate=True):
    return values.new_empty(num_segments, values.shape[1])


@torch.library.custom_op("molix::segment_sum_backward", mutates_args=(), device_types="cuda")
def segment_sum_backward(grad: Tensor, index: Tensor, values: Tensor, weights: Tensor | None, need_values: bool,
                         need_weights: bool) -> tuple[Tensor, Tensor]:
    g = _f32_rows(grad, grad.shape[-1], "grad")
    v = _f32_rows(values, g.shape[1], "values")
    idx = index.to(torch.int64).contiguous()
    w = None if weights is None else _f32_rows(weights, 1, "weights").reshape(-1)
    gv = torch.empty_like(v) if need_values else v.new_empty(0)
    gw = v.new_empty(v.shape[0]) if (need_weights and w is not None) else v.new_empty(0)
    check(_lib.load().mnx_segment_sum_bwd_f32(ptr(g), ptr(idx), ptr(w), ptr(v), v.shape[0], g.shape[1], g.shape[0],
                                              ptr(gv), ptr(gw), _stream(g)), "segment_sum backward")
    return gv, gw


@segment_sum_backward.register_fake
def _(grad, index, values, weights, need_values, need_weights):
    return (torch.empty_like(values) if need_values else values.new_empty(0),
            values.new_empty(values.shape[0]) if (need_weights and weights is not None) else values.new_empty(0))


def _seg_setup(ctx, inputs, output):
    values, index, num_segments, weights, validate = inputs
    ctx.save_for_backward(values, index, weights)


def _seg_backward(ctx, grad):
    values, index, weights = ctx.saved_tensors
    nig = ctx.needs_input_grad  # one flag per argument given (defaults left out)
    nv, nw = nig[0], len(nig) > 3 and nig[3] and weights is not None
    gv, gw = segment_sum_backward(grad.contiguous(), index, values, weights, nv, nw)
    grads = [gv.reshape(values.shape) if nv else None, None, None, gw.reshape(weights.shape) if nw else None, None]
    return tuple(grads[:len(nig)])


segment_sum.register_autograd(_seg_backward, setup_context=_seg_setup)


# second-order formulas (autograd of the backward ops): registered on import, after every op above
from . import second_order  # noqa: E402,F401
