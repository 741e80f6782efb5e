"""Segment sums on the HIP path (molix::segment_sum): molix.F.scatter_sum / batch_add
(src/molix/F/scatter.py:13-51) and MessageAggregation (src/molrep/interaction/aggregation.py:93-117)
against the fp64 oracle (oracle.equivariant.scatter_add, a sparse incidence product) and torch fp64
autograd for the gradients."""

import numpy as np
import pytest
import torch

import molnex_amd.kernels  # noqa: F401  (registers torch.ops.molix.*)
from oracle import equivariant as O
from oracle import mace_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(got, ref, tol=1e-6):
    got = got.detach().double().cpu()
    ref = torch.as_tensor(ref, dtype=torch.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    den = ref.norm().clamp_min(1e-30)
    assert (got - ref).norm() / den <= tol, float((got - ref).norm() / den)


@pytest.mark.parametrize("rows,dim,num", [(1000, 128, 37), (777, 3, 50), (4096, 130, 9), (1, 8, 1), (300, 2048, 64),
                                          # few long segments (a workgroup per segment and column block)
                                          (50000, 1, 1), (50000, 2, 1), (20000, 300, 3), (5000, 2048, 2),
                                          (70000, 5, 16)])
def test_segment_sum_matches_oracle(rows, dim, num):
    g = torch.Generator().manual_seed(rows + dim)
    v = torch.randn(rows, dim, generator=g)
    idx = torch.randint(0, num, (rows,), generator=g)
    w = torch.rand(rows, generator=g)
    out = torch.ops.molix.segment_sum(v.to(DEV), idx.to(DEV), num, w.to(DEV))
    # fp32 sums of thousands of rows per segment carry ~1e-6 of rounding: the 1e-5 contract there
    tol = 1e-6 if rows <= 1000 * num else 1e-5
    _close(out, O.scatter_add(idx.numpy(), (v.double() * w.double()[:, None]).numpy(), num), tol)
    out2 = torch.ops.molix.segment_sum(v.to(DEV), idx.to(DEV), num, w.to(DEV))
    assert torch.equal(out, out2)  # fixed summation order


def test_segment_sum_gradients():
    g = torch.Generator().manual_seed(3)
    rows, dim, num = 500, 40, 23
    v = torch.randn(rows, dim, generator=g, dtype=torch.float64)
    idx = torch.randint(0, num, (rows,), generator=g)
    w = torch.rand(rows, generator=g, dtype=torch.float64)
    go = torch.randn(num, dim, generator=g, dtype=torch.float64)
    vg = v.float().to(DEV).requires_grad_(True)
    wg = w.float().to(DEV).requires_grad_(True)
    gv, gw = torch.autograd.grad(torch.ops.molix.segment_sum(vg, idx.to(DEV), num, wg), (vg, wg), go.float().to(DEV))
    v64, w64 = v.clone().requires_grad_(True), w.clone().requires_grad_(True)
    ref = torch.zeros(num, dim, dtype=torch.float64).index_add(0, idx, v64 * w64[:, None])
    rv, rw = torch.autograd.grad(ref, (v64, w64), go)
    _close(gv, rv)
    _close(gw, rw)


def test_scatter_sum_dims_and_index_forms():
    from molnex_amd.molix.F import batch_add, scatter_sum

    g = torch.Generator().manual_seed(4)
    src = torch.randn(6, 50, 5, generator=g)
    idx = torch.randint(0, 11, (50,), generator=g)
    ref = torch.zeros(6, 11, 5, dtype=torch.float64).index_add(1, idx, src.double())
    _close(scatter_sum(src.to(DEV), idx.to(DEV), dim=1, dim_size=11), ref)
    _close(scatter_sum(src.to(DEV), idx.to(DEV), dim=-2, dim_size=11), ref)
    # an index of src's rank broadcast from the 1-D one, as the reference builds it
    full = idx.view(1, 50, 1).expand_as(src)
    _close(scatter_sum(src.to(DEV), full.to(DEV), dim=1, dim_size=11), ref)
    _close(scatter_sum(src.to(DEV), idx.view(1, 50, 1).to(DEV), dim=1, dim_size=11), ref)
    # dim_size from the largest index
    assert scatter_sum(src.to(DEV), idx.to(DEV), dim=1).shape[1] == int(idx.max()) + 1
    # a full-rank index that varies along other axes: an element-wise scatter
    var = torch.randint(0, 4, src.shape, generator=g)
    ref_var = torch.zeros(6, 4, 5, dtype=torch.float64).scatter_add(1, var, src.double())
    _close(scatter_sum(src.to(DEV), var.to(DEV), dim=1, dim_size=4), ref_var)
    # batch_add on a per-atom vector
    batch = torch.tensor([0, 0, 1, 1, 1, 3])
    e = torch.randn(6, generator=g)
    _close(batch_add(e.to(DEV), batch.to(DEV)), torch.zeros(4, dtype=torch.float64).index_add(0, batch, e.double()))
    # empty input
    assert scatter_sum(torch.zeros(0, 4, device=DEV), torch.zeros(0, dtype=torch.long, device=DEV), 0, 3).abs().sum() == 0


def test_segment_sum_rejects_out_of_range_index():
    v = torch.randn(10, 4, device=DEV)
    with pytest.raises(ValueError, match="outside"):
        torch.ops.molix.segment_sum(v, torch.tensor([0, 1, 2, 3, 4, 5, 6, 7, 8, 9], device=DEV), 5)


@pytest.mark.parametrize("apply_cutoff", [True, False])
def test_message_aggregation_vs_oracle(apply_cutoff):
    from molnex_amd.molrep.interaction import MessageAggregation

    torch.manual_seed(5)
    irreps = "16x0e+8x1o+4x2e"
    blocks = [(16, 0, 1), (8, 1, -1), (4, 2, 1)]
    agg = MessageAggregation(irreps=irreps, apply_cutoff=apply_cutoff).to(DEV)
    n, E = 40, 600
    g = torch.Generator().manual_seed(6)
    ei = torch.randint(0, n, (E, 2), generator=g)
    msg = torch.randn(E, 16 + 24 + 20, generator=g)
    cut = torch.rand(E, generator=g)
    out = agg(msg.to(DEV), ei.to(DEV), cut.to(DEV))
    assert out.shape == (int(ei.max()) + 1, msg.shape[1])
    m64 = msg.double() * (cut.double()[:, None] if apply_cutoff else 1.0)
    summed = torch.tensor(O.scatter_add(ei[:, 1].numpy(), m64.numpy(), out.shape[0]))
    ref = mace_ref.linear(summed, agg.linear.linear.weight.detach().double().cpu(), blocks, blocks)
    _close(out, ref, 1e-5)
    # gradients of messages and cutoff weights against fp64 autograd of the same composition
    mg = msg.to(DEV).requires_grad_(True)
    cg = cut.to(DEV).requires_grad_(True)
    go = torch.randn(out.shape, generator=g)
    gm, gc = torch.autograd.grad(agg(mg, ei.to(DEV), cg, n_nodes=out.shape[0]), (mg, cg), go.to(DEV),
                                 allow_unused=True)
    m64r = msg.double().requires_grad_(True)
    c64r = cut.double().requires_grad_(True)
    s64 = torch.zeros(out.shape[0], msg.shape[1], dtype=torch.float64).index_add(
        0, ei[:, 1], m64r * (c64r[:, None] if apply_cutoff else 1.0))
    r64 = mace_ref.linear(s64, agg.linear.linear.weight.detach().double().cpu(), blocks, blocks)
    rm, rc = torch.autograd.grad(r64, (m64r, c64r), go.double(), allow_unused=True)
    _close(gm, rm, 1e-5)
    if apply_cutoff:
        _close(gc, rc, 1e-5)
    else:
        assert gc is None


def test_scatter_sum_other_dtypes():
    """float64, half and integer src go to torch's scatter_add on the GPU (the fp32 kernel does
    not compute them), with the reference's results."""
    from molnex_amd.molix.F import batch_add, scatter_sum

    g = torch.Generator().manual_seed(7)
    idx = torch.randint(0, 9, (70,), generator=g)
    src64 = torch.randn(70, 3, generator=g, dtype=torch.float64)
    ref64 = torch.zeros(9, 3, dtype=torch.float64).index_add(0, idx, src64)
    out64 = scatter_sum(src64.to(DEV), idx.to(DEV), 0, 9)
    assert out64.dtype == torch.float64
    assert torch.allclose(out64.cpu(), ref64, rtol=1e-14, atol=1e-14)
    # along dim 1 with a 1-D index
    src64t = src64.t().contiguous()
    assert torch.allclose(scatter_sum(src64t.to(DEV), idx.to(DEV), 1, 9).cpu(), ref64.t(), rtol=1e-14, atol=1e-14)
    counts = torch.randint(0, 5, (70,), generator=g)
    outi = batch_add(counts.to(DEV), idx.to(DEV), 9)
    assert outi.dtype == torch.int64
    assert torch.equal(outi.cpu(), torch.zeros(9, dtype=torch.int64).index_add(0, idx, counts))
    assert torch.equal(batch_add(counts.to(DEV), idx.to(DEV)).cpu()[: int(idx.max()) + 1],
                       torch.zeros(9, dtype=torch.int64).index_add(0, idx, counts)[: int(idx.max()) + 1])
    h = torch.randn(70, 4, generator=g).half()
    outh = scatter_sum(h.to(DEV), idx.to(DEV), 0, 9)
    assert outh.dtype == torch.float16
    assert torch.allclose(outh.float().cpu(), torch.zeros(9, 4).index_add(0, idx, h.float()), atol=2e-2)


def test_message_aggregation_float64():
    from molnex_amd.molrep.interaction import MessageAggregation

    torch.manual_seed(8)
    irreps = "8x0e+8x1o"
    blocks = [(8, 0, 1), (8, 1, -1)]
    agg = MessageAggregation(irreps=irreps).to(DEV).double()
    g = torch.Generator().manual_seed(9)
    ei = torch.randint(0, 30, (400, 2), generator=g)
    msg = torch.randn(400, 32, generator=g, dtype=torch.float64)
    cut = torch.rand(400, generator=g, dtype=torch.float64)
    out = agg(msg.to(DEV), ei.to(DEV), cut.to(DEV), n_nodes=30)
    assert out.dtype == torch.float64
    summed = torch.zeros(30, 32, dtype=torch.float64).index_add(0, ei[:, 1], msg * cut[:, None])
    ref = mace_ref.linear(summed, agg.linear.linear.weight.detach().cpu(), blocks, blocks)
    assert torch.allclose(out.cpu(), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_energy_aggregation_vs_fp64(pooling):
    """Per-graph sum / mean of per-atom energies on the segment-sum kernel against an fp64
    index_add (and a float64 model's energies through torch), empty graphs included."""
    from molnex_amd.molpot import EnergyAggregation

    g = torch.Generator().manual_seed(10)
    batch = torch.sort(torch.randint(0, 12, (3000,), generator=g)).values
    batch[batch == 5] = 6  # graph 5 has no atoms
    e = torch.randn(3000, generator=g)
    tot = torch.zeros(13, dtype=torch.float64).index_add(0, batch, e.double())
    cnt = torch.zeros(13, dtype=torch.float64).index_add(0, batch, torch.ones(3000, dtype=torch.float64))
    ref = tot if pooling == "sum" else tot / cnt.clamp(min=1)
    agg = EnergyAggregation(pooling)
    out = agg(e.to(DEV), batch.to(DEV), 13)
    assert out.shape == (13,) and out.dtype == torch.float32
    _close(out, ref, 1e-6)
    assert float(out[5]) == 0.0
    assert torch.equal(out, agg(e.to(DEV), batch.to(DEV), 13))  # fixed summation order
    # num_graphs from the largest id (trailing graphs without atoms are not counted)
    assert agg(e.to(DEV), batch.to(DEV)).shape == (int(batch.max()) + 1,)
    out64 = agg(e.double().to(DEV), batch.to(DEV), 13)
    assert out64.dtype == torch.float64 and torch.allclose(out64.cpu(), ref, rtol=1e-12, atol=1e-12)
    # gradient: every atom of graph b receives dL/dE[b] (divided by the graph's count for mean)
    eg = e.to(DEV).requires_grad_(True)
    go = torch.randn(13, generator=g)
    (ge,) = torch.autograd.grad(agg(eg, batch.to(DEV), 13), eg, go.to(DEV))
    rg = go[batch] / (1.0 if pooling == "sum" else cnt.float()[batch])
    assert torch.allclose(ge.cpu(), rg, rtol=1e-6, atol=1e-7)


def test_aggregations_with_sizes_have_no_host_sync():
    """With the sizes given, EnergyAggregation and MessageAggregation enqueue their work without a
    device-to-host copy or synchronisation (torch's sync debug mode raises on one)."""
    from molnex_amd.molpot import EnergyAggregation
    from molnex_amd.molrep.interaction import MessageAggregation

    g = torch.Generator().manual_seed(11)
    batch = torch.sort(torch.randint(0, 4, (500,), generator=g)).values.to(DEV)
    e = torch.randn(500, generator=g).to(DEV).requires_grad_(True)
    agg = MessageAggregation(irreps="8x0e").to(DEV)
    ei = torch.randint(0, 50, (300, 2), generator=g).to(DEV)
    msg = torch.randn(300, 8, generator=g).to(DEV).requires_grad_(True)
    cut = torch.rand(300, generator=g).to(DEV)
    ea = EnergyAggregation("mean")
    for sync_mode in (0, "error"):  # warm-up pass first (library load, lazy buffers)
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode(sync_mode)
        try:
            E = ea(e, batch, 4)
            m = agg(msg, ei, cut, n_nodes=50)
            ge, gm = torch.autograd.grad((E.sum(), m.sum()), (e, msg))
        finally:
            torch.cuda.set_sync_debug_mode(0)
    assert torch.isfinite(ge).all() and torch.isfinite(gm).all()
