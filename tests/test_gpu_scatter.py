"""Segment sums on the HIP path (molix::segment_sum): molix.F.scatter_sum / batch_add
(src/molix/F/scatter.py:13-51) and MessageAggregation (src/molrep/interaction/aggregation.py:93-117)
against the fp64 oracle (oracle.equivariant.scatter_add, a sparse incidence product) and torch fp64
autograd for the gradients."""

import numpy as np
import pytest
import torch

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


@pytest.mark.parametrize("rows,dim,num", [(1000, 128, 37), (777, 3, 50), (4096, 130, 9), (1, 8, 1), (300, 2048, 64)])
def test_segment_sum_matches_oracle(rows, dim, num):
    g = torch.Generator().manual_seed(rows + dim)
    v = torch.randn(rows, dim, generator=g)
    idx = torch.randint(0, num, (rows,), generator=g)
    w = torch.rand(rows, generator=g)
    out = torch.ops.molix.segment_sum(v.to(DEV), idx.to(DEV), num, w.to(DEV))
    _close(out, O.scatter_add(idx.numpy(), (v.double() * w.double()[:, None]).numpy(), num))
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
