"""The oracle of the table-driven product (any irreps, l <= 3) is pinned before it is trusted, and
the host side of ``molix::tp_any`` (path tables, their validation, the module's choice of kernel) is
checked against it (CPU only).

* coupling tensors of every triple, odd l1 + l2 + l3 included: two independent constructions agree
  (oracle null space of fitted Wigner matrices vs the product's Haar average / Gaunt integral),
  each is invariant, isotropic, and (1, 1 -> 1) is the Levi-Civita tensor / sqrt(6);
* ``ChannelwiseTPMul``: equal to ``ChannelwiseTP`` on uniform natural irreps, equal block by block
  to one-block products (the multiplicity bookkeeping), O(3)-equivariant including inversion for
  mixed parities, gradients against finite differences; planted mistakes fail.

The sign of an odd triple's tensor is a convention (first entry above 1e-9 x max positive); it is
not pinned against cuequivariance, which is absent here.
"""

import itertools
import math

import numpy as np
import pytest

from oracle import equivariant as O


def _triples():
    return [(a, b, c) for a, b, c in itertools.product(range(4), repeat=3) if abs(a - b) <= c <= a + b]


def test_coupling_all_triples_two_constructions_agree():
    from molnex_amd import irreps as P

    rng = np.random.default_rng(21)
    R = O.random_rotation(rng)
    odd = 0
    for l1, l2, l3 in _triples():
        c = O.coupling(l1, l2, l3)
        np.testing.assert_allclose(c, P.coupling(l1, l2, l3), atol=1e-12, err_msg=str((l1, l2, l3)))
        rot = np.einsum("ad,be,cf,def->abc", O.wigner_d(l1, R), O.wigner_d(l2, R), O.wigner_d(l3, R), c)
        np.testing.assert_allclose(rot, c, atol=1e-10)
        np.testing.assert_allclose((c ** 2).sum((0, 1)), 1 / (2 * l3 + 1), atol=1e-12)
        odd += (l1 + l2 + l3) % 2
    assert odd == 11
    # textbook case: the l = 1 blocks are sqrt(3) (x, y, z), so (1, 1 -> 1) is epsilon_abc / sqrt(6)
    eps = np.zeros((3, 3, 3))
    for (a, b, c), s in (((0, 1, 2), 1), ((1, 2, 0), 1), ((2, 0, 1), 1), ((0, 2, 1), -1), ((2, 1, 0), -1),
                         ((1, 0, 2), -1)):
        eps[a, b, c] = s
    np.testing.assert_allclose(O.coupling(1, 1, 1), eps / math.sqrt(6), atol=1e-12)


def _parity(feat, irreps):
    out = np.array(feat, dtype=np.float64, copy=True)
    off = 0
    for mul, l, p in O._irrep_list(irreps):
        d = (2 * l + 1) * mul
        out[..., off:off + d] *= p
        off += d
    return out


def _out_irreps(tp):
    order = sorted(tp.out_pos, key=tp.out_pos.get)
    return " + ".join(f"{tp.muls[k]}x{tp.paths[k][4]}{'e' if tp.paths[k][5] == 1 else 'o'}" for k in order)


def _case(rng, in1, in2, filt, N=6, E=25):
    tp = O.ChannelwiseTPMul(in1, in2, filt)
    x = rng.normal(size=(N, tp.nx))
    Y = rng.normal(size=(E, tp.ny))
    w = rng.normal(size=(E, tp.nw))
    ei = rng.integers(0, N, (E, 2))
    return tp, x, Y, w, ei, N


MIXED = ("3x0e + 2x1o + 2x1e + 1x2o + 2x3o", "0e + 1o + 1e + 2e", "0e + 0o + 1o + 1e + 2e + 2o + 3o + 3e")


def test_tp_mul_equals_uniform_product():
    rng = np.random.default_rng(22)
    C, N, E = 3, 7, 30
    irr = "0e+1o+2e+3o"
    xirr = "+".join(f"{C}x{t}" for t in irr.split("+"))
    ref = O.ChannelwiseTP(xirr, irr, irr, C)
    tp = O.ChannelwiseTPMul(xirr, irr, irr)
    assert tp.nx == ref.nx * C and tp.no == ref.no * C and tp.nw == len(ref.paths) * C
    x, Y = rng.normal(size=(N, tp.nx)), rng.normal(size=(E, tp.ny))
    w, ei = rng.normal(size=(E, tp.nw)), rng.integers(0, N, (E, 2))
    g = rng.normal(size=(N, tp.no))
    np.testing.assert_allclose(tp.forward(x, Y, w, ei, N), ref.forward(x, Y, w, ei, N), atol=1e-12)
    for a, b in zip(tp.backward(x, Y, w, ei, g), ref.backward(x, Y, w, ei, g)):
        np.testing.assert_allclose(a, b, atol=1e-12)


def test_tp_mul_blockwise_equals_one_block_products():
    """Each in1 block alone gives the paths of that block: their weight segments and output blocks
    must be the full product's, at the offsets of its bookkeeping."""
    rng = np.random.default_rng(23)
    in1, in2, filt = MIXED
    tp, x, Y, w, ei, N = _case(rng, in1, in2, filt)
    full = tp.forward(x, Y, w, ei, N)
    seen = 0
    blocks = O._irrep_list(in1)
    for b, (mul, l, p) in enumerate(blocks):
        sub = O.ChannelwiseTPMul(f"{mul}x{l}{'e' if p == 1 else 'o'}", in2, filt)
        ks = [k for k, pp in enumerate(tp.paths) if pp[0] == b]
        assert len(ks) == len(sub.paths)
        xs = x[:, tp.off1[b]:tp.off1[b + 1]]
        ws = np.concatenate([w[:, tp.offw[k]:tp.offw[k + 1]] for k in ks], axis=1)
        out = sub.forward(xs, Y, ws, ei, N)
        for j, k in enumerate(ks):
            pf, ps = tp.out_pos[k], sub.out_pos[j]
            np.testing.assert_allclose(out[:, sub.off3[ps]:sub.off3[ps + 1]], full[:, tp.off3[pf]:tp.off3[pf + 1]],
                                       atol=1e-12)
            seen += 1
    assert seen == len(tp.paths)


def _equivariant(f, x, Y, R, improper, in1, in2, out_irr):
    def act(feat, irreps):
        r = O.rotate_irreps(feat, R, irreps, None)
        return _parity(r, irreps) if improper else r
    return np.allclose(f(act(x, in1), act(Y, in2)), act(f(x, Y), out_irr), atol=1e-9)


def test_tp_mul_o3_equivariance_mixed_parity():
    rng = np.random.default_rng(24)
    in1, in2, filt = MIXED
    tp, x, Y, w, ei, N = _case(rng, in1, in2, filt)
    assert any((p[2] + p[3] + p[4]) % 2 for p in tp.paths)  # odd couplings present
    assert {p[5] for p in tp.paths} == {1, -1}
    f = lambda x_, Y_: tp.forward(x_, Y_, w, ei, N)  # noqa: E731
    R = O.random_rotation(rng)
    out_irr = _out_irreps(tp)
    for improper in (False, True):
        assert _equivariant(f, x, Y, R, improper, in1, in2, out_irr)
    # planted: a path whose output parity label is wrong passes rotations but fails inversion
    tp.paths = [pp[:5] + (-pp[5],) if k == 3 else pp for k, pp in enumerate(tp.paths)]
    assert _equivariant(f, x, Y, R, False, in1, in2, _out_irreps(tp))
    assert not _equivariant(f, x, Y, R, True, in1, in2, _out_irreps(tp))


def test_tp_mul_planted_zero_odd_coupling_is_caught():
    """The odd-sum Gaunt integral is zero; a product that used it for 1 x 1 -> 1 would output zero
    there, which the textbook check and the output of the odd path itself reject."""
    rng = np.random.default_rng(25)
    tp, x, Y, w, ei, N = _case(rng, "2x1o", "1o", "1e")
    assert len(tp.paths) == 1
    out = tp.forward(x, Y, w, ei, N)
    assert np.abs(out).max() > 1e-3
    # the cross product: with one edge, x = sqrt(3) a, Y = sqrt(3) b -> out = sqrt(3) w (3/sqrt(6)) a x b
    a, b = rng.normal(size=3), rng.normal(size=3)
    x1 = np.zeros((2, 6))
    x1[0] = (math.sqrt(3) * a[:, None] * np.ones((1, 2))).ravel()
    got = tp.forward(x1, math.sqrt(3) * b[None, :], np.ones((1, 2)), np.array([[0, 1]]), 2)[1].reshape(3, 2)[:, 0]
    np.testing.assert_allclose(got, math.sqrt(3) * 3 / math.sqrt(6) * np.cross(a, b), atol=1e-12)


def test_tp_mul_gradients_finite_differences():
    rng = np.random.default_rng(26)
    in1, in2, filt = MIXED
    tp, x, Y, w, ei, N = _case(rng, in1, in2, filt, N=5, E=12)
    g = rng.normal(size=(N, tp.no))
    grads = tp.backward(x, Y, w, ei, g)
    f = lambda args: (tp.forward(*args, ei, N) * g).sum()  # noqa: E731
    h = 1e-6
    for k, gr in enumerate(grads):
        base = [x, Y, w][k]
        for _ in range(10):
            idx = tuple(rng.integers(0, s) for s in base.shape)
            a, b = base.copy(), base.copy()
            a[idx] += h
            b[idx] -= h
            ap, am = [x, Y, w], [x, Y, w]
            ap[k], am[k] = a, b
            fd = (f(ap) - f(am)) / (2 * h)
            assert abs(fd - gr[idx]) < 1e-6 * max(1, abs(fd))


# ---------------------------------------------------------------------------
# host side of molix::tp_any (no GPU calls)
# ---------------------------------------------------------------------------

def test_tp_any_table_matches_oracle_bookkeeping():
    from molnex_amd import _lib
    from molnex_amd import kernels as K
    from molnex_amd.irreps import ChannelwiseTPDescriptor

    lib = _lib.load()
    in1, in2, filt = MIXED
    tp = O.ChannelwiseTPMul(in1, in2, filt)
    d = ChannelwiseTPDescriptor(in1, in2, filt)
    t = K.tp_any_table(d)
    P = len(tp.paths)
    assert t[:5] == [P, tp.nx, tp.ny, tp.no, tp.nw]
    for k, pp in enumerate(tp.paths):
        tri, xo, yo, oo, wo, mul = t[5 + 6 * k: 11 + 6 * k]
        assert tri == lib.mnx_tp_any_triple(*pp[2:5])
        assert (xo, yo, oo, wo, mul) == (tp.off1[pp[0]], tp.off2[pp[1]], tp.off3[tp.out_pos[k]], tp.offw[k],
                                         tp.muls[k])
    assert str(d.irreps_out).replace(" ", "") == _out_irreps(tp).replace(" ", "")
    assert lib.mnx_tp_any_triple(3, 3, 4) == -1 and lib.mnx_tp_any_triple(1, 1, 3) == -1


def test_tp_any_rejects_bad_tables():
    import ctypes as C

    from molnex_amd import _lib

    lib = _lib.load()
    one = [lib.mnx_tp_any_triple(0, 0, 0)]

    def call(table):
        arr = (C.c_int32 * len(table))(*table)
        rc = lib.mnx_tp_any_fwd_f32(arr, len(table), None, None, None, None, None, None, 1, 1, None, None)
        return rc, lib.mnx_last_error().decode()

    # two paths whose output blocks overlap (each 4 channels of 0e, row of 8)
    rc, msg = call([2, 8, 1, 8, 8] + one + [0, 0, 0, 0, 4] + one + [4, 0, 2, 4, 4])
    assert rc != 0 and "overlap" in msg
    # an x block outside the row
    rc, msg = call([1, 4, 1, 4, 4] + one + [2, 0, 0, 0, 4])
    assert rc != 0 and "x block" in msg
    # output blocks that do not cover the row
    rc, msg = call([1, 4, 1, 8, 4] + one + [0, 0, 0, 0, 4])
    assert rc != 0 and "tile" in msg
    # length that does not match the path count; an unknown triple
    assert call([1, 4, 1, 4, 4, 0])[0] != 0
    rc, msg = call([1, 4, 1, 4, 4, 99, 0, 0, 0, 0, 4])
    assert rc != 0 and "triple" in msg


@pytest.mark.parametrize("in1,in2,filt,compiled", [
    ("8x0e + 8x1o + 8x2e", "0e + 1o + 2e", "0e + 1o + 2e", True),
    ("8x0e + 4x1o", "0e + 1o", "0e + 1o", False),  # non-uniform multiplicity
    ("8x0e + 8x1e", "0e + 1o", "0e + 1o + 1e", False),  # non-natural parity
    ("8x0e + 8x0e + 8x1o", "0e + 1o", "0e + 1o", False),  # two blocks of one l
    ("8x0e + 8x1o", "0e + 1o", "0e + 1o + 1e", False),  # odd coupling 1o x 1o -> 1e in the output
])
def test_module_selects_kernel(in1, in2, filt, compiled):
    from molnex_amd.molrep.interaction.tensor_product import ChannelWiseTensorProduct

    m = ChannelWiseTensorProduct(in1, in2, filt)
    assert (m.config_id >= 0) == compiled
    assert (m.any_table is None) == compiled
    tp = O.ChannelwiseTPMul(in1, in2, filt)
    assert m.weight_numel == tp.nw and m.irreps_out.dim == tp.no
