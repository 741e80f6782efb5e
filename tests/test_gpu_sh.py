"""GPU spherical harmonics vs the fp64 oracle (scipy-based), forward and backward."""

import numpy as np
import pytest
import torch

from oracle import equivariant as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    import molnex_amd.kernels  # noqa: F401

    return torch.ops.molix


@pytest.mark.parametrize("l_max", [0, 1, 2, 3])
def test_sh_forward_backward(ops, l_max):
    rng = np.random.default_rng(l_max)
    v = rng.normal(size=(4099, 3)) * rng.uniform(0.5, 5.0, (4099, 1))
    v[0] = 0.0  # zero vector: Y^0 = 1, rest 0, zero gradient
    vt = torch.tensor(v, dtype=torch.float32, device="cuda", requires_grad=True)
    Y = ops.spherical_harmonics(vt, l_max)
    ref = O.sh(range(l_max + 1), v.astype(np.float32).astype(np.float64))
    np.testing.assert_allclose(Y.detach().cpu().numpy(), ref, atol=2e-6, rtol=0)
    g = rng.normal(size=Y.shape)
    (gv,) = torch.autograd.grad(Y, vt, torch.tensor(g, dtype=torch.float32, device="cuda"))
    vv = v.astype(np.float32).astype(np.float64)
    if l_max == 0:
        assert np.all(gv.cpu().numpy() == 0)
        return
    ref_g = O.sh_grad_fd(range(l_max + 1), vv[1:], g[1:])
    out = gv.cpu().numpy()
    assert np.all(out[0] == 0)
    err = np.linalg.norm(out[1:] - ref_g) / np.linalg.norm(ref_g)
    assert err < 1e-5, err


def test_sh_batched_shape(ops):
    v = torch.randn(4, 5, 3, device="cuda")
    assert ops.spherical_harmonics(v, 3).shape == (4, 5, 16)
