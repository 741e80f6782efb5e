"""Class grouping (mnx_class_groups): a stable counting sort of nodes by element, against numpy's
stable argsort with out-of-range classes moved last; class boundaries against the class counts.
Sizes around the 1024-node segment, empty input, one class, many classes, invalid classes."""

import numpy as np
import pytest
import torch

import molnex_amd.kernels as K

pytestmark = pytest.mark.gpu


def _expected(z, S):
    key = np.where((z >= 0) & (z < S), z, S)
    order = np.argsort(key, kind="stable").astype(np.int32)
    counts = np.bincount(key, minlength=S + 1)
    return order, np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


@pytest.mark.parametrize("n,S,invalid", [(0, 10, False), (1, 1, False), (63, 3, False), (1024, 10, True),
                                         (1025, 10, True), (50_000, 10, True), (200_003, 89, True),
                                         (5000, 4096, True), (3000, 1, True)])
def test_class_groups_vs_numpy(n, S, invalid):
    rng = np.random.default_rng(n + S)
    z = rng.integers(0, S, n)
    if invalid and n:
        bad = rng.random(n) < 0.05
        z[bad] = rng.choice([-1, -7, S, S + 3], bad.sum())
    order, start = K.class_groups(torch.tensor(z, device="cuda"), S)
    ro, rs = _expected(z, S)
    assert order.dtype == torch.int32 and start.dtype == torch.int32
    assert np.array_equal(order.cpu().numpy(), ro)
    assert np.array_equal(start.cpu().numpy(), rs)


def test_class_groups_int32_classes_and_sorted_input():
    z = torch.arange(5000, device="cuda", dtype=torch.int32) // 700  # already grouped, 8 classes
    order, start = K.class_groups(z, 8)
    assert torch.equal(order.cpu(), torch.arange(5000, dtype=torch.int32))
    assert start.cpu().tolist() == [0, 700, 1400, 2100, 2800, 3500, 4200, 4900, 5000, 5000]


def test_class_groups_rejects_cpu_tensors():
    with pytest.raises(RuntimeError, match="GPU only"):
        K.class_groups(torch.zeros(0, dtype=torch.long), 4)
