"""Host-side contract of the molix data task (no GPU): the NeighborList task is GPU-only and
says so, including inside a DataLoader worker forked from a process that uses the GPU; the
receiver-sorted mode rejects symmetry=False."""

import pytest
import torch

from molnex_amd.molix.data.tasks.neighbor_list import NeighborList


def test_receiver_sorted_requires_symmetry():
    with pytest.raises(ValueError, match="symmetry=False"):
        NeighborList(receiver_sorted=True, symmetry=False)
    assert NeighborList(receiver_sorted=True).task_id.endswith(":rs")


def test_task_id_matches_reference_format():
    # src/molix/data/tasks/neighbor_list.py:60-65
    assert NeighborList(cutoff=4.5, max_num_pairs=100, pbc=True, symmetry=False).task_id == \
        "nlist:cut=4.5:max=100:pbc=True:sym=False"


def test_cpu_sample_without_gpu_raises_clearly():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(RuntimeError, match="no GPU is visible and there is no CPU implementation"):
        NeighborList()({"pos": torch.zeros((4, 3))})


def test_forked_worker_of_a_gpu_process_raises_clearly(monkeypatch):
    # the state torch reports in a child forked after the parent initialised the GPU
    monkeypatch.setattr(torch.cuda, "_is_in_bad_fork", lambda: True)
    with pytest.raises(RuntimeError, match="forked from a process that already uses the GPU"):
        NeighborList()({"pos": torch.zeros((4, 3))})
