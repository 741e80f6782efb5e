"""Per-sample neighbor-list task (src/molix/data/tasks/neighbor_list.py:22-103) on the HIP cell list.

Same output as the reference task: half pairs (row > col) in (row, col) order
with ``bond_diff = pos[target] - pos[source] = -deltas``
(``neighbor_list.py:86-89``), followed by the reversed edges when
``symmetry=True`` (``:91-96``); ``bond_diff`` / ``bond_dist`` cast to fp32
(``:101-102``).  The pair list comes from the exact-size cell list, so it is
the reference CPU op's list (all pairs, bit-identical geometry) regardless of
``max_num_pairs``, which is kept for the task id (the reference CPU op also
returns every found pair when there are more than ``max_num_pairs``,
``get_neighbor_pairs.cpp:55-73``).

Where it runs: the search is the HIP cell list, there is no CPU
implementation.  Samples on the CPU are moved to the current GPU for the
search and the results moved back, which works in the main process and in
DataLoader workers started with ``multiprocessing_context="spawn"``.  The
reference runs this task inside forked DataLoader workers
(``src/molix/data/datamodule.py:172-184``); a worker forked from a process that
already uses the GPU cannot use it, and the task then raises a RuntimeError
that says so (run it with ``num_workers=0``, with spawned workers, or on the
collated batch on the GPU) instead of failing inside the HIP runtime.

``receiver_sorted=True`` (not in the reference) returns every directed edge
once, sorted by (target, source), which is the order the tensor-product
kernels consume without a re-sort; it is the full (symmetric) list by
construction, so it requires ``symmetry=True``.
"""

from __future__ import annotations

import torch

from ...F.locality import neighbor_list


def _normalize_to_E2(edge_index: torch.Tensor) -> torch.Tensor:
    """Normalise edge_index to canonical ``[E, 2]`` (neighbor_list.py:11-19)."""
    if edge_index.ndim != 2:
        raise ValueError(f"edge_index must be 2D, got {tuple(edge_index.shape)}")
    if edge_index.shape[1] == 2:
        return edge_index.long()
    if edge_index.shape[0] == 2:
        return edge_index.t().contiguous().long()
    raise ValueError(f"edge_index shape {tuple(edge_index.shape)} is invalid")


def _search_device(pos: torch.Tensor) -> torch.device:
    """The GPU the cell list runs on for a sample stored on ``pos.device``."""
    if pos.device.type == "cuda":
        return pos.device
    if torch.cuda._is_in_bad_fork():
        worker = torch.utils.data.get_worker_info()
        where = f"DataLoader worker {worker.id}" if worker is not None else "this forked process"
        raise RuntimeError(
            f"molix NeighborList runs on the GPU (HIP cell list) and {where} was forked from a process that "
            "already uses the GPU, so it cannot start a GPU context. Run the task with num_workers=0, with "
            "multiprocessing_context='spawn', or on the collated batch on the GPU.")
    if not torch.cuda.is_available():
        raise RuntimeError("molix NeighborList runs on the GPU (HIP cell list); no GPU is visible and there is no "
                           "CPU implementation")
    return torch.device("cuda", torch.cuda.current_device())


class NeighborList:
    """Compute the neighbor list of one sample (a ``SampleTask`` in the reference)."""

    def __init__(self, cutoff: float = 5.0, max_num_pairs: int = 512, pbc: bool = False,
                 filter_padding: bool = True, symmetry: bool = True, receiver_sorted: bool = False) -> None:
        if receiver_sorted and not symmetry:
            raise ValueError("receiver_sorted=True returns the full directed list; it cannot be combined with "
                             "symmetry=False")
        self.cutoff = cutoff
        self.max_num_pairs = max_num_pairs
        self.pbc = pbc
        self.filter_padding = filter_padding
        self.symmetry = symmetry
        self.receiver_sorted = receiver_sorted

    @property
    def task_id(self) -> str:
        tid = f"nlist:cut={self.cutoff}:max={self.max_num_pairs}:pbc={self.pbc}:sym={self.symmetry}"
        return tid + (":rs" if self.receiver_sorted else "")

    def __call__(self, data: dict) -> dict:
        return self.execute(data)

    def execute(self, data: dict) -> dict:
        pos = data["pos"]
        home = pos.device
        dev = _search_device(pos)
        box = data.get("cell") if self.pbc else None
        p = pos.to(dev)
        b = box.to(device=dev, dtype=p.dtype) if box is not None else None
        if self.receiver_sorted:
            i, j, _, deltas, dist = neighbor_list(p, self.cutoff, b, full=True)
            # edge (source j -> target i): bond_diff = pos[i] - image(pos[j]) = deltas
            edge_index = torch.stack([j.long(), i.long()], dim=1)
            bond_diff = deltas
        else:
            i, j, _, deltas, dist = neighbor_list(p, self.cutoff, b, full=False)
            edge_index = torch.stack([i.long(), j.long()], dim=1)
            bond_diff = -deltas
            if self.symmetry:
                edge_index = torch.cat([edge_index, edge_index[:, [1, 0]]], dim=0)
                bond_diff = torch.cat([bond_diff, -bond_diff], dim=0)
                dist = torch.cat([dist, dist], dim=0)
        return {
            **data,
            "edge_index": edge_index.to(home),
            "bond_diff": bond_diff.float().to(home),
            "bond_dist": dist.float().to(home),
        }
