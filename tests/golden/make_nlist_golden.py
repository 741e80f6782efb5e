"""Write tests/golden/nlist_golden.npz from the reference's own CPU op.

Runs in the build container only: it loads oracle/_ref/libmolix_ref.so, which
oracle/Makefile (`make ref`) compiles from the reference sources
src/molix/op/src/{molix_library,molix_meta}.cpp, neighbors/get_neighbor_pairs.cpp
and pme/pme_cpu.cpp, and calls torch.ops.molix.get_neighbor_pairs on seeded
inputs.  The fixture holds inputs and the reference outputs only.

    python tests/golden/make_nlist_golden.py
"""

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.path.join(HERE, "..", "..", "oracle", "_ref", "libmolix_ref.so")


def molecule(rng, n, side=6.0, dmin=0.9):
    pts = []
    while len(pts) < n:
        p = rng.uniform(0, side, 3)
        if all(np.linalg.norm(p - q) >= dmin for q in pts):
            pts.append(p)
    return np.array(pts)


def tric_box():
    return np.array([[18.0, 0, 0], [3.0, 17.0, 0], [-2.0, 4.0, 16.0]])


def cases():
    rng = np.random.default_rng(1234)
    out = []
    mol = molecule(rng, 32)
    out.append(("open_f32_m512", mol, None, 5.0, 512, np.float32))
    out.append(("open_f32_all", mol, None, 5.0, -1, np.float32))
    out.append(("open_f64_m512", mol, None, 5.0, 512, np.float64))
    dense = rng.uniform(0, 6.0, (64, 3))
    out.append(("open_f32_truncated", dense, None, 5.0, 100, np.float32))
    L = 16.0
    out.append(("cubic_f32", rng.uniform(0, L, (400, 3)), np.eye(3) * L, 5.0, 20000, np.float32))
    L2 = (1500 / 0.1) ** (1 / 3)
    out.append(("cubic_f32_n1500", rng.uniform(0, L2, (1500, 3)), np.eye(3) * L2, 5.0, 60000, np.float32))
    out.append(("cubic_f64", rng.uniform(0, L, (400, 3)), np.eye(3) * L, 5.0, 20000, np.float64))
    B = tric_box()
    frac = rng.uniform(0, 1, (500, 3))
    out.append(("tric_f32", frac @ B, B, 5.0, 30000, np.float32))
    out.append(("tric_f64", frac @ B, B, 5.0, 30000, np.float64))
    out.append(("smallbox_f32", rng.uniform(0, 8.0, (50, 3)), np.eye(3) * 8.0, 3.9, 2000, np.float32))
    # outside the box (unwrapped coordinates) and negative coordinates
    out.append(("cubic_unwrapped_f32", rng.uniform(-20, 40, (300, 3)), np.eye(3) * 16.0, 5.0, 20000, np.float32))
    # boundary cases: exact cutoff distance, duplicate positions, half-box minimum image tie
    edge = np.array([[0, 0, 0], [5, 0, 0], [5, 0, 0], [0, 3, 4], [1, 1, 1], [9.5, 1, 1], [2, 2, 2]], float)
    out.append(("edge_open_f32", edge, None, 5.0, 64, np.float32))
    out.append(("edge_pbc_f32", edge, np.eye(3) * 10.0, 5.0, 64, np.float32))
    out.append(("single_atom", np.zeros((1, 3)), None, 5.0, 8, np.float32))
    return out


def main():
    torch.ops.load_library(REF)
    data = {}
    names = []
    for name, pos, box, cut, mnp, dt in cases():
        tdt = torch.float32 if dt == np.float32 else torch.float64
        p = torch.tensor(pos, dtype=tdt)
        b = torch.empty((0, 0), dtype=tdt) if box is None else torch.tensor(box, dtype=tdt)
        nb, d, dist, npairs = torch.ops.molix.get_neighbor_pairs(p, cut, mnp, b)
        names.append(name)
        data[f"{name}/positions"] = p.numpy()
        data[f"{name}/box"] = b.numpy()
        data[f"{name}/cutoff"] = np.array(cut)
        data[f"{name}/max_num_pairs"] = np.array(mnp)
        data[f"{name}/neighbors"] = nb.numpy()
        data[f"{name}/deltas"] = d.detach().numpy()
        data[f"{name}/distances"] = dist.detach().numpy()
        data[f"{name}/num_pairs"] = npairs.numpy()
        print(f"{name}: n={len(pos)} pairs={int(npairs[0])} width={nb.shape[1]}")
    data["cases"] = np.array(names)
    np.savez_compressed(os.path.join(HERE, "nlist_golden.npz"), **data)


if __name__ == "__main__":
    main()
