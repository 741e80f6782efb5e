"""Write tests/golden/pme_golden.npz from the reference's own CPU PME ops.

Build-container only: loads oracle/_ref/libmolix_ref.so (oracle/Makefile `make ref`,
compiled from src/molix/op/src/pme/pme_cpu.cpp and the op schema files) and records
energies and their gradients (positions, charges) of torch.ops.molix.pme_reciprocal
and torch.ops.molix.pme_direct on seeded inputs.  Moduli come from
oracle/pme.bspline_moduli and are stored as inputs.

    python tests/golden/make_pme_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", ".."))
from oracle.pme import bspline_moduli  # noqa: E402

REF = os.path.join(HERE, "..", "..", "oracle", "_ref", "libmolix_ref.so")


def charges(rng, n):
    q = rng.normal(size=n)
    return q - q.mean()


def main():
    torch.ops.load_library(REF)
    rng = np.random.default_rng(77)
    data, names = {}, []
    tric = np.array([[12.0, 0, 0], [2.0, 11.0, 0], [-1.5, 1.0, 10.0]])
    recip_cases = [
        ("cubic_o4_f64", 40, np.eye(3) * 10.0, (16, 16, 16), 4, 0.35, np.float64),
        ("cubic_o5_f64", 40, np.eye(3) * 10.0, (16, 18, 20), 5, 0.35, np.float64),
        ("cubic_o6_f64", 60, np.eye(3) * 12.0, (20, 20, 20), 6, 0.3, np.float64),
        ("tric_o6_f64", 50, tric, (16, 16, 16), 6, 0.4, np.float64),
        ("cubic_o6_f32", 60, np.eye(3) * 12.0, (20, 20, 20), 6, 0.3, np.float32),
        ("cubic_o4_f32", 40, np.eye(3) * 10.0, (16, 16, 16), 4, 0.35, np.float32),
    ]
    coulomb = 14.399645
    for name, n, box, grid, order, alpha, dt in recip_cases:
        tdt = torch.float32 if dt == np.float32 else torch.float64
        frac = rng.uniform(-0.2, 1.2, (n, 3))  # some atoms outside the cell
        pos = torch.tensor(frac @ box, dtype=tdt, requires_grad=True)
        q = torch.tensor(charges(rng, n), dtype=tdt, requires_grad=True)
        b = torch.tensor(box, dtype=tdt)
        mods = [torch.tensor(bspline_moduli(g, order), dtype=tdt) for g in grid]
        e = torch.ops.molix.pme_reciprocal(pos, q, b, grid[0], grid[1], grid[2], order, alpha, coulomb, *mods)
        gp, gq = torch.autograd.grad(e, (pos, q))
        key = f"recip_{name}"
        names.append(key)
        data.update({f"{key}/positions": pos.detach().numpy(), f"{key}/charges": q.detach().numpy(),
                     f"{key}/box": box.astype(dt), f"{key}/grid": np.array(grid), f"{key}/order": np.array(order),
                     f"{key}/alpha": np.array(alpha), f"{key}/coulomb": np.array(coulomb),
                     f"{key}/xmoduli": mods[0].numpy(), f"{key}/ymoduli": mods[1].numpy(),
                     f"{key}/zmoduli": mods[2].numpy(), f"{key}/energy": e.detach().numpy(),
                     f"{key}/grad_positions": gp.numpy(), f"{key}/grad_charges": gq.numpy()})
        print(key, float(e))
    direct_cases = [("cubic_f64", 80, 12.0, 4.5, 0.35, np.float64, True),
                    ("cubic_f32", 80, 12.0, 4.5, 0.35, np.float32, True),
                    ("cubic_noexcl_f64", 60, 11.0, 4.0, 0.3, np.float64, False)]
    for name, n, L, rc, alpha, dt, with_excl in direct_cases:
        tdt = torch.float32 if dt == np.float32 else torch.float64
        pos = torch.tensor(rng.uniform(0, L, (n, 3)), dtype=tdt, requires_grad=True)
        q = torch.tensor(charges(rng, n), dtype=tdt, requires_grad=True)
        box = torch.eye(3, dtype=tdt) * L
        nb, d, dist, npairs = torch.ops.molix.get_neighbor_pairs(pos.detach(), rc, -1, box)
        keep = (nb[0] >= 0)
        nb, d, dist = nb[:, keep].contiguous(), d[keep].contiguous(), dist[keep].contiguous()
        if with_excl:
            # each atom excludes up to 3 of its lower-index pair partners; lists descending, -1 padded
            excl = -np.ones((n, 4), np.int32)
            for i in range(n):
                cand = sorted({int(c) for r, c in zip(nb[0].tolist(), nb[1].tolist()) if r == i}, reverse=True)[:3]
                excl[i, :len(cand)] = cand
                # symmetric entries so both atoms list each other
            for i in range(n):
                for c in excl[i]:
                    if c >= 0 and i not in excl[c]:
                        free = np.where(excl[c] < 0)[0]
                        if len(free):
                            excl[c, free[0]] = i
            excl = -np.sort(-excl, axis=1)
        else:
            excl = -np.ones((n, 1), np.int32)
        ex = torch.tensor(excl, dtype=torch.int32)
        e = torch.ops.molix.pme_direct(pos, q, nb, d, dist, ex, alpha, coulomb)
        gp, gq = torch.autograd.grad(e, (pos, q))
        key = f"direct_{name}"
        names.append(key)
        data.update({f"{key}/positions": pos.detach().numpy(), f"{key}/charges": q.detach().numpy(),
                     f"{key}/neighbors": nb.numpy(), f"{key}/deltas": d.numpy(), f"{key}/distances": dist.numpy(),
                     f"{key}/exclusions": excl, f"{key}/alpha": np.array(alpha), f"{key}/coulomb": np.array(coulomb),
                     f"{key}/energy": e.detach().numpy(), f"{key}/grad_positions": gp.numpy(),
                     f"{key}/grad_charges": gq.numpy()})
        print(key, float(e), nb.shape[1])
    data["cases"] = np.array(names)
    np.savez_compressed(os.path.join(HERE, "pme_golden.npz"), **data)


if __name__ == "__main__":
    main()
