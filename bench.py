"""Benchmark of the equivariant edge step on one MI355X.

Workload: 50,000 atoms uniform in a periodic cube at
0.1 atoms/A^3 (L = 79.37 A), directed cell list at rc = 5 A (E ~ 2.62 M edges,
built by this package's HIP neighbor list), node features 128 x (0e+1o+2e+3o)
~ N(0,1) fp32 in ir_mul layout, real harmonics l <= 3 of the edge vectors and
per-edge weights from 8 Bessel functions x cosine cutoff -> 64 -> 64 -> 2944
SiLU MLP (random init, seeded).  One step = forward (harmonics, radial basis,
MLP, channelwise TP + scatter-sum to receivers) and backward with respect to
node features and edge vectors.  Metric: M edges/s = E * steps / time.

Prints one JSON line (the driver's contract) with a ``roofline`` object for the
dominant HIP kernel (timed with HIP events on the stream it runs on) and a
``cpu_baseline`` (the same step in torch on the host cores, fp32 and fp64, on a
bounded sample of the graph; rank 0, N=1).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import copy
import json
import math
import os
import platform
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--atoms", type=int, default=50_000)
    p.add_argument("--channels", type=int, default=128)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--unsorted", action="store_true", help="keep atoms in random order (no spatial sort)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--workload", choices=["tp", "full", "sc", "nl", "pme", "train", "allegro", "tpgh"], default="tp",
                   help="tp: config 3 edge step (default, the headline line); full: config 5 energy + forces; "
                        "sc / nl / pme: config 4, config 2, config 5's PME term alone; train: config 5 "
                        "force-matching training step; allegro: Allegro energy + forces on the 50k-atom graph; "
                        "tpgh: the config-3 tensor-product backward fused with the output layer's input "
                        "gradient against the unfused pair (off by default in the library)")
    p.add_argument("--no-secondary", action="store_true",
                   help="skip the secondary figures (config 2 neighbor list, config 5 energy + forces)")
    p.add_argument("--literal", action="store_true",
                   help="with --workload full: the literal MACE (hidden 128x0e+128x1o, polynomial cutoff)")
    p.add_argument("--kernels-only", action="store_true",
                   help="profiling aid: a 1 GiB device copy (counter calibration), then 3 TP forward and "
                        "3 TP backward launches; prints their event times")
    return p.parse_args()


def bessel_cutoff(r: torch.Tensor, rc: float, n: int, mu: torch.Tensor, sigma: torch.Tensor) -> torch.Tensor:
    """8-Bessel basis with the reference's shift/scale (radial.py:117-147) times the cosine cutoff
    (cutoff.py:56-75), as combined in MACE's EmbeddingBlock (mace.py:180-182)."""
    freqs = torch.arange(1, n + 1, device=r.device, dtype=r.dtype) * (math.pi / rc)
    rr = r.unsqueeze(-1)
    phi = math.sqrt(2.0 / rc) * torch.sin(rr * freqs) / (rr + 1e-8)
    phi = (phi - mu) / sigma
    cut = 0.5 * (torch.cos(math.pi * r / rc) + 1.0) * (r < rc)
    return phi * cut.unsqueeze(-1)


def bessel_stats(rc: float, n: int):
    r = torch.linspace(1e-8, rc, 4096, dtype=torch.float32)
    freqs = torch.arange(1, n + 1, dtype=torch.float32) * (math.pi / rc)
    phi = math.sqrt(2.0 / rc) * torch.sin(r[:, None] * freqs) / (r[:, None] + 1e-8)
    return phi.mean(0), phi.std(0).clamp(min=1e-8)


def make_system(n_atoms: int, seed: int, sort: bool, dev):
    import molnex_amd.kernels  # noqa: F401

    L = (n_atoms / 0.1) ** (1.0 / 3.0)
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand((n_atoms, 3), generator=g, dtype=torch.float32) * L
    if sort:
        # spatial (cell) order, as MD codes and data pipelines keep atoms
        cell = torch.floor(pos / (L / 16)).long().clamp(max=15)
        key = (cell[:, 2] * 16 + cell[:, 1]) * 16 + cell[:, 0]
        pos = pos[torch.argsort(key, stable=True)]
    pos = pos.to(dev)
    box = torch.eye(3, device=dev) * L
    i, j, shifts, deltas, dist = torch.ops.molix.neighbor_list(pos, 5.0, box, True)
    # edge (sender j -> receiver i); bond vector pos[receiver] - image(pos[sender]) = deltas
    edge_index = torch.stack([j.long(), i.long()], dim=1)
    return pos, box, edge_index, deltas.contiguous(), L


class EdgeStep:
    """forward + backward of SH x radial-MLP x channelwise TP + scatter (config 3)."""

    def __init__(self, n_atoms, edge_index, vec, C, seed, dev):
        from molnex_amd import kernels as K

        self.K = K
        self.N, self.E, self.C = n_atoms, edge_index.shape[0], C
        self.config = K.tp_config_id([0, 1, 2, 3], [0, 1, 2, 3], [0, 1, 2, 3])
        self.num_paths, self.nx, self.ny, self.no = K.tp_config_info(self.config)
        g = torch.Generator(device="cpu").manual_seed(seed + 1)
        self.x = torch.randn((n_atoms, self.nx * C), generator=g).to(dev).requires_grad_(True)
        self.vec = vec.detach().clone().requires_grad_(True)
        self.edge_index = edge_index
        torch.manual_seed(seed + 2)
        from molnex_amd.molrep.interaction import RadialWeightMLP

        self.mlp = RadialWeightMLP(in_dim=8, hidden_dim=64, out_dim=self.num_paths * C, num_layers=2).to(dev)
        for p in self.mlp.parameters():
            p.requires_grad_(False)
        self.mu, self.sigma = (t.to(dev) for t in bessel_stats(5.0, 8))
        self.gout = torch.randn((n_atoms, self.no * C), generator=g).to(dev)
        from molnex_amd.config import config as mcfg

        self.fused = mcfg.fused_weight_grad is True and self.K.tp_weight_grad_supported(self.config, C, 64)
        self.paired = mcfg.paired_radial
        self.graph = None  # (row_ptr, perm, senders, pairs), built on the first step

    def step(self):
        ops = torch.ops.molix
        Y = ops.spherical_harmonics(self.vec, 3)
        r = torch.linalg.vector_norm(self.vec, dim=-1)
        # 8-Bessel x cosine cutoff in one kernel each way (bessel_cutoff below is its torch form)
        feats = ops.bessel_cutoff(r, 8, 5.0, 1e-8, self.mu, self.sigma, 1, 0)
        if self.graph is None:
            # the receiver CSR and the undirected-edge pairing belong to the graph: built on its
            # first step and kept, as an MD loop keeps its neighbor list between rebuilds (the
            # pairing holds for any positions: a neighbor list's two directions have bond vectors
            # that are exact negations).  Indices come from the neighbor list: no validation sync.
            row_ptr, perm, snd = ops.edge_csr(self.edge_index, self.N, False)
            pairs = self.K.EdgePairs.build(self.edge_index, self.N, row_ptr, perm, snd, feats.detach()) \
                if self.paired else None
            self.graph = (row_ptr, perm, snd, pairs)
        row_ptr, perm, snd, pairs = self.graph
        if pairs is not None:
            # the output layer once per undirected pair (both directions have the same distance,
            # hence the same weights); edge mode: every edge vector gets its own gradient
            last = self.mlp.mlp[-1]
            # with config.fused_weight_grad = True: the input gradient without the per-edge weight
            # gradient in memory (its work list costs one more synchronisation per step here)
            batches = self.K.tp_gh_batches(row_ptr) if self.fused else None
            out, _ = ops.radial_tp_pairs(self.x, Y, self.mlp.hidden(feats), last.weight, last.bias, row_ptr, perm,
                                         snd, pairs.wrow, pairs.pairs, self.config, self.C, batches)
        elif self.fused:
            # output layer + TP as one op: the backward forms the weight gradient in registers
            last = self.mlp.mlp[-1]
            out, _ = ops.radial_tp(self.x, Y, self.mlp.hidden(feats), last.weight, last.bias, row_ptr, perm, snd,
                                   self.edge_index, self.config, self.C)
        else:
            w = self.mlp(feats)
            out = ops.tp_scatter(self.x, Y, w, row_ptr, perm, snd, self.config, self.C)
        self.x.grad = None
        self.vec.grad = None
        out.backward(self.gout)
        return out


def time_tp_kernels(step: EdgeStep, reps: int = 5):
    """Average duration of the TP forward and backward launches (HIP events on the
    current stream, which is the stream the kernels are enqueued on)."""
    ops = torch.ops.molix
    K = step.K
    row_ptr, perm, snd = ops.edge_csr(step.edge_index, step.N)
    with torch.no_grad():
        Y = ops.spherical_harmonics(step.vec, 3)
        r = torch.linalg.vector_norm(step.vec, dim=-1)
        w = step.mlp(bessel_cutoff(r, 5.0, 8, step.mu, step.sigma))
    x = step.x.detach()
    fwd, bwd = [], []
    for _ in range(reps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record()
        ops.tp_scatter(x, Y, w, row_ptr, perm, snd, step.config, step.C)
        e[1].record()
        e[2].record()
        K.tp_scatter_backward(step.gout, x, Y, w, row_ptr, perm, snd, step.config, step.C, True, True, True)
        e[3].record()
        fwd.append(e[:2])
        bwd.append(e[2:])
    torch.cuda.synchronize()
    tf = sum(a.elapsed_time(b) for a, b in fwd) / reps
    tb = sum(a.elapsed_time(b) for a, b in bwd) / reps
    return tf, tb


def time_edge_weight_kernels(step: EdgeStep, reps: int = 5):
    """Average duration of the radial MLP's output-layer kernels (molix::edge_weights forward and
    input-gradient backward) at the step's shapes; HIP events on the current stream."""
    K = step.K
    with torch.no_grad():
        r = torch.linalg.vector_norm(step.vec, dim=-1)
        h = K.radial_hidden(bessel_cutoff(r, 5.0, 8, step.mu, step.sigma).contiguous(),
                            torch.cat([t.reshape(-1) for m in step.mlp.mlp[:-1:2] for t in (m.weight, m.bias)]),
                            8, 64, 2)
    last = step.mlp.mlp[-1]
    gw = torch.randn(h.shape[0], last.out_features, device=h.device)
    # with the pairing the step's forward runs on one row per undirected pair (E / 2)
    hf = h[: h.shape[0] // 2].contiguous() if step.paired else h
    fwd, bwd = [], []
    for i in range(reps + 1):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record()
        w = K.edge_weights(hf, last.weight, last.bias)
        e[1].record()
        e[2].record()
        K.edge_weights_backward(gw, last.weight)
        e[3].record()
        del w
        if i:
            fwd.append(e[:2])
            bwd.append(e[2:])
    torch.cuda.synchronize()
    tf = sum(a.elapsed_time(b) for a, b in fwd) / reps
    tb = sum(a.elapsed_time(b) for a, b in bwd) / reps
    # each direction: one rows x K and one rows x N tensor
    nbytes_f = 4 * hf.shape[0] * (h.shape[1] + last.out_features)
    nbytes_b = 4 * h.shape[0] * (h.shape[1] + last.out_features)
    return tf, tb, nbytes_f, nbytes_b


def measured_traffic(kernel: str):
    """HBM bytes per launch (FETCH_SIZE x calibration + WRITE_SIZE) of `kernel` at config 3,
    recorded from rocprofv3 --pmc runs in profiles/tp_scatter_config3_traffic.{json,md}."""
    path = os.path.join(ROOT, "profiles", "tp_scatter_config3_traffic.json")
    try:
        rec = json.load(open(path))[kernel]
        return int(rec["read_bytes"] + rec["write_bytes"])
    except (OSError, KeyError, ValueError):
        return None


def tp_bytes(N, E, C, P=23, NX=16, NY=16, NO=99):
    """Algorithmic HBM bytes (each tensor once at its width; fp32, int32 CSR)."""
    csr = E * 8 + (N + 1) * 4
    fwd = 4 * (E * P * C + N * NO * C + N * NX * C + E * NY) + csr
    bwd = 4 * (2 * E * P * C + N * NO * C + 2 * N * NX * C + 2 * E * NY) + csr
    return fwd, bwd


def mace_step_bytes(enc, N, E, mlp_rows=None):
    """Algorithmic HBM bytes of one energy + forces step of `enc` (fp32, each tensor once per kernel):
    per interaction layer the radial MLP hidden stack (fwd: features in, h out; bwd: features and
    grad_h in, grad_features out), its output layer (fwd: h in, weights out; bwd: the per-edge weight
    gradient in, grad_h out) and the TP + scatter forward and backward (tp_bytes, per directed edge);
    once per step the harmonics (vectors in, 16 components out, and back) and the bond vectors
    (positions and edge list in, vectors out, and back).  ``mlp_rows``: the rows the radial MLP runs
    on -- E per directed edge (the reference's form), E / 2 once per undirected pair (what MACE here
    runs): the hidden stack, the output layer's input and its weights written then have E / 2 rows,
    while the per-edge weight gradient it reads back stays E rows.  Node-level kernels (linears,
    contraction, element updates, PME on 50k atoms) move < 2 % of these bytes and are left out."""
    from molnex_amd import kernels as K

    R = E if mlp_rows is None else mlp_rows
    total = 2 * (4 * E * 3 + 4 * E * 16) + 4 * E * 3  # harmonics fwd + bwd
    total += 2 * (8 * E * 2 + 4 * E * 3 + 4 * N * 3)  # bond vectors fwd + bwd
    for blk in enc.interactions:
        P, NX, NY, NO = K.tp_config_info(blk.conv_tp.cue_tp.config_id)
        C = blk.conv_tp.cue_tp.channels
        rc = blk.radial_mlp.config
        kin, H = rc.in_dim, rc.hidden_dim
        tf, tb = tp_bytes(N, E, C, P, NX, NY, NO)
        total += 4 * R * (kin + H) + 4 * R * (H + P * C) + tf  # forward
        total += tb + 4 * E * P * C + 4 * R * H + 4 * R * (kin + H + kin)  # backward
    return total


def host_cores() -> int:
    """Cores this process may use: its affinity set, capped by OMP_NUM_THREADS when that is set."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() else n


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(edge_index, vec, x, C, mlp, mu, sigma, gout, target_s=8.0, chunk_edges=5_000):
    """The GPU line's step on the host cores, per dtype (fp32, then fp64), on a bounded sample:
    harmonics + 8-Bessel x cosine cutoff -> the radial MLP -> channelwise TP + scatter, forward and
    backward to the node features and the edge vectors (torch autograd through the oracle's torch
    restatement, oracle/mace_ref.py: sh_torch, conv_tp), over receiver-ordered chunks of the
    config-3 graph (each chunk: the edges of consecutive receivers, with their senders' rows) until
    ~target_s of CPU time per dtype."""
    from oracle import mace_ref

    cores = host_cores()
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    order = torch.argsort(edge_index[:, 1], stable=True).cpu()
    ei_all = edge_index.cpu()[order]
    vec_all = vec.detach().cpu()[order]
    rates = {}
    try:
        for dt in (torch.float32, torch.float64):
            mlp_c = copy.deepcopy(mlp.mlp).cpu().to(dt)  # the plain Sequential: Linear/SiLU layers
            mu_c, sig_c = mu.cpu().to(dt), sigma.cpu().to(dt)
            done, t_used, start, warm = 0, 0.0, 0, True
            while (t_used < target_s or warm) and start < len(ei_all):
                ei = ei_all[start:start + chunk_edges]
                # whole receivers only: stop at the last receiver boundary of the chunk
                if start + chunk_edges < len(ei_all):
                    last = int(ei[-1, 1])
                    ei = ei[ei[:, 1] != last] if (ei[:, 1] != last).any() else ei
                n_e = len(ei)
                senders, s_loc = torch.unique(ei[:, 0], return_inverse=True)
                recv, r_loc = torch.unique(ei[:, 1], return_inverse=True)
                xs = x.detach()[senders.to(x.device)].cpu().to(dt).requires_grad_(True)
                v = vec_all[start:start + n_e].to(dt).requires_grad_(True)
                g = gout[recv.to(gout.device)].cpu().to(dt)
                t0 = time.perf_counter()
                r = torch.linalg.vector_norm(v, dim=-1)
                Y = mace_ref.sh_torch(3, v)
                w = mlp_c(bessel_cutoff(r, 5.0, 8, mu_c, sig_c))
                out, _ = mace_ref.conv_tp(xs, Y, w, torch.stack([s_loc, r_loc], 1), len(recv), 3, C)
                gx, gv = torch.autograd.grad(out, (xs, v), g)
                dt_chunk = time.perf_counter() - t0
                start += n_e
                if warm:
                    warm = False
                    continue
                t_used += dt_chunk
                done += n_e
            rates[dt] = (done / t_used / 1e6 if t_used else 0.0, done, t_used)
    finally:
        torch.set_num_threads(prev)
    f32, f64 = rates[torch.float32], rates[torch.float64]
    return {
        "value": round(f32[0], 6),
        "unit": "M edges/s",
        "cores": cores,
        "kind": "port",
        "dtype": "fp32",
        "fp64_value": round(f64[0], 6),
        "cpu_model": cpu_model(),
        "sample": f"the GPU line's step (harmonics, Bessel x cutoff, 8->64->64->{mlp.config.out_dim} SiLU MLP, channelwise "
                  f"TP + scatter, backward to x and edge vectors) in torch on {cores} host cores over "
                  f"receiver-ordered chunks of the config-3 graph: fp32 {f32[1]} edges in {f32[2]:.1f} s, fp64 "
                  f"{f64[1]} edges in {f64[2]:.1f} s (after one warm-up chunk each)",
    }


def lattice_positions(n: int, L: float, g: torch.Generator) -> torch.Tensor:
    """Jittered cubic lattice in a periodic cube of side L: uniform density with every pair
    >= 0.9 A apart, atoms in spatial (cell) order."""
    k = math.ceil(n ** (1 / 3))
    sites = torch.stack(torch.meshgrid(*[torch.arange(k)] * 3, indexing="ij"), -1).reshape(-1, 3).float()
    sites = sites[torch.randperm(sites.shape[0], generator=g)[:n]]
    a = L / k
    pos = (sites + 0.5) * a + (torch.rand((n, 3), generator=g) - 0.5) * (a - 0.9)
    cell = torch.floor(pos / (L / 16)).long().clamp(max=15)
    return pos[torch.argsort((cell[:, 2] * 16 + cell[:, 1]) * 16 + cell[:, 0], stable=True)]


def pme_bench(dev, reps=10):
    """BASELINE config 5's long-range term alone: 50k atoms (jittered lattice, 0.1 A^-3), neutral
    random charges, PME alpha 0.3, 128^3, order 6, real-space cutoff 5 A (half list built inside);
    energy + forces by autograd."""
    from molnex_amd.molpot import PMEPotential

    n = 50_000
    L = (n / 0.1) ** (1.0 / 3.0)
    g = torch.Generator().manual_seed(5)
    pos = lattice_positions(n, L, g).to(dev)
    q = torch.randn(n, generator=g) * 0.3
    q = (q - q.mean()).to(dev)
    box = torch.eye(3, device=dev) * L
    pme = PMEPotential(alpha=0.3, grid=(128, 128, 128), order=6, cutoff=5.0).to(dev)

    def step():
        p = pos.clone().requires_grad_(True)
        e = pme(p, q, box)
        (f,) = torch.autograd.grad(e, p)
        return e, f

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        e, f = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    return {"workload": "config 5 PME term: 50k atoms, alpha 0.3, 128^3, order 6, rc 5 A, energy + forces",
            "ms_per_step": round(dt * 1e3, 3), "energy_finite": bool(torch.isfinite(e).item())}


def full_step_bench(args, dev):
    """MACE (as coded: 128 x (0e..3o), 2 layers, correlation 3) on 50k atoms in a
    periodic box with 10 elements, ChargeHead charges (per-system neutral) into PME (alpha 0.3, 128^3,
    order 6, real-space cutoff 5 A); energy + forces (one backward).  Metric: atoms/s."""
    from molnex_amd.molpot import ChargeHead, PMEPotential
    from molnex_amd.molpot.pipeline import EnergyForceModel
    from molnex_amd.molrep.embedding import DiscreteEmbeddingSpec
    from molnex_amd.molzoo import MACE

    n = args.atoms
    L = (n / 0.1) ** (1.0 / 3.0)
    g = torch.Generator().manual_seed(args.seed)
    pos = lattice_positions(n, L, g).to(dev)
    Z = torch.randint(0, 10, (n,), generator=g).to(dev)
    box = torch.eye(3, device=dev) * L
    # periodic images enter the recomputed bond vectors through the shifts: bond = pos[i] - pos[j] - shift
    i, j, shifts, deltas, _ = torch.ops.molix.neighbor_list(pos, 5.0, box, True)
    edge_index = torch.stack([j.long(), i.long()], 1)
    torch.manual_seed(args.seed)
    C = args.channels
    literal = getattr(args, "literal", False)
    enc = MACE(node_attr_specs=[DiscreteEmbeddingSpec(input_key="Z", num_classes=10, emb_dim=C)], num_elements=10,
               num_features=C, r_max=5.0, num_bessel=8, l_max=3, num_interactions=2, correlation=3,
               avg_num_neighbors=float(edge_index.shape[0]) / n, cutoff="polynomial" if literal else "cosine",
               hidden_irreps=f"{C}x0e+{C}x1o" if literal else None)
    model = EnergyForceModel(enc, C).to(dev)
    charge_head = ChargeHead(C, hidden_dim=64).to(dev)
    pme = PMEPotential(alpha=0.3, grid=(128, 128, 128), order=6, cutoff=5.0).to(dev)
    batch = torch.zeros(n, dtype=torch.long, device=dev)
    # PME's real-space pairs: the MACE graph's half list (same 5 A minimum-image cutoff), built once
    # like the graph itself; deltas pos[i] - pos[j] - shift are the bond vectors of those edges
    half = torch.nonzero(edge_index[:, 1] > edge_index[:, 0]).squeeze(1)
    pme_nb = torch.stack([edge_index[half, 1], edge_index[half, 0]]).to(torch.int32).contiguous()
    for p in list(model.parameters()) + list(charge_head.parameters()):
        p.requires_grad_(False)
    # inference (energy + forces with a fixed model, no second derivatives): eval mode
    model.eval()
    charge_head.eval()

    def step():
        p = pos.detach().clone().requires_grad_(True)
        bond_diff = torch.ops.molix.bond_vectors(p, edge_index, shifts)
        bond_dist = bond_diff.norm(dim=-1).clamp(min=1e-6)
        feats = enc(Z=Z, bond_dist=bond_dist, bond_diff=bond_diff, edge_index=edge_index)
        pooled = model.pool(feats)
        e_mace = model.aggregate(model.energy(pooled), batch, 1)
        q = charge_head(pooled, batch=batch, num_graphs=1)["charge"]
        d = bond_diff.detach()[half]
        e = e_mace.sum() + pme(p, q, box, pairs=(pme_nb, d, bond_dist.detach()[half]))
        (f,) = torch.autograd.grad(e, p)
        return e, -f

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    E = int(edge_index.shape[0])
    # the radial MLP runs once per undirected pair (E / 2 rows); the per-edge form beside it
    nbytes = mace_step_bytes(enc, n, E, E // 2)
    nbytes_edge = mace_step_bytes(enc, n, E)
    achieved = nbytes / dt / 1e9
    roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "whole step",
            "algorithmic_bytes": nbytes, "algorithmic_bytes_mlp_per_edge": nbytes_edge,
            "frac_mlp_per_edge": round(nbytes_edge / dt / 1e9 / HBM_PEAK_GBS, 4)}
    return {"metric": "atoms/s energy+forces (MACE + PME)", "value": round(n / dt, 1), "unit": "atoms/s",
            "roofline": roof,
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
            "data": "synthetic (jittered lattice, random-init weights)",
            "config": {"workload": ("config 5: MACE literal (hidden 128x0e+128x1o, polynomial cutoff, equivariant "
                                    "product basis)" if literal else "config 5: MACE as coded 128 ch l<=3") +
                                   " x2 layers + PME 128^3 order 6, 50k atoms",
                       "atoms": n, "edges": int(edge_index.shape[0]), "channels": C,
                       "neighbor_lists": "built once outside the timed steps (MACE directed graph; PME real "
                                         "space: its half list)"}}


def train_step_bench(args, dev, steps=2, warmup=1):
    """Force-matching training step on the config-5 literal MACE (50k atoms, 2.6 M edges): energy,
    forces with create_graph (ForceDerivation in training mode), loss = E^2 + mean |F|^2, backward
    to every parameter through the second-order formulas of the molix ops."""
    from molnex_amd.molpot.pipeline import EnergyForceModel
    from molnex_amd.molrep.embedding import DiscreteEmbeddingSpec
    from molnex_amd.molzoo import MACE

    n = args.atoms
    L = (n / 0.1) ** (1.0 / 3.0)
    g = torch.Generator().manual_seed(args.seed)
    pos = lattice_positions(n, L, g).to(dev)
    Z = torch.randint(0, 10, (n,), generator=g).to(dev)
    box = torch.eye(3, device=dev) * L
    i, j, shifts, _, _ = torch.ops.molix.neighbor_list(pos, 5.0, box, True)
    edge_index = torch.stack([j.long(), i.long()], 1)
    torch.manual_seed(args.seed)
    C = args.channels
    enc = MACE(node_attr_specs=[DiscreteEmbeddingSpec(input_key="Z", num_classes=10, emb_dim=C)], num_elements=10,
               num_features=C, r_max=5.0, num_bessel=8, l_max=3, num_interactions=2, correlation=3,
               avg_num_neighbors=float(edge_index.shape[0]) / n, cutoff="polynomial",
               hidden_irreps=f"{C}x0e+{C}x1o")
    model = EnergyForceModel(enc, C).to(dev)
    model.train()
    params = [q for q in model.parameters() if q.requires_grad]

    def step():
        p = pos.detach().clone().requires_grad_(True)
        bond_diff = torch.ops.molix.bond_vectors(p, edge_index, shifts)
        feats = enc(Z=Z, bond_dist=bond_diff.norm(dim=-1).clamp(min=1e-6), bond_diff=bond_diff,
                    edge_index=edge_index)
        e = model.aggregate(model.energy(model.pool(feats)), torch.zeros(n, dtype=torch.long, device=dev), 1)
        f = model.forces(e, p)
        loss = (e ** 2).sum() + (f ** 2).sum(-1).mean()
        for q in params:
            q.grad = None
        loss.backward()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return {"workload": "config 5 literal MACE, force-matching training step (energy + forces with create_graph, "
                        "loss backward to all parameters), 50k atoms", "ms_per_step": round(dt * 1e3, 3),
            "atoms_per_s": round(n / dt, 1), "edges": int(edge_index.shape[0])}


def nlist_bench(dev, reps=10, warmup=3):
    """directed cell list of 100k atoms in a periodic 100 A cube, rc 5 A.
    Times the whole op (bin, count, scan, host read of the count, emit) after warm-up calls
    (the caching allocator holds the outputs' blocks by then)."""
    g = torch.Generator().manual_seed(2)
    L = 100.0
    pos = (torch.rand((100_000, 3), generator=g) * L).to(dev)
    box = torch.eye(3, device=dev) * L
    for _ in range(warmup):
        out = torch.ops.molix.neighbor_list(pos, 5.0, box, True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        out = torch.ops.molix.neighbor_list(pos, 5.0, box, True)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    E = out[0].shape[0]
    return {"workload": "config 2: 100k atoms, periodic 100 A cube, rc 5 A, directed pairs + shifts",
            "pairs": E, "ms": round(dt * 1e3, 3), "M_pairs_per_s": round(E / dt / 1e6, 1)}


def tp_gh_bench(dev, reps=5):
    """The config-3 tensor-product backward in its two forms, event-timed on the same inputs:
    unfused -- molix::tp_scatter_backward writing the per-edge weight gradient gw (E x 23*128),
    then the output layer's input gradient gw W (molix::edge_weights backward, K 64) -- and fused,
    molix::tp_scatter_backward_gh (gw staged in LDS and multiplied on the matrix cores, never
    written)."""
    import molnex_amd.kernels as K

    torch.manual_seed(0)
    pos, box, ei, vec, L = make_system(50_000, 0, True, dev)
    N, E, C, Kh = pos.shape[0], ei.shape[0], 128, 64
    ls = [0, 1, 2, 3]
    cfg = K.tp_config_id(ls, ls, ls)
    P, NX, NY, NO = K.tp_config_info(cfg)
    row_ptr, perm, snd = torch.ops.molix.edge_csr(ei, N)
    Y = torch.ops.molix.spherical_harmonics(vec, 3)
    x = torch.randn(N, NX * C, device=dev)
    w = torch.randn(E, P * C, device=dev)
    W = torch.randn(P * C, Kh, device=dev) / Kh ** 0.5
    g = torch.randn(N, NO * C, device=dev)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(reps + 1)]
    for i in range(reps + 1):
        e = ev[i]
        e[0].record()
        _, _, gw = K.tp_scatter_backward(g, x, Y, w, row_ptr, perm, snd, cfg, C, True, True, True)
        e[1].record()
        K.edge_weights_backward(gw, W)
        e[2].record()
        del gw
        K.tp_scatter_backward_gh(g, x, Y, w, row_ptr, perm, snd, None, W, cfg, C, True, True)
        e[3].record()
    torch.cuda.synchronize()
    tb = sum(e[0].elapsed_time(e[1]) for e in ev[1:]) / reps
    te = sum(e[1].elapsed_time(e[2]) for e in ev[1:]) / reps
    tf = sum(e[2].elapsed_time(e[3]) for e in ev[1:]) / reps
    return {"workload": "config 3 TP backward (50k atoms, 2.6 M edges, 128 x (0e+1o+2e+3o), K 64), "
                        "fused with the output layer's input gradient vs unfused",
            "edges": E, "unfused_tp_bwd_ms": round(tb, 3), "unfused_edge_weights_bwd_ms": round(te, 3),
            "unfused_ms": round(tb + te, 3), "fused_ms": round(tf, 3)}


def sc_flops(l_in=3, l_out=1, nu=3):
    """FLOPs per (node, channel) of the generated symmetric-contraction code, each distinct
    pair product A_i A_j counted once (the compiler shares them between monomials and
    product-rule terms): forward = monomials + one FMA per basis coefficient + the weight
    mix; backward (both gradients) = monomials + per (monomial, path) h = coef . g, the
    grad_W and grad-monomial FMAs + the product-rule FMAs."""
    from molnex_amd.csrc.gen_sc import Cfg, config_list

    c = Cfg(config_list().index((l_in, l_out, nu)), l_in, l_out, nu)
    pairs = {m[:2] for m, _ in c.terms if len(m) >= 2} | {m[1:] for m, _ in c.terms if len(m) == 3} | \
        {(m[0], m[2]) for m, _ in c.terms if len(m) == 3}
    monos = len(pairs) + sum(1 for m, _ in c.terms if len(m) == 3)
    accs = {(p, M) for _, ts in c.terms for p, M, _ in ts}
    fwd = monos + 2 * c.nnz + 2 * len(accs)
    bwd = monos
    for mono, ts in c.terms:
        per_path = {}
        for p, _, _ in ts:
            per_path[p] = per_path.get(p, 0) + 1
        bwd += sum(2 * t - 1 + 4 for t in per_path.values())
        for x in set(mono):
            bwd += 1 if len(mono) == 1 else 2 + (1 if mono.count(x) > 1 else 0)
    return fwd, bwd


def sc_bench(dev, reps=10):
    """equivariant symmetric contraction of 50k nodes, 128 x (0e+1o+2e+3o)
    -> 128 x (0e+1o), correlation 3, 10 elements, then the 128 -> 128 channel mixing per (l, m);
    forward and backward (grad wrt A and both weights).  Kernel times by HIP events."""
    from molnex_amd import kernels as K
    from molnex_amd.molrep.interaction import EquivariantSymmetricContraction, Linear

    g = torch.Generator().manual_seed(4)
    N, C, S = 50_000, 128, 10
    A = torch.randn((N, 16 * C), generator=g).to(dev).requires_grad_(True)
    z = torch.randint(0, S, (N,), generator=g).to(dev)
    torch.manual_seed(4)
    sc = EquivariantSymmetricContraction(f"{C}x0e+{C}x1o+{C}x2e+{C}x3o", f"{C}x0e+{C}x1o", 3, S).to(dev)
    with torch.no_grad():
        sc.weight.mul_(0.1)
    mix = Linear(f"{C}x0e+{C}x1o", f"{C}x0e+{C}x1o").to(dev)
    gout = torch.randn((N, 4 * C), generator=g).to(dev)

    params = [A, *sc.parameters(), *mix.parameters()]

    def step():
        for p in params:  # a training step's zero_grad(set_to_none=True): no accumulation adds
            p.grad = None
        out = mix(sc(A, z))
        out.backward(gout)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / reps
    # the two contraction kernels alone
    with torch.no_grad():
        B = sc(A, z)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    tf = tb = 0.0
    for _ in range(reps):
        ev[0].record()
        torch.ops.molix.symmetric_contraction(A.detach(), z, sc.weight.detach(), 3, 1, 3)
        ev[1].record()
        K.symmetric_contraction_backward(gout, A.detach(), z, sc.weight.detach(), 3, 1, 3, True, True)
        ev[3].record()
        torch.cuda.synchronize()
        tf += ev[0].elapsed_time(ev[1])
        tb += ev[1].elapsed_time(ev[3])
    tf, tb = tf / reps, tb / reps  # ms (the backward figure includes the element argsort)
    ff, fb = sc_flops()
    fwd_bytes = 4 * N * (16 * C + 4 * C) + 8 * N
    return {"workload": "config 4: symmetric contraction 50k nodes, 128 x (0e+1o+2e+3o) -> 128 x (0e+1o), "
                        "correlation 3, 10 elements, + 128->128 mixing; fwd + bwd",
            "ms_per_step": round(dt * 1e3, 3), "nodes_per_s": round(N / dt, 1), "B_finite": bool(torch.isfinite(B).all()),
            "sc_fwd_ms": round(tf, 4), "sc_bwd_ms": round(tb, 4),
            "sc_fwd_TFLOPs": round(ff * N * C / (tf * 1e-3) / 1e12, 2),
            "sc_bwd_TFLOPs": round(fb * N * C / (tb * 1e-3) / 1e12, 2),
            "sc_fwd_GBs": round(fwd_bytes / (tf * 1e-3) / 1e9, 1),
            "flops_per_node_channel": {"fwd": ff, "bwd": fb}}


def allegro_bench(args, dev, steps=5, warmup=2, reps=5):
    """Allegro encoder (src/molzoo/allegro.py, reference defaults: 64 scalar / 16 tensor channels,
    l_max 2, 2 layers) on the config-3/5 graph (50k atoms, periodic, rc 5 A): edge features, a
    fixed linear readout summed to an energy, forces by one backward to the positions.  Also the
    molix::edge_tp_proj kernels (the layer's product fused with its projection, which the frozen
    encoder runs) at the layer's shape, HIP events on the current stream; algorithmic bytes per
    edge forward 4 (NX + NI) C + 4 NY, backward 4 (2 NX + NI) C + 8 NY (x, Y, projected out / grad
    once; NI = 9 projected components at l_max 2)."""
    import molnex_amd.kernels as K
    from molnex_amd.molzoo.allegro import Allegro

    n = args.atoms
    L = (n / 0.1) ** (1.0 / 3.0)
    g = torch.Generator().manual_seed(args.seed)
    pos = lattice_positions(n, L, g).to(dev)
    Z = torch.randint(0, 10, (n,), generator=g).to(dev)
    box = torch.eye(3, device=dev) * L
    i, j, shifts, _, _ = torch.ops.molix.neighbor_list(pos, 5.0, box, True)
    edge_index = torch.stack([j.long(), i.long()], 1)
    E = int(edge_index.shape[0])
    torch.manual_seed(args.seed)
    enc = Allegro(num_elements=10, num_scalar_features=64, num_tensor_features=16, r_max=5.0, l_max=2,
                  num_layers=2, avg_num_neighbors=E / n).to(dev)
    for p in enc.parameters():
        p.requires_grad_(False)
    readout = torch.randn(2, 64, device=dev) / 8

    def step():
        p = pos.detach().clone().requires_grad_(True)
        bond_diff = torch.ops.molix.bond_vectors(p, edge_index, shifts)
        bond_dist = bond_diff.norm(dim=-1).clamp(min=1e-6)
        feats = enc(Z=Z, bond_dist=bond_dist, bond_diff=bond_diff, edge_index=edge_index)
        e = (feats * readout).sum()
        (f,) = torch.autograd.grad(e, p)
        return e, -f

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        e, f = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    finite = bool(torch.isfinite(f).all())
    layer = enc.layers[0]
    tp = layer.tp
    P, NX, NY, NO = K.tp_config_info(tp.config_id)
    C = tp.channels
    blocks = K.edge_tp_proj_blocks(tp.config_id)
    NI = sum(2 * l + 1 for l, _, _, _ in blocks)
    x = torch.randn(E, NX * C, device=dev)
    Y = torch.randn(E, NY, device=dev)
    w = torch.randn(P, C, device=dev)
    proj = layer.tp_linear.weight.reshape(-1, C) * layer._proj_scale
    gout = torch.randn(E, NI * C, device=dev)
    fwd, bwd = [], []
    for r in range(reps + 1):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        ev[0].record()
        K.edge_tp_proj(x, Y, w, tp.config_id, proj)
        ev[1].record()
        ev[2].record()
        K.edge_tp_proj_backward(gout, x, Y, w, tp.config_id, proj, True, True, True)
        ev[3].record()
        if r:
            fwd.append(ev[:2])
            bwd.append(ev[2:])
    torch.cuda.synchronize()
    tf = sum(a.elapsed_time(b) for a, b in fwd) / reps
    tb = sum(a.elapsed_time(b) for a, b in bwd) / reps
    bf = E * (4 * (NX + NI) * C + 4 * NY)
    bb = E * (4 * (2 * NX + NI) * C + 8 * NY)
    return {"workload": "Allegro (64 scalar / 16 tensor ch, l_max 2, 2 layers) on 50k atoms, rc 5 A, energy + forces",
            "edges": E, "ms_per_step": round(dt * 1e3, 3), "M_edges_per_s": round(E / dt / 1e6, 2),
            "forces_finite": finite, "edge_tp_proj_fwd_ms": round(tf, 3), "edge_tp_proj_bwd_ms": round(tb, 3),
            "edge_tp_proj_fwd_GBs": round(bf / tf / 1e6, 1), "edge_tp_proj_bwd_GBs": round(bb / tb / 1e6, 1),
            "edge_tp_proj_fwd_hbm_frac": round(bf / tf / 1e6 / HBM_PEAK_GBS, 4),
            "edge_tp_proj_bwd_hbm_frac": round(bb / tb / 1e6 / HBM_PEAK_GBS, 4)}


def unsorted_bench(args, dev, steps=3, warmup=2):
    """The headline step with the atoms left in random order (no spatial sort): the reference's data
    path (collate.py:65-177) does not reorder atoms, so sender gathers then hit random rows."""
    pos, box, edge_index, vec, L = make_system(args.atoms, args.seed, False, dev)
    N, E = pos.shape[0], edge_index.shape[0]
    step = EdgeStep(N, edge_index, vec, args.channels, args.seed, dev)
    for _ in range(warmup):
        step.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step.step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    tf, tb = time_tp_kernels(step, reps=3)
    return {"workload": "config 3 with atoms in random order", "edges": E, "ms_per_step": round(dt * 1e3, 3),
            "M_edges_per_s": round(E / dt / 1e6, 2), "tp_scatter_fwd_ms": round(tf, 3),
            "tp_scatter_bwd_ms": round(tb, 3)}


def secondary_figures(args, dev):
    out = {"config3_unsorted_atoms": unsorted_bench(args, dev)}
    torch.cuda.empty_cache()
    sc = sc_bench(dev)
    nl = nlist_bench(dev)
    out.update({"config2_neighbor_list": nl, "config4_symmetric_contraction": sc,
                "config5_pme_term": pme_bench(dev)})
    for key, lit in (("config5_energy_forces", False), ("config5_literal_energy_forces", True)):
        sub = argparse.Namespace(**{**vars(args), "steps": 3, "warmup": 2, "literal": lit})
        full = full_step_bench(sub, dev)
        out[key] = {"atoms_per_s": full["value"], "ms_per_step": full["ms_per_step"],
                    "workload": full["config"]["workload"], "edges": full["config"]["edges"],
                    "hbm_frac": full["roofline"]["frac"], "algorithmic_GB": round(full["roofline"]["algorithmic_bytes"] / 1e9, 2),
                    "hbm_frac_mlp_per_edge": full["roofline"]["frac_mlp_per_edge"],
                    "algorithmic_GB_mlp_per_edge": round(full["roofline"]["algorithmic_bytes_mlp_per_edge"] / 1e9, 2)}
        torch.cuda.empty_cache()
    out["config5_literal_training_step"] = train_step_bench(args, dev)
    torch.cuda.empty_cache()
    out["allegro_energy_forces"] = allegro_bench(args, dev)
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus > 1 is not supported (the path would "
                                   "shard by space: owned atoms plus a halo of rc x interactions per GPU)"}))
        sys.exit(2)
    if args.workload == "full":
        dev = torch.device("cuda:0")
        print(json.dumps(full_step_bench(args, dev)), flush=True)
        return
    if args.workload == "train":
        dev = torch.device("cuda:0")
        out = train_step_bench(args, dev, steps=args.steps, warmup=args.warmup)
        out["peak_GB"] = round(torch.cuda.max_memory_allocated() / 1e9, 1)
        print(json.dumps(out), flush=True)
        return
    if args.workload == "allegro":
        print(json.dumps(allegro_bench(args, torch.device("cuda:0"), steps=args.steps, warmup=args.warmup)),
              flush=True)
        return
    if args.workload in ("sc", "nl", "pme", "tpgh"):
        import molnex_amd.kernels  # noqa: F401

        fn = {"sc": sc_bench, "nl": nlist_bench, "pme": pme_bench, "tpgh": tp_gh_bench}[args.workload]
        print(json.dumps(fn(torch.device("cuda:0"))), flush=True)
        return
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    pos, box, edge_index, vec, L = make_system(args.atoms, args.seed, not args.unsorted, dev)
    N, E = pos.shape[0], edge_index.shape[0]
    step = EdgeStep(N, edge_index, vec, args.channels, args.seed, dev)
    if args.kernels_only:
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        tf, tb = time_tp_kernels(step, reps=3)
        print(json.dumps({"copy_bytes": 2 * src.numel() * 4, "tp_fwd_ms": tf, "tp_bwd_ms": tb, "edges": E}))
        return
    for _ in range(args.warmup):
        step.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step.step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt / args.steps * 1e3
    value = E * args.steps / dt / 1e6

    tf, tb = time_tp_kernels(step)
    ewf, ewb, ewf_bytes, ewb_bytes = time_edge_weight_kernels(step)
    step_paired = step.paired
    bf, bb = tp_bytes(N, E, args.channels)
    dom_t, dom_b, dom_name = (tb, bb, "tp_scatter_bwd") if tb >= tf else (tf, bf, "tp_scatter_fwd")
    achieved = dom_b / (dom_t * 1e-3) / 1e9
    traffic = measured_traffic(dom_name) if args.channels == 128 and args.atoms == 50_000 else None
    roof = {
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": dom_name,
        "kernel_ms": round(dom_t, 3), "algorithmic_bytes": dom_b,
        "other": {"tp_scatter_fwd_ms": round(tf, 3), "tp_scatter_fwd_GBs": round(bf / (tf * 1e-3) / 1e9, 1),
                  "tp_scatter_bwd_ms": round(tb, 3), "tp_scatter_bwd_GBs": round(bb / (tb * 1e-3) / 1e9, 1),
                  "edge_weights_fwd_ms": round(ewf, 3), "edge_weights_fwd_GBs": round(ewf_bytes / (ewf * 1e-3) / 1e9, 1),
                  "edge_weights_bwd_ms": round(ewb, 3), "edge_weights_bwd_GBs": round(ewb_bytes / (ewb * 1e-3) / 1e9, 1)},
    }
    secondary = None
    if not args.no_secondary:
        del step
        torch.cuda.empty_cache()
        secondary = secondary_figures(args, dev)
    cpu = None
    if not args.no_cpu_baseline:
        step = EdgeStep(N, edge_index, vec, args.channels, args.seed, dev)
        cpu = cpu_baseline(edge_index, step.vec, step.x, args.channels, step.mlp, step.mu, step.sigma, step.gout)
    line = {
        "metric": "M edges/s TP+scatter (fwd+bwd wrt node features and edge vectors)",
        "value": round(value, 3),
        "unit": "M edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded uniform periodic box, random-init MLP weights, N(0,1) node features)",
        "config": {"workload": "config 3: edge TP + scatter, 50k atoms, rc 5 A, 128 ch, l<=3, fwd+bwd",
                   "atoms": N, "edges": E, "channels": args.channels, "box_A": round(L, 3),
                   "spatially_sorted": not args.unsorted,
                   "radial_output_layer": ("once per undirected pair (both directions have the same distance, "
                                           "hence the same weights; per-edge gradients)" if step_paired
                                           else "per directed edge"),
                   "graph": "receiver CSR and edge pairing built on the graph's first step and kept"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
