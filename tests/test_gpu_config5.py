"""BASELINE config 5 on the HIP path: MACE (128 channels, the literal and the as-coded
variants) + ChargeHead (per-system neutral charges) + PMEPotential (direct + reciprocal - self),
energy and forces.

(i)  a small periodic system against the fp64 composition ``oracle.config5_ref`` (1e-5);
(ii) the full 50k-atom, 128^3 system through size-independent properties: finite results,
     zero net charge, translation invariance, and forces against central differences of the
     energy at sampled atoms."""

import math

import numpy as np
import pytest
import torch

from oracle import config5_ref
from oracle import nlist as NL
from oracle import pme as P

pytestmark = pytest.mark.gpu
DEV = "cuda"
ALPHA, ORDER, RC = 0.3, 6, 5.0


def lattice(n: int, seed: int):
    """Jittered cubic lattice at 0.1 atoms/A^3 in a periodic cube (pairs >= 0.9 A apart), atoms in
    spatial cell order; fp32 positions."""
    L = (n / 0.1) ** (1.0 / 3.0)
    rng = np.random.default_rng(seed)
    k = math.ceil(n ** (1 / 3))
    sites = np.stack(np.meshgrid(*[np.arange(k)] * 3, indexing="ij"), -1).reshape(-1, 3).astype(np.float64)
    sites = sites[rng.permutation(len(sites))[:n]]
    a = L / k
    pos = (sites + 0.5) * a + (rng.uniform(size=(n, 3)) - 0.5) * (a - 0.9)
    cell = np.minimum(np.floor(pos / (L / 8)).astype(np.int64), 7)
    pos = pos[np.argsort((cell[:, 2] * 8 + cell[:, 1]) * 8 + cell[:, 0], kind="stable")]
    return pos.astype(np.float32), L


def image_shifts(pos, i, j, deltas, L):
    """Image offset of j per pair: deltas = pos[i] - (pos[j] + shift), shift a multiple of L per axis."""
    p = pos.astype(np.float64)
    return L * np.rint((p[i] - p[j] - deltas.astype(np.float64)) / L)


def build_models(n_elem, C, literal, avg_nbrs, seed=0):
    from molnex_amd.molpot import ChargeHead
    from molnex_amd.molpot.pipeline import EnergyForceModel
    from molnex_amd.molrep.embedding import DiscreteEmbeddingSpec
    from molnex_amd.molzoo import MACE

    torch.manual_seed(seed)
    enc = MACE(node_attr_specs=[DiscreteEmbeddingSpec(input_key="Z", num_classes=n_elem, emb_dim=C)],
               num_elements=n_elem, num_features=C, r_max=RC, num_bessel=8, l_max=3, num_interactions=2,
               correlation=3, avg_num_neighbors=avg_nbrs, cutoff="polynomial" if literal else "cosine",
               hidden_irreps=f"{C}x0e+{C}x1o" if literal else None)
    model = EnergyForceModel(enc, C).to(DEV)
    head = ChargeHead(C, hidden_dim=64).to(DEV)
    for p in list(model.parameters()) + list(head.parameters()):
        p.requires_grad_(False)
    return model, head


class System:
    """One periodic system on the GPU with a fixed directed edge list (MACE) and a fixed half
    pair list (PME real space), both with image shifts, so the energy is a smooth function of
    the positions for finite differences."""

    def __init__(self, pos, L, Z, model, head, pme):
        self.L = L
        self.box = torch.eye(3, device=DEV) * L
        p = torch.tensor(pos, device=DEV)
        i, j, sh, _, _ = torch.ops.molix.neighbor_list(p, RC, self.box, True)
        self.edge_index = torch.stack([j.long(), i.long()], 1)
        self.shifts = sh
        hi, hj, hsh, _, _ = torch.ops.molix.neighbor_list(p, RC, self.box, False)
        self.half = (torch.stack([hi, hj]), hsh)
        self.Z = torch.tensor(Z, device=DEV)
        self.batch = torch.zeros(len(Z), dtype=torch.long, device=DEV)
        self.model, self.head, self.pme = model, head, pme

    def parts(self, p, dtype_pme=torch.float32):
        """(per-atom MACE energies, charges, PME energy) at positions p (fp32, may require grad)."""
        ops = torch.ops.molix
        bond = ops.bond_vectors(p, self.edge_index, self.shifts)
        enc = self.model.encoder
        feats = enc(Z=self.Z, bond_dist=bond.norm(dim=-1).clamp(min=1e-6), bond_diff=bond,
                    edge_index=self.edge_index)
        pooled = self.model.pool(feats)
        e_atoms = self.model.energy(pooled)
        q = self.head(pooled, batch=self.batch, num_graphs=1)["charge"]
        nb, hsh = self.half
        pp = p.to(dtype_pme)
        d = (pp[nb[0].long()] - pp[nb[1].long()] - hsh.to(dtype_pme)).detach()
        e_pme = self.pme(pp, q.to(dtype_pme), self.box.to(dtype_pme), pairs=(nb, d, d.norm(dim=-1)))
        return e_atoms, q, e_pme

    def energy_forces(self, pos_t):
        p = pos_t.detach().clone().requires_grad_(True)
        e_atoms, q, e_pme = self.parts(p)
        e = self.model.aggregate(e_atoms, self.batch, 1).sum() + e_pme
        (g,) = torch.autograd.grad(e, p)
        return e.detach(), -g, q.detach(), e_atoms.detach(), e_pme.detach()


def _stats(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    rms = np.sqrt(np.mean(b * b))
    return np.linalg.norm(a - b) / np.linalg.norm(b), np.abs(a - b).max() / rms


@pytest.mark.parametrize("literal", [True, False], ids=["literal", "as_coded"])
def test_config5_small_system_vs_fp64_oracle(literal):
    """~400 atoms at the config-5 density, 128 channels, 10 elements, PME alpha 0.3 / order 6 /
    rc 5 A on a 32^3 mesh: energy and forces against the fp64 composition (1e-5)."""
    from molnex_amd.molpot import PMEPotential

    n, C = 400, 128
    pos, L = lattice(n, seed=3)
    Z = np.random.default_rng(4).integers(0, 10, n)
    grid = (32, 32, 32)
    ii, jj, dd, _ = NL.directed_pairs(pos, RC, np.eye(3, dtype=np.float32) * np.float32(L))
    model, head = build_models(10, C, literal, avg_nbrs=len(ii) / n)
    pme = PMEPotential(alpha=ALPHA, grid=grid, order=ORDER, cutoff=RC).to(DEV)
    sysm = System(pos, L, Z, model, head, pme)
    # the GPU neighbor lists are the oracle's, bit for bit (checked elsewhere): reuse their order
    assert np.array_equal(sysm.edge_index[:, 1].cpu().numpy(), ii) and np.array_equal(
        sysm.edge_index[:, 0].cpu().numpy(), jj)
    e, f, q, e_atoms, e_pme = sysm.energy_forces(torch.tensor(pos, device=DEV))

    sd_model = {k.removeprefix("encoder."): v for k, v in model.state_dict().items()}
    edge_shifts = image_shifts(pos, ii, jj, dd, L)
    rows, cols, hd, _ = NL.half_pairs(pos, RC, np.eye(3, dtype=np.float32) * np.float32(L))
    half_shifts = image_shifts(pos, rows, cols, hd, L)
    cfg = dict(num_features=C, num_interactions=2, l_max=3, correlation=3, r_max=RC, num_bessel=8,
               avg_num_neighbors=len(ii) / n, cutoff="polynomial" if literal else "cosine")
    if literal:
        cfg["hidden_ls"] = [0, 1]
    re, rf, rq, re_mace, re_pme = config5_ref.energy_forces(
        sd_model, head.state_dict(), cfg, torch.tensor(Z), torch.tensor(pos, dtype=torch.float64),
        torch.tensor(np.stack([jj, ii], 1).astype(np.int64)), edge_shifts, torch.zeros(n, dtype=torch.long), 1,
        np.eye(3) * L, (rows, cols, half_shifts), grid, ORDER, ALPHA, 14.399645478425668)
    rel_e = abs(e.item() - re.sum().item()) / abs(re.sum().item())
    rel_mace = abs(e_atoms.double().sum().item() - re_mace.sum().item()) / abs(re_mace.sum().item())
    rel_pme = abs(e_pme.item() - re_pme.item()) / abs(re_pme.item())
    # The charges are raw - mean(raw) per graph (heads.py:158-171); with random-init weights the raw
    # charges are much larger than their spread, so an fp32 evaluation carries the rounding of
    # raw: their error is measured against the raw charges' scale.  The PME term is then checked on
    # its own arithmetic: the oracle's PME of the GPU's charges.
    raw_rms = _raw_charge_rms(head, sysm, torch.tensor(pos, device=DEV))
    dq = (q.double().cpu() - rq).numpy()
    q_norm = np.linalg.norm(dq) / (raw_rms * np.sqrt(n))
    q_max = np.abs(dq).max() / raw_rms
    pme_own = config5_ref._PMEEnergy.apply(
        torch.tensor(pos, dtype=torch.float64), q.double().cpu(),
        config5_ref.half_pair_geometry(torch.tensor(pos, dtype=torch.float64), rows, cols, half_shifts),
        np.eye(3) * L, grid, ORDER, ALPHA, 14.399645478425668,
        [P.bspline_moduli(g, ORDER) for g in grid]).item()
    rel_pme = abs(e_pme.item() - pme_own) / abs(pme_own)
    f_norm, f_max = _stats(f.cpu(), rf)
    print(f"config 5 small ({'literal' if literal else 'as coded'}): E {re.sum().item():.6g} (MACE "
          f"{re_mace.sum().item():.6g}, PME {re_pme.item():.6g}); rel err E {rel_e:.2e} MACE {rel_mace:.2e} "
          f"PME of the same charges {rel_pme:.2e}; charges {q_norm:.2e} (max {q_max:.2e}) of the raw charges' "
          f"RMS {raw_rms:.3g} (|q| RMS {q.pow(2).mean().sqrt().item():.3g}); forces {f_norm:.2e} (max {f_max:.2e} RMS)")
    assert rel_e <= 1e-5 and rel_mace <= 1e-5 and rel_pme <= 1e-5
    assert q_norm <= 1e-5 and q_max <= 1e-5
    assert f_norm <= 1e-5 and f_max <= 1e-5
    # neutrality up to the fp32 rounding of the per-graph sum of the raw charges
    assert abs(q.double().sum().item()) <= 1e-5 * raw_rms * n


def _raw_charge_rms(head, sysm, p):
    """RMS of the charge MLP's raw output (before the per-graph shift)."""
    with torch.no_grad():
        bond = torch.ops.molix.bond_vectors(p, sysm.edge_index, sysm.shifts)
        feats = sysm.model.encoder(Z=sysm.Z, bond_dist=bond.norm(dim=-1).clamp(min=1e-6), bond_diff=bond,
                                   edge_index=sysm.edge_index)
        raw = head.mlp(sysm.model.pool(feats)).squeeze(-1)
    return raw.double().pow(2).mean().sqrt().item()


@pytest.mark.parametrize("literal", [True], ids=["literal"])
def test_config5_full_size_properties(literal):
    """50,000 atoms, 128 channels, 10 elements, PME 128^3 order 6: finite energy, forces and
    charges; zero net charge; the MACE energy is translation invariant; forces match central
    differences of the energy at sampled atoms.  Differences take the per-atom MACE energies
    (fp32) summed in fp64 and the PME energy in fp64 with the same charges, so the difference
    quotient is not lost in the rounding of a 50k-atom fp32 sum."""
    from molnex_amd.molpot import PMEPotential

    n, C = 50_000, 128
    pos, L = lattice(n, seed=0)
    Z = np.random.default_rng(1).integers(0, 10, n)
    model, head = build_models(10, C, literal, avg_nbrs=52.0)
    pme = PMEPotential(alpha=ALPHA, grid=(128, 128, 128), order=ORDER, cutoff=RC).to(DEV)
    sysm = System(pos, L, Z, model, head, pme)
    p0 = torch.tensor(pos, device=DEV)
    e, f, q, e_atoms, e_pme = sysm.energy_forces(p0)
    assert torch.isfinite(e) and torch.isfinite(f).all() and torch.isfinite(q).all()
    net = abs(q.double().sum().item())
    print(f"config 5 full: E {e.item():.6g} (PME {e_pme.item():.6g}), |F| rms {f.pow(2).mean().sqrt().item():.3g}, "
          f"net charge {net:.2e} of sum|q| {q.abs().sum().item():.3g}")
    assert net <= 1e-5 * q.abs().sum().item()

    # translation by a non-lattice vector: per-atom MACE energies unchanged
    t = torch.tensor([0.37, -1.21, 2.05], device=DEV)
    with torch.no_grad():
        e_atoms_t, q_t, _ = sysm.parts(p0 + t)
    d_e = (e_atoms_t - e_atoms).abs().max().item()
    d_q = (q_t - q).abs().max().item()
    print(f"translation: max |de_atom| {d_e:.2e} (max |e_atom| {e_atoms.abs().max().item():.3g}), "
          f"max |dq| {d_q:.2e}")
    assert d_e <= 1e-5 * e_atoms.abs().max().item() and d_q <= 1e-5 * q.abs().max().item()

    # central differences (4-point stencil, truncation O(h^4)) at 10 sampled atoms, 3 axes each,
    # and along a random +-1 direction of every atom.  Random-init weights give small forces (RMS
    # ~3e-4 eV/A) against per-atom energies ~1e-2 eV whose fp32 rounding (~1e-9 eV each) is the
    # noise floor: h = 0.05 A keeps it ~0.3 % for a single atom (a displacement that moves ~6 of
    # its 52 edges across the C^2 polynomial cutoff, a smaller error still); along the global
    # direction h = 4e-3 A per atom sums ~sqrt(N) force components against ~sqrt(N) roundings --
    # including the fp32 rounding of every displaced coordinate (ulp 7.6e-6 A at 80 A, up to 0.4 %
    # of a 1e-3 A step, which put that check's noise near 1 %).
    nb, hsh = sysm.half

    def energy(p):
        ea, qq, _ = sysm.parts(p)
        pd = p.double()
        d = pd[nb[0].long()] - pd[nb[1].long()] - hsh.double()
        ep = sysm.pme(pd, qq.double(), sysm.box.double(), pairs=(nb, d, d.norm(dim=-1)))
        return ea.double().sum().item() + ep.item()

    def stencil(direction, h):
        with torch.no_grad():
            v = [energy(p0 + k * h * direction) for k in (1, -1, 2, -2)]
        return -(8 * (v[0] - v[1]) - (v[2] - v[3])) / (12 * h)

    rng = np.random.default_rng(2)
    atoms = rng.choice(n, 10, replace=False)
    fd = np.zeros((10, 3))
    for a_i, a in enumerate(atoms):
        for ax in range(3):
            u = torch.zeros_like(p0)
            u[a, ax] = 1.0
            fd[a_i, ax] = stencil(u, 5e-2)
    fa = f[torch.tensor(atoms, device=DEV)].double().cpu().numpy()
    rel = np.linalg.norm(fa - fd) / np.linalg.norm(fd)
    u = torch.randint(0, 2, p0.shape, generator=torch.Generator(device=DEV).manual_seed(5), device=DEV) * 2.0 - 1.0
    fu = stencil(u, 4e-3)
    ref_u = (f.double() * u.double()).sum().item()
    rel_u = abs(fu - ref_u) / abs(ref_u)
    print(f"finite differences at {len(atoms)} atoms: rel err {rel:.2e} (|F| {np.linalg.norm(fd):.3g}); "
          f"along a random +-1 direction of all atoms: {fu:.6g} vs F.u {ref_u:.6g}, rel err {rel_u:.2e}")
    assert rel <= 1e-2 and rel_u <= 1e-2


@pytest.mark.parametrize("literal", [True, False], ids=["literal", "as_coded"])
def test_energy_forces_step_has_no_host_sync(literal):
    """A whole MACE + ChargeHead + PME energy + forces step at new positions on a known graph, with
    the graph count given and the first step's edge pairing trusted (config.verify_pairs = False),
    enqueues without a device-to-host copy or synchronisation (torch's sync debug mode raises on
    one); its energy and forces agree with the same step under the per-step pairing check."""
    from molnex_amd.config import config
    from molnex_amd.molpot import PMEPotential

    n, C = 400, 32
    pos, L = lattice(n, seed=5)
    Z = np.random.default_rng(6).integers(0, 10, n)
    model, head = build_models(10, C, literal, 30.0, seed=1)
    pme = PMEPotential(alpha=ALPHA, grid=(32, 32, 32), order=ORDER, cutoff=RC).to(DEV)
    system = System(pos, L, Z, model, head, pme)
    pos_t = torch.tensor(pos, device=DEV)
    moved = pos_t + 0.01 * torch.randn(pos_t.shape, generator=torch.Generator(device=DEV).manual_seed(7),
                                       device=DEV)
    prev = config.verify_pairs
    try:
        config.verify_pairs = False
        system.energy_forces(pos_t)  # first step on the graph: CSR, pairing, lazy buffers
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            e, f, *_ = system.energy_forces(moved)
        finally:
            torch.cuda.set_sync_debug_mode(0)
        config.verify_pairs = True
        e2, f2, *_ = system.energy_forces(moved.clone())
    finally:
        config.verify_pairs = prev
    assert torch.isfinite(f).all()
    assert abs(float(e) - float(e2)) <= 1e-6 * abs(float(e2))
    assert float((f - f2).norm() / f2.norm()) <= 1e-6
