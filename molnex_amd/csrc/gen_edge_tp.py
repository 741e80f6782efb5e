"""Generates edge_tp_gen.inc: the per-edge channelwise tensor product with shared
weights (no scatter) of Allegro's layers, forward and backward, one kernel per
configuration and channel width.

    out[e][row(p, m3)][c] = w[p][c] * sum_{m1, m2} cf_p[m1][m2][m3] x[e][o1 + m1][c] Y[e][o2 + m2]

with the rows of the paths that share an output irrep interleaved (out_row below)

(src/molzoo/allegro.py:352-359 builds it as cuet.ChannelWiseTensorProduct(irreps_in,
sh_irreps, shared_weights=True); :457-458 applies it to the pre-scaled edge features
and the aggregated neighbourhood harmonics of each edge's source).  Only the paths
whose output irrep appears in irreps_in are computed: the projection that follows
(:363-367, cuet.Linear(tp.irreps_out, irreps_in)) connects nothing else.

An optional per-edge, per-channel scale xs[e][c] multiplies x first (Allegro's env weights,
allegro.py:447-450: TP(s x) = s TP(x) channel by channel); its gradient is
sum_m1 grad_(s x)[m1] x[m1] per edge and channel.

Lane layout: a wavefront holds 64 / CW edges side by side, CW = min(C, 64) lanes
per edge, one channel per lane (CPL = 2 channels per lane for C = 128), so small
channel counts (Allegro's default is 16) still fill the wave.  Backward per lane
and channel: v_p[m1][m2] = sum_m3 cf g[row(p, m3)] (g the output gradient), then
grad_x[m1] = sum_p w_p sum_m2 Y[m2] v_p[m1][m2] (stored once: x is per edge),
grad_Y[m2] = sum_c sum_p w_p sum_m1 x[m1] v_p[m1][m2] (reduced over the CW lanes of
the edge by xor shuffles), grad_w[p][c] = sum_e sum_m1 x[m1] (sum_m2 Y v)[m1]
accumulated in registers over the edges a wavefront walks, reduced over its edge
slots and written as one partial per wavefront (summed in a fixed order by a
second kernel).
"""

from __future__ import annotations

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from molnex_amd.csrc.gen_tp import EPS, Cfg, config_list, f32  # noqa: E402

# (channels per edge slot, channels per lane): C = CW * CPL
VARIANTS = ((8, 1), (16, 1), (32, 1), (64, 1), (64, 2))


def out_row(cfg: Cfg):
    """Output row of (path k, m3).  The paths sharing an output irrep form one block of
    multiplicity (paths x C), irrep component outermost: row = first row of the irrep's rows
    + m3 * (paths of that irrep) + the path's rank among them (ascending path order), C channels
    per row.  The projection after the product then reads one input segment per output irrep, and
    its input gradient is one launch per irrep instead of one per path (the per-path blocks of the
    irreps sorted by irrep, in the same path order, hold the same numbers with the rows permuted)."""
    rows = {}
    groups = {}
    for p in sorted(cfg.paths, key=lambda p: p["o3"]):
        groups.setdefault(p["l3"], []).append(p)
    for l3, ps in groups.items():
        base = min(p["o3"] for p in ps)
        nb = len(ps)
        assert max(p["o3"] for p in ps) == base + (nb - 1) * (2 * l3 + 1), "blocks of one irrep not adjacent"
        for b, p in enumerate(ps):
            for m3 in range(2 * l3 + 1):
                rows[(p["k"], m3)] = base + m3 * nb + b
    return rows


def fwd_groups(cfg: Cfg) -> int:
    """Edge groups per forward wavefront, their loads all in flight before any arithmetic: 2 up to
    l_max = 2 (1.99 -> 1.39 ms at l_max 2, C = 16, 2.6 M edges), 1 for l_max = 3 (registers)."""
    return 2 if cfg.NX <= 9 else 1


def supported(cfg: Cfg) -> bool:
    """Allegro's product: input, harmonics and kept outputs all l = 0 .. l_max."""
    return cfg.in_ls == cfg.sh_ls == cfg.out_ls


def _fwd(cfg: Cfg) -> str:
    L = []
    a = L.append
    NX, NY, NO, NP = cfg.NX, cfg.NY, cfg.NO, cfg.NP
    EPW = fwd_groups(cfg)
    rows = out_row(cfg)
    a(f"template <int CW, int CPL>\n__global__ void __launch_bounds__(256) etp_fwd_c{cfg.idx}("
      "const float* __restrict__ x, const float* __restrict__ Y, const float* __restrict__ w, "
      "const float* __restrict__ xs, int64_t E, int C, float* __restrict__ out) {")
    a("  constexpr int G = 64 / CW;")
    a("  const int lane = threadIdx.x & 63, c0 = lane % CW;")
    a(f"  const int64_t e0 = (int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * ({EPW} * G) + lane / CW;")
    a(f"  // {EPW} edge groups per wavefront: every load of all of them issued before any arithmetic")
    a(f"  float y[{EPW}][{NY}], xv[{EPW}][CPL][{NX}];")
    a("#pragma unroll")
    a(f"  for (int q = 0; q < {EPW}; ++q) {{")
    a("    const int64_t e = e0 + q * G;")
    a("    if (e >= E) break;")
    a(f"    const float* __restrict__ Ye = Y + e * {NY};")
    a(f"    const float* __restrict__ xe = x + e * ({NX} * int64_t(C));")
    a(f"#pragma unroll\n    for (int i = 0; i < {NY}; ++i) y[q][i] = Ye[i];")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k)")
    a("    {")
    a("      const float sc = xs ? xs[e * C + c0 + 64 * k] : 1.f;")
    a(f"#pragma unroll\n      for (int i = 0; i < {NX}; ++i) xv[q][k][i] = xe[i * C + c0 + 64 * k] * sc;")
    a("    }")
    a("  }")
    a("#pragma unroll")
    a(f"  for (int q = 0; q < {EPW}; ++q) {{")
    a("    const int64_t e = e0 + q * G;")
    a("    if (e >= E) break;")
    a(f"    float* __restrict__ oe = out + e * ({NO} * int64_t(C));")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k) {")
    a("      const int c = c0 + 64 * k;")
    for j, p in enumerate(cfg.paths):
        cf = p["c"]
        a("      {")
        a(f"        const float wj = w[{j} * C + c];")
        for m3 in range(2 * p["l3"] + 1):
            row = []
            for m1 in range(2 * p["l1"] + 1):
                terms = [(m2, cf[m1, m2, m3]) for m2 in range(2 * p["l2"] + 1) if abs(cf[m1, m2, m3]) > EPS]
                if not terms:
                    continue
                expr = f"{f32(terms[0][1])} * y[q][{p['o2'] + terms[0][0]}]"
                for m2, v in terms[1:]:
                    expr = f"fmaf({f32(v)}, y[q][{p['o2'] + m2}], {expr})"
                row.append((m1, expr))
            o = rows[(p["k"], m3)]
            if not row:
                a(f"        oe[{o} * C + c] = 0.f;")
                continue
            s = f"({row[0][1]}) * xv[q][k][{p['o1'] + row[0][0]}]"
            for m1, expr in row[1:]:
                s = f"fmaf({expr}, xv[q][k][{p['o1'] + m1}], {s})"
            a(f"        oe[{o} * C + c] = wj * ({s});")
        a("      }")
    a("    }")
    a("  }")
    a("}")
    return "\n".join(L)


def _bwd(cfg: Cfg) -> str:
    L = []
    a = L.append
    NX, NY, NO, NP = cfg.NX, cfg.NY, cfg.NO, cfg.NP
    rows = out_row(cfg)
    a(f"template <int CW, int CPL>\n__global__ void __launch_bounds__(256) etp_bwd_c{cfg.idx}("
      "const float* __restrict__ gout, const float* __restrict__ x, const float* __restrict__ Y, "
      "const float* __restrict__ w, const float* __restrict__ xs, int64_t E, int C, float* __restrict__ gx, "
      "float* __restrict__ gY, float* __restrict__ gw_part, float* __restrict__ gxs) {")
    a("  constexpr int G = 64 / CW;")
    a("  const int lane = threadIdx.x & 63, c0 = lane % CW;")
    a("  const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6), nwaves = int64_t(gridDim.x) * 4;")
    a("  const int64_t ngroups = (E + G - 1) / G;")
    a(f"  float wv[CPL][{NP}], gwa[CPL][{NP}];")
    a("#pragma unroll")
    a("  for (int k = 0; k < CPL; ++k)")
    a("#pragma unroll")
    a(f"    for (int j = 0; j < {NP}; ++j) {{ wv[k][j] = w[j * C + c0 + 64 * k]; gwa[k][j] = 0.f; }}")
    a("  for (int64_t grp = wave; grp < ngroups; grp += nwaves) {")
    a("    const int64_t e = grp * G + lane / CW;")
    a("    const bool valid = e < E;")
    a("    const int64_t es = valid ? e : 0;")
    a(f"    const float* __restrict__ Ye = Y + es * {NY};")
    a("    " + " ".join(f"const float y{i} = Ye[{i}];" for i in range(NY)))
    a(f"    float gYp[{NY}];")
    a(f"#pragma unroll\n    for (int i = 0; i < {NY}; ++i) gYp[i] = 0.f;")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k) {")
    a("      const int c = c0 + 64 * k;")
    a(f"      const float* __restrict__ xe = x + es * ({NX} * int64_t(C)) + c;")
    a(f"      const float* __restrict__ ge = gout + es * ({NO} * int64_t(C)) + c;")
    a(f"      float xv[{NX}], gv[{NO}], gxv[{NX}];")
    a("      const float sc = (xs && valid) ? xs[es * C + c] : 1.f;")
    a(f"      float xr[{NX}];  // x as given; xv = sc * xr enters the product")
    a(f"#pragma unroll\n      for (int i = 0; i < {NX}; ++i) {{ xr[i] = valid ? xe[i * C] : 0.f; xv[i] = xr[i] * sc; gxv[i] = 0.f; }}")
    a(f"#pragma unroll\n      for (int i = 0; i < {NO}; ++i) gv[i] = valid ? ge[i * C] : 0.f;")
    for j, p in enumerate(cfg.paths):
        cf = p["c"]
        a("      {")
        a(f"        const float wj = wv[k][{j}];")
        for m1 in range(2 * p["l1"] + 1):
            vs = []
            for m2 in range(2 * p["l2"] + 1):
                terms = [(m3, cf[m1, m2, m3]) for m3 in range(2 * p["l3"] + 1) if abs(cf[m1, m2, m3]) > EPS]
                if not terms:
                    continue
                expr = f"{f32(terms[0][1])} * gv[{rows[(p['k'], terms[0][0])]}]"
                for m3, v in terms[1:]:
                    expr = f"fmaf({f32(v)}, gv[{rows[(p['k'], m3)]}], {expr})"
                vs.append((m2, expr))
            if not vs:
                continue
            xi = p["o1"] + m1
            a("        {")
            for m2, expr in vs:
                a(f"          const float v{m2} = {expr};")
            u = f"y{p['o2'] + vs[0][0]} * v{vs[0][0]}"
            for m2, _ in vs[1:]:
                u = f"fmaf(y{p['o2'] + m2}, v{m2}, {u})"
            a(f"          const float u = {u};")
            a(f"          gxv[{xi}] = fmaf(wj, u, gxv[{xi}]);")
            a(f"          gwa[k][{j}] = fmaf(xv[{xi}], u, gwa[k][{j}]);")
            a(f"          const float xw = xv[{xi}] * wj;")
            for m2, _ in vs:
                a(f"          gYp[{p['o2'] + m2}] = fmaf(xw, v{m2}, gYp[{p['o2'] + m2}]);")
            a("        }")
        a("      }")
    a(f"      if (gx && valid) {{ float* __restrict__ gxe = gx + es * ({NX} * int64_t(C)) + c;")
    a(f"#pragma unroll\n        for (int i = 0; i < {NX}; ++i) gxe[i * C] = gxv[i] * sc; }}")
    a("      if (gxs && valid) {")
    a("        float t = 0.f;")
    a(f"#pragma unroll\n        for (int i = 0; i < {NX}; ++i) t = fmaf(gxv[i], xr[i], t);")
    a("        gxs[es * C + c] = t;")
    a("      }")
    a("    }")
    a("    if (gY) {")
    a("#pragma unroll")
    a(f"      for (int i = 0; i < {NY}; ++i) {{")
    a("#pragma unroll")
    a("        for (int s = 1; s < CW; s <<= 1) gYp[i] += __shfl_xor(gYp[i], s);")
    a("      }")
    a(f"      if (valid && c0 == 0) {{ float* __restrict__ gYe = gY + es * {NY};")
    a(f"#pragma unroll\n        for (int i = 0; i < {NY}; ++i) gYe[i] = gYp[i]; }}")
    a("    }")
    a("  }")
    a("  // one partial per wavefront: sum over its edge slots (lanes of equal channel)")
    a("#pragma unroll")
    a("  for (int k = 0; k < CPL; ++k)")
    a("#pragma unroll")
    a(f"    for (int j = 0; j < {NP}; ++j)")
    a("#pragma unroll")
    a("      for (int s = CW; s < 64; s <<= 1) gwa[k][j] += __shfl_xor(gwa[k][j], s);")
    a("  if (lane < CW) {")
    a(f"    float* __restrict__ pw = gw_part + wave * ({NP} * int64_t(C));")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k)")
    a("#pragma unroll")
    a(f"      for (int j = 0; j < {NP}; ++j) pw[j * C + c0 + 64 * k] = gwa[k][j];")
    a("  }")
    a("}")
    return "\n".join(L)




def proj_layout(cfg: Cfg):
    """Blocks of the projection that follows the product (cuet.Linear(tp.irreps_out, irreps_in),
    src/molzoo/allegro.py:363-367) for the fused kernels: per output irrep in merged-row order
    (l3, its paths in rank order, first block index J0, the irrep's component offset O in the
    projected rows, whose irreps are l = 0..l_max in order); and the projected components."""
    rows = out_row(cfg)
    groups = {}
    for p in sorted(cfg.paths, key=lambda p: p["o3"]):
        groups.setdefault(p["l3"], []).append(p)
    offs, o = {}, 0
    for l in sorted(groups):
        offs[l] = o
        o += 2 * l + 1
    blocks, J = [], 0
    for l3, ps in sorted(groups.items(), key=lambda kv: min(rows[(p["k"], 0)] for p in kv[1])):
        blocks.append((l3, ps, J, offs[l3]))
        J += len(ps)
    return blocks, o


def _row_terms(p, m3):
    """[(m1, expr of Y)] of output component m3 of path p (Y in y[...])."""
    cf = p["c"]
    row = []
    for m1 in range(2 * p["l1"] + 1):
        terms = [(m2, cf[m1, m2, m3]) for m2 in range(2 * p["l2"] + 1) if abs(cf[m1, m2, m3]) > EPS]
        if not terms:
            continue
        expr = f"{f32(terms[0][1])} * y[{p['o2'] + terms[0][0]}]"
        for m2, v in terms[1:]:
            expr = f"fmaf({f32(v)}, y[{p['o2'] + m2}], {expr})"
        row.append((m1, expr))
    return row


def _stage_proj(a, cfg: Cfg):
    """LDS copy of the projection weights wp (rows J*16 + c, 16 columns) as the forward's matrix-core
    B operands, sw[J][q][n][j] = wp[J][4q + j][n] w[j(J)][4q + j] (k = input channel 4 q + j,
    column n = output channel; the product's path weight folded in, j(J) the compiled path of block
    row J): lane l = 16 q + n reads its four j as one float4 at J*256 + 4 l."""
    blocks, _ = proj_layout(cfg)
    jidx = {p["k"]: j for j, p in enumerate(cfg.paths)}
    a(f"  __shared__ __align__(16) float sw[{cfg.NP * 256}];")
    a("  {")
    a("    const int q = threadIdx.x >> 6, n = (threadIdx.x >> 2) & 15, j = threadIdx.x & 3;")
    a("    const int src = (4 * q + j) * 16 + n;")
    for l3, ps, J0, O in blocks:
        for b, p in enumerate(ps):
            J = J0 + b
            a(f"    sw[{J * 256} + threadIdx.x] = wp[{J * 256} + src] * w[{jidx[p['k']]} * 16 + 4 * q + j];")
    a("  }")


def _fwdp(cfg: Cfg) -> str:
    """Product and projection in one pass (16 channels) on the matrix cores.  A wavefront walks
    groups of 16 edges: lane l holds edge r = l mod 16 of the group and channels 4 q .. 4 q + 3
    (q = l / 16).  Per output irrep, component m3 and path b, the product's values t_b[m3] are
    exactly the A operand of four fp32 16x16x4 products (A[edge][k] = t_b[m3][edge][4 k + j]), whose
    B operands are the projection weights of input channels 4 k + j (staged in LDS in operand
    order); the 16x16 result holds out[edge 4 q + v][channel r] in lane l, register v.  Only the
    projected rows (irreps l = 0..l_max, 16 channels each) are written."""
    L = []
    a = L.append
    NX, NY = cfg.NX, cfg.NY
    blocks, ncomp = proj_layout(cfg)
    a(f"template <bool XB>\n__global__ void __launch_bounds__(256) etp_fwdp_c{cfg.idx}("
      "const float* __restrict__ x, const float* __restrict__ Y, const float* __restrict__ w, "
      "const float* __restrict__ xs, const float* __restrict__ xs2, const float* __restrict__ wp, int64_t E, "
      "float* __restrict__ out) {")
    _stage_proj(a, cfg)
    a("  __syncthreads();")
    a("  const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;")
    a("  const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6), nwaves = int64_t(gridDim.x) * 4;")
    a("  const int64_t ngroups = (E + 15) / 16;")
    a("  const f4* __restrict__ sw4 = reinterpret_cast<const f4*>(sw) + lane;")
    a("  for (int64_t grp = wave; grp < ngroups; grp += nwaves) {")
    a("    asm volatile(\"\" ::: \"memory\");  // the LDS operands are re-read every group")
    a("    const int64_t e = grp * 16 + r;")
    a("    const int64_t es = e < E ? e : E - 1;  // edges past the end compute edge E - 1, unstored")
    a(f"    const float* __restrict__ Ye = Y + es * {NY};")
    a(f"    float y[{NY}];")
    a("#pragma unroll")
    a(f"    for (int i = 0; i < {NY}; ++i) y[i] = Ye[i];")
    a("    f4 sc = xs ? *reinterpret_cast<const f4*>(xs + es * 16 + 4 * q) : f4{1.f, 1.f, 1.f, 1.f};")
    a("    if (xs2) sc *= *reinterpret_cast<const f4*>(xs2 + es * 16 + 4 * q);  // a second channel scale")
    a(f"    f4 xv[{NX}];")
    a("    if constexpr (XB) {  // x[e][i] shared by every channel")
    a(f"      const float* __restrict__ xe = x + es * {NX};")
    a("#pragma unroll")
    a(f"      for (int i = 0; i < {NX}; ++i) xv[i] = xe[i] * sc;")
    a("    } else {")
    a(f"      const f4* __restrict__ xe = reinterpret_cast<const f4*>(x + es * {NX * 16}) + q;")
    a("#pragma unroll")
    a(f"      for (int i = 0; i < {NX}; ++i) xv[i] = xe[i * 4] * sc;")
    a("    }")
    for l3, ps, J0, O in blocks:
        M = 2 * l3 + 1
        a("    {")
        a(f"      f4 acc[{M}];")
        a("#pragma unroll")
        a(f"      for (int m = 0; m < {M}; ++m) acc[m] = f4{{0.f, 0.f, 0.f, 0.f}};")
        for b, p in enumerate(ps):
            a("      __builtin_amdgcn_sched_barrier(0);  // one path at a time (register pressure)")
            a("      {")
            a(f"        const f4 bw = sw4[{(J0 + b) * 64}];")
            a(f"        f4 t[{M}];")
            for m3 in range(M):
                row = _row_terms(p, m3)
                if not row:
                    a(f"        t[{m3}] = f4{{0.f, 0.f, 0.f, 0.f}};")
                    continue
                sx = f"({row[0][1]}) * xv[{p['o1'] + row[0][0]}]"
                for m1, expr in row[1:]:
                    sx = f"({expr}) * xv[{p['o1'] + m1}] + {sx}"
                a(f"        t[{m3}] = {sx};")
            a("#pragma unroll")
            a(f"        for (int m = 0; m < {M}; ++m) {{")
            a("          acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(t[m][0], bw[0], acc[m], 0, 0, 0);")
            a("          acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(t[m][1], bw[1], acc[m], 0, 0, 0);")
            a("          acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(t[m][2], bw[2], acc[m], 0, 0, 0);")
            a("          acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(t[m][3], bw[3], acc[m], 0, 0, 0);")
            a("        }")
            a("      }")
        a("#pragma unroll")
        a("      for (int v = 0; v < 4; ++v) {")
        a("        const int64_t eo = grp * 16 + 4 * q + v;")
        a("        if (eo < E) {")
        a(f"          float* __restrict__ oe = out + eo * {ncomp * 16} + {O * 16} + r;")
        a("#pragma unroll")
        a(f"          for (int m = 0; m < {M}; ++m) oe[m * 16] = acc[m][v];")
        a("        }")
        a("      }")
        a("    }")
    a("  }")
    a("}")
    return "\n".join(L)


def _stage_proj_rot(a, cfg: Cfg):
    """LDS copy of the projection weights wp (rows J*16 + c, 16 columns) for the backward's row
    rotations, sw[J][c][k] = wp[J][c][(c - k) mod 16] in rows of 20 floats (float4 reads of four k
    at once by the 16 lanes of a row hit distinct banks)."""
    a(f"  __shared__ __align__(16) float sw[{cfg.NP * 320}];")
    a("  {")
    a("    const int cc = threadIdx.x >> 4, k = threadIdx.x & 15;")
    a("    const int src = cc * 16 + ((cc - k) & 15), dst = cc * 20 + k;")
    for J in range(cfg.NP):
        a(f"    sw[{J * 320} + dst] = wp[{J * 256} + src];")
    a("  }")
    a("  __syncthreads();")


def _bwdp(cfg: Cfg) -> str:
    """Backward of ``_fwdp``.  Per output irrep, the gradient of each path's components is
    projected back in registers: lane c accumulates s_b[m3][c] = sum_k W[(J0 + b)*16 + c][(c - k)
    mod 16] g[m3][(c - k) mod 16] over the 16 rotations of the row (the rotated g shared by the
    irrep's paths); then each of those paths' product backward as in ``_bwd`` (16 channels, one
    channel per lane), so at most one irrep's path gradients are live at a time."""
    L = []
    a = L.append
    NX, NY, NP = cfg.NX, cfg.NY, cfg.NP
    blocks, ncomp = proj_layout(cfg)
    jidx = {p["k"]: j for j, p in enumerate(cfg.paths)}
    a(f"template <bool XB>\n__global__ void __launch_bounds__(256) etp_bwdp_c{cfg.idx}("
      "const float* __restrict__ gproj, const float* __restrict__ x, const float* __restrict__ Y, "
      "const float* __restrict__ w, const float* __restrict__ xs, const float* __restrict__ xs2, "
      "const float* __restrict__ wp, int64_t E, float* __restrict__ gx, float* __restrict__ gY, "
      "float* __restrict__ gw_part, float* __restrict__ gxs, float* __restrict__ gxs2) {")
    _stage_proj_rot(a, cfg)
    a("  constexpr int G = 4, C = 16;")
    a("  const int lane = threadIdx.x & 63, c = lane & 15;")
    a("  const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6), nwaves = int64_t(gridDim.x) * 4;")
    a("  const int64_t ngroups = (E + G - 1) / G;")
    a("  const float4* __restrict__ sw4 = reinterpret_cast<const float4*>(sw) + c * 5;")
    a(f"  float wv[{NP}], gwa[{NP}];")
    a("#pragma unroll")
    a(f"  for (int j = 0; j < {NP}; ++j) {{ wv[j] = w[j * C + c]; gwa[j] = 0.f; }}")
    a("  for (int64_t grp = wave; grp < ngroups; grp += nwaves) {")
    a("    // the LDS weights are re-read every iteration (hoisted, they would not fit in registers)")
    a("    asm volatile(\"\" ::: \"memory\");")
    a("    const int64_t e = grp * G + lane / 16;")
    a("    const bool valid = e < E;")
    a("    const int64_t es = valid ? e : 0;")
    a(f"    const float* __restrict__ Ye = Y + es * {NY};")
    a("    " + " ".join(f"const float y{i} = Ye[{i}];" for i in range(NY)))
    a(f"    float gYp[{NY}];")
    a("#pragma unroll")
    a(f"    for (int i = 0; i < {NY}; ++i) gYp[i] = 0.f;")
    a(f"    const float* __restrict__ xe = XB ? x + es * {NX} : x + es * ({NX} * int64_t(C)) + c;")
    a("    constexpr int XS = XB ? 1 : C;  // stride between x's components (x shared by the channels: 1)")
    a(f"    const float* __restrict__ ge = gproj + es * {ncomp * 16} + c;")
    a("    const float s1 = xs ? xs[es * C + c] : 1.f, s2 = xs2 ? xs2[es * C + c] : 1.f, sc = s1 * s2;")
    a(f"    float xr[{NX}], xv[{NX}], gxv[{NX}];  // x as given; xv = sc * xr enters the product")
    a("#pragma unroll")
    a(f"    for (int i = 0; i < {NX}; ++i) {{ xr[i] = xe[i * XS]; xv[i] = xr[i] * sc; gxv[i] = 0.f; }}")
    for l3, ps, J0, O in blocks:
        M, nb = 2 * l3 + 1, len(ps)
        a("    {")
        a(f"      float gl[{M}], s[{nb}][{M}];")
        a("#pragma unroll")
        a(f"      for (int m = 0; m < {M}; ++m) {{ const float g = ge[({O} + m) * 16]; gl[m] = valid ? g : 0.f; }}")
        a("#pragma unroll")
        a(f"      for (int m = 0; m < {M}; ++m)")
        a("#pragma unroll")
        a(f"        for (int b = 0; b < {nb}; ++b) s[b][m] = 0.f;")
        for kq in range(4):
            a("      __builtin_amdgcn_sched_barrier(0);")
            a("      {")
            for b in range(nb):
                a(f"        const float4 v{b} = sw4[{(J0 + b) * 80 + kq}];")
            for kk, comp in enumerate("xyzw"):
                k = 4 * kq + kk
                a("#pragma unroll")
                a(f"        for (int m = 0; m < {M}; ++m) {{")
                a(f"          const float r = ror16<{k}>(gl[m]);")
                for b in range(nb):
                    a(f"          s[{b}][m] = fmaf(v{b}.{comp}, r, s[{b}][m]);")
                a("        }")
            a("      }")
        a("      __builtin_amdgcn_sched_barrier(0);")
        for b, p in enumerate(ps):
            cf = p["c"]
            j = jidx[p["k"]]
            a("      {")
            a(f"        const float wj = wv[{j}];")
            for m1 in range(2 * p["l1"] + 1):
                vs = []
                for m2 in range(2 * p["l2"] + 1):
                    terms = [(m3, cf[m1, m2, m3]) for m3 in range(M) if abs(cf[m1, m2, m3]) > EPS]
                    if not terms:
                        continue
                    expr = f"{f32(terms[0][1])} * s[{b}][{terms[0][0]}]"
                    for m3, v in terms[1:]:
                        expr = f"fmaf({f32(v)}, s[{b}][{m3}], {expr})"
                    vs.append((m2, expr))
                if not vs:
                    continue
                xi = p["o1"] + m1
                a("        {")
                for m2, expr in vs:
                    a(f"          const float v{m2} = {expr};")
                u = f"y{p['o2'] + vs[0][0]} * v{vs[0][0]}"
                for m2, _ in vs[1:]:
                    u = f"fmaf(y{p['o2'] + m2}, v{m2}, {u})"
                a(f"          const float u = {u};")
                a(f"          gxv[{xi}] = fmaf(wj, u, gxv[{xi}]);")
                a(f"          gwa[{j}] = fmaf(xv[{xi}], u, gwa[{j}]);")
                a(f"          const float xw = xv[{xi}] * wj;")
                for m2, _ in vs:
                    a(f"          gYp[{p['o2'] + m2}] = fmaf(xw, v{m2}, gYp[{p['o2'] + m2}]);")
                a("        }")
            a("      }")
        a("    }")
    a("    if constexpr (XB) {  // grad of x shared by the channels: the row's sum over its 16 lanes")
    a("      if (gx) {")
    a(f"        float gxr[{NX}];")
    a("#pragma unroll")
    a(f"        for (int i = 0; i < {NX}; ++i) {{")
    a("          float t = gxv[i] * sc;")
    a("          t += ror16<8>(t);")
    a("          t += ror16<4>(t);")
    a("          t += ror16<2>(t);")
    a("          t += ror16<1>(t);")
    a("          gxr[i] = t;")
    a("        }")
    a(f"        if (valid && c == 0) {{ float* __restrict__ gxe = gx + es * {NX};")
    a("#pragma unroll")
    a(f"          for (int i = 0; i < {NX}; ++i) gxe[i] = gxr[i]; }}")
    a("      }")
    a("    } else if (gx && valid) {")
    a(f"      float* __restrict__ gxe = gx + es * ({NX} * int64_t(C)) + c;")
    a("#pragma unroll")
    a(f"      for (int i = 0; i < {NX}; ++i) gxe[i * C] = gxv[i] * sc;")
    a("    }")
    a("    if ((gxs || gxs2) && valid) {")
    a("      float t = 0.f;  // the gradient of the combined scale s1 s2")
    a("#pragma unroll")
    a(f"      for (int i = 0; i < {NX}; ++i) t = fmaf(gxv[i], xr[i], t);")
    a("      if (gxs) gxs[es * C + c] = t * s2;")
    a("      if (gxs2) gxs2[es * C + c] = t * s1;")
    a("    }")
    a("    if (gY) {")
    a("#pragma unroll")
    a(f"      for (int i = 0; i < {NY}; ++i) {{")
    a("        gYp[i] += ror16<8>(gYp[i]);  // every lane of the row ends with the row's sum")
    a("        gYp[i] += ror16<4>(gYp[i]);")
    a("        gYp[i] += ror16<2>(gYp[i]);")
    a("        gYp[i] += ror16<1>(gYp[i]);")
    a("      }")
    a(f"      if (valid && c == 0) {{ float* __restrict__ gYe = gY + es * {NY};")
    a("#pragma unroll")
    a(f"        for (int i = 0; i < {NY}; ++i) gYe[i] = gYp[i]; }}")
    a("    }")
    a("  }")
    a("  // one partial per wavefront: sum over its edge slots (lanes of equal channel)")
    a("#pragma unroll")
    a(f"  for (int j = 0; j < {NP}; ++j)")
    a("#pragma unroll")
    a("    for (int s2 = 16; s2 < 64; s2 <<= 1) gwa[j] += __shfl_xor(gwa[j], s2);")
    a("  if (lane < 16) {")
    a(f"    float* __restrict__ pw = gw_part + wave * ({NP} * int64_t(C));")
    a("#pragma unroll")
    a(f"    for (int j = 0; j < {NP}; ++j) pw[j * C + c] = gwa[j];")
    a("  }")
    a("}")
    return "\n".join(L)


def generate() -> str:
    cfgs = [Cfg(i, *c) for i, c in enumerate(config_list())]
    out = ["// Generated by gen_edge_tp.py -- do not edit.", "// clang-format off", ""]
    for cfg in cfgs:
        if not supported(cfg):
            continue
        out.append(f"// config {cfg.idx}: l={cfg.in_ls}; {cfg.NP} paths, NX={cfg.NX} NY={cfg.NY} NO={cfg.NO}")
        out.append(_fwd(cfg))
        out.append("")
        out.append(_bwd(cfg))
        out.append("")
        out.append(_fwdp(cfg))
        out.append("")
        out.append(_bwdp(cfg))
        out.append("")
    out.append(f"static constexpr int kETPNumConfigs = {len(cfgs)};")
    out.append(f"static constexpr int kETPNumVariants = {len(VARIANTS)};")
    out.append("static const int kETPVariantCW[] = {" + ", ".join(str(v[0]) for v in VARIANTS) + "};")
    out.append("static const int kETPVariantCPL[] = {" + ", ".join(str(v[1]) for v in VARIANTS) + "};")
    out.append("static const ETPInfo kETPInfo[] = {")
    for cfg in cfgs:
        out.append(f"  {{{int(supported(cfg))}, {cfg.NP}, {cfg.NX}, {cfg.NY}, {cfg.NO}, {fwd_groups(cfg)}}},")
    out.append("};")
    # fused product + projection (16 channels): kernels, projected components, projection blocks
    # [config][x shared by the channels]
    out.append("static const ETPFwdPFn kETPFwdP[][2] = {" + ", ".join(
        f"{{etp_fwdp_c{c.idx}<false>, etp_fwdp_c{c.idx}<true>}}" if supported(c) else "{nullptr, nullptr}"
        for c in cfgs) + "};")
    out.append("static const ETPBwdPFn kETPBwdP[][2] = {" + ", ".join(
        f"{{etp_bwdp_c{c.idx}<false>, etp_bwdp_c{c.idx}<true>}}" if supported(c) else "{nullptr, nullptr}"
        for c in cfgs) + "};")
    out.append("static const int kETPProjComps[] = {" + ", ".join(
        str(proj_layout(c)[1]) if supported(c) else "0" for c in cfgs) + "};")
    out.append("static const int kETPProjBlocks[][4 * 4 + 1] = {")
    for c in cfgs:
        if supported(c):
            bl = proj_layout(c)[0]
            flat = [len(bl)] + [v for l3, ps, J0, O in bl for v in (l3, len(ps), J0, O)]
        else:
            flat = [0]
        flat += [0] * (17 - len(flat))
        out.append("  {" + ", ".join(str(v) for v in flat) + "},")
    out.append("};")
    for kind in ("fwd", "bwd"):
        typ = "ETPFwdFn" if kind == "fwd" else "ETPBwdFn"
        out.append(f"static const {typ} kETP{kind.capitalize()}[][{len(VARIANTS)}] = {{")
        for cfg in cfgs:
            if supported(cfg):
                fns = [f"etp_{kind}_c{cfg.idx}<{cw}, {cpl}>" for cw, cpl in VARIANTS]
            else:
                fns = ["nullptr"] * len(VARIANTS)
            out.append("  {" + ", ".join(fns) + "},")
        out.append("};")
    return "\n".join(out) + "\n"


def main():
    path = os.path.join(HERE, "edge_tp_gen.inc")
    text = generate()
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as f:
            f.write(text)
    return path


if __name__ == "__main__":
    print(main())
