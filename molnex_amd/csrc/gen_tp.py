"""Generate the channelwise tensor-product kernels (``tp_gen.inc``).

Each supported configuration (the l's of irreps_in1, of the harmonics and of
the output filter) becomes straight-line HIP code with the real coupling
coefficients of ``molnex_amd.irreps`` baked in as constants, so every register
index is static.  Paths are split into groups by the l of irreps_in1; each
group is one wavefront kernel per (receiver, channel block).

Per-edge weights are read from row wrow[e] of w when wrow is given (edges that share
their weights, e.g. the two directions of an undirected pair), else from row e.

Forward (per edge, per channel):   out_p[m3] += w_p * sum_m1 M_p[m3][m1] x[m1]
  with the uniform matrix M_p[m3][m1] = sum_m2 c_p[m1,m2,m3] Y[m2].
Backward (per receiver, per channel), with v_p[m1][m2] = sum_m3 c_p g_p[m3]
computed once per receiver:
  u_p[m1] = sum_m2 Y[m2] v_p[m1][m2]      -> grad_x[m1] += w_p u_p[m1]
  s_p[m2] = sum_m1 x[m1] v_p[m1][m2]      -> grad_w_p = sum_m2 Y[m2] s_p[m2]
                                           -> grad_Y[m2] += w_p s_p[m2] (summed over channels)

Run as ``python -m molnex_amd.csrc.gen_tp`` (``build()`` does this).
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from molnex_amd.irreps import ChannelwiseTPDescriptor, coupling  # noqa: E402

EPS = 1e-12


def _irreps(ls, mul=1):
    return " + ".join(f"{mul}x{l}{'e' if l % 2 == 0 else 'o'}" for l in ls)


def _mask(ls):
    m = 0
    for l in ls:
        m |= 1 << l
    return m


def _ls(mask):
    return [l for l in range(4) if mask >> l & 1]


# (in1 l's, harmonics l's, output filter l's)
def config_list():
    cfgs = []
    for L in range(4):  # MACE as coded: hidden = C x (0..L), harmonics 0..L
        cfgs.append((list(range(L + 1)), list(range(L + 1)), list(range(L + 1))))
    for ins in ([0], [0, 1]):  # MACE with hidden 0e+1o, harmonics l <= 3
        for outs in ([0, 1, 2, 3], [0, 1]):
            cfgs.append((ins, [0, 1, 2, 3], outs))
    # small shapes used by the reference's module tests
    cfgs += [
        ([0], [0, 1], [0]),
        ([1], [0, 1], [1]),
        ([0], [0, 1, 2], [0]),
        ([0], [0, 1], [0, 1]),
        ([0, 1], [0, 1, 2, 3], [0, 1, 2, 3]),
    ]
    seen, out = set(), []
    for c in cfgs:
        key = (_mask(c[0]), _mask(c[1]), _mask(c[2]))
        if key not in seen:
            seen.add(key)
            out.append(c)
    return out


def f32(v: float) -> str:
    return f"{float(np.float32(v)):.9e}f"


class Cfg:
    def __init__(self, idx, in_ls, sh_ls, out_ls):
        self.idx = idx
        self.in_ls, self.sh_ls, self.out_ls = in_ls, sh_ls, out_ls
        d = ChannelwiseTPDescriptor(_irreps(in_ls), _irreps(sh_ls), _irreps(out_ls))
        self.d = d
        self.NX = sum(2 * l + 1 for l in in_ls)
        self.NY = sum(2 * l + 1 for l in sh_ls)
        self.NO = sum(b.ir.dim for b in d.irreps_out)
        self.NP = d.num_paths
        off1 = np.cumsum([0] + [2 * l + 1 for l in in_ls])
        off2 = np.cumsum([0] + [2 * l + 1 for l in sh_ls])
        off3 = np.cumsum([0] + [b.ir.dim for b in d.irreps_out])
        self.paths = []
        for k, p in enumerate(d.paths):
            coef = math.sqrt(2 * p.l3 + 1) * coupling(p.l1, p.l2, p.l3)
            self.paths.append(
                dict(k=k, l1=p.l1, l2=p.l2, l3=p.l3, o1=int(off1[p.i1]), o2=int(off2[p.i2]),
                     o3=int(off3[p.out_block]), c=coef)
            )
        self.groups = []
        for l1 in in_ls:
            ps = [p for p in self.paths if p["l1"] == l1]
            if ps:
                self.groups.append(ps)

    @property
    def masks(self):
        return _mask(self.in_ls), _mask(self.sh_ls), _mask(self.out_ls)


def _uniq(seq):
    out = []
    for s in seq:
        if s not in out:
            out.append(s)
    return out


def _group_layout(ps):
    xs = _uniq([p["o1"] + m for p in ps for m in range(2 * p["l1"] + 1)])
    ys = _uniq([p["o2"] + m for p in ps for m in range(2 * p["l2"] + 1)])
    outs = [p["o3"] + m for p in ps for m in range(2 * p["l3"] + 1)]
    return xs, ys, outs


def _v_count(ps):
    return sum(1 for p in ps for m1 in range(2 * p["l1"] + 1) for m2 in range(2 * p["l2"] + 1)
               if np.any(np.abs(p["c"][m1, m2, :]) > EPS))


def bwd_cpl(ps) -> int:
    """Channels per lane for a backward group: 2 when the per-channel register
    state (folded gradient v, x, w, partial sums) stays small, else 1."""
    xs, ys, outs = _group_layout(ps)
    per_channel = _v_count(ps) + 2 * (len(xs) + len(ps)) + len(xs)
    return 2 if per_channel <= 60 else 1


def _emit_prefetch(a, cfg, ps, xs, ys, xi, indent, cpl_expr="CPL"):
    """Load the harmonics, sender row and weight row of the edge whose ids are (ne, ns, nw) into
    the n* registers."""
    a(f"{indent}{{")
    a(f"{indent}  const float* __restrict__ Yn = Y + int64_t(ne) * {cfg.NY};")
    for c in ys:
        a(f"{indent}  ny{c} = Yn[{c}];")
    a(f"{indent}  const float* __restrict__ xn = x + int64_t(ns) * XS;")
    a(f"{indent}  const float* __restrict__ wn = w + int64_t(nw) * WS;")
    a("#pragma unroll")
    a(f"{indent}  for (int k = 0; k < {cpl_expr}; ++k) {{")
    for c in xs:
        a(f"{indent}    nxv[k][{xi[c]}] = ok[k] ? xn[{c} * C + cc[k]] : 0.f;")
    for j, p in enumerate(ps):
        a(f"{indent}    nwv[k][{j}] = ok[k] ? __builtin_nontemporal_load(wn + {p['k']} * C + cc[k]) : 0.f;")
    a(f"{indent}  }}")
    a(f"{indent}}}")


def _emit_ids(a, indent, t_expr, dst=("ie", "is", "iw")):
    """Edge, sender and weight-row ids of CSR slot t_expr (wave-uniform scalar loads)."""
    e, s_, w = dst
    a(f"{indent}{e} = perm[{t_expr}]; {s_} = snd[{t_expr}]; {w} = wrow ? wrow[{e}] : {e};")


def _emit_edge_loop_head(a, cfg, ps, xs, ys, xi, flush=None):
    """The receiver's CSR walk with a two-stage prefetch: the ids of edge t + 2 (including the
    dependent weight-row lookup) are loaded while edge t is processed, and the rows of edge t + 1
    are loaded at the top of iteration t from ids that are already in registers.  `flush`: lines
    emitted at the top of each iteration after the rows of edge t are taken and before the loads
    of edge t + 1 are issued (the backward's deferred writes of edge t - 1)."""
    a("  const int beg = row_ptr[n], end = row_ptr[n + 1];")
    a("  int ne = 0, ns = 0, nw = 0, ie = 0, is = 0, iw = 0;")
    a("  " + " ".join(f"float ny{c} = 0.f;" for c in ys))
    a(f"  float nxv[CPL][{len(xs)}], nwv[CPL][{len(ps)}];")
    a("  if (beg < end) {")
    _emit_ids(a, "    ", "beg", ("ne", "ns", "nw"))
    _emit_prefetch(a, cfg, ps, xs, ys, xi, "    ")
    a("  }")
    a("  if (beg + 1 < end) {")
    _emit_ids(a, "    ", "beg + 1")
    a("  }")
    a("  for (int t = beg; t < end; ++t) {")
    a("    const int e = ne, s = ns;")
    a("    " + " ".join(f"const float y{c} = ny{c};" for c in ys))
    a(f"    float xv[CPL][{len(xs)}], wv[CPL][{len(ps)}];")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k) {")
    a(f"#pragma unroll\n      for (int i = 0; i < {len(xs)}; ++i) xv[k][i] = nxv[k][i];")
    a(f"#pragma unroll\n      for (int i = 0; i < {len(ps)}; ++i) wv[k][i] = nwv[k][i];")
    a("    }")
    for line in flush or []:
        a(line)
    a("    if (t + 1 < end) {")
    a("      ne = ie; ns = is; nw = iw;")
    _emit_prefetch(a, cfg, ps, xs, ys, xi, "      ")
    a("      if (t + 2 < end) {")
    _emit_ids(a, "        ", "t + 2")
    a("      }")
    a("    }")


def gen_fwd(cfg: Cfg, g: int) -> str:
    ps = cfg.groups[g]
    xs, ys, outs = _group_layout(ps)
    xi = {c: i for i, c in enumerate(xs)}
    oi = {c: i for i, c in enumerate(outs)}
    L = []
    a = L.append
    name = f"tp_fwd_c{cfg.idx}_g{g}"
    a(f"template <int CPL, bool FULL>\n__global__ void __launch_bounds__(64) {name}(const float* __restrict__ x, "
      "const float* __restrict__ Y, const float* __restrict__ w, const int32_t* __restrict__ row_ptr, "
      "const int32_t* __restrict__ perm, const int32_t* __restrict__ snd, const int32_t* __restrict__ wrow, "
      "int64_t N, int C, float* __restrict__ out) {")
    a("  const int64_t n = xcd_node(blockIdx.x, gridDim.x);")
    a("  if (n >= N) return;")
    a("  const int lane = threadIdx.x;")
    a("  int cc[CPL]; bool ok[CPL];")
    a("#pragma unroll")
    a("  for (int k = 0; k < CPL; ++k) { cc[k] = blockIdx.y * (64 * CPL) + 64 * k + lane; ok[k] = FULL || cc[k] < C; }")
    a(f"  float acc[CPL][{len(outs)}];")
    a("#pragma unroll")
    a(f"  for (int k = 0; k < CPL; ++k)\n#pragma unroll\n    for (int i = 0; i < {len(outs)}; ++i) acc[k][i] = 0.f;")
    a(f"  const int64_t XS = int64_t({cfg.NX}) * C, WS = int64_t({cfg.NP}) * C;")
    _emit_edge_loop_head(a, cfg, ps, xs, ys, xi)
    a("    (void)e; (void)s;")
    # per output row (path j, m3): the wave-uniform coupling row M_j[m3][m1] = sum_m2 c y,
    # used at once for every channel of the lane (short live ranges, no hoisted M table)
    for j, p in enumerate(ps):
        c = p["c"]
        for m3 in range(2 * p["l3"] + 1):
            row = []
            for m1 in range(2 * p["l1"] + 1):
                terms = [(m2, c[m1, m2, m3]) for m2 in range(2 * p["l2"] + 1) if abs(c[m1, m2, m3]) > EPS]
                if not terms:
                    continue
                expr = f"{f32(terms[0][1])} * y{p['o2'] + terms[0][0]}"
                for m2, v in terms[1:]:
                    expr = f"fmaf({f32(v)}, y{p['o2'] + m2}, {expr})"
                row.append((m1, expr))
            if not row:
                continue
            a("    {")
            for m1, expr in row:
                a(f"      const float M{m1} = {expr};")
            o = oi[p["o3"] + m3]
            a("#pragma unroll")
            a("      for (int k = 0; k < CPL; ++k) {")
            expr = f"M{row[0][0]} * xv[k][{xi[p['o1'] + row[0][0]]}]"
            for m1, _ in row[1:]:
                expr = f"fmaf(M{m1}, xv[k][{xi[p['o1'] + m1]}], {expr})"
            a(f"        acc[k][{o}] = fmaf(wv[k][{j}], {expr}, acc[k][{o}]);")
            a("      }")
            a("    }")
    a("  }")
    a(f"  float* __restrict__ on = out + n * int64_t({cfg.NO}) * C;")
    a("#pragma unroll")
    a("  for (int k = 0; k < CPL; ++k) {")
    a("    if (!ok[k]) continue;")
    for c in outs:
        a(f"    on[{c} * C + cc[k]] = acc[k][{oi[c]}];")
    a("  }")
    a("}")
    return "\n".join(L)


def gen_bwd(cfg: Cfg, g: int) -> str:
    ps = cfg.groups[g]
    xs, ys, outs = _group_layout(ps)
    xi = {c: i for i, c in enumerate(xs)}
    oi = {c: i for i, c in enumerate(outs)}
    V = 1
    while V < cfg.NY:
        V *= 2
    L = []
    a = L.append
    name = f"tp_bwd_c{cfg.idx}_g{g}"
    a(f"template <int CPL, bool FULL>\n__global__ void __launch_bounds__(64) {name}(const float* __restrict__ x, "
      "const float* __restrict__ Y, const float* __restrict__ w, const float* __restrict__ gout, "
      "const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ perm, const int32_t* __restrict__ snd, "
      "const int32_t* __restrict__ wrow, "
      "int64_t N, int C, float* __restrict__ gx, float* __restrict__ gw, float* __restrict__ gyp, int npart, "
      "int pbase) {")
    a("  const int64_t n = xcd_node(blockIdx.x, gridDim.x);")
    a("  if (n >= N) return;")
    a("  const int lane = threadIdx.x;")
    a("  int cc[CPL]; bool ok[CPL];")
    a("#pragma unroll")
    a("  for (int k = 0; k < CPL; ++k) { cc[k] = blockIdx.y * (64 * CPL) + 64 * k + lane; ok[k] = FULL || cc[k] < C; }")
    a("  const int pidx = pbase + blockIdx.y;")
    a(f"  const int64_t XS = int64_t({cfg.NX}) * C, WS = int64_t({cfg.NP}) * C;")
    a(f"  const float* __restrict__ gn = gout + n * int64_t({cfg.NO}) * C;")
    vnames = {}
    a(f"  float v[CPL][{_v_count(ps)}];")
    a("#pragma unroll")
    a("  for (int k = 0; k < CPL; ++k) {")
    a(f"    float gv[{len(outs)}];")
    for c in outs:
        a(f"    gv[{oi[c]}] = ok[k] ? gn[{c} * C + cc[k]] : 0.f;")
    vi = 0
    for j, p in enumerate(ps):
        c = p["c"]
        for m1 in range(2 * p["l1"] + 1):
            for m2 in range(2 * p["l2"] + 1):
                terms = [(m3, c[m1, m2, m3]) for m3 in range(2 * p["l3"] + 1) if abs(c[m1, m2, m3]) > EPS]
                if not terms:
                    continue
                expr = f"{f32(terms[0][1])} * gv[{oi[p['o3'] + terms[0][0]]}]"
                for m3, val in terms[1:]:
                    expr = f"fmaf({f32(val)}, gv[{oi[p['o3'] + m3]}], {expr})"
                a(f"    v[k][{vi}] = {expr};")
                vnames[(j, m1, m2)] = vi
                vi += 1
    a("  }")
    # Writes are deferred by one edge: edge t's weight gradient, grad_x atomics and grad_Y partial
    # stay in registers (dgw, dgx, dgy) and are issued at the top of iteration t + 1, after the
    # rows of edge t + 1 have arrived and before the loads of edge t + 2.  Waiting for loads with
    # writes outstanding drains the whole vector memory counter (loads and writes retire out of
    # order on gfx9), so writes issued after the next edge's loads -- the natural order -- made
    # every iteration wait for its own atomics to complete.
    flush = []
    f = flush.append
    f("    if (pend) {")
    f("      float* __restrict__ gwe = gw ? gw + int64_t(de) * WS : nullptr;")
    f("      float* __restrict__ gxs = gx ? gx + int64_t(ds) * XS : nullptr;")
    f("#pragma unroll")
    f("      for (int k = 0; k < CPL; ++k) {")
    f("        if (!ok[k]) continue;")
    for j, p in enumerate(ps):
        f(f"        if (gwe) __builtin_nontemporal_store(dgw[k][{j}], gwe + {p['k']} * C + cc[k]);")
    f("        if (gxs) {")
    for c in xs:
        f(f"          atomicAdd(gxs + {c} * C + cc[k], dgx[k][{xi[c]}]);")
    f("        }")
    f("      }")
    f(f"      if (gyp && (lane & (64 / {V} - 1)) == 0 && dcomp < {cfg.NY}) "
      f"gyp[(int64_t(de) * npart + pidx) * {cfg.NY} + dcomp] = dgy;")
    f("    }")
    a(f"  float dgw[CPL][{len(ps)}], dgx[CPL][{len(xs)}], dgy = 0.f;")
    a(f"  const int dcomp = reduce_scatter_index<{V}>(lane);")
    a("  int de = 0, ds = 0;")
    a("  bool pend = false;")
    _emit_edge_loop_head(a, cfg, ps, xs, ys, xi, flush)
    a(f"    float gy[{V}];")
    a("#pragma unroll")
    a(f"    for (int i = 0; i < {V}; ++i) gy[i] = 0.f;")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k) {")
    a(f"      float gxl[{len(xs)}];")
    for c in xs:
        a(f"      gxl[{xi[c]}] = 0.f;")
    for j, p in enumerate(ps):
        n1, n2 = 2 * p["l1"] + 1, 2 * p["l2"] + 1
        for m1 in range(n1):
            ts = [m2 for m2 in range(n2) if (j, m1, m2) in vnames]
            if not ts:
                continue
            expr = f"y{p['o2'] + ts[0]} * v[k][{vnames[(j, m1, ts[0])]}]"
            for m2 in ts[1:]:
                expr = f"fmaf(y{p['o2'] + m2}, v[k][{vnames[(j, m1, m2)]}], {expr})"
            a(f"      const float u{j}_{m1} = {expr};")
            a(f"      gxl[{xi[p['o1'] + m1]}] = fmaf(wv[k][{j}], u{j}_{m1}, gxl[{xi[p['o1'] + m1]}]);")
        svals = []
        for m2 in range(n2):
            ts = [m1 for m1 in range(n1) if (j, m1, m2) in vnames]
            if not ts:
                continue
            expr = f"xv[k][{xi[p['o1'] + ts[0]]}] * v[k][{vnames[(j, ts[0], m2)]}]"
            for m1 in ts[1:]:
                expr = f"fmaf(xv[k][{xi[p['o1'] + m1]}], v[k][{vnames[(j, m1, m2)]}], {expr})"
            a(f"      const float s{j}_{m2} = {expr};")
            a(f"      gy[{p['o2'] + m2}] = fmaf(wv[k][{j}], s{j}_{m2}, gy[{p['o2'] + m2}]);")
            svals.append(m2)
        if svals:
            expr = f"y{p['o2'] + svals[0]} * s{j}_{svals[0]}"
            for m2 in svals[1:]:
                expr = f"fmaf(y{p['o2'] + m2}, s{j}_{m2}, {expr})"
        else:
            expr = "0.f"
        a(f"      dgw[k][{j}] = {expr};")
    for c in xs:
        a(f"      dgx[k][{xi[c]}] = gxl[{xi[c]}];")
    a("    }")
    a(f"    if (gyp) dgy = wave_reduce_scatter<{V}>(gy, lane);")
    a("    de = e; ds = s; pend = true;")
    a("  }")
    for line in flush:
        a(line[2:] if line.startswith("  ") else line)
    a("}")
    return "\n".join(L)

# ---------------------------------------------------------------------------
# Sender-major backward: one wavefront per (sender, channel block, path subgroup)
# walks the sender's out-edges (sender CSR), so grad_x of the sender accumulates in
# registers and is stored once -- no atomics.  Per sender and channel the table
# N_p[m2][m3] = sum_m1 c[m1,m2,m3] x[m1] is formed once; per edge, with the
# receiver's output gradient g gathered (read-only, cache resident):
#   u_p[m1] = sum_m3 M_p[m3][m1] g_p[m3]  (M from the wave-uniform harmonics)
#       -> grad_x[m1] += w_p u_p[m1]
#   s_p[m2] = sum_m3 N_p[m2][m3] g_p[m3]
#       -> grad_w_p = sum_m2 Y[m2] s_p[m2],  grad_Y[m2] += w_p s_p[m2] (channel sum)
# Paths of one input l are split into subgroups whose per-channel register state
# stays within SENDER_BUDGET; the first subgroup of an l stores grad_x, later ones add.
# ---------------------------------------------------------------------------

SENDER_BUDGET = 60


def _npairs(p):
    c = p["c"]
    return [(m2, m3) for m2 in range(2 * p["l2"] + 1) for m3 in range(2 * p["l3"] + 1)
            if np.any(np.abs(c[:, m2, m3]) > EPS)]


def _sstate(ps):
    nx = 2 * ps[0]["l1"] + 1
    return sum(len(_npairs(p)) + 2 * (2 * p["l3"] + 1) + 2 for p in ps) + nx


def sender_subgroups(cfg):
    """[(paths, first_of_its_l)] in launch order."""
    subs = []
    for ps in cfg.groups:
        cur, first = [], True
        for p in ps:
            if cur and _sstate(cur + [p]) > SENDER_BUDGET:
                subs.append((cur, first))
                cur, first = [p], False
            else:
                cur = cur + [p]
        if cur:
            subs.append((cur, first))
    return subs


def sender_cpl(ps) -> int:
    return 2 if _sstate(ps) <= SENDER_BUDGET else 1


def _sub_layout(ps):
    xs = [ps[0]["o1"] + m for m in range(2 * ps[0]["l1"] + 1)]
    ys = _uniq([p["o2"] + m for p in ps for m in range(2 * p["l2"] + 1)])
    outs = [p["o3"] + m for p in ps for m in range(2 * p["l3"] + 1)]
    return xs, ys, outs


def gen_bwd_sender(cfg: Cfg, sg: int, ps, first: bool) -> str:
    xs, ys, outs = _sub_layout(ps)
    xi = {c: i for i, c in enumerate(xs)}
    oi = {c: i for i, c in enumerate(outs)}
    yi = {c: i for i, c in enumerate(ys)}
    V = 1
    while V < len(ys):
        V *= 2
    nidx = {}
    for j, p in enumerate(ps):
        for (m2, m3) in _npairs(p):
            nidx[(j, m2, m3)] = len(nidx)
    L = []
    a = L.append
    name = f"tp_bws_c{cfg.idx}_s{sg}"
    a(f"template <int CPL>\n__global__ void __launch_bounds__(64) {name}(const float* __restrict__ x, "
      "const float* __restrict__ Y, const float* __restrict__ w, const float* __restrict__ gout, "
      "const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ perm, const int32_t* __restrict__ rcv, "
      "const int32_t* __restrict__ wrow, "
      "int64_t N, int C, float* __restrict__ gx, float* __restrict__ gw, float* __restrict__ gyp, int, int) {")
    a("  const int64_t s = xcd_node(blockIdx.x, gridDim.x);")
    a("  if (s >= N) return;")
    a("  const int lane = threadIdx.x;")
    a("  int cc[CPL]; bool ok[CPL];")
    a("#pragma unroll")
    a("  for (int k = 0; k < CPL; ++k) { cc[k] = blockIdx.y * (64 * CPL) + 64 * k + lane; ok[k] = cc[k] < C; }")
    a(f"  const int64_t XS = int64_t({cfg.NX}) * C, WS = int64_t({cfg.NP}) * C, OS = int64_t({cfg.NO}) * C;")
    a(f"  float nv[CPL][{max(len(nidx), 1)}], gxa[CPL][{len(xs)}];")
    a("#pragma unroll")
    a("  for (int k = 0; k < CPL; ++k) {")
    a(f"    const float* __restrict__ xr = x + s * XS;")
    for c in xs:
        a(f"    const float x{xi[c]} = ok[k] ? xr[{c} * C + cc[k]] : 0.f;")
    for (j, m2, m3), i in nidx.items():
        p = ps[j]
        terms = [(m1, p["c"][m1, m2, m3]) for m1 in range(2 * p["l1"] + 1) if abs(p["c"][m1, m2, m3]) > EPS]
        expr = f"{f32(terms[0][1])} * x{xi[p['o1'] + terms[0][0]]}"
        for m1, v in terms[1:]:
            expr = f"fmaf({f32(v)}, x{xi[p['o1'] + m1]}, {expr})"
        a(f"    nv[k][{i}] = {expr};")
    for c in xs:
        a(f"    gxa[k][{xi[c]}] = 0.f;")
    a("  }")
    a("  const int beg = row_ptr[s], end = row_ptr[s + 1];")
    a("  int ne = 0, nr = 0;")
    a("  " + " ".join(f"float ny{c} = 0.f;" for c in ys))
    a(f"  float ngv[CPL][{len(outs)}], nwv[CPL][{len(ps)}];")

    def prefetch(indent, t_expr):
        a(f"{indent}{{")
        a(f"{indent}  ne = perm[{t_expr}]; nr = rcv[{t_expr}];")
        a(f"{indent}  const float* __restrict__ Yn = Y + int64_t(ne) * {cfg.NY};")
        for c in ys:
            a(f"{indent}  ny{c} = Yn[{c}];")
        a(f"{indent}  const float* __restrict__ gn = gout + int64_t(nr) * OS;")
        a(f"{indent}  const float* __restrict__ wn = w + int64_t(wrow ? wrow[ne] : ne) * WS;")
        a("#pragma unroll")
        a(f"{indent}  for (int k = 0; k < CPL; ++k) {{")
        for c in outs:
            a(f"{indent}    ngv[k][{oi[c]}] = ok[k] ? gn[{c} * C + cc[k]] : 0.f;")
        for j, p in enumerate(ps):
            a(f"{indent}    nwv[k][{j}] = ok[k] ? __builtin_nontemporal_load(wn + {p['k']} * C + cc[k]) : 0.f;")
        a(f"{indent}  }}")
        a(f"{indent}}}")

    a("  if (beg < end)")
    prefetch("  ", "beg")
    a("  for (int t = beg; t < end; ++t) {")
    a("    const int e = ne;")
    a("    " + " ".join(f"const float y{c} = ny{c};" for c in ys))
    a(f"    float gv[CPL][{len(outs)}], wv[CPL][{len(ps)}];")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k) {")
    a(f"#pragma unroll\n      for (int i = 0; i < {len(outs)}; ++i) gv[k][i] = ngv[k][i];")
    a(f"#pragma unroll\n      for (int i = 0; i < {len(ps)}; ++i) wv[k][i] = nwv[k][i];")
    a("    }")
    a("    if (t + 1 < end)")
    prefetch("    ", "t + 1")
    a("    float* __restrict__ gwe = gw ? gw + int64_t(e) * WS : nullptr;")
    a(f"    float gy[{V}];")
    a("#pragma unroll")
    a(f"    for (int i = 0; i < {V}; ++i) gy[i] = 0.f;")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k) {")
    for j, p in enumerate(ps):
        c = p["c"]
        n1, n2, n3 = 2 * p["l1"] + 1, 2 * p["l2"] + 1, 2 * p["l3"] + 1
        # u_j[m1] = sum_m3 M[m3][m1] g[m3]
        for m1 in range(n1):
            ents = []
            for m3 in range(n3):
                terms = [(m2, c[m1, m2, m3]) for m2 in range(n2) if abs(c[m1, m2, m3]) > EPS]
                if not terms:
                    continue
                expr = f"{f32(terms[0][1])} * y{p['o2'] + terms[0][0]}"
                for m2, v in terms[1:]:
                    expr = f"fmaf({f32(v)}, y{p['o2'] + m2}, {expr})"
                ents.append((m3, expr))
            if not ents:
                continue
            a("      {")
            for m3, expr in ents:
                a(f"        const float M{m3} = {expr};")
            uexpr = f"M{ents[0][0]} * gv[k][{oi[p['o3'] + ents[0][0]]}]"
            for m3, _ in ents[1:]:
                uexpr = f"fmaf(M{m3}, gv[k][{oi[p['o3'] + m3]}], {uexpr})"
            a(f"        gxa[k][{xi[p['o1'] + m1]}] = fmaf(wv[k][{j}], {uexpr}, gxa[k][{xi[p['o1'] + m1]}]);")
            a("      }")
        # s_j[m2] = sum_m3 N[m2][m3] g[m3]
        svals = []
        for m2 in range(n2):
            m3s = [m3 for m3 in range(n3) if (j, m2, m3) in nidx]
            if not m3s:
                continue
            expr = f"nv[k][{nidx[(j, m2, m3s[0])]}] * gv[k][{oi[p['o3'] + m3s[0]]}]"
            for m3 in m3s[1:]:
                expr = f"fmaf(nv[k][{nidx[(j, m2, m3)]}], gv[k][{oi[p['o3'] + m3]}], {expr})"
            a(f"      const float s{j}_{m2} = {expr};")
            a(f"      gy[{yi[p['o2'] + m2]}] = fmaf(wv[k][{j}], s{j}_{m2}, gy[{yi[p['o2'] + m2]}]);")
            svals.append(m2)
        if svals:
            expr = f"y{p['o2'] + svals[0]} * s{j}_{svals[0]}"
            for m2 in svals[1:]:
                expr = f"fmaf(y{p['o2'] + m2}, s{j}_{m2}, {expr})"
        else:
            expr = "0.f"
        a(f"      if (gwe && ok[k]) __builtin_nontemporal_store({expr}, gwe + {p['k']} * C + cc[k]);")
    a("    }")
    # grad_Y accumulates in place (zeroed by the caller): one wave per (edge, component)
    # when the channels fit one block, atomics otherwise
    ymap = "{" + ", ".join(str(c) for c in ys) + "}"
    a("    if (gyp) {")
    a(f"      float r = wave_reduce_scatter<{V}>(gy, lane);")
    a(f"      const int comp = reduce_scatter_index<{V}>(lane);")
    a(f"      constexpr int ymap[{len(ys)}] = {ymap};")
    a(f"      if ((lane & (64 / {V} - 1)) == 0 && comp < {len(ys)}) {{")
    a(f"        float* __restrict__ dst = gyp + int64_t(e) * {cfg.NY} + ymap[comp];")
    a("        if (gridDim.y == 1) *dst += r; else atomicAdd(dst, r);")
    a("      }")
    a("    }")
    a("  }")
    a("  if (gx) {")
    a("#pragma unroll")
    a("    for (int k = 0; k < CPL; ++k) {")
    a("      if (!ok[k]) continue;")
    a("      float* __restrict__ gxs = gx + s * XS;")
    for c in xs:
        if first:
            a(f"      gxs[{c} * C + cc[k]] = gxa[k][{xi[c]}];")
        else:
            a(f"      gxs[{c} * C + cc[k]] += gxa[k][{xi[c]}];")
    a("    }")
    a("  }")
    a("}")
    return "\n".join(L)



# ---------------------------------------------------------------------------
# Backward fused with the radial MLP output layer's input gradient
#   grad_h[e][k] = sum_{p, c} gw[e][p][c] W[p*C + c][k]
# without writing gw.  Persistent workgroups of NWAVE wavefronts; each wavefront
# walks an equal share of the CSR slots (receivers change along the way: the
# receiver's output gradient is folded into v again), one channel block of 64
# per lane row (blockIdx.y).  Every SW edges per wavefront (a phase) the
# workgroup has SLOTS = NWAVE * SW edges' gw rows (this group's P paths x 64
# channels, fp32) in LDS; after a barrier each wavefront multiplies 16-row x
# 16-column tiles of them by the group's slice of W (pre-split fp16 fragments,
# LDS-resident for the whole kernel) on v_mfma_f32_16x16x32_f16, three products
# per k-step (the split-fp16 scheme of edge_weights.hip: rows scaled by a power
# of two from their largest magnitude, W columns likewise), and writes the tile
# into a partial grad_h row per (group, channel block) at the edge's CSR slot;
# a second barrier frees the staging for the next phase.
# ---------------------------------------------------------------------------

FUSED_LDS_BYTES = 160 * 1024
FUSED_KH = (64, 128)


def fused_lds(P: int, KH: int, nwave: int, sw: int) -> int:
    """LDS bytes: the W slice, the staged gw rows (two fp16 planes, rows padded by 16 bytes) and
    per-row exponents and CSR slots."""
    slots = nwave * sw
    return P * KH * 256 + 2 * slots * (P * 64 + 8) * 2 + slots * 8


def fused_shape(ps, KH: int):
    """(NWAVE, SW) of the fused backward for a group ``ps`` of paths and a hidden width KH, or None
    when the group's W slice and the staging do not fit the LDS.  Groups whose folded output
    gradient is small (at most 30 values per lane) fit four wavefronts per SIMD without spilling:
    sixteen per workgroup; larger ones eight."""
    P = len(ps)
    for nw in ((16, 8) if _v_count(ps) <= 30 else (8,)):
        # as many staged rows (slots) per phase as the LDS holds
        for slots in range(128, 7, -8):
            if slots % nw == 0 and fused_lds(P, KH, nw, slots // nw) <= FUSED_LDS_BYTES:
                return nw, slots // nw
    return None


def gen_bwd_fused(cfg: Cfg, g: int) -> str:
    ps = cfg.groups[g]
    P = len(ps)
    xs, ys, outs = _group_layout(ps)
    xi = {c: i for i, c in enumerate(xs)}
    oi = {c: i for i, c in enumerate(outs)}
    V = 1
    while V < cfg.NY:
        V *= 2
    L = []
    a = L.append
    name = f"tp_bwf_c{cfg.idx}_g{g}"
    a(f"template <int NWAVE, int SW, int KH>\n__global__ void __launch_bounds__(64 * NWAVE, NWAVE / 4) {name}("
      "const float* __restrict__ x, const float* __restrict__ Y, const float* __restrict__ w, "
      "const float* __restrict__ gout, const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ perm, "
      "const int32_t* __restrict__ snd, const int32_t* __restrict__ wrow, int64_t N, int64_t E, int C, "
      "float* __restrict__ gx, float* __restrict__ gyp, int npart, int pbase, const f16x8* __restrict__ wfrag, "
      "const float* __restrict__ kscale, float* __restrict__ hpart) {")
    a(f"  constexpr int P = {P}, SLOTS = NWAVE * SW, AST = P * 64 + 8, KSTEPS = P * 2, CT = KH / 16;")
    a("  extern __shared__ __align__(16) unsigned char smem[];")
    a("  f16x8* __restrict__ sW = reinterpret_cast<f16x8*>(smem);  // [CT][KSTEPS][2][64]")
    a("  _Float16* __restrict__ sA = reinterpret_cast<_Float16*>(smem + P * KH * 256);  // [2][SLOTS][AST]")
    a("  int* __restrict__ sE = reinterpret_cast<int*>(sA + 2 * SLOTS * AST);  // row exponents")
    a("  int* __restrict__ sT = sE + SLOTS;  // CSR slot of each row, -1 if none")
    a("  const int lane = threadIdx.x & 63;")
    a("  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);")
    a("  const int cb = blockIdx.y;")
    a("  const int cc = cb * 64 + lane;")
    a("  {  // this (group, channel block)'s W fragments, resident for the whole kernel")
    a("    constexpr int NV = P * KH * 16;")
    a("    const f16x8* __restrict__ src = wfrag + int64_t(cb) * NV;")
    a("    for (int i = threadIdx.x; i < NV; i += 64 * NWAVE) sW[i] = src[i];")
    a("  }")
    a("  // this wavefront's share of the CSR slots; each XCD walks one contiguous range")
    a("  const int64_t nwg = gridDim.x;")
    a("  const int64_t lb = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);")
    a("  const int64_t nwaves = nwg * NWAVE, wid = lb * NWAVE + wave;")
    a("  const int t0 = int(wid * E / nwaves), t1 = int((wid + 1) * E / nwaves);")
    a("  const int nph = int(((E + nwaves - 1) / nwaves + SW - 1) / SW);")
    a(f"  const int64_t XS = int64_t({cfg.NX}) * C, WS = int64_t({cfg.NP}) * C;")
    a("  // receiver of slot t0: the last n with row_ptr[n] <= t0")
    a("  int n = 0, rend = 0;")
    a("  if (t0 < t1) {")
    a("    int lo = 0, hi = int(N);")
    a("    while (hi - lo > 1) { const int mid = (lo + hi) >> 1; if (row_ptr[mid] <= t0) lo = mid; else hi = mid; }")
    a("    n = lo; rend = row_ptr[n + 1];")
    a("  }")
    # folded output gradient of the current receiver
    vnames = {}
    nv = _v_count(ps)
    a(f"  float v[{nv}];")

    def emit_fold(indent):
        a(f"{indent}{{")
        a(f"{indent}  const float* __restrict__ gn = gout + int64_t(n) * {cfg.NO} * C;")
        a(f"{indent}  float gv[{len(outs)}];")
        for c in outs:
            a(f"{indent}  gv[{oi[c]}] = gn[{c} * C + cc];")
        vi = 0
        for j, p in enumerate(ps):
            c = p["c"]
            for m1 in range(2 * p["l1"] + 1):
                for m2 in range(2 * p["l2"] + 1):
                    terms = [(m3, c[m1, m2, m3]) for m3 in range(2 * p["l3"] + 1) if abs(c[m1, m2, m3]) > EPS]
                    if not terms:
                        continue
                    expr = f"{f32(terms[0][1])} * gv[{oi[p['o3'] + terms[0][0]]}]"
                    for m3, val in terms[1:]:
                        expr = f"fmaf({f32(val)}, gv[{oi[p['o3'] + m3]}], {expr})"
                    a(f"{indent}  v[{vi}] = {expr};")
                    vnames[(j, m1, m2)] = vi
                    vi += 1
        a(f"{indent}}}")

    a(f"#pragma unroll\n  for (int i = 0; i < {nv}; ++i) v[i] = 0.f;")
    a("  if (t0 < t1)")
    emit_fold("  ")
    # prefetch pipeline over [t0, t1)
    a("  int ne = 0, ns = 0, nw = 0, ie = 0, is = 0, iw = 0;")
    a("  " + " ".join(f"float ny{c} = 0.f;" for c in ys))
    a(f"  float nxv[1][{len(xs)}], nwv[1][{len(ps)}];")
    a("  if (t0 < t1) {")
    _emit_ids(a, "    ", "t0", ("ne", "ns", "nw"))
    _emit_prefetch_c(a, cfg, ps, xs, ys, xi, "    ")
    a("  }")
    a("  if (t0 + 1 < t1) {")
    _emit_ids(a, "    ", "t0 + 1")
    a("  }")
    a("  int t = t0;")
    a("  for (int ph = 0; ph < nph; ++ph) {")
    a("    for (int i = 0; i < SW; ++i) {")
    a("      const int slot = wave * SW + i;")
    a("      _Float16* __restrict__ arow = sA + slot * AST;")
    a("      if (t >= t1) {")
    a("        if (lane == 0) { sT[slot] = -1; sE[slot] = 0; }")
    a("        continue;")
    a("      }")
    a("      if (t == rend) {  // next receiver (skipping empty ones): fold its output gradient")
    a("        do { ++n; rend = row_ptr[n + 1]; } while (rend == t);")
    emit_fold("        ")
    a("      }")
    a("      const int e = ne, s = ns;")
    a("      " + " ".join(f"const float y{c} = ny{c};" for c in ys))
    a(f"      float xv[{len(xs)}], wv[{len(ps)}];")
    a(f"#pragma unroll\n      for (int q = 0; q < {len(xs)}; ++q) xv[q] = nxv[0][q];")
    a(f"#pragma unroll\n      for (int q = 0; q < {len(ps)}; ++q) wv[q] = nwv[0][q];")
    a("      if (t + 1 < t1) {")
    a("        ne = ie; ns = is; nw = iw;")
    _emit_prefetch_c(a, cfg, ps, xs, ys, xi, "        ")
    a("        if (t + 2 < t1) {")
    _emit_ids(a, "          ", "t + 2")
    a("        }")
    a("      }")
    a(f"      float gy[{V}];")
    a(f"#pragma unroll\n      for (int q = 0; q < {V}; ++q) gy[q] = 0.f;")
    a(f"      float gxl[{len(xs)}], gwv[{P}];")
    for c in xs:
        a(f"      gxl[{xi[c]}] = 0.f;")
    for j, p in enumerate(ps):
        n1, n2 = 2 * p["l1"] + 1, 2 * p["l2"] + 1
        for m1 in range(n1):
            ts = [m2 for m2 in range(n2) if (j, m1, m2) in vnames]
            if not ts:
                continue
            expr = f"y{p['o2'] + ts[0]} * v[{vnames[(j, m1, ts[0])]}]"
            for m2 in ts[1:]:
                expr = f"fmaf(y{p['o2'] + m2}, v[{vnames[(j, m1, m2)]}], {expr})"
            a(f"      const float u{j}_{m1} = {expr};")
            a(f"      gxl[{xi[p['o1'] + m1]}] = fmaf(wv[{j}], u{j}_{m1}, gxl[{xi[p['o1'] + m1]}]);")
        svals = []
        for m2 in range(n2):
            ts = [m1 for m1 in range(n1) if (j, m1, m2) in vnames]
            if not ts:
                continue
            expr = f"xv[{xi[p['o1'] + ts[0]]}] * v[{vnames[(j, ts[0], m2)]}]"
            for m1 in ts[1:]:
                expr = f"fmaf(xv[{xi[p['o1'] + m1]}], v[{vnames[(j, m1, m2)]}], {expr})"
            a(f"      const float s{j}_{m2} = {expr};")
            a(f"      gy[{p['o2'] + m2}] = fmaf(wv[{j}], s{j}_{m2}, gy[{p['o2'] + m2}]);")
            svals.append(m2)
        if svals:
            expr = f"y{p['o2'] + svals[0]} * s{j}_{svals[0]}"
            for m2 in svals[1:]:
                expr = f"fmaf(y{p['o2'] + m2}, s{j}_{m2}, {expr})"
        else:
            expr = "0.f"
        a(f"      gwv[{j}] = {expr};")
    a("      if (gx) {")
    a("        float* __restrict__ gxs = gx + int64_t(s) * XS;")
    for c in xs:
        a(f"        atomicAdd(gxs + {c} * C + cc, gxl[{xi[c]}]);")
    a("      }")
    a("      if (gyp) {")
    a(f"        float r = wave_reduce_scatter<{V}>(gy, lane);")
    a(f"        const int comp = reduce_scatter_index<{V}>(lane);")
    a(f"        if ((lane & (64 / {V} - 1)) == 0 && comp < {cfg.NY}) "
      f"gyp[(int64_t(e) * npart + pbase + cb) * {cfg.NY} + comp] = r;")
    a("      }")
    a("      // gw row of this edge into the staging, scaled by the row's power of two and split")
    a("      // into two fp16 parts (the matrix-core operand planes)")
    a(f"      float m = fabsf(gwv[0]);")
    a(f"#pragma unroll\n      for (int q = 1; q < {P}; ++q) m = fmaxf(m, fabsf(gwv[q]));")
    a("      const int ex = ew_exp(wave_max(m));")
    a("      const float sc = ldexpf(1.f, -ex);")
    a(f"#pragma unroll\n      for (int q = 0; q < {P}; ++q) {{")
    a("        const float v = gwv[q] * sc;")
    a("        const _Float16 h0 = (_Float16)v;")
    a("        arow[q * 64 + lane] = h0;")
    a("        arow[SLOTS * AST + q * 64 + lane] = (_Float16)(v - (float)h0);")
    a("      }")
    a("      if (lane == 0) { sT[slot] = t; sE[slot] = ex; }")
    a("      ++t;")
    a("    }")
    a("    __syncthreads();")
    a("    fused_gh_tiles<P, NWAVE, SW, KH>(sW, sA, sE, sT, kscale, hpart + int64_t(cb) * E * KH, lane, wave);")
    a("    __syncthreads();")
    a("  }")
    a("}")
    return "\n".join(L)


def _emit_prefetch_c(a, cfg, ps, xs, ys, xi, indent):
    """_emit_prefetch for one channel per lane, channel ``cc`` (no guards: C % 64 == 0)."""
    a(f"{indent}{{")
    a(f"{indent}  const float* __restrict__ Yn = Y + int64_t(ne) * {cfg.NY};")
    for c in ys:
        a(f"{indent}  ny{c} = Yn[{c}];")
    a(f"{indent}  const float* __restrict__ xn = x + int64_t(ns) * XS;")
    a(f"{indent}  const float* __restrict__ wn = w + int64_t(nw) * WS;")
    for c in xs:
        a(f"{indent}  nxv[0][{xi[c]}] = xn[{c} * C + cc];")
    for j, p in enumerate(ps):
        a(f"{indent}  nwv[0][{j}] = __builtin_nontemporal_load(wn + {p['k']} * C + cc);")
    a(f"{indent}}}")


def fused_configs():
    """(config index, group, KH, NWAVE, SW) of every fused backward instantiation."""
    out = []
    for i, c in enumerate(config_list()):
        cfg = Cfg(i, *c)
        for g, ps in enumerate(cfg.groups):
            for KH in FUSED_KH:
                sh = fused_shape(ps, KH)
                if sh:
                    out.append((i, g, KH, *sh))
    return out


def generate_fused() -> str:
    cfgs = [Cfg(i, *c) for i, c in enumerate(config_list())]
    out = ["// Generated by gen_tp.py -- do not edit.", "// clang-format off", ""]
    for cfg in cfgs:
        for g in range(len(cfg.groups)):
            out.append(gen_bwd_fused(cfg, g))
            out.append("")
    inst = fused_configs()
    out.append(f"static constexpr int kNumFusedKH = {len(FUSED_KH)};")
    out.append("static constexpr int kFusedKH[] = {" + ", ".join(str(k) for k in FUSED_KH) + "};")
    # per config and group: paths (weight-row indices), then per hidden width the kernel, its shape and LDS bytes
    out.append("static const TPFusedGroup kTPFused[][4] = {")
    for cfg in cfgs:
        row = []
        for g in range(4):
            if g >= len(cfg.groups):
                row.append("{0, {0}, {{nullptr, 0, 0, 0}, {nullptr, 0, 0, 0}}}")
                continue
            ps = cfg.groups[g]
            pk = "{" + ", ".join(str(p["k"]) for p in ps) + "}"
            ks = []
            for KH in FUSED_KH:
                sh = fused_shape(ps, KH)
                if sh:
                    nw, sw = sh
                    ks.append(f"{{tp_bwf_c{cfg.idx}_g{g}<{nw}, {sw}, {KH}>, {nw}, {sw}, "
                              f"{fused_lds(len(ps), KH, nw, sw)}}}")
                else:
                    ks.append("{nullptr, 0, 0, 0}")
            row.append(f"{{{len(ps)}, {pk}, {{{', '.join(ks)}}}}}")
        out.append("  {" + ", ".join(row) + "},")
    out.append("};")
    return "\n".join(out) + "\n"


def generate() -> str:
    cfgs = [Cfg(i, *c) for i, c in enumerate(config_list())]
    out = ["// Generated by gen_tp.py -- do not edit.", "// clang-format off", ""]
    for cfg in cfgs:
        im, sm, om = cfg.masks
        out.append(f"// config {cfg.idx}: in l={cfg.in_ls} sh l={cfg.sh_ls} out l={cfg.out_ls}; "
                   f"{cfg.NP} paths, NX={cfg.NX} NY={cfg.NY} NO={cfg.NO}")
        for g in range(len(cfg.groups)):
            out.append(gen_fwd(cfg, g))
            out.append("")
            out.append(gen_bwd(cfg, g))
            out.append("")
        for sg, (ps, first) in enumerate(sender_subgroups(cfg)):
            out.append(gen_bwd_sender(cfg, sg, ps, first))
            out.append("")
    # dispatch tables
    out.append("static const TPConfigInfo kTPConfigs[] = {")
    for cfg in cfgs:
        im, sm, om = cfg.masks
        out.append(f"  {{{im}, {sm}, {om}, {cfg.NP}, {cfg.NX}, {cfg.NY}, {cfg.NO}, {len(cfg.groups)}}},")
    out.append("};")
    out.append(f"static constexpr int kNumTPConfigs = {len(cfgs)};")
    # FULL: every lane's channels exist (C a multiple of 64 x CPL), no per-load guards
    for full, tag in ((False, ""), (True, "F")):
        fl = "true" if full else "false"
        for cpl in (1, 2):
            out.append(f"static const TPFwdFn kTPFwd{tag}{cpl}[][4] = {{")
            for cfg in cfgs:
                fns = [f"tp_fwd_c{cfg.idx}_g{g}<{cpl}, {fl}>" for g in range(len(cfg.groups))]
                fns += ["nullptr"] * (4 - len(fns))
                out.append("  {" + ", ".join(fns) + "},")
            out.append("};")
        # backward: one instantiation per group, channels per lane chosen by register budget
        out.append(f"static const TPBwdFn kTPBwd{tag}[][4] = {{")
        for cfg in cfgs:
            fns = [f"tp_bwd_c{cfg.idx}_g{g}<{bwd_cpl(ps)}, {fl}>" for g, ps in enumerate(cfg.groups)]
            fns += ["nullptr"] * (4 - len(fns))
            out.append("  {" + ", ".join(fns) + "},")
        out.append("};")
    out.append("static const int kTPBwdCPL[][4] = {")
    for cfg in cfgs:
        cp = [str(bwd_cpl(ps)) for ps in cfg.groups] + ["0"] * (4 - len(cfg.groups))
        out.append("  {" + ", ".join(cp) + "},")
    out.append("};")
    # path range of each group: groups hold consecutive paths (paths are enumerated by input block)
    out.append("static const int kTPGroupPaths[][5] = {")
    for cfg in cfgs:
        bounds = [cfg.groups[0][0]["k"]]
        for ps in cfg.groups:
            ks = [p["k"] for p in ps]
            assert ks == list(range(bounds[-1], bounds[-1] + len(ks))), "group paths must be consecutive"
            bounds.append(bounds[-1] + len(ks))
        assert bounds[0] == 0 and bounds[-1] == cfg.NP
        bounds += [bounds[-1]] * (5 - len(bounds))
        out.append("  {" + ", ".join(str(b) for b in bounds) + "},")
    out.append("};")
    # sender-major backward: subgroups, channels per lane, harmonics components per subgroup
    subs = [sender_subgroups(cfg) for cfg in cfgs]
    ms = max(len(x) for x in subs)
    out.append(f"static constexpr int kTPMaxSub = {ms};")
    out.append("static const int kTPBwSNum[] = {" + ", ".join(str(len(x)) for x in subs) + "};")
    out.append(f"static const TPBwdFn kTPBwS[][{ms}] = {{")
    for cfg, sl in zip(cfgs, subs):
        fns = [f"tp_bws_c{cfg.idx}_s{sg}<{sender_cpl(ps)}>" for sg, (ps, _) in enumerate(sl)]
        fns += ["nullptr"] * (ms - len(fns))
        out.append("  {" + ", ".join(fns) + "},")
    out.append("};")
    out.append(f"static const int kTPBwSCPL[][{ms}] = {{")
    for sl in subs:
        cp = [str(sender_cpl(ps)) for ps, _ in sl] + ["0"] * (ms - len(sl))
        out.append("  {" + ", ".join(cp) + "},")
    out.append("};")
    return "\n".join(out) + "\n"


# ---------------------------------------------------------------------------
# Fused weight gradient (tp_gh.hip): per edge lane and path p, the gradient of the
# per-edge weights for 8 consecutive channels,
#   gw_p[c] = sum_m3 g[r][o3 + m3][c] * sum_m1 M_p[m3][m1] x[s][o1 + m1][c],
#   M_p[m3][m1] = sum_m2 c_p[m1, m2, m3] Y[e][o2 + m2]
# (the same quantity the receiver-walked backward stores as grad_w), produced in
# registers for the matrix-core product with the output layer's weights.
# ---------------------------------------------------------------------------


def gen_grad_h(cfg: Cfg) -> str:
    L = []
    a = L.append
    a(f"template <> struct TPGH<{cfg.idx}> {{")
    a(f"  static constexpr int NX = {cfg.NX}, NY = {cfg.NY}, NO = {cfg.NO}, NP = {cfg.NP};")
    a("  // gw[j] for path p, channels c + j (xr, gr already offset by c); y: the edge's harmonics")
    a(f"  __device__ static __forceinline__ void gw(int p, const float* __restrict__ xr, "
      f"const float* __restrict__ gr, int C, const float (&y)[{cfg.NY}], float (&out)[8]) {{")
    a("    switch (p) {")
    for p in cfg.paths:
        c = p["c"]
        n1, n3 = 2 * p["l1"] + 1, 2 * p["l3"] + 1
        a(f"      case {p['k']}: {{")
        a(f"        f32x4 xv[{n1}][2], gv[{n3}][2];")
        for m1 in range(n1):
            a(f"        xv[{m1}][0] = *reinterpret_cast<const f32x4*>(xr + {p['o1'] + m1} * C);")
            a(f"        xv[{m1}][1] = *reinterpret_cast<const f32x4*>(xr + {p['o1'] + m1} * C + 4);")
        for m3 in range(n3):
            a(f"        gv[{m3}][0] = *reinterpret_cast<const f32x4*>(gr + {p['o3'] + m3} * C);")
            a(f"        gv[{m3}][1] = *reinterpret_cast<const f32x4*>(gr + {p['o3'] + m3} * C + 4);")
        rows = []
        for m3 in range(n3):
            row = []
            for m1 in range(n1):
                terms = [(m2, c[m1, m2, m3]) for m2 in range(2 * p["l2"] + 1) if abs(c[m1, m2, m3]) > EPS]
                if not terms:
                    continue
                expr = f"{f32(terms[0][1])} * y[{p['o2'] + terms[0][0]}]"
                for m2, v in terms[1:]:
                    expr = f"fmaf({f32(v)}, y[{p['o2'] + m2}], {expr})"
                a(f"        const float M{m3}_{m1} = {expr};")
                row.append(m1)
            rows.append(row)
        a("#pragma unroll")
        a("        for (int j = 0; j < 8; ++j) {")
        a("          const int h = j >> 2, i = j & 3;")
        a("          float acc = 0.f;")
        for m3, row in enumerate(rows):
            if not row:
                continue
            expr = f"M{m3}_{row[0]} * xv[{row[0]}][h][i]"
            for m1 in row[1:]:
                expr = f"fmaf(M{m3}_{m1}, xv[{m1}][h][i], {expr})"
            a(f"          acc = fmaf(gv[{m3}][h][i], {expr}, acc);")
        a("          out[j] = acc;")
        a("        }")
        a("      } break;")
    a("      default:")
    a("#pragma unroll")
    a("        for (int j = 0; j < 8; ++j) out[j] = 0.f;")
    a("    }")
    a("  }")
    a("};")
    return "\n".join(L)


# ---------------------------------------------------------------------------
# Receiver-batched fused weight gradient (tp_gh.hip, k_tp_gh2): the contraction
# index n = p*C + c of grad_h = gw W is walked group by group (paths sharing l1),
# within a group by 16-channel chunk, within a chunk by path.  Per (group,
# chunk) a lane holds its edge's sender rows of the group (n1 rows x 8 channels)
# in registers, and the wavefront -- 32 edges of one receiver -- stages that
# receiver's output-gradient rows of the group's paths (16 channels each) in
# LDS; each k-step then forms gw for one path and 8 channels from registers and
# LDS only.
# ---------------------------------------------------------------------------


def gh2_layout(cfg: Cfg):
    """Per group: (paths, x row offset o1, n1, g rows [(path j, m3) -> LDS row], rows)."""
    out = []
    for ps in cfg.groups:
        rows = []
        for j, p in enumerate(ps):
            for m3 in range(2 * p["l3"] + 1):
                rows.append(p["o3"] + m3)
        out.append(dict(paths=ps, o1=ps[0]["o1"], n1=2 * ps[0]["l1"] + 1, grows=rows))
    return out


def gh2_order(cfg: Cfg, C: int):
    """W rows in the kernel's contraction order (the order of its k-steps' 16 rows each)."""
    rows = []
    for grp in gh2_layout(cfg):
        for cc in range(C // 16):
            for p in grp["paths"]:
                rows.extend(range(p["k"] * C + 16 * cc, p["k"] * C + 16 * cc + 16))
    return rows


def gen_grad_h2(cfg: Cfg) -> str:
    """TPGH2<cfg>::run: the whole contraction of k_tp_gh2 for one configuration, groups and paths
    unrolled (every register index static), the 16-channel chunks a runtime loop.  Per chunk the
    lane's sender rows and its share of the receiver's output-gradient rows for the next chunk are
    loaded into registers while the current chunk's k-steps run; the gradient rows go to the
    wavefront's LDS area (two buffers) at the end of the chunk.  Each k-step hands the lane's 8 gw
    values to the caller's sink (S::step), which does the matrix-core part."""
    lay = gh2_layout(cfg)
    NG = len(lay)
    gmax = max(len(g["grows"]) for g in lay)
    L = []
    a = L.append
    a(f"template <> struct TPGH2<{cfg.idx}> {{")
    a(f"  static constexpr int NG = {NG}, NX = {cfg.NX}, NY = {cfg.NY}, NO = {cfg.NO}, NP = {cfg.NP}, "
      f"GROWS = {gmax};")
    order = [p["k"] for g in lay for p in g["paths"]]
    a(f"  static constexpr int GP[NG] = {{{', '.join(str(len(g['paths'])) for g in lay)}}};")
    a(f"  static constexpr int ORDER[NP] = {{{', '.join(str(k) for k in order)}}};  // paths, group by group")
    a("  template <class S>")
    a("  __device__ static __forceinline__ void run(S& st, const float* __restrict__ xr, const float* __restrict__ grow,")
    a(f"                                              int C, float* __restrict__ lds, int lane, bool eok, bool bok,")
    a(f"                                              const float (&y)[{cfg.NY}]) {{")
    a("    const int cpk = C >> 4;")
    a("    const int hoff = 8 * (lane >> 5);")
    a("    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};")
    for gi, g in enumerate(lay):
        n1, o1, rows = g["n1"], g["o1"], g["grows"]
        nsh = -(-len(rows) * 4 // 64)  # this lane's shares of the gradient rows
        a(f"    {{  // group {gi}: l1 = {g['paths'][0]['l1']}, {len(g['paths'])} paths, {len(rows)} gradient rows")
        a("      " + " ".join(f"f32x4 a{m}, b{m}, na{m}, nb{m};" for m in range(n1)))
        a("      " + " ".join(f"f32x4 gp{k}; int go{k} = -1;" for k in range(nsh)))
        for k in range(nsh):
            a(f"      if (lane + {64 * k} < {len(rows) * 4}) go{k} = kGH2Rows_c{cfg.idx}_g{gi}[(lane + {64 * k}) >> 2] * C + "
              f"4 * ((lane + {64 * k}) & 3);")
        # chunk 0: x and gradient rows directly
        a("      if (eok) {")
        for m in range(n1):
            a(f"        a{m} = *reinterpret_cast<const f32x4*>(xr + {o1 + m} * C);")
            a(f"        b{m} = *reinterpret_cast<const f32x4*>(xr + {o1 + m} * C + 4);")
        a("      } else {")
        a("        " + " ".join(f"a{m} = z4; b{m} = z4;" for m in range(n1)))
        a("      }")
        a("      if (bok) {")
        for k in range(nsh):
            a(f"        if (go{k} >= 0) *reinterpret_cast<f32x4*>(lds + 4 * (lane + {64 * k})) = "
              f"*reinterpret_cast<const f32x4*>(grow + go{k});")
        a("      }")
        a("      for (int cc = 0; cc < cpk; ++cc) {")
        a(f"        const float* __restrict__ gl = lds + (cc & 1) * {gmax * 16} + hoff;")
        a("        const bool more = cc + 1 < cpk;")
        a("        if (more && eok) {")
        for m in range(n1):
            a(f"          na{m} = *reinterpret_cast<const f32x4*>(xr + 16 * (cc + 1) + {o1 + m} * C);")
            a(f"          nb{m} = *reinterpret_cast<const f32x4*>(xr + 16 * (cc + 1) + {o1 + m} * C + 4);")
        a("        }")
        a("        if (more && bok) {")
        for k in range(nsh):
            a(f"          if (go{k} >= 0) gp{k} = *reinterpret_cast<const f32x4*>(grow + 16 * (cc + 1) + go{k});")
        a("        }")
        base = 0
        for j, p in enumerate(g["paths"]):
            c = p["c"]
            n3 = 2 * p["l3"] + 1
            a(f"        {{  // path {p['k']}: ({p['l1']}, {p['l2']}) -> {p['l3']}")
            a("          f32x4 o0 = z4, o1 = z4;")
            a("          if (eok) {")
            rws = []
            for m3 in range(n3):
                row = []
                for m1 in range(n1):
                    terms = [(m2, c[m1, m2, m3]) for m2 in range(2 * p["l2"] + 1) if abs(c[m1, m2, m3]) > EPS]
                    if not terms:
                        continue
                    expr = f"{f32(terms[0][1])} * y[{p['o2'] + terms[0][0]}]"
                    for m2, v in terms[1:]:
                        expr = f"fmaf({f32(v)}, y[{p['o2'] + m2}], {expr})"
                    a(f"            const float M{m3}_{m1} = {expr};")
                    row.append(m1)
                rws.append(row)
            for m3, row in enumerate(rws):
                if not row:
                    continue
                a("            {")
                a(f"              const f32x4 g0 = *reinterpret_cast<const f32x4*>(gl + {(base + m3) * 16});")
                a(f"              const f32x4 g1 = *reinterpret_cast<const f32x4*>(gl + {(base + m3) * 16 + 4});")
                for q in range(8):
                    h, i = q >> 2, q & 3
                    xn = "ab"[h]
                    expr = f"M{m3}_{row[0]} * {xn}{row[0]}[{i}]"
                    for m1 in row[1:]:
                        expr = f"fmaf(M{m3}_{m1}, {xn}{m1}[{i}], {expr})"
                    a(f"              o{h}[{i}] = fmaf(g{h}[{i}], {expr}, o{h}[{i}]);")
                a("            }")
            a("          }")
            a("          st.step(o0, o1);")
            a("        }")
            base += n3
        a("        if (more) {")
        a("          " + " ".join(f"a{m} = na{m}; b{m} = nb{m};" for m in range(n1)))
        a("          if (bok) {")
        a(f"            float* __restrict__ gn = lds + ((cc + 1) & 1) * {gmax * 16};")
        for k in range(nsh):
            a(f"            if (go{k} >= 0) *reinterpret_cast<f32x4*>(gn + 4 * (lane + {64 * k})) = gp{k};")
        a("          }")
        a("        }")
        a("      }")
        a("    }")
    a("  }")
    a("};")
    return "\n".join(L)


def gen_gh2_tables(cfg: Cfg) -> str:
    """Constant-memory row lists of the groups' output-gradient rows (stage_g)."""
    out = []
    for gi, g in enumerate(gh2_layout(cfg)):
        rows = g["grows"]
        out.append(f"__constant__ int kGH2Rows_c{cfg.idx}_g{gi}[{len(rows)}] = "
                   f"{{{', '.join(str(r) for r in rows)}}};")
    return "\n".join(out)


def generate_gh() -> str:
    cfgs = [Cfg(i, *c) for i, c in enumerate(config_list())]
    out = ["// Generated by molnex_amd/csrc/gen_tp.py -- do not edit.",
           "// Fused tensor-product weight gradient: per-path gw producers (TPGH<config>) and the",
           "// receiver-batched form (TPGH2<config>)."]
    for cfg in cfgs:
        out.append(f"// config {cfg.idx}: in l={cfg.in_ls} sh l={cfg.sh_ls} out l={cfg.out_ls}")
        out.append(gen_grad_h(cfg))
        out.append(gen_gh2_tables(cfg))
        out.append(gen_grad_h2(cfg))
        out.append("")
    out.append(f"static constexpr int kNumTPGHConfigs = {len(cfgs)};")
    return "\n".join(out) + "\n"


def _write(path, text):
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as f:
            f.write(text)


def main():
    path = os.path.join(HERE, "tp_gen.inc")
    _write(path, generate())
    _write(os.path.join(HERE, "tp_gh_gen.inc"), generate_gh())
    _write(os.path.join(HERE, "tp_bwf_gen.inc"), generate_fused())
    return path


if __name__ == "__main__":
    print(main())
