"""Generate the equivariant symmetric-contraction kernels (``sc_gen.inc``).

Per node n of element z and channel c, with A the node features (irreps
0e + 1o + ... + l_in, one block per l, ir_mul layout) and the product basis of
``molnex_amd.symmetric`` (U_{L,nu,k} stored on sorted index tuples q with the
permutation multiplicity folded into coef[k, M, q]):

    P_k[M]  = sum_q coef_k[M, q] * A[q_1] ... A[q_nu]          (generated FMAs)
    B[L, M] = sum_{nu, k} W[z, p(L, nu, k), c] * P_k[M]

Backward, with g = dLoss/dB and h_{k,q} = sum_M coef_k[M, q] g[L_k, M]:
    dW[z, p, c] += sum_q h_{p,q} * mono_q(A)
    dA[x]        = sum_q (sum_k W_k h_{k,q}) * d mono_q / d A[x]

Every supported configuration (l_in in 1..3, L_out in 0..1, correlation 1..3)
becomes straight-line HIP code with the coefficients as constants.  Paths are
ordered by output L, then correlation, then basis index; the weight tensor is
W[element][path][channel].

Run as ``python -m molnex_amd.csrc.gen_sc`` (``build()`` does this).
"""

from __future__ import annotations

import os
import sys
from collections import defaultdict

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from molnex_amd.symmetric import ProductBasisDescriptor  # noqa: E402

EPS = 1e-10


def config_list():
    return [(li, lo, nu) for li in (1, 2, 3) for lo in (0, 1) for nu in (1, 2, 3)]


def f32(v: float) -> str:
    return f"{float(np.float32(v)):.9e}f"


class Cfg:
    def __init__(self, idx, l_in, l_out, nu):
        self.idx, self.l_in, self.l_out, self.nu = idx, l_in, l_out, nu
        self.desc = ProductBasisDescriptor(tuple(range(l_in + 1)), tuple(range(l_out + 1)), nu)
        self.ni = (l_in + 1) ** 2
        self.no = (l_out + 1) ** 2
        self.paths = self.desc.num_paths
        # terms[q] = (monomial, [(path, M_global, coef)]) over all parts, monomials in sorted order
        by_mono = defaultdict(list)
        p0 = 0
        for L, nu_, r, monos, coef in self.desc.parts:
            moff = L * L
            for qi, mono in enumerate(monos):
                for k in range(r):
                    for M in range(2 * L + 1):
                        v = coef[k, M, qi]
                        if abs(v) > EPS:
                            by_mono[mono].append((p0 + k, moff + M, float(v)))
            p0 += r
        self.terms = sorted(by_mono.items(), key=lambda t: (len(t[0]), t[0]))
        self.path_L = []
        for L, nu_, r, _, _ in self.desc.parts:
            self.path_L += [L] * r
        self.nnz = sum(len(t) for _, t in self.terms)
        self.used = sorted({i for mono, _ in self.terms for i in mono})


def _mono_expr(mono):
    if len(mono) == 1:
        return f"a{mono[0]}"
    if len(mono) == 2:
        return f"a{mono[0]} * a{mono[1]}"
    return f"(a{mono[0]} * a{mono[1]}) * a{mono[2]}"


def _deriv_terms(mono):
    """[(x, count, expr of the other factors)] for d mono / d a_x."""
    out = []
    for x in sorted(set(mono)):
        cnt = mono.count(x)
        rest = list(mono)
        rest.remove(x)
        if not rest:
            expr = None
        elif len(rest) == 1:
            expr = f"a{rest[0]}"
        else:
            expr = f"a{rest[0]} * a{rest[1]}"
        out.append((x, cnt, expr))
    return out


def emit_fwd(c: Cfg) -> str:
    L = []
    w = L.append
    w(f"// config {c.idx}: l_in {c.l_in}, L_out <= {c.l_out}, correlation {c.nu}: {c.paths} paths, "
      f"{len(c.terms)} monomials, {c.nnz} coefficients")
    w(f"__global__ void __launch_bounds__(256) k_scg_fwd_{c.idx}(const float* __restrict__ A, "
      f"const int64_t* __restrict__ z, const float* __restrict__ W, int64_t N, int C, int S, "
      f"float* __restrict__ B) {{")
    w("    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;")
    w("    if (t >= N * C) return;")
    w("    const int64_t n = t / C;")
    w("    const int c = int(t - n * C);")
    w("    const int64_t e = z[n];")
    w(f"    float* bp = B + n * ({c.no} * int64_t(C)) + c;")
    w("    if (e < 0 || e >= S) {")
    w(f"        for (int M = 0; M < {c.no}; ++M) bp[M * C] = 0.f;")
    w("        return;")
    w("    }")
    w(f"    const float* ap = A + n * ({c.ni} * int64_t(C)) + c;")
    for i in c.used:
        w(f"    const float a{i} = ap[{i} * C];")
    w(f"    const float* wp = W + e * ({c.paths} * int64_t(C)) + c;")
    accs = sorted({(p, M) for _, ts in c.terms for p, M, _ in ts})
    for p, M in accs:
        w(f"    float u{p}_{M} = 0.f;")
    for mono, ts in c.terms:
        w("    {")
        w(f"        const float m = {_mono_expr(mono)};")
        for p, M, v in ts:
            w(f"        u{p}_{M} = fmaf({f32(v)}, m, u{p}_{M});")
        w("    }")
    for M in range(c.no):
        terms = [p for p, MM in accs if MM == M]
        w(f"    {{  // output component {M}")
        w("        float b = 0.f;")
        for p in terms:
            w(f"        b = fmaf(wp[{p} * C], u{p}_{M}, b);")
        w(f"        bp[{M} * C] = b;")
        w("    }")
    w("}")
    return "\n".join(L)


def emit_bwd(c: Cfg) -> str:
    L = []
    w = L.append
    w(f"template <bool GA, bool GW>")
    w(f"__global__ void __launch_bounds__(256) k_scg_bwd_{c.idx}(const float* __restrict__ A, "
      f"const int64_t* __restrict__ z, const float* __restrict__ W, const float* __restrict__ G, "
      f"const int32_t* __restrict__ order, int64_t N, int C, int S, int chunk, float* __restrict__ gA, "
      f"float* __restrict__ gW) {{")
    w("    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;")
    w("    const int64_t q = t / C;")
    w("    const int c = int(t - q * C);")
    w("    const int64_t s0 = q * chunk;")
    w("    if (s0 >= N) return;")
    w("    const int64_t s1 = s0 + chunk < N ? s0 + chunk : N;")
    for p in range(c.paths):
        w(f"    float gw{p} = 0.f;")
    w("    int64_t ecur = -1;")
    w("    for (int64_t s = s0; s < s1; ++s) {")
    w("        const int64_t n = order ? int64_t(order[s]) : s;")
    w("        const int64_t e = z[n];")
    w("        if (GW && e != ecur) {")
    w("            if (ecur >= 0 && ecur < S) {")
    w(f"                float* gp = gW + ecur * ({c.paths} * int64_t(C)) + c;")
    for p in range(c.paths):
        w(f"                atomicAdd(gp + {p} * C, gw{p});")
    w("            }")
    for p in range(c.paths):
        w(f"            gw{p} = 0.f;")
    w("            ecur = e;")
    w("        }")
    w(f"        float* dp = gA + n * ({c.ni} * int64_t(C)) + c;")
    w("        if (e < 0 || e >= S) {")
    w(f"            if (GA) for (int i = 0; i < {c.ni}; ++i) dp[i * C] = 0.f;")
    w("            continue;")
    w("        }")
    w(f"        const float* ap = A + n * ({c.ni} * int64_t(C)) + c;")
    for i in c.used:
        w(f"        const float a{i} = ap[{i} * C];")
    w(f"        const float* gp = G + n * ({c.no} * int64_t(C)) + c;")
    for M in range(c.no):
        w(f"        const float g{M} = gp[{M} * C];")
    w(f"        const float* wp = W + e * ({c.paths} * int64_t(C)) + c;")
    w("        float " + ", ".join(f"w{p} = 0.f" for p in range(c.paths)) + ";")
    w("        if (GA) {")
    for p in range(c.paths):
        w(f"            w{p} = wp[{p} * C];")
    w("        }")
    for i in range(c.ni):
        w(f"        float d{i} = 0.f;")
    for mono, ts in c.terms:
        w("        {")
        byp = defaultdict(list)
        for p, M, v in ts:
            byp[p].append((M, v))
        w(f"            const float m = {_mono_expr(mono)};")
        w("            float gm = 0.f;")
        for p, lst in byp.items():
            expr = f"{f32(lst[0][1])} * g{lst[0][0]}"
            for M, v in lst[1:]:
                expr = f"fmaf({f32(v)}, g{M}, {expr})"
            w(f"            {{ const float h = {expr};")
            w(f"              if (GW) gw{p} = fmaf(m, h, gw{p});")
            w(f"              if (GA) gm = fmaf(w{p}, h, gm); }}")
        w("            if (GA) {")
        for x, cnt, expr in _deriv_terms(mono):
            if expr is None:
                w(f"                d{x} += gm;")
            elif cnt == 1:
                w(f"                d{x} = fmaf(gm, {expr}, d{x});")
            else:
                w(f"                d{x} = fmaf({float(cnt):.1f}f * gm, {expr}, d{x});")
        w("            }")
        w("        }")
    w("        if (GA) {")
    for i in range(c.ni):
        w(f"            dp[{i} * C] = d{i};")
    w("        }")
    w("    }")
    w("    if (GW && ecur >= 0 && ecur < S) {")
    w(f"        float* gp = gW + ecur * ({c.paths} * int64_t(C)) + c;")
    for p in range(c.paths):
        w(f"        atomicAdd(gp + {p} * C, gw{p});")
    w("    }")
    w("}")
    return "\n".join(L)


def _dir_terms(mono):
    """D = d mono along the seed s: [(count, x, rest)] with s_x * prod(a_rest), duplicates merged."""
    acc = defaultdict(int)
    for p in range(len(mono)):
        rest = tuple(sorted(mono[r] for r in range(len(mono)) if r != p))
        acc[(mono[p], rest)] += 1
    return [(cnt, x, rest) for (x, rest), cnt in sorted(acc.items())]


def _dir_deriv_terms(mono):
    """d D / d a_y for D = sum_p s_{t_p} prod_{r != p} a_{t_r}: [(y, count, x, rest)] with
    s_x * prod(a_rest) over ordered position pairs (p, q), p != q, y = t_q, duplicates merged."""
    acc = defaultdict(int)
    n = len(mono)
    for p in range(n):
        for q in range(n):
            if p != q:
                rest = tuple(sorted(mono[r] for r in range(n) if r not in (p, q)))
                acc[(mono[q], mono[p], rest)] += 1
    return [(y, cnt, x, rest) for (y, x, rest), cnt in sorted(acc.items())]


def _prod(names):
    return " * ".join(names) if names else "1.f"


def emit_bwd2(c: Cfg) -> str:
    """Second order: with first-order gradients gA, gW of <G, B> and seeds sA, sW,
    L2 = <sA, gA> + <sW, gW> = sum_q H_q D_q + Hw_q m_q where D_q = d m_q along sA,
    h_{k,q} = sum_M coef_k[M, q] G[M], H_q = sum_k W_k h_{k,q}, Hw_q = sum_k sW_k h_{k,q}:
        dG[M] = sum_{q,k} coef_k[M, q] (W_k D_q + sW_k m_q)
        dW_k  = sum_q h_{k,q} D_q
        dA_y  = sum_q H_q dD_q/dA_y + Hw_q dm_q/dA_y."""
    L = []
    w = L.append
    w(f"__global__ void __launch_bounds__(256) k_scg_bwd2_{c.idx}(const float* __restrict__ A, "
      f"const int64_t* __restrict__ z, const float* __restrict__ W, const float* __restrict__ G, "
      f"const float* __restrict__ sA, const float* __restrict__ sW, const int32_t* __restrict__ order, int64_t N, "
      f"int C, int S, int chunk, float* __restrict__ dG, float* __restrict__ dA, float* __restrict__ dW) {{")
    w("    const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;")
    w("    const int64_t q = t / C;")
    w("    const int c = int(t - q * C);")
    w("    const int64_t s0 = q * chunk;")
    w("    if (s0 >= N) return;")
    w("    const int64_t s1 = s0 + chunk < N ? s0 + chunk : N;")
    w("    const bool hasA = sA != nullptr, hasW = sW != nullptr;")
    for p in range(c.paths):
        w(f"    float dw{p} = 0.f;")
    w("    int64_t ecur = -1;")
    w("    for (int64_t s = s0; s < s1; ++s) {")
    w("        const int64_t n = order ? int64_t(order[s]) : s;")
    w("        const int64_t e = z[n];")
    w("        if (dW && e != ecur) {")
    w("            if (ecur >= 0 && ecur < S && hasA) {")
    w(f"                float* wq = dW + ecur * ({c.paths} * int64_t(C)) + c;")
    for p in range(c.paths):
        w(f"                atomicAdd(wq + {p} * C, dw{p});")
    w("            }")
    for p in range(c.paths):
        w(f"            dw{p} = 0.f;")
    w("            ecur = e;")
    w("        }")
    w(f"        float* gq = dG ? dG + n * ({c.no} * int64_t(C)) + c : nullptr;")
    w(f"        float* aq = dA ? dA + n * ({c.ni} * int64_t(C)) + c : nullptr;")
    w("        if (e < 0 || e >= S) {")
    w(f"            if (gq) for (int i = 0; i < {c.no}; ++i) gq[i * C] = 0.f;")
    w(f"            if (aq) for (int i = 0; i < {c.ni}; ++i) aq[i * C] = 0.f;")
    w("            continue;")
    w("        }")
    w(f"        const float* ap = A + n * ({c.ni} * int64_t(C)) + c;")
    for i in c.used:
        w(f"        const float a{i} = ap[{i} * C];")
    w(f"        const float* sp = hasA ? sA + n * ({c.ni} * int64_t(C)) + c : nullptr;")
    for i in c.used:
        w(f"        const float s{i} = hasA ? sp[{i} * C] : 0.f;")
    w(f"        const float* gp = G + n * ({c.no} * int64_t(C)) + c;")
    for M in range(c.no):
        w(f"        const float g{M} = gp[{M} * C];")
    w(f"        const float* wp = W + e * ({c.paths} * int64_t(C)) + c;")
    w(f"        const float* vp = hasW ? sW + e * ({c.paths} * int64_t(C)) + c : nullptr;")
    for p in range(c.paths):
        w(f"        const float w{p} = wp[{p} * C];")
        w(f"        const float v{p} = hasW ? vp[{p} * C] : 0.f;")
    for M in range(c.no):
        w(f"        float dg{M} = 0.f;")
    for i in range(c.ni):
        w(f"        float d{i} = 0.f;")
    for mono, ts in c.terms:
        w("        {")
        byp = defaultdict(list)
        for p, M, v in ts:
            byp[p].append((M, v))
        w(f"            const float m = {_mono_expr(mono)};")
        dterms = " + ".join((f"{float(cnt):.1f}f * " if cnt > 1 else "") + _prod([f"s{x}"] + [f"a{r}" for r in rest])
                            for cnt, x, rest in _dir_terms(mono))
        w(f"            const float D = {dterms};")
        w("            float H = 0.f, Hw = 0.f;")
        for p, lst in byp.items():
            expr = f"{f32(lst[0][1])} * g{lst[0][0]}"
            for M, v in lst[1:]:
                expr = f"fmaf({f32(v)}, g{M}, {expr})"
            w(f"            {{ const float h = {expr};")
            w(f"              H = fmaf(w{p}, h, H); Hw = fmaf(v{p}, h, Hw); dw{p} = fmaf(h, D, dw{p}); }}")
        for p, M, v in ts:
            w(f"            dg{M} = fmaf({f32(v)}, fmaf(w{p}, D, v{p} * m), dg{M});")
        for x, cnt, expr in _deriv_terms(mono):
            val = "Hw" if expr is None else f"Hw * {expr}"
            w(f"            d{x} = fmaf({float(cnt):.1f}f, {val}, d{x});")
        for y, cnt, x, rest in _dir_deriv_terms(mono):
            w(f"            d{y} = fmaf({float(cnt):.1f}f * H, {_prod([f's{x}'] + [f'a{r}' for r in rest])}, d{y});")
        w("        }")
    w("        if (gq) {")
    for M in range(c.no):
        w(f"            gq[{M} * C] = dg{M};")
    w("        }")
    w("        if (aq) {")
    for i in range(c.ni):
        w(f"            aq[{i} * C] = d{i};")
    w("        }")
    w("    }")
    w("    if (dW && hasA && ecur >= 0 && ecur < S) {")
    w(f"        float* wq = dW + ecur * ({c.paths} * int64_t(C)) + c;")
    for p in range(c.paths):
        w(f"        atomicAdd(wq + {p} * C, dw{p});")
    w("    }")
    w("}")
    return "\n".join(L)


def generate() -> str:
    cfgs = [Cfg(i, *t) for i, t in enumerate(config_list())]
    out = ["// Generated by molnex_amd/csrc/gen_sc.py -- do not edit.", ""]
    for c in cfgs:
        out.append(emit_fwd(c))
        out.append("")
        out.append(emit_bwd(c))
        out.append("")
        out.append(emit_bwd2(c))
        out.append("")
    out.append("struct SCConfig { int l_in, l_out, nu, ni, no, paths, nnz; };")
    out.append("constexpr SCConfig kSCConfigs[] = {")
    for c in cfgs:
        out.append(f"    {{{c.l_in}, {c.l_out}, {c.nu}, {c.ni}, {c.no}, {c.paths}, {c.nnz}}},")
    out.append("};")
    out.append(f"constexpr int kNumSCConfigs = {len(cfgs)};")
    out.append("using SCFwdFn = void (*)(const float*, const int64_t*, const float*, int64_t, int, int, float*);")
    out.append("using SCBwdFn = void (*)(const float*, const int64_t*, const float*, const float*, const int32_t*, "
               "int64_t, int, int, int, float*, float*);")
    out.append("constexpr SCFwdFn kSCFwd[] = {" + ", ".join(f"k_scg_fwd_{c.idx}" for c in cfgs) + "};")
    for ga, gw in ((1, 1), (1, 0), (0, 1)):
        name = {(1, 1): "kSCBwdAW", (1, 0): "kSCBwdA", (0, 1): "kSCBwdW"}[(ga, gw)]
        tb = "true" if ga else "false"
        tw = "true" if gw else "false"
        out.append(f"constexpr SCBwdFn {name}[] = {{" +
                   ", ".join(f"k_scg_bwd_{c.idx}<{tb}, {tw}>" for c in cfgs) + "};")
    out.append("using SCBwd2Fn = void (*)(const float*, const int64_t*, const float*, const float*, const float*, "
               "const float*, const int32_t*, int64_t, int, int, int, float*, float*, float*);")
    out.append("constexpr SCBwd2Fn kSCBwd2[] = {" + ", ".join(f"k_scg_bwd2_{c.idx}" for c in cfgs) + "};")
    return "\n".join(out) + "\n"


def main():
    path = os.path.join(HERE, "sc_gen.inc")
    text = generate()
    old = open(path).read() if os.path.exists(path) else None
    if text != old:
        with open(path, "w") as f:
            f.write(text)


if __name__ == "__main__":
    main()
