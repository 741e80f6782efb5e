"""Build the HIP library ``molnex_amd/lib/libmolnex_hip.so`` for gfx950.

Plain ``hipcc`` invocations (no CMake): each ``csrc/*.hip`` / ``*.cpp`` is
compiled to an object in parallel, then linked into one shared library that
exports the C ABI of ``include/molnex.h``.  ``python -m molnex_amd.build``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libmolnex_hip.so")
ARCH = os.environ.get("MOLNEX_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-munsafe-fp-atomics",
    # packed fp32 VALU ops are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# per-source extra flags
EXTRA = {
    # bit-exact reference geometry: no fused multiply-add contraction
    "nlist.hip": ["-ffp-contract=off"],
}
SOURCES = ["errors.cpp", "nlist.hip", "csr.hip", "sh.hip", "tp.hip", "pme.hip", "symcon.hip", "radial.hip", "edges.hip", "linear.hip", "edge_weights.hip", "edge_tp.hip", "segment.hip", "tp_gh.hip", "embed.hip", "pairs.hip", "tp_any.hip", "tall_gemm.hip", "tp_fused.hip", "chscale.hip"]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    t0 = time.time()
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return f"{src}: {time.time() - t0:.1f}s"


def build(verbose: bool = True) -> str:
    sys.path.insert(0, os.path.dirname(PKG))
    from molnex_amd.csrc import gen_edge_tp, gen_sc, gen_tp, gen_tp_any

    gen_tp.main()
    gen_sc.main()
    gen_edge_tp.main()
    gen_tp_any.main()
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        for msg in ex.map(_compile, SOURCES):
            if verbose:
                print("  built", msg, flush=True)
    objs = [os.path.join(BUILD, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("  linked", LIB, flush=True)
    return LIB


if __name__ == "__main__":
    build()
