"""ctypes binding of the C ABI in ``include/molnex.h`` (``lib/libmolnex_hip.so``).

The library is loaded on first use.  There is no CPU fallback: if the shared
library is missing the import of an op raises, and every entry point raises
``MolnexError`` with the library's message when a call fails.
"""

from __future__ import annotations

import ctypes as C
import os
import threading

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libmolnex_hip.so")

_lock = threading.Lock()
_lib = None

c_i32, c_i64, c_f64, c_sz = C.c_int32, C.c_int64, C.c_double, C.c_size_t
vp = C.c_void_p

# name -> (restype, argtypes); mirrors include/molnex.h
SIGNATURES = {
    "mnx_last_error": (C.c_char_p, []),
    "mnx_abi_version": (C.c_int, []),
    "mnx_nlist_workspace_bytes": (c_sz, [c_i64]),
    "mnx_nlist_count_f32": (C.c_int, [vp, c_i64, c_f64, vp, c_i32, vp, c_sz, vp, vp]),
    "mnx_nlist_count_f64": (C.c_int, [vp, c_i64, c_f64, vp, c_i32, vp, c_sz, vp, vp]),
    "mnx_nlist_emit_f32": (C.c_int, [vp, c_i64, c_f64, vp, c_i32, c_i32, vp, c_sz, c_i64, vp, vp, vp, vp, vp, vp]),
    "mnx_nlist_emit_f64": (C.c_int, [vp, c_i64, c_f64, vp, c_i32, c_i32, vp, c_sz, c_i64, vp, vp, vp, vp, vp, vp]),
    "mnx_nlist_backward_f32": (C.c_int, [vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp]),
    "mnx_nlist_backward_f64": (C.c_int, [vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp]),
    "mnx_csr_workspace_bytes": (c_sz, [c_i64, c_i64]),
    "mnx_csr_build": (C.c_int, [vp, c_i64, c_i64, vp, vp, vp, vp, vp, c_sz, vp]),
    "mnx_csr_build_noalloc": (C.c_int, [vp, c_i64, c_i64, vp, vp, vp, vp, vp]),
    "mnx_segment_sum_f32": (C.c_int, [vp, c_i64, c_i32, vp, vp, vp, c_i64, vp, vp]),
    "mnx_class_groups_workspace_bytes": (c_sz, [c_i64, c_i32]),
    "mnx_class_groups": (C.c_int, [vp, c_i64, c_i32, vp, vp, vp, c_sz, vp]),
    "mnx_segment_sum_bwd_f32": (C.c_int, [vp, vp, vp, vp, c_i64, c_i32, c_i64, vp, vp, vp]),
    "mnx_sh_fwd_f32": (C.c_int, [vp, c_i64, c_i32, vp, vp]),
    "mnx_sh_bwd_f32": (C.c_int, [vp, vp, c_i64, c_i32, vp, vp]),
    "mnx_tp_config": (C.c_int, [c_i32, c_i32, c_i32]),
    "mnx_tp_config_info": (C.c_int, [c_i32, C.POINTER(c_i32)]),
    "mnx_tp_fwd_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp]),
    "mnx_tp_bwd_workspace_bytes": (c_sz, [c_i32, c_i32, c_i64]),
    "mnx_tp_bwd_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp, vp, vp, c_sz, vp]),
    "mnx_tp_bwd_sender_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp, vp, vp]),
    "mnx_tp_fwd_rows_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp]),
    "mnx_tp_any_triple": (C.c_int, [c_i32, c_i32, c_i32]),
    "mnx_tp_any_fwd_f32": (C.c_int, [vp, c_i32, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp]),
    "mnx_tp_any_bwd_f32": (C.c_int, [vp, c_i32, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp, vp, vp]),
    "mnx_tall_tn_workspace_bytes": (C.c_size_t, [c_i64, c_i32, c_i32]),
    "mnx_silu_bwd2_f32": (C.c_int, [vp, vp, vp, c_i64, vp, vp, vp]),
    "mnx_tall_tn_f32": (C.c_int, [vp, c_i64, vp, c_i64, c_i64, c_i32, c_i32, vp, vp, vp, C.c_size_t, vp]),
    "mnx_tp_bwd_rows_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp, vp, vp,
                                      c_sz, vp]),
    "mnx_tp_bwd_sender_rows_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp,
                                             vp, vp]),
    "mnx_edge_reverse": (C.c_int, [vp, c_i64, c_i64, vp, vp, vp, vp, c_i32, vp, vp, vp]),
    "mnx_edge_pairs_workspace_bytes": (c_sz, [c_i64]),
    "mnx_gather_rows_f32": (C.c_int, [vp, vp, c_i64, c_i32, vp, vp]),
    "mnx_edge_pairs_verify": (C.c_int, [vp, c_i64, vp, c_i32, vp, vp]),
    "mnx_scatter_rows_f32": (C.c_int, [vp, vp, c_i64, c_i32, vp, vp]),
    "mnx_pair_sum_rows_f32": (C.c_int, [vp, vp, c_i64, c_i32, vp, vp]),
    "mnx_edge_pairs": (C.c_int, [vp, c_i64, c_i64, vp, vp, vp, vp, c_i32, vp, vp, vp, vp, vp, c_sz, vp]),
    "mnx_pme_spread_workspace_bytes": (c_sz, [c_i64, c_i32, c_i32, c_i32]),
    "mnx_pme_spread_f32": (C.c_int, [vp, vp, vp, c_i64, c_i32, c_i32, c_i32, c_i32, c_f64, vp, vp, c_sz, vp]),
    "mnx_pme_spread_f64": (C.c_int, [vp, vp, vp, c_i64, c_i32, c_i32, c_i32, c_i32, c_f64, vp, vp, c_sz, vp]),
    "mnx_pme_convolve_workspace_bytes": (c_sz, [c_i32, c_i32, c_i32]),
    "mnx_pme_convolve_f32": (C.c_int, [vp, vp, c_i32, c_i32, c_i32, c_f64, vp, vp, vp, vp, vp, c_sz, vp]),
    "mnx_pme_convolve_f64": (C.c_int, [vp, vp, c_i32, c_i32, c_i32, c_f64, vp, vp, vp, vp, vp, c_sz, vp]),
    "mnx_pme_gather_f32": (C.c_int, [vp, vp, vp, c_i64, vp, c_i32, c_i32, c_i32, c_i32, c_f64, vp, vp, vp]),
    "mnx_pme_gather_f64": (C.c_int, [vp, vp, vp, c_i64, vp, c_i32, c_i32, c_i32, c_i32, c_f64, vp, vp, vp]),
    "mnx_pme_direct_workspace_bytes": (c_sz, [c_i64, c_i64]),
    "mnx_pme_direct_f32": (C.c_int, [vp, vp, c_i64, vp, c_i64, vp, vp, vp, c_i32, c_f64, c_f64, vp, vp, vp, vp, c_sz,
                                     vp]),
    "mnx_pme_direct_f64": (C.c_int, [vp, vp, c_i64, vp, c_i64, vp, vp, vp, c_i32, c_f64, c_f64, vp, vp, vp, vp, c_sz,
                                     vp]),
    "mnx_sc_scalar_fwd_f32": (C.c_int, [vp, vp, vp, c_i64, c_i32, c_i32, c_i32, vp, vp]),
    "mnx_sc_scalar_bwd_f32": (C.c_int, [vp, vp, vp, vp, c_i64, c_i32, c_i32, c_i32, vp, vp, vp]),
    "mnx_sc_config": (C.c_int, [c_i32, c_i32, c_i32]),
    "mnx_sc_config_info": (C.c_int, [c_i32, vp]),
    "mnx_sc_fwd_f32": (C.c_int, [c_i32, vp, vp, vp, c_i64, c_i32, c_i32, vp, vp]),
    "mnx_sc_bwd_f32": (C.c_int, [c_i32, vp, vp, vp, vp, vp, c_i64, c_i32, c_i32, vp, vp, vp]),
    "mnx_sc_bwd2_f32": (C.c_int, [c_i32, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i32, c_i32, vp, vp, vp, vp]),
    "mnx_block_linear_frag_floats": (c_i64, [c_i32, c_i32]),
    "mnx_block_linear_f32": (C.c_int, [vp, c_i64, c_i32, vp, vp, vp, vp, c_i32, c_i64, c_i32, vp, c_i64, c_i64,
                                        c_i32, vp]),
    "mnx_indexed_block_linear_f32": (C.c_int, [vp, c_i64, c_i32, vp, vp, vp, vp, c_i64, c_i32, vp, vp, c_i32,
                                                c_i64, c_i32, vp, c_i64, c_i64, c_i32, vp]),
    "mnx_bond_vectors_f32": (C.c_int, [vp, c_i64, vp, vp, c_i64, vp, vp]),
    "mnx_bond_vectors_bwd_f32": (C.c_int, [vp, vp, c_i64, c_i64, vp, vp]),
    "mnx_bessel_cutoff_f32": (C.c_int, [vp, c_i64, c_i32, c_f64, c_f64, vp, vp, c_i32, c_i32, vp, vp]),
    "mnx_bessel_cutoff_bwd_f32": (C.c_int, [vp, c_i64, c_i32, c_f64, c_f64, vp, vp, c_i32, c_i32, vp, vp, vp]),
    "mnx_radial_raw_floats": (c_i64, [c_i32, c_i32, c_i32]),
    "mnx_radial_frag_floats": (c_i64, [c_i32, c_i32, c_i32]),
    "mnx_radial_pack_f32": (C.c_int, [vp, c_i32, c_i32, c_i32, vp, vp]),
    "mnx_radial_fwd_f32": (C.c_int, [vp, c_i64, c_i32, c_i32, c_i32, vp, vp, vp]),
    "mnx_radial_bwd_f32": (C.c_int, [vp, c_i64, c_i32, c_i32, c_i32, vp, vp, vp, vp]),
    "mnx_edge_weights_frag_elems": (c_i64, [c_i32, c_i32, c_i32]),
    "mnx_edge_weights_pack_f32": (C.c_int, [vp, c_i32, c_i32, c_i32, vp, vp]),
    "mnx_edge_weights_f32": (C.c_int, [vp, c_i64, c_i32, vp, vp, c_i32, vp, vp]),
    "mnx_edge_weights_bwd_f32": (C.c_int, [vp, c_i64, c_i32, vp, c_i32, vp, vp]),
    "mnx_edge_weights_bwd_pairs_f32": (C.c_int, [vp, vp, c_i64, c_i32, vp, c_i32, vp, vp]),
    "mnx_edge_weights_rows_f32": (C.c_int, [vp, vp, c_i64, c_i32, vp, vp, c_i32, vp, vp]),
    "mnx_tp_weight_grad_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, c_i64, c_i64, vp, c_i32, vp, vp]),
    "mnx_tp_weight_grad_rows": (C.c_int, [c_i32, c_i32, vp]),
    "mnx_tp_weight_grad_batched_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_i64, vp,
                                                  c_i32, vp, vp]),
    "mnx_tp_group_paths": (C.c_int, [c_i32, vp]),
    "mnx_tp_bwd_group_rows_f32": (C.c_int, [c_i32, c_i32, c_i32, vp, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, vp, vp,
                                             vp, c_sz, vp]),
    "mnx_tp_bwd_reduce_gy_f32": (C.c_int, [c_i32, c_i32, c_i64, vp, c_sz, vp, vp]),
    "mnx_edge_weights_bwd_cols_f32": (C.c_int, [vp, c_i64, vp, c_i64, c_i32, vp, c_i32, vp, c_i32, vp]),
    "mnx_edge_weights_bwd_into_f32": (C.c_int, [vp, c_i64, vp, c_i64, c_i32, vp, c_i32, vp, c_i64, c_i32, vp]),
    "mnx_tp_bwd_gh_supported": (C.c_int, [c_i32, c_i32, c_i32]),
    "mnx_tp_bwd_gh_workspace_bytes": (c_sz, [c_i32, c_i32, c_i64, c_i32, c_i32]),
    "mnx_tp_bwd_gh_rows_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, vp, vp, vp, c_i64, c_i64, c_i32, vp,
                                          c_i32, vp, vp, vp, vp, c_sz, vp]),
    "mnx_edge_tp_fwd_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, c_i64, vp, vp]),
    "mnx_channel_scale_f32": (C.c_int, [vp, vp, c_i64, c_i32, c_i32, vp, vp]),
    "mnx_channel_scale_bwd_f32": (C.c_int, [vp, vp, vp, c_i64, c_i32, c_i32, vp, vp, vp]),
    "mnx_channel_outer_f32": (C.c_int, [vp, vp, c_i64, c_i32, c_i32, vp, vp]),
    "mnx_channel_outer_bwd_f32": (C.c_int, [vp, vp, vp, c_i64, c_i32, c_i32, vp, vp, vp]),
    "mnx_channel_outer_stack_f32": (C.c_int, [vp, vp, c_i32, c_i64, c_i32, vp, vp]),
    "mnx_channel_outer_stack_bwd_f32": (C.c_int, [vp, vp, vp, c_i32, c_i64, c_i32, vp, vp, vp]),
    "mnx_edge_tp_bwd_workspace_bytes": (c_sz, [c_i32, c_i32, c_i64]),
    "mnx_edge_tp_bwd_f32": (C.c_int, [c_i32, c_i32, vp, vp, vp, vp, vp, c_i64, vp, vp, vp, vp, vp, c_sz, vp]),
    "mnx_edge_tp_proj_info": (c_i32, [c_i32, vp]),
    "mnx_edge_tp_proj_bwd_workspace_bytes": (c_sz, [c_i32, c_i64]),
    "mnx_edge_tp_proj_fwd_f32": (C.c_int, [c_i32, vp, c_i32, vp, vp, vp, vp, vp, c_i64, vp, vp]),
    "mnx_edge_tp_proj_bwd_f32": (C.c_int, [c_i32, vp, c_i32, vp, vp, vp, vp, vp, vp, c_i64, vp, vp, vp, vp, vp, vp,
                                           c_sz, vp]),
}


class MolnexError(RuntimeError):
    pass


def load(path: str = LIB_PATH):
    """Load the library (once) and bind every symbol of the C ABI."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise MolnexError(
                f"molnex HIP library not found at {path}; build it with `python -m molnex_amd.build`"
            )
        lib = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().mnx_last_error().decode(errors="replace")
        raise MolnexError(f"{what} failed (status {rc}): {msg}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None / empty)."""
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()
