"""The C-ABI library loads and exports every symbol include/molnex.h declares (no GPU calls)."""

import ctypes
import os
import re

from molnex_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "molnex.h")).read()
    return sorted(set(re.findall(r"\b(mnx_\w+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "mnx_tp_fwd_f32" in syms and "mnx_nlist_count_f32" in syms
    assert len(syms) >= 15


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_bindings_cover_header():
    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_host_only_queries():
    lib = _lib.load()
    assert lib.mnx_abi_version() == 1
    assert lib.mnx_nlist_workspace_bytes(1000) > 1000 * 12
    assert lib.mnx_csr_workspace_bytes(100, 1000) > 0
    cfg = lib.mnx_tp_config(0b1111, 0b1111, 0b1111)
    assert cfg >= 0
    assert lib.mnx_tp_config(0b10000, 1, 1) == -1
    assert lib.mnx_tp_bwd_workspace_bytes(cfg, 128, 10) >= 10 * 16 * 4
    # error path: invalid config reports a message
    rc = lib.mnx_tp_fwd_f32(9999, 16, None, None, None, None, None, None, 1, 1, None, None)
    assert rc != 0 and b"invalid tp config" in lib.mnx_last_error()
