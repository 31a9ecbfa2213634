"""The C-ABI library loads on a machine without a GPU and exports every symbol that
include/coldpress_hip.h declares (no compute calls)."""
import ctypes
import os
import re

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "coldpress_hip.h")
LIB = os.path.join(ROOT, "perm_amd", "libcoldpress_hip.so")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(cp_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "cp_kq_quantize" in syms and "cp_last_error" in syms


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "libcoldpress_hip.so missing: run `python -m perm_amd.build`"
    lib = ctypes.CDLL(LIB)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"


def test_binding_table_matches_header():
    from perm_amd import _lib
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_error_path_without_gpu():
    """Argument validation answers before touching the device."""
    lib = ctypes.CDLL(LIB)
    lib.cp_kq_block_bytes.restype = ctypes.c_int
    lib.cp_last_error.restype = ctypes.c_char_p
    assert lib.cp_kq_block_bytes(10) == 84 and lib.cp_kq_block_bytes(14) == 210
    assert lib.cp_kq_block_bytes(99) == -2
    assert b"unsupported" in lib.cp_last_error()
