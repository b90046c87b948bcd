"""CPU checks of the C-ABI library: it is built, loads without a GPU, and
exports every entry point include/dbi_kv.h declares (no compute calls here)."""
import ctypes
import os
import subprocess

import pytest

from dbinfer_amd import _lib


def test_library_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    _lib.load()


def test_exports_every_declared_symbol():
    declared = _lib.header_symbols()
    assert len(declared) >= 20
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    # the Python binding types every declared entry point
    assert sorted(_lib.SIGNATURES) == declared


def test_exports_are_c_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    names = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for s in _lib.header_symbols():
        assert s in names, f"{s} is not an unmangled C symbol"


def test_last_error_is_empty_string_initially():
    lib = _lib.load()
    assert lib.dbi_last_error() == b""


def test_create_rejects_bad_config_without_gpu():
    """Argument validation runs before any device call."""
    lib = _lib.load()
    h = ctypes.c_void_p()
    cfg = _lib.KvConfig(0, 16, 1, 64, 0, 0, 0, 1e4)
    assert lib.dbi_kv_create(ctypes.byref(cfg), ctypes.byref(h)) == _lib.DBI_ERR_INVALID
    assert b"positive" in lib.dbi_last_error()
    cfg = _lib.KvConfig(1, 16, 1, 64, 4, 8, 0, 0.0)
    assert lib.dbi_kv_create(ctypes.byref(cfg), ctypes.byref(h)) == _lib.DBI_ERR_INVALID
    assert b"rope_theta" in lib.dbi_last_error()
    cfg = _lib.KvConfig(1, 16, 1, 64, 0, 0, 7, 1e4)
    assert lib.dbi_kv_create(ctypes.byref(cfg), ctypes.byref(h)) == _lib.DBI_ERR_INVALID
    assert lib.dbi_kv_create(None, ctypes.byref(h)) == _lib.DBI_ERR_INVALID
    # one head's fp32 K array at 2^22 positions x hd 128 is 2 GiB: refused
    cfg = _lib.KvConfig(1, 1 << 22, 1, 128, 0, 0, 0, 1e4)
    assert lib.dbi_kv_create(ctypes.byref(cfg), ctypes.byref(h)) == _lib.DBI_ERR_INVALID
    assert b"below 2 GiB" in lib.dbi_last_error()


def test_no_oracle_in_product_library():
    """The product library links nothing from oracle/ (no CPU fallback)."""
    out = subprocess.run(["nm", "-D", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    assert "okv_" not in out and "ok_rope" not in out
    deps = subprocess.run(["ldd", _lib.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle" not in deps
