"""CPU checks of the C ABI: the library loads (no GPU needed to dlopen) and
exports every function include/klearu_hip.h declares; the Python binding
covers each of them."""
import ctypes
import os

import pytest

from klearu_amd import _lib


def test_header_symbols_exported():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libklearu_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = _lib.header_functions()
    assert len(names) > 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    names = set(_lib.header_functions())
    assert names == set(_lib.SIGS), (names ^ set(_lib.SIGS))


def test_error_reporting_without_gpu():
    lib = _lib.load()
    # argument validation happens before any device call
    rc = lib.kh_sparse_ffn_forward(None, None, 1, None, 0, None, None, 0, None)
    assert rc == _lib.KH_ERR_ARG
    assert b"null" in lib.kh_last_error()
    assert lib.kh_version() >= 1
