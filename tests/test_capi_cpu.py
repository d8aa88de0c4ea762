"""The C-ABI library loads and exports every function include/mi355x_decode.h declares.
No compute calls (this runs without a GPU)."""
import ctypes as C
import os

import pytest

from mipkg import mi


def test_library_exports_every_declared_function():
    L = mi.lib()
    names = mi.header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_signatures_cover_the_header():
    names = set(mi.header_functions())
    assert names == set(mi.SIGNATURES), (names ^ set(mi.SIGNATURES))


def test_argument_errors_are_reported_without_a_gpu():
    L = mi.lib()
    rc = L.mi_gemv_w4a16(None, None, None, None, 1, 64, 64, 1, None)
    assert rc == -1
    assert b"null" in L.mi_last_error()
    rc = L.mi_gemv_w4a16(8, 8, 8, 8, 1, 100, 64, 1, None)
    assert rc == -2
    assert L.mi_gemv_pick_s(5120, 5120) >= 1
