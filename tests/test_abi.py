"""The C-ABI library builds, loads without a GPU, and exports exactly what
include/fastdms_amd.h declares with the signatures the ctypes binding uses."""
import ctypes

import pytest

from abi_signatures import header_signatures, source_signatures


def test_header_matches_hip_sources():
    assert header_signatures() == source_signatures()


def test_ctypes_table_matches_header():
    from fastdms_amd import _native
    assert _native.SIGNATURES == header_signatures()


def test_library_loads_and_exports_every_symbol():
    from fastdms_amd import _native
    if not _native.LIB_PATH.exists():
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = _native.lib()
    for name in header_signatures():
        assert hasattr(lib, name), name
    assert lib.fdms_abi_version() == 4


def test_rejected_arguments_return_invalid_value_without_launching():
    from fastdms_amd import _native
    if not _native.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _native.lib()
    # unaligned / odd-sized copy and a bad dtype code are rejected before any launch
    assert lib.fdms_copy_bytes(None, None, 15, 1, None) == 1
    assert lib.fdms_convert(ctypes.c_void_p(16), 9, ctypes.c_void_p(16), 0, 4, None) == 1
