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
    # the norm prologue (2) sums one statistic per 16-column producer strip:
    # x_amax_n must be k / 16 (here k = 2048: 128), 127 and 129 are rejected
    # (distinct aligned addresses, never dereferenced: every other argument is valid)
    x, w, nw, y, st = (ctypes.c_void_p(i << 12) for i in range(1, 6))
    for bad_n in (127, 129):
        assert lib.fdms_linear_small_m(x, 2048, 8, 2048, w, _native.DT_BF16, 2048, None, None, 4096, 2, nw, 1e-5,
                                       None, 0, None, 0, 0, 0, 1, None, None, y, 4096, st, bad_n, 128, None,
                                       None, _native.DT_F32, None) == 1


def _integration_python_blocks():
    from pathlib import Path
    import re
    text = (Path(__file__).resolve().parents[1] / "INTEGRATION.md").read_text()
    return re.findall(r"```python\n(.*?)```", text, flags=re.S)


def test_integration_stub_signatures_match_header():
    """Every ctypes signature string and every library call in the integration
    guide's reference-side stub (its python blocks) agree with
    include/fastdms_amd.h (argument kinds and the number of arguments passed)."""
    import ast
    header = header_signatures()
    blocks = _integration_python_blocks()
    assert blocks, "the integration guide has no python stub"
    sigs, calls = {}, []
    for code in blocks:
        tree = ast.parse(code)
        for node in ast.walk(tree):
            if isinstance(node, ast.Assign) and any(isinstance(t, ast.Name) and t.id == "_SIG" for t in node.targets):
                sigs.update(ast.literal_eval(node.value))
            if (isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute)
                    and node.func.attr.startswith("fdms_")):
                calls.append((node.func.attr, len(node.args)))
    assert sigs and calls
    for name, sig in sigs.items():
        assert header.get(name) == sig, f"{name}: stub {sig!r} vs header {header.get(name)!r}"
    for name, nargs in calls:
        assert name in sigs, f"{name} is called in the stub without a _SIG entry"
        assert nargs == len(header[name]), f"{name}: the stub passes {nargs} arguments, the header takes {len(header[name])}"
