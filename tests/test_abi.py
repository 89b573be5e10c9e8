"""C ABI checks that need no GPU: the library loads, exports every entry point
include/synapse_hip.h declares, and the Python binding declares the same set."""
import ctypes
import os
import re

import pytest

from synapse_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "synapse_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(syn_\w+)\s*\(", text)))


def test_header_declares_reference_entry_points():
    syms = declared_symbols()
    for name in ("syn_qgemm_int8", "syn_quantize_per_channel_int8", "syn_q4_0_gemv"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    if not os.path.exists(hip.LIB_PATH):
        pytest.fail("libsynapse_hip.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(hip.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_header():
    assert set(declared_symbols()) == set(hip.SIGNATURES), (
        set(declared_symbols()) ^ set(hip.SIGNATURES))


def test_status_codes_match_reference():
    # synapse.h:27-35
    text = open(os.path.join(ROOT, "include", "synapse_hip.h")).read()
    want = {"SYN_OK": 0, "SYN_ERR_NULL_PTR": 1, "SYN_ERR_INVALID_ARG": 2,
            "SYN_ERR_OUT_OF_MEMORY": 3, "SYN_ERR_SHAPE_MISMATCH": 4,
            "SYN_ERR_NOT_CONTIGUOUS": 5, "SYN_ERR_INVALID_AXIS": 6,
            "SYN_ERR_INVALID_DIMENSIONS": 7, "SYN_ERR_INTERNAL": 8}
    for k, v in want.items():
        assert re.search(rf"#define {k} {v}\b", text), k
