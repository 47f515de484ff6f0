"""CPU checks of the C-ABI library: it builds, loads, and exports every entry
point include/qma_gpu.h declares; without a GPU it reports unavailability
(no compute calls are made here)."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qma_gpu.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b((?:qmag?_|dequantize_row_|dot_q)[A-Za-z0-9_]+)\s*\(", src)
    return sorted(set(names))


@pytest.fixture(scope="module")
def built():
    import qmag
    if not os.path.exists(qmag.LIB_PATH):
        import build as b
        b.build()
    return qmag


def test_header_declares_reference_entries():
    names = declared_functions()
    for ref in ("qma_q8k_available", "qma_q8k_quant", "qma_q8k_dot", "qma_q8k_gateup",
                "dequantize_row_q4_K", "dequantize_row_q6_K", "dot_q4_K_f32", "dot_q6_K_f32"):
        assert ref in names


def test_library_exports_every_declared_symbol(built):
    import ctypes
    L = ctypes.CDLL(built.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_python_binding_covers_header(built):
    assert sorted(built.SIGNATURES) == declared_functions()


def test_no_gpu_reports_unavailable(built):
    L = built.lib()
    st = L.qmag_init(0)
    if st == 0:
        pytest.skip("a gfx950 GPU is visible")
    assert st == -3
    assert L.qma_q8k_available() == 0
    assert b"gfx950" in L.qmag_last_error() or b"device" in L.qmag_last_error()
