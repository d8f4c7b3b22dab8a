"""The C ABI (CPU): the library loads without a GPU and exports every function include/geode_verify.h declares; the
Python host module binds each of them. No compute call is made here."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "geode_verify.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(gv_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_verify_contract():
    names = declared_functions()
    for must in ("gv_model_create", "gv_verify", "gv_verify_keep", "gv_gemv_q4", "gv_q4_pack", "gv_q4_dequant",
                 "gv_open", "gv_adopt_q4", "gv_gemm", "gv_mlp"):
        assert must in names


def test_library_exports_every_declared_symbol():
    import ctypes

    import geode_amd

    lib = ctypes.CDLL(geode_amd.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_the_header():
    import geode_amd

    assert set(declared_functions()) <= set(geode_amd.SIGNATURES), \
        set(declared_functions()) - set(geode_amd.SIGNATURES)
