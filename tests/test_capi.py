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


def test_sampler_refuses_a_vocabulary_past_its_chunk_table():
    """the sampler's work buffers hold 64 chunks of 4096 values a row: every entry point refuses a larger vocabulary
    before any device work (checked here without a GPU: the refusal comes before the library's init)"""
    import ctypes

    import geode_amd

    lib = geode_amd.lib
    V = 64 * 4096 + 1
    logits = (ctypes.c_float * 4)()
    out = (ctypes.c_int32 * 32)()
    batch = (ctypes.c_int32 * 2)(0, 1)
    kept = ctypes.c_int(0)
    u = (ctypes.c_double * 2)(0.5, 0.5)
    uf = (ctypes.c_float * 2)(0.5, 0.5)
    rcs = {
        "gv_sample_rows": lib.gv_sample_rows(logits, V, 1, V, 0.0, 1.0, 0, 0, u, out),
        "gv_accept_match": lib.gv_accept_match(logits, V, V, batch, 2, 0.0, 1.0, 0, 0, u, out, ctypes.byref(kept)),
        "gv_accept_textbook": lib.gv_accept_textbook(logits, logits, V, V, 1, 0.7, 0.95, 0, uf, uf, 0.5, out),
    }
    for name, rc in rcs.items():
        assert rc == -1, name
    assert "262,144" in lib.gv_last_error().decode()


def test_library_leaves_none_of_its_own_symbols_undefined():
    """every function of the library's own namespace is defined in it (a declaration without a definition in the
    same namespace would surface only when a GPU call reaches it)"""
    import subprocess

    import geode_amd

    out = subprocess.run(["nm", "-D", "--undefined-only", geode_amd.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    own = [line.split()[-1] for line in out.splitlines() if "_ZN2gv" in line or " gv_" in line]
    assert not own, f"undefined: {own}"
