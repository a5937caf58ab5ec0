"""The C-ABI library loads and exports every symbol include/*.h declares
(no compute calls: this runs without a GPU)."""
import ctypes
import os

import iro_hip


def test_library_exports_every_declared_symbol():
    names = iro_hip.declared_symbols()
    assert len(names) > 30
    lib = ctypes.CDLL(iro_hip.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_every_declared_symbol():
    lib = iro_hip.load()
    for n in iro_hip.declared_symbols():
        fn = getattr(lib, n)
        assert fn.argtypes is not None, f"{n} has no ctypes signature"


def test_ops_dropin_names_match_reference_header():
    # include/iro_int8_ops.h mirrors the int8 section of ops.h:18-78
    want = {"iro_int8_weight_quantize", "iro_int8_weight_quantize_transposed",
            "iro_int8_weight_free", "iro_int8_weight_bytes", "iro_int8_quantize_rows",
            "iro_int8_linear", "iro_int8_linear_ex", "iro_int8_quantize_rows_residual",
            "iro_int8_fast_available", "iro_int8_prepare_backend", "iro_int8_selfcheck"}
    assert want <= set(iro_hip.declared_symbols())


def test_library_is_gfx950_code_object():
    # the offload bundle id of the embedded device code object
    data = open(iro_hip.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_no_cpu_fallback_in_product_path():
    # The HIP library must not link the oracle or call back into it.
    data = open(iro_hip.LIB_PATH, "rb").read()
    assert b"orc_" not in data and b"liboracle" not in data
    src = os.path.join(os.path.dirname(iro_hip.LIB_PATH), "csrc")
    for f in os.listdir(src):
        text = open(os.path.join(src, f)).read()
        assert "oracle" not in text.lower(), f
