"""The C ABI: the library loads (no GPU needed) and exports every entry point include/dsv41_amd.h declares,
with the Python binding's argument counts matching the header."""
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "dsv41_amd.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for m in re.finditer(r"\bint\s+(dsv41_\w+)\s*\(([^)]*)\)\s*;", src):
        out[m.group(1)] = len([a for a in m.group(2).split(",") if a.strip()])
    return out


def test_header_parses():
    d = declared()
    assert len(d) >= 10 and "dsv41_fp4_grouped_gemm" in d and "dsv41_moe_down_sum" in d


def test_library_exports_every_declared_symbol():
    from dsv41_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (dsv41_\w+)", nm))
    for name, nargs in declared().items():
        assert name in exported, f"{name} declared but not exported"
        assert hasattr(L, name)
        assert name in _lib.SIGNATURES, f"{name} has no Python binding"
        assert len(_lib.SIGNATURES[name]) == nargs, f"{name}: binding has {len(_lib.SIGNATURES[name])} args, header {nargs}"
    assert exported == set(declared()), f"undeclared exports: {exported - set(declared())}"


def test_invalid_arguments_are_rejected_without_launch():
    """Argument checks run on the host before any launch: no GPU is touched."""
    import ctypes
    from dsv41_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    L = _lib.lib()
    assert L.dsv41_dequant_fp4(None, None, 16, 64, 0, None, None) == -1
    assert L.dsv41_quant_fp8(ctypes.c_void_p(16), 0, 4, 33, 33, 0, ctypes.c_void_p(16), None, None, None) == -1  # K % 32
    assert L.dsv41_moe_dispatch(ctypes.c_void_p(16), None, 8, 8, 1000, 64, *[ctypes.c_void_p(16)] * 5, None, None) == -1  # E > 512
    assert L.dsv41_dense_gemv_bf16(ctypes.c_void_p(16), 64, 16, 64, ctypes.c_void_p(16), 64, 17, ctypes.c_void_p(16), 16, None, 0, None) == -1
    # decode down projection: h rows shorter than K (codes or scales), an output row stride below N
    p = ctypes.c_void_p(16)
    down = lambda ldh, ldhs, ldy: L.dsv41_moe_down_sum(p, 7168 * 832, p, 7168 * 52, 1, 7168, 1664, p, ldh, p, ldhs, 8, p, p, p, 8, 1,
                                                      p, ldy, None, 7168, None, 7168, 0, 384, None)
    assert down(1600, 52, 7168) == -1
    assert down(1664, 51, 7168) == -1
    assert down(1664, 52, 7000) == -1
