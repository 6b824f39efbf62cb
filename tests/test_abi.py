"""The C-ABI library loads and exports every symbol include/mtl.h declares
(CPU only: no kernel is launched)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mtl.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mtl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for n in ("mtl_selective_scan_fwd", "mtl_causal_conv1d_fwd", "mtl_conv_step", "mtl_selective_state_update",
              "mtl_add_rmsnorm", "mtl_quant_dequant_sum_int8_tok", "mtl_quant_dequant_sum_fp16",
              "mtl_last_error", "mtl_abi_version"):
        assert n in names


def test_library_loads_and_exports_every_declared_symbol():
    from mamba_lite import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: build with python mamba-tp-lite_amd/build.py")
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.mtl_abi_version() == _lib.ABI_VERSION
    assert lib.mtl_last_error() == b""


def test_struct_layouts_match_header():
    """ctypes mirrors follow the header field order: 8-byte fields, then four
    int32 flags."""
    from mamba_lite import _lib

    assert ctypes.sizeof(_lib.ScanParams) == 8 * (6 * 4 + 5 + 4) + 4 * 4
    assert ctypes.sizeof(_lib.ConvParams) == 8 * (2 * 4 + 4 + 3) + 4 * 4


def test_invalid_arguments_are_rejected_without_a_gpu():
    """Host-side validation in the library returns an error code and a
    message before any launch."""
    from mamba_lite import _lib

    lib = _lib.load()
    p = _lib.ScanParams()
    p.batch, p.seqlen, p.dim, p.dstate = 1, 4, 8, 64   # dstate > 32
    rc = lib.mtl_selective_scan_fwd(ctypes.byref(p), None)
    assert rc == 1 and b"dstate" in lib.mtl_last_error()
    rc = lib.mtl_quant_dequant_sum_int8_tok(None, 2, 4, 4, None, None, None)
    assert rc == 1 and b"parts" in lib.mtl_last_error()
    c = _lib.ConvParams()
    c.batch, c.seqlen, c.dim, c.width = 1, 4, 8, 9     # width > 8
    assert lib.mtl_causal_conv1d_fwd(ctypes.byref(c), None) == 1
    assert b"width" in lib.mtl_last_error()
