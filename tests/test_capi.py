"""The C ABI library (libfdm.so) on the CPU: it loads, it exports every
entry point include/fdm.h declares, and its error paths answer without a
GPU.  No compute call is made here."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fdm.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fdm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("fdm_init", "fdm_dequant_q4k", "fdm_matvec_q4k", "fdm_route",
                 "fdm_moe_forward", "fdm_moe_layer"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from flash_deepseek_amd import _lib
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding knows every one of them
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_error_strings():
    from flash_deepseek_amd import _lib
    for code in range(0, -8, -1):
        assert _lib.lib.fdm_strerror(code)
    assert _lib.lib.fdm_strerror(-99) == b"unknown error"


def test_calls_before_init_are_rejected():
    from flash_deepseek_amd import _lib
    if _lib.lib.fdm_available():
        pytest.skip("library already initialised in this process")
    rc = _lib.lib.fdm_dequant_q4k(None, None, 256, None)
    assert rc == _lib.FDM_E_STATE
    rc = _lib.lib.fdm_moe_layer(3, None, None, 8, None, None, None, None)
    assert rc == _lib.FDM_E_STATE


def test_init_without_device_reports_nodev():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from flash_deepseek_amd import _lib
    assert _lib.lib.fdm_init(0) == _lib.FDM_E_NODEV
    assert _lib.lib.fdm_available() == 0
    with pytest.raises(_lib.FdmError):
        _lib.call("fdm_init", 0)
