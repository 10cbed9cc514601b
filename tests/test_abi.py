"""CPU tests of the boundary: the HIP library loads and exports every entry point
include/ovnative_amd.h declares (no compute: there is no GPU here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "ovnative_amd.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ovh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    import ovnative_amd
    if not os.path.exists(ovnative_amd.LIB_PATH):
        pytest.fail("libovnative_amd.so is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(ovnative_amd.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 18
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []
    # the Python binding covers exactly the declared surface
    assert sorted(ovnative_amd.SIGNATURES) == names


def test_pure_host_entry_points():
    import ovnative_amd
    lib = ovnative_amd.load()
    assert lib.ovh_abi_version() == 1
    assert lib.ovh_quant_bytes(7, 69) == 7 * 96
    assert lib.ovh_quant_scales(7, 69) == 7 * 3
    assert lib.ovh_quant_bytes(0, 69) == 0 and lib.ovh_quant_scales(5, 0) == 0
    assert lib.ovh_last_error() == b""


def test_copy_last_error_caller_buffer():
    """The reference's convention: the message into a caller-owned buffer,
    truncated with a NUL, the full length returned."""
    import ovnative_amd as ov
    lib = ov.load()
    h = ctypes.c_void_p()
    assert lib.ovh_weight_upload(0, 5, None, None, 0, None, ctypes.byref(h)) == ov.OV_ERR_INVALID_ARG
    msg = lib.ovh_last_error()
    n = len(msg)
    buf = ctypes.create_string_buffer(256)
    assert lib.ovh_copy_last_error(buf, 256) == n and buf.value == msg
    small = ctypes.create_string_buffer(b"x" * 8)
    assert lib.ovh_copy_last_error(small, 5) == n
    assert small.raw[:5] == msg[:4] + b"\0"
    assert lib.ovh_copy_last_error(None, 0) == n


def test_f16_form_switch():
    """The f16-operand GEMM form is off by default; the setter returns the
    previous threshold and a negative value only queries."""
    import ovnative_amd as ov
    assert ov.set_f16_min_rows(-1) == 0
    assert ov.set_f16_min_rows(4096) == 0
    assert ov.set_f16_min_rows(-1) == 4096
    assert ov.set_f16_min_rows(0) == 4096
    assert ov.set_f16_min_rows(-1) == 0


def test_argument_errors_without_device():
    """Argument checks run before any device work, so they are testable here."""
    import ovnative_amd as ov
    lib = ov.load()
    h = ctypes.c_void_p()
    assert lib.ovh_weight_upload(0, 5, None, None, 0, None, ctypes.byref(h)) == ov.OV_ERR_INVALID_ARG
    assert b"positive" in lib.ovh_last_error()
    assert lib.ovh_weight_from_device(4, 4, None, None, 2, None, ctypes.byref(h)) == ov.OV_ERR_INVALID_ARG
    # degenerate sizes are a silent no-op, as in the reference (gemm.cpp:761)
    assert lib.ovh_s8_nk_quantize(0, 10, None, None, None, None) == ov.OV_OK
    assert lib.ovh_linear_q(0, None, None, None, None, 0, 0, None) == ov.OV_OK
    assert lib.ovh_linear_q(3, None, None, None, None, 0, 0, None) == ov.OV_ERR_INVALID_ARG
