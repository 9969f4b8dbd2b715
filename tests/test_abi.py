"""The C ABI library loads and exports every entry point of include/vva.h.

CPU only: no compute call is made.  vva_create on a machine without a GPU
must fail with a status and a message rather than crash.
"""
import ctypes
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "vva.h")
LIB = os.path.join(REPO, "vibevoice.cpp_amd", "lib", "libvva.so")


def header_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"VVA_API\s+[\w\s\*]+?\b(vva_\w+)\s*\(", text)))


def test_header_declares_the_binding_list():
    import vva
    assert header_symbols() == sorted(vva.EXPORTS)


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "build the library first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT\s+(vva_\w+)", out))
    missing = [s for s in header_symbols() if s not in exported]
    assert not missing, missing


def test_library_loads_and_reports_version():
    import vva
    lib = vva.load_library()
    assert lib.vva_version().decode().startswith("vva ")


def test_status_codes_follow_vv_status():
    text = open(HEADER).read()
    expect = {"VVA_OK": 0, "VVA_ERR_GENERIC": -1, "VVA_ERR_INVALID_ARG": -2, "VVA_ERR_OUT_OF_MEMORY": -5,
              "VVA_ERR_NOT_IMPLEMENTED": -6}
    for name, val in expect.items():
        assert re.search(rf"{name}\s*=\s*{val}\b", text), name


def test_create_without_gpu_fails_cleanly():
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible")
    import vva
    lib = vva.load_library()
    h = ctypes.c_void_p()
    st = lib.vva_create(0, None, ctypes.byref(h))
    assert st < 0 and not h.value
    assert lib.vva_last_error(None).decode()


def test_null_arguments_are_rejected_without_a_device():
    import vva
    lib = vva.load_library()
    assert lib.vva_kv_get_len(None, 0, None) == vva.ERR_INVALID_ARG
    assert lib.vva_synchronize(None) == vva.ERR_INVALID_ARG
    assert lib.vva_supports(None, 128, 28, 4, vva.F16, vva.Q8_0) == 0
    assert lib.vva_attn(None, None, 0, None, None, None, 0.0, None) == vva.ERR_INVALID_ARG


def test_log_callback_receives_failed_calls():
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is visible")
    import vva
    got = []
    vva.set_log_callback(lambda lvl, msg: got.append((lvl, msg)), vva.LOG_DEBUG)
    lib = vva.load_library()
    h = ctypes.c_void_p()
    try:
        assert lib.vva_create(0, None, ctypes.byref(h)) < 0
        assert lib.vva_create(-1, None, ctypes.byref(h)) < 0
    finally:
        vva.set_log_callback(None)
    assert [lvl for lvl, _ in got] == [vva.LOG_ERROR, vva.LOG_ERROR], got
    assert got[1][1] == lib.vva_last_error(None).decode()
    # removed: nothing more is delivered
    assert lib.vva_create(0, None, ctypes.byref(h)) < 0
    assert len(got) == 2
