"""The C++ host layer (vibevoice.cpp_amd/host/qwen2_attn.{hpp,cpp}) and its
test program tests/cpp/test_qwen2_resident, which replays the call sequences
of the reference's tests/test_qwen2_resident.cpp through it.

CPU: the host layer's archive defines its entry points and the test program
links and loads (its --list makes no HIP call).  GPU: the whole program runs
(one process, every case) and must exit 0."""
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "tests", "cpp", "bin", "test_qwen2_resident")
HOSTLIB = os.path.join(REPO, "vibevoice.cpp_amd", "lib", "libvva_qwen2.a")
CASES = ["chunks", "stack", "cfg", "q8", "step", "timing", "block", "errors", "supports", "order"]


def _need_built():
    if not (os.path.exists(BIN) and os.path.exists(HOSTLIB)):
        pytest.fail("C++ host layer not built: run __graft_entry__.build()")


def test_host_archive_defines_entry_points():
    _need_built()
    syms = subprocess.run(["nm", "-C", "--defined-only", HOSTLIB], capture_output=True, text=True,
                          check=True).stdout
    for name in ("vva::qwen2_attention_resident", "vva::qwen2_attention_block_resident", "vva::ResidentKV::init",
                 "vva::ResidentKV::free", "vva::ResidentKV::upload"):
        assert name in syms, name


def test_program_links_and_lists_cases():
    _need_built()
    r = subprocess.run([BIN, "--list"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert r.stdout.split() == CASES


@pytest.mark.gpu
def test_resident_call_sequences_through_cpp_host():
    _need_built()
    print("tests/cpp/bin/test_qwen2_resident (all cases)", flush=True)
    r = subprocess.run(["timeout", "-k", "10", "240", BIN], capture_output=True, text=True)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, f"exit {r.returncode}"
    for c in CASES:
        assert f"[{c}] PASS" in r.stdout, c
