"""The ggml side of the drop-in (vibevoice.cpp_amd/host/ggml/qwen2_vva.cpp)
cannot be built here: ggml is not in the image.  It is compiled with
g++ -fsyntax-only against stand-in declarations of the part of ggml's API it
uses (tests/ggml_standin/ggml/), together with

  - the reference's own src/backend.hpp, src/qwen2.hpp and src/rms_norm.hpp
    where the reference tree is present (the declarations the adapter must
    match), and
  - stand-ins of those three (tests/ggml_standin/vv/) in every case,

so that a change of the host layer's signatures, a typo or a wrong member
name in the adapter fails on the CPU."""
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
STANDIN = os.path.join(REPO, "tests", "ggml_standin")
REF_SRC = "/root/reference/src"
ADAPTER = os.path.join(REPO, "vibevoice.cpp_amd", "host", "ggml", "qwen2_vva.cpp")


def _syntax(vv_dir):
    cmd = ["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(STANDIN, "ggml"), "-I", vv_dir,
           "-I", os.path.join(REPO, "include"), "-I", os.path.join(REPO, "vibevoice.cpp_amd", "host"),
           "-I", "/opt/rocm/include", ADAPTER]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "warning" not in r.stderr, r.stderr


def test_adapter_syntax_against_standin_declarations():
    _syntax(os.path.join(STANDIN, "vv"))


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="reference tree absent")
def test_adapter_syntax_against_reference_headers():
    _syntax(REF_SRC)
