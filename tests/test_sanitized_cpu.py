"""The oracle (oracle/vvo.c) and the host code of the C ABI
(vibevoice.cpp_amd/csrc/vva.cpp) built under AddressSanitizer and
UndefinedBehaviorSanitizer (`make -C oracle san`, `make -C vibevoice.cpp_amd
san`: lib/san/), and the CPU tests of the oracle and of the ABI run against
those builds in a child process with clang's sanitizer runtime preloaded.
CPU only: the GPU tests and the shipped libraries are the regular builds.

A planted out-of-bounds write through the sanitized oracle (a conversion
told to write more elements than its buffer holds) must stop the child with
AddressSanitizer's report, so a run that quietly lost its instrumentation
fails here too."""
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN_VVO = os.path.join(REPO, "oracle", "lib", "san", "libvvo.so")
SAN_VVA = os.path.join(REPO, "vibevoice.cpp_amd", "lib", "san", "libvva.so")
CLANG = "/opt/rocm/llvm/bin/clang"
SUITE = ["tests/test_oracle_attention.py", "tests/test_oracle_linear.py", "tests/test_oracle_numerics.py",
         "tests/test_abi.py"]


def _runtime():
    r = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    if r.returncode != 0 or not os.path.isfile(path):
        pytest.skip("clang's AddressSanitizer runtime is not installed")
    return path


@pytest.fixture(scope="module")
def san_env():
    if not os.path.exists(CLANG):
        pytest.skip("ROCm clang absent")
    for d in ("oracle", "vibevoice.cpp_amd"):
        r = subprocess.run(["make", "-C", os.path.join(REPO, d), "san"], capture_output=True, text=True,
                           timeout=600)
        assert r.returncode == 0, r.stdout + r.stderr
    env = dict(os.environ)
    env.update(LD_PRELOAD=_runtime(), ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", VVO_LIB=SAN_VVO, VVA_LIB=SAN_VVA)
    return env


def test_cpu_suite_under_asan_and_ubsan(san_env):
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *SUITE],
                       cwd=REPO, env=san_env, capture_output=True, text=True, timeout=900)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "passed" in r.stdout


def test_sanitized_builds_are_the_ones_loaded(san_env):
    code = ("import sys; sys.path[:0] = ['oracle', 'vibevoice.cpp_amd']\n"
            "import vvo, vva\n"
            "vvo.lib(); vva.load_library()\n"
            "maps = open('/proc/self/maps').read()\n"
            "print('asan' in maps and 'lib/san/libvvo.so' in maps and 'lib/san/libvva.so' in maps)\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=REPO, env=san_env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    assert r.stdout.strip().endswith("True"), r.stdout


def test_planted_overflow_is_caught(san_env):
    """vvo_from_f32 asked for 64 f16 values into a 32-value buffer."""
    code = ("import sys, ctypes; sys.path[:0] = ['oracle']\n"
            "import numpy as np, vvo\n"
            "L = vvo.lib()\n"
            "x = np.ones(64, np.float32); out = np.zeros(32, np.uint16)\n"
            "L.vvo_from_f32(x.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(ctypes.c_void_p), 1,\n"
            "               ctypes.c_int64(64))\n"
            "print('not caught')\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=REPO, env=san_env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode != 0 and "not caught" not in r.stdout
    assert "AddressSanitizer" in r.stderr and "buffer-overflow" in r.stderr, r.stderr[-2000:]
