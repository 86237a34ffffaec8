"""The oracle and the library's host-only C ABI (xwen_amd/csrc/xs_host.cpp)
built with -fsanitize=address,undefined (oracle/Makefile, target asan), and
tests/test_oracle.py plus tests/test_host_abi.py run against those builds in a
child process: any out-of-bounds access, use after free or undefined
behaviour in the C code aborts the child and fails this test.  CPU only."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN_DIR = os.path.join(ROOT, "oracle", "_build", "asan")


def _runtime():
    if not shutil.which("gcc") or not shutil.which("make"):
        return None
    out = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True,
                         text=True).stdout.strip()
    return out if os.path.isabs(out) and os.path.exists(out) else None


def test_oracle_and_host_abi_under_asan_and_ubsan():
    rt = _runtime()
    if rt is None:
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    env = dict(os.environ)
    env.update(
        LD_PRELOAD=rt,  # the runtime must come first; python itself is not instrumented
        ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1",
        UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
        XS_ORACLE_LIB=os.path.join(ASAN_DIR, "libxs_oracle.so"),
        XS_HOST_LIB=os.path.join(ASAN_DIR, "libxs_host.so"),
    )
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        "-m", "not gpu", "tests/test_oracle.py", "tests/test_host_abi.py"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    tail = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, tail
    assert "passed" in r.stdout and "ERROR: AddressSanitizer" not in r.stderr, tail
    assert "runtime error:" not in r.stderr, tail


PROBE = r"""
import ctypes as C, os, sys
L = C.CDLL(os.environ["XS_HOST_LIB"])
libc = C.CDLL(None)
libc.malloc.restype = C.c_void_p
p = libc.malloc(16)             # four floats, with the sanitizer's red zone after them
C.memset(p, 0, 16)
L.xs_keep_confident.restype = C.c_int64
L.xs_keep_confident.argtypes = [C.c_void_p, C.c_int64, C.c_float]
print("kept", L.xs_keep_confident(p, 5, -1.0))  # n = 5 overstates the array by one
sys.exit(0)
"""


def test_the_sanitizer_is_live():
    """The same runtime set-up reports a one-element overread of a host buffer
    (a caller's mistake, made on the CPU), so a clean run above means something."""
    rt = _runtime()
    if rt is None:
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True)
    env = dict(os.environ, LD_PRELOAD=rt, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               XS_HOST_LIB=os.path.join(ASAN_DIR, "libxs_host.so"))
    r = subprocess.run([sys.executable, "-c", PROBE], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr, r.stdout + r.stderr[-2000:]
