"""The C oracle and the library's host code under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only).  `make -C oracle sanitize` builds the
oracle with both and drives every function over edge cases
(oracle/san_check.c); `make -C haste_amd sanitize` builds the library with both
on its host code (the device code as usual) and drives the argument checks,
workspace sizing and bwd-features planning over a grid of shapes, every build
and dtype (tests/native/host_check.cpp), with no GPU.  A sanitizer report
aborts the program, so the test sees a non-zero status."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(args, marker, timeout):
    p = subprocess.run(args, cwd=ROOT, capture_output=True, text=True, timeout=timeout)
    out = p.stdout + p.stderr
    assert p.returncode == 0, out[-4000:]
    assert marker in p.stdout, out[-4000:]


def test_oracle_under_asan_ubsan():
    _run(["make", "-s", "-C", "oracle", "sanitize"], "san_check OK", 300)


def test_host_code_under_asan_ubsan():
    if not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("hipcc not found")
    _run(["make", "-s", "-j8", "-C", "haste_amd", "sanitize"], "host_check OK", 1200)
