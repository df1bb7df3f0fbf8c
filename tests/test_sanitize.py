"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

* libmdgl's C ABI host code (capi.cpp: argument validation, broadcast
  descriptors, workspace sizes, softmax geometry) built with the host side
  instrumented (tests/sanitize/Makefile), driven by
  tests/sanitize/abi_host_check.cpp through calls that return before any
  launch;
* the CPU oracle built instrumented and run on seeded cases of every
  function (tests/sanitize/oracle_cases.py), whose results must equal the
  regular build's bit for bit.

A sanitizer report fails the run (recovery off for UBSan)."""

import os
import subprocess
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SAN = os.path.join(HERE, "sanitize")
ROOT = os.path.dirname(HERE)


def _make(target):
    from mojodgl import _lib

    _lib.build()  # the library's objects, which the ABI check links
    proc = subprocess.run(["make", "-C", SAN, target], capture_output=True, text=True,
                          timeout=900)
    if proc.returncode != 0:
        pytest.fail("sanitizer build failed:\n" + (proc.stderr or proc.stdout)[-3000:])
    return os.path.join(SAN, target)


def _clean(stderr):
    return "AddressSanitizer" not in stderr and "runtime error" not in stderr


@pytest.mark.parametrize("roctx", ["0", "1"])
def test_abi_host_code_under_sanitizers(roctx):
    """The host checks with the roctx ranges off and on (the roctx library
    opened at run time and a range pushed and popped around every call)."""
    exe = _make("_build/abi_host_check")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", MDGL_ROCTX=roctx)
    proc = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert proc.returncode == 0 and _clean(proc.stderr), proc.stdout + proc.stderr
    assert "abi host checks passed" in proc.stdout


def test_oracle_under_sanitizers(tmp_path):
    lib = _make("_build/liboracle_san.so")
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True,
                          text=True).stdout.strip()
    if not os.path.isabs(asan) or not os.path.exists(asan):
        pytest.skip("gcc's AddressSanitizer runtime is not installed")
    script = os.path.join(SAN, "oracle_cases.py")
    san_out, ref_out = str(tmp_path / "san.npz"), str(tmp_path / "ref.npz")
    env = dict(os.environ, LD_PRELOAD=asan, MDGL_ORACLE_LIB=lib,
               ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="halt_on_error=1")
    proc = subprocess.run([sys.executable, script, san_out], capture_output=True, text=True,
                          timeout=600, env=env)
    assert proc.returncode == 0 and _clean(proc.stderr), proc.stdout + proc.stderr[-3000:]
    env = {k: v for k, v in os.environ.items() if k != "MDGL_ORACLE_LIB"}
    proc = subprocess.run([sys.executable, script, ref_out], capture_output=True, text=True,
                          timeout=600, env=env)
    assert proc.returncode == 0, proc.stderr[-3000:]
    san, ref = np.load(san_out), np.load(ref_out)
    assert sorted(san.files) == sorted(ref.files) and len(ref.files) > 40
    for key in ref.files:
        np.testing.assert_array_equal(san[key], ref[key], err_msg=key)
