"""Runs the C++ restatement of the reference's tests (tests/cpp/test_facade.cpp) against the
C++ host API include/vector_hip.hpp.  The binary is built by vector-rs_amd/Makefile."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "vector-rs_amd")
BIN = os.path.join(PKG, "_build", "test_facade")


def _binary():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-s", "-C", PKG, "_build/test_facade"], check=True)
    return BIN


def _run(args, timeout):
    p = subprocess.run([_binary()] + args, capture_output=True, text=True, timeout=timeout)
    print(p.stdout)
    fails = [l for l in p.stdout.splitlines() if l.startswith("FAIL")]
    assert p.returncode == 0 and not fails, "\n".join(fails) or p.stderr
    return p.stdout


def test_facade_host_semantics():
    out = _run(["--host"], 60)
    assert out.count("PASS") >= 9


@pytest.mark.gpu
def test_facade_reference_tests_on_gpu():
    out = _run([], 110)
    assert out.count("PASS") >= 40
