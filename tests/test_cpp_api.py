"""The C++ mirror of the reng-fp8 crate API (reciprocating-engine_amd/host):
tests/cpp/test_reng_fp8.cpp ports the crate's unit tests
(crates/reng-fp8/src/lib.rs:633-926) and fixture tests
(crates/reng-fp8/tests/fixtures.rs:113-292) onto it. Without a GPU only the
tests that touch no device run (constants, names, bf16 helpers, the
exponent-bias choice, the asserts' messages, the fixture file)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
BIN = os.path.join(CPP, "build", "test_reng_fp8")
FIXTURE = os.path.join(ROOT, "tests", "golden", "fp8_cast.json")


def _binary():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-C", CPP], check=True, capture_output=True)
    return BIN


def _run(*args, timeout):
    r = subprocess.run([_binary(), "--fixture", FIXTURE, *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    return r.stdout


def test_cpp_api_host_side():
    out = _run("--cpu-only", timeout=60)
    assert "5 run, 0 failed" in out


@pytest.mark.gpu
def test_cpp_api_on_the_device():
    out = _run(timeout=110)
    assert " 0 failed" in out and "FAILED" not in out
    # Every test ran, device ones included.
    assert int(out.strip().splitlines()[-1].split()[0]) >= 27
