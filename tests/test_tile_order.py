"""The fp8 wide GEMM's workgroup -> tile order (csrc/tile_order.h, the same
header the kernel includes): tests/cpp/test_tile_order.cpp checks that every
grid's workgroups reach every tile exactly once, with and without the 2-D XCD
blocks, and which blocks the launcher picks on the Qwen2.5-32B prefill shapes."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP = os.path.join(ROOT, "tests", "cpp")
BIN = os.path.join(CPP, "build", "test_tile_order")


def test_every_workgroup_reaches_a_distinct_tile():
    subprocess.run(["make", "-C", CPP, "build/test_tile_order"], check=True, capture_output=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("0 failed")
