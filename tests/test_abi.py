"""The C ABI without a GPU: the library loads, exports every entry point that
include/reng_hip.h declares with the documented signature, and refuses bad
arguments with EINVAL and the reference's messages before touching a device."""
import ctypes
import os
import re

import pytest

import reng_hip as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "reng_hip.h")


def declared():
    text = open(HEADER).read()
    return re.findall(r"RENG_HIP_API\s+[\w\s\*]+?\b(reng_hip_\w+)\s*\(", text)


def test_every_declared_entry_point_is_exported():
    names = declared()
    assert len(names) >= 15
    R.lib()   # loads torch's HIP runtime first, as the binding does
    lib = ctypes.CDLL(R.LIB_PATH)
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(R.SIGNATURES), set(names) ^ set(R.SIGNATURES)


def test_header_constants_match_the_binding():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (RENG_HIP_\w+) (\d+)", text))
    assert int(consts["RENG_HIP_E4M3"]) == R.E4M3 and int(consts["RENG_HIP_E5M2"]) == R.E5M2
    assert int(consts["RENG_HIP_PCS"]) == R.PCS and int(consts["RENG_HIP_HW"]) == R.HW
    assert int(consts["RENG_HIP_UNIT"]) == R.UNIT
    assert int(consts["RENG_HIP_BF16"]) == R.BF16 and int(consts["RENG_HIP_F32"]) == R.F32
    assert int(consts["RENG_HIP_EINVAL"]) == R.EINVAL


def test_version():
    assert R.version().startswith("reng-hip ")


def test_choose_exp_bias_is_the_reference_rule():
    # lib.rs:757-766
    for a, want in [(0.5, 15), (0.9375, 15), (1.0, 11), (15.0, 11), (16.0, 7), (1000.0, 3), (1e9, 3)]:
        assert R.choose_exp_bias(a, "e4m3") == want
    assert R.choose_exp_bias(1e9, "e5m2") == 15


def test_refusals_happen_before_any_device_work():
    L = R.lib()
    p = ctypes.c_void_p(16)   # never dereferenced: the checks come first
    rc = L.reng_hip_quantize(p, R.BF16, 0, 16, 16, R.E4M3, R.PCS, 1.0, p, p, None, None)
    assert rc == R.EINVAL and L.reng_hip_last_error() == b"empty shape 0 x 16"
    rc = L.reng_hip_quantize(p, R.BF16, 4, 16, 16, R.E4M3, R.PCS, 0.0, p, p, None, None)
    assert rc == R.EINVAL and b"is not positive and finite" in L.reng_hip_last_error()
    rc = L.reng_hip_quantize(p, R.BF16, 4, 16, 16, R.E4M3, R.PCS, float("inf"), p, p, None, None)
    assert rc == R.EINVAL
    rc = L.reng_hip_quantize(p, R.BF16, 4, 16, 8, R.E4M3, R.PCS, 1.0, p, p, None, None)
    assert rc == R.EINVAL and b"row pitch" in L.reng_hip_last_error()
    rc = L.reng_hip_quantize(p, 7, 4, 16, 16, R.E4M3, R.PCS, 1.0, p, p, None, None)
    assert rc == R.EINVAL
    rc = L.reng_hip_quantize(p, R.BF16, 4, 16, 16, 9, R.PCS, 1.0, p, p, None, None)
    assert rc == R.EINVAL
    rc = L.reng_hip_gemm_w8a16(p, p, None, 1, 8, 40, R.E4M3, p, None)
    assert rc == R.EINVAL and b"multiple of 16" in L.reng_hip_last_error()
    rc = L.reng_hip_gemm_fp8_scaled(p, R.E4M3, None, 0, p, R.E4M3, p, 5, 4, 8, 128, p, None)
    assert rc == R.EINVAL and b"scale_b" in L.reng_hip_last_error()
    rc = L.reng_hip_gemm_fp8_scaled(p, R.E4M3, None, 0, p, R.E4M3, None, 0, 4, 8, 100, p, None)
    assert rc == R.EINVAL and b"multiple of 128" in L.reng_hip_last_error()
    arr = (R._Matrix * 1)()
    rc = L.reng_hip_quantize_batch(arr, 0, R.BF16, R.E4M3, R.PCS, 1.0, None)
    assert rc == R.EINVAL


def test_the_binding_rejects_unknown_names():
    with pytest.raises(ValueError):
        R._fmt("fp4")
    with pytest.raises(ValueError):
        R._sc("bogus")
    assert R._fmt("HF8") == R.E4M3 and R._fmt("f8") == R.E5M2
    assert R._sc("per-channel") == R.PCS and R._sc("none") == R.UNIT
