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
    # The three yardsticks bench.py measures with.
    rc = L.reng_hip_stream_stage(p, p, 16, 512, 3584, p, None)
    assert rc == R.EINVAL and b"outside 17..64" in L.reng_hip_last_error()
    rc = L.reng_hip_stream_stage(p, p, 64, 512, 3600, p, None)
    assert rc == R.EINVAL and b"multiple of 128" in L.reng_hip_last_error()
    rc = L.reng_hip_stream_stage(ctypes.c_void_p(8), p, 64, 512, 3584, p, None)
    assert rc == R.EINVAL and b"16-byte aligned" in L.reng_hip_last_error()
    rc = L.reng_hip_stream_read(p, 1000, p, None)
    assert rc == R.EINVAL and b"multiple of 1024" in L.reng_hip_last_error()
    rc = L.reng_hip_stream_narrow(p, 12, p, None)
    assert rc == R.EINVAL and b"multiple of 8" in L.reng_hip_last_error()
    rc = L.reng_hip_stream_narrow(ctypes.c_void_p(8), 16, p, None)
    assert rc == R.EINVAL and b"16-byte aligned" in L.reng_hip_last_error()


def test_the_binding_rejects_unknown_names():
    with pytest.raises(ValueError):
        R._fmt("fp4")
    with pytest.raises(ValueError):
        R._sc("bogus")
    assert R._fmt("HF8") == R.E4M3 and R._fmt("f8") == R.E5M2
    assert R._sc("per-channel") == R.PCS and R._sc("none") == R.UNIT


class _FakeDev:
    """Stands in for a GPU tensor in the binding's argument checks, which run
    before any library call (a check that passed would hand the library this
    address, so every case below must be refused)."""

    def __init__(self, nbytes, dtype=None):
        import torch

        self.dtype = torch.uint8 if dtype is None else dtype
        self._n = nbytes // torch.empty(0, dtype=self.dtype).element_size()
        self.is_cuda = True
        self.device = torch.device("cpu")   # where a wrapper allocates its outputs (never reached)

    def is_contiguous(self):
        return True

    def numel(self):
        return self._n

    def element_size(self):
        import torch

        return torch.empty(0, dtype=self.dtype).element_size()

    def data_ptr(self):
        return 16


def test_the_binding_refuses_short_buffers():
    import numpy as np
    import torch

    bf, f32 = torch.bfloat16, torch.float32
    rows, cols = 8, 64
    codes, scales = _FakeDev(rows * cols), _FakeDev(4 * rows, f32)
    with pytest.raises(ValueError, match="weight length against the shape"):
        R.quantize_into(_FakeDev(2 * rows * cols - 2, bf), rows, cols, "e4m3", "pcs", 1.0, codes, scales)
    with pytest.raises(ValueError, match="weight length"):   # a row pitch widens the span
        R.quantize_into(_FakeDev(2 * rows * cols, bf), rows, cols, "e4m3", "pcs", 1.0, codes, scales, ld=72)
    with pytest.raises(ValueError, match="weight length"):   # f32 weights: 4 bytes an element
        R.quantize_into(_FakeDev(2 * rows * cols, f32), rows, cols, "e4m3", "pcs", 1.0, codes, scales)
    with pytest.raises(ValueError, match="codes length"):
        R.quantize_into(_FakeDev(2 * rows * cols, bf), rows, cols, "e4m3", "pcs", 1.0, _FakeDev(rows * cols - 1),
                        scales)
    with pytest.raises(ValueError, match="scales length"):
        R.quantize_into(_FakeDev(2 * rows * cols, bf), rows, cols, "e4m3", "pcs", 1.0, codes, _FakeDev(4 * rows - 4, f32))
    with pytest.raises(ValueError, match="exp_bias length"):
        R.quantize_into(_FakeDev(2 * rows * cols, bf), rows, cols, "e4m3", "pcs", 1.0, codes, scales, _FakeDev(2))
    with pytest.raises(ValueError, match="weight length"):
        R.row_absmax(_FakeDev(2 * rows * cols - 2, bf), rows, cols)
    # quantize_batch: the dtype comes from the tensors, one dtype a batch.
    good = (_FakeDev(2 * rows * cols, bf), rows, cols, codes, scales, None)
    with pytest.raises(ValueError, match="one weight dtype"):
        R.quantize_batch([good, (_FakeDev(4 * rows * cols, f32), rows, cols, codes, scales, None)], "e4m3", "pcs")
    with pytest.raises(ValueError, match="weight 1 length"):
        R.quantize_batch([good, (_FakeDev(2 * rows * cols, f32), rows, cols, codes, scales, None)][:1] +
                         [(_FakeDev(2 * rows * cols - 2, bf), rows, cols, codes, scales, None)], "e4m3", "pcs")
    with pytest.raises(ValueError, match="empty batch"):
        R.quantize_batch([], "e4m3", "pcs")
    # The consumer.
    M, N, K = 4, 32, 128
    x, c, s, y = _FakeDev(2 * M * K, bf), _FakeDev(N * K), _FakeDev(4 * N, f32), _FakeDev(2 * M * N, bf)
    for args, what in [((_FakeDev(2 * M * K - 2, bf), c, s), "x"), ((x, _FakeDev(N * K - 1), s), "codes"),
                       ((x, c, _FakeDev(4 * N - 4, f32)), "scales")]:
        with pytest.raises(ValueError, match=f"{what} length"):
            R.gemm_w8a16(*args, M, N, K, "e4m3", y)
    with pytest.raises(ValueError, match="y length"):
        R.gemm_w8a16(x, c, s, M, N, K, "e4m3", _FakeDev(2 * M * N - 2, bf))
    a = _FakeDev(M * K)
    with pytest.raises(ValueError, match="b length"):
        R.gemm_fp8_scaled(a, "e4m3", None, _FakeDev(N * K - 1), "e4m3", None, M, N, K, y)
    with pytest.raises(ValueError, match="out length"):
        R.gemm_fp8_scaled(a, "e4m3", None, c, "e4m3", None, M, N, K, _FakeDev(2 * M * N - 2, bf))
    # The host entry: the reference's own refusal of a wrong-length slice.
    with pytest.raises(ValueError, match="weight length against the shape"):
        R.quantize_host(np.zeros(rows * cols - 1, dtype=np.uint16), rows, cols, "e4m3", "pcs")
    with pytest.raises(ValueError, match="weight length against the shape"):
        R.quantize_host(np.zeros(rows * cols + 1, dtype=np.float32), rows, cols, "e4m3", "pcs")
    # The decode-step helpers.
    with pytest.raises(ValueError, match="residual length"):
        R.gemv_residual(_FakeDev(2 * K, bf), c, s, N, K, "e4m3", _FakeDev(4 * N - 4, f32), _FakeDev(4 * N, f32))
    with pytest.raises(ValueError, match="gamma length"):
        R.rms_norm_bf16(_FakeDev(4 * rows * cols, f32), _FakeDev(4 * cols - 4, f32), rows, cols, 1e-5,
                        _FakeDev(2 * rows * cols, bf))
    with pytest.raises(ValueError, match="k_cache length"):
        R.attention_decode(_FakeDev(2 * 32 * 128, bf), _FakeDev(2 * 100 * 8 * 128 - 2, bf),
                           _FakeDev(2 * 100 * 8 * 128, bf), 32, 8, 128, 100, 0.1, _FakeDev(2 * 32 * 128, bf))
    with pytest.raises(ValueError, match="v_row length"):
        R.rope_append(_FakeDev(2 * 4 * 64, bf), _FakeDev(2 * 2 * 64, bf), _FakeDev(2 * 2 * 64, bf), 4, 2, 64,
                      _FakeDev(4 * 64, f32), _FakeDev(4 * 64, f32), _FakeDev(2 * 2 * 64, bf), _FakeDev(2 * 64, bf))
