"""The kernel-level roofline (reciprocating-engine_amd/reng_ceiling.py) against
crates/reng-ceiling/src/lib.rs: the reference's Gaudi2 constants (lib.rs:39-51),
the Precision table and parser (lib.rs:66-105), ceiling_from's closed form
(lib.rs:230-247) on hand-computed cases, and the MI355X figures the bench's
roofline fractions are taken against."""
import math

import pytest

import reng_ceiling as RC


def test_gaudi2_figures_are_the_reference_constants():
    hw = RC.HardwareSpec.gaudi2()
    assert hw.name == "Gaudi2 (HL-225)"
    assert (hw.flops_bf16, hw.flops_fp16, hw.flops_fp8, hw.flops_fp32) == (432.0e12, 432.0e12, 865.0e12, 45.0e12)
    assert hw.hbm_bytes == 96 * 2**30 and hw.hbm_bw == 2.45e12
    assert hw.sram_bytes == 48 * 2**20 and hw.pcie_bw == 32.0e9


def test_mi355x_figures():
    hw = RC.HardwareSpec.mi355x()
    assert hw.hbm_bw == 8.0e12 and hw.hbm_bytes == 288 * 10**9
    assert hw.flops_fp8 == 5.0e15 and hw.flops_bf16 == hw.flops_fp16 == 2.5e15
    assert hw.flops_fp32 == 157.3e12
    assert hw.sram_bytes == 256 * 2**20


def test_precision_table():
    P = RC.Precision
    assert [p.weight_bytes() for p in (P.FP32, P.BF16, P.FP16, P.FP8, P.INT8, P.INT4)] == [4, 2, 2, 1, 1, 0.5]
    hw = RC.HardwareSpec.gaudi2()
    # Integer weight-only formats dequantize to bf16 and take its rate.
    assert P.INT8.compute_flops(hw) == P.INT4.compute_flops(hw) == P.BF16.compute_flops(hw) == hw.flops_bf16
    assert P.FP8.compute_flops(hw) == hw.flops_fp8 and P.FP32.compute_flops(hw) == hw.flops_fp32
    assert P.FP16.compute_flops(hw) == hw.flops_fp16


@pytest.mark.parametrize("name,want", [
    ("bf16", "BF16"), ("BFloat16", "BF16"), ("fp16", "FP16"), ("float16", "FP16"), ("HALF", "FP16"),
    ("fp8", "FP8"), ("float8", "FP8"), ("fp32", "FP32"), ("float32", "FP32"), ("int8", "INT8"),
    ("i8", "INT8"), ("Int4", "INT4"), ("i4", "INT4")])
def test_precision_parse(name, want):
    assert RC.Precision.parse(name) is RC.Precision[want]


def test_precision_parse_refuses_with_the_reference_message():
    with pytest.raises(ValueError, match=r'^unknown precision "fp4"$'):
        RC.Precision.parse("FP4")
    with pytest.raises(ValueError, match=r'^unknown precision "a\\"b"$'):
        RC.Precision.parse('a"b')
    # Only ASCII letters fold, as Rust's to_ascii_lowercase.
    with pytest.raises(ValueError):
        RC.Precision.parse("ＢＦ16")


def test_ceiling_from_closed_forms():
    # 1 TFLOP against 1 PFLOP/s: 1 ms of compute; 1 GB against 2 TB/s: 0.5 ms.
    c = RC.ceiling_from(1e12, 1e9, 1e15, 2e12, 100.0)
    assert c.bottleneck is RC.Bottleneck.COMPUTE
    assert math.isclose(c.compute_time_s, 1e-3) and math.isclose(c.memory_time_s, 5e-4)
    assert math.isclose(c.latency_s, 1e-3) and math.isclose(c.tokens_per_s, 1e5)
    assert math.isclose(c.arithmetic_intensity, 1000.0)
    # The memory side sets it when it is the larger.
    m = RC.ceiling_from(1e9, 1e9, 1e15, 1e12, 1.0)
    assert m.bottleneck is RC.Bottleneck.HBM_BANDWIDTH
    assert math.isclose(m.latency_s, 1e-3) and math.isclose(m.compute_time_s, 1e-6)
    # A tie is compute-bound (compute_time >= memory_time).
    t = RC.ceiling_from(2e12, 1e9, 2e15, 1e12, 1.0)
    assert t.bottleneck is RC.Bottleneck.COMPUTE and t.compute_time_s == t.memory_time_s
    # fraction: ceiling over measured.
    assert math.isclose(c.fraction(2e-3), 0.5)


def test_kernel_ceilings_on_mi355x():
    hw = RC.HardwareSpec.mi355x()
    # The quantizer: 3 bytes per bf16 element + 4 per row, HBM-bound.
    q = RC.quantize_ceiling(hw, 4096, 14336)
    assert RC.quantize_bytes(4096, 14336) == 4096 * 14336 * 3 + 4 * 4096
    assert q.bottleneck is RC.Bottleneck.HBM_BANDWIDTH and math.isclose(q.latency_s, q.memory_time_s)
    assert math.isclose(q.latency_s, (4096 * 14336 * 3 + 4 * 4096) / 8e12)
    # w8a16 on bf16 MFMA against 1-byte codes: 2m flops per code byte against
    # 2.5e15 / 8e12 = 312.5 flops per byte, so HBM-bound up to m = 156.
    for m in (1, 8, 64, 128):
        assert RC.w8a16_ceiling(hw, m, 18944, 3584).bottleneck is RC.Bottleneck.HBM_BANDWIDTH, m
    assert RC.w8a16_ceiling(hw, 256, 18944, 3584).bottleneck is RC.Bottleneck.COMPUTE
    g = RC.w8a16_ceiling(hw, 1, 14336, 4096)
    assert math.isclose(g.memory_time_s, (14336 * 4096 + 4 * 14336 + 2 * 4096 + 2 * 14336) / 8e12)
    # The M = 1024 prefill GEMM on fp8 MFMA: compute-bound at every Qwen2.5-32B shape.
    for n, k in ((5120, 5120), (1024, 5120), (27648, 5120), (5120, 27648)):
        c = RC.fp8_gemm_ceiling(hw, 1024, n, k)
        assert c.bottleneck is RC.Bottleneck.COMPUTE, (n, k)
        assert math.isclose(c.compute_time_s, 2 * 1024 * n * k / 5.0e15)
