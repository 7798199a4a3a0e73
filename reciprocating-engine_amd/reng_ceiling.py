"""reng_ceiling - the kernel-level roofline of reng-ceiling with an MI355X spec.

Mirrors the part of crates/reng-ceiling/src/lib.rs that a kernel's
roofline needs: `HardwareSpec` (lib.rs:13-51, with the reference's Gaudi2
figures and an MI355X entry), `Precision` (lib.rs:53-106: bytes per weight,
the compute rate a format's matmuls run at, the name parser), `Bottleneck`,
`Ceiling` and `ceiling_from` (lib.rs:210-247: time = max(flops / peak,
bytes / bandwidth)). The model-level prefill / decode ceilings, the
configuration grid and the strategy planner (lib.rs:249-483, strategy.rs)
are not part of this library.

On top of `ceiling_from`, the per-kernel ceilings bench.py reports: the
quantizer and the w8a16 GEMV / skinny GEMM are bounded by HBM bytes, the
fp8 x fp8 prefill GEMM by the fp8 MFMA rate.
"""
from dataclasses import dataclass
from enum import Enum


@dataclass(frozen=True)
class HardwareSpec:
    """Peak throughput and bandwidth figures for one accelerator (lib.rs:13-31).

    flops_* are dense matrix-core rates in FLOP/s (no structured-sparsity
    doubling); hbm_bw and pcie_bw in bytes/s (PCIe per direction)."""
    name: str
    flops_bf16: float
    flops_fp16: float
    flops_fp8: float
    flops_fp32: float
    hbm_bytes: int
    hbm_bw: float
    sram_bytes: int
    pcie_bw: float

    @staticmethod
    def gaudi2():
        """The reference's Intel Gaudi2 (HL-225) figures (lib.rs:33-51)."""
        return HardwareSpec(name="Gaudi2 (HL-225)", flops_bf16=432.0e12, flops_fp16=432.0e12,
                            flops_fp8=865.0e12, flops_fp32=45.0e12, hbm_bytes=98_304 * 1024 * 1024,
                            hbm_bw=2.45e12, sram_bytes=48 * 1024 * 1024, pcie_bw=32.0e9)

    @staticmethod
    def mi355x():
        """AMD Instinct MI355X, one GPU: 288 GB HBM3E at 8 TB/s; dense MFMA
        2.5 PFLOP/s bf16 / fp16, 5.0 PFLOP/s fp8, 157.3 TFLOP/s fp32 (AMD's
        published figures without 2:1 sparsity); the 256 MB Infinity Cache
        as the on-die memory; PCIe Gen5 x16, 64 GB/s per direction."""
        return HardwareSpec(name="MI355X", flops_bf16=2.5e15, flops_fp16=2.5e15, flops_fp8=5.0e15,
                            flops_fp32=157.3e12, hbm_bytes=288 * 10**9, hbm_bw=8.0e12,
                            sram_bytes=256 * 1024 * 1024, pcie_bw=64.0e9)


class Precision(Enum):
    """Storage and compute format of the weights (lib.rs:53-63)."""
    BF16 = "bf16"
    FP16 = "fp16"
    FP8 = "fp8"
    FP32 = "fp32"
    INT8 = "int8"
    INT4 = "int4"

    def weight_bytes(self):
        """Bytes per weight element (lib.rs:66-74)."""
        return {Precision.FP32: 4.0, Precision.BF16: 2.0, Precision.FP16: 2.0, Precision.FP8: 1.0,
                Precision.INT8: 1.0, Precision.INT4: 0.5}[self]

    def compute_flops(self, hw):
        """Peak matrix rate for this format's matmuls (lib.rs:76-88): the
        integer weight-only formats dequantize to bf16 and take its rate."""
        if self is Precision.FP8:
            return hw.flops_fp8
        if self is Precision.FP32:
            return hw.flops_fp32
        if self is Precision.FP16:
            return hw.flops_fp16
        return hw.flops_bf16

    @staticmethod
    def parse(s):
        """A precision name, case-insensitive (lib.rs:90-105); ValueError for
        an unknown one, with the reference's message."""
        names = {"bf16": Precision.BF16, "bfloat16": Precision.BF16, "fp16": Precision.FP16,
                 "float16": Precision.FP16, "half": Precision.FP16, "fp8": Precision.FP8,
                 "float8": Precision.FP8, "fp32": Precision.FP32, "float32": Precision.FP32,
                 "int8": Precision.INT8, "i8": Precision.INT8, "int4": Precision.INT4, "i4": Precision.INT4}
        low = "".join(chr(ord(c) + 32) if "A" <= c <= "Z" else c for c in s)   # ASCII only, as Rust's
        p = names.get(low)
        if p is None:
            raise ValueError(f"unknown precision {_debug_str(low)}")
        return p


def _debug_str(s):
    """Rust's {:?} of a str: quoted, with backslash, quote, tab, CR and LF escaped."""
    esc = {"\\": "\\\\", '"': '\\"', "\t": "\\t", "\r": "\\r", "\n": "\\n"}
    return '"' + "".join(esc.get(c, c) for c in s) + '"'


class Bottleneck(Enum):
    """Which resource sets the ceiling (lib.rs:210-217)."""
    COMPUTE = "compute"
    HBM_BANDWIDTH = "hbm"


@dataclass(frozen=True)
class Ceiling:
    """A computed ceiling (lib.rs:219-228)."""
    latency_s: float
    tokens_per_s: float
    bottleneck: Bottleneck
    compute_time_s: float
    memory_time_s: float
    arithmetic_intensity: float

    def fraction(self, measured_s):
        """The share of this ceiling a measured time reaches (ceiling / measured)."""
        return self.latency_s / measured_s


def ceiling_from(flops, bytes_, peak_flops, hbm_bw, tokens):
    """time = max(flops / peak, bytes / bandwidth); compute-bound on a tie
    (lib.rs:230-247)."""
    compute_time = flops / peak_flops
    memory_time = bytes_ / hbm_bw
    latency = max(compute_time, memory_time)
    bottleneck = Bottleneck.COMPUTE if compute_time >= memory_time else Bottleneck.HBM_BANDWIDTH
    return Ceiling(latency_s=latency, tokens_per_s=tokens / latency, bottleneck=bottleneck,
                   compute_time_s=compute_time, memory_time_s=memory_time,
                   arithmetic_intensity=flops / bytes_)


# ------------------------------------------------------------ per-kernel ceilings

def quantize_bytes(rows, cols, in_bytes=2):
    """HBM bytes of one quantize_with pass: the weights read once, one code
    byte per element and one f32 scale per row written."""
    return rows * cols * (in_bytes + 1) + 4 * rows


def quantize_ceiling(hw, rows, cols, in_bytes=2):
    """The quantizer moves bytes and does no matrix work: HBM-bound."""
    return ceiling_from(0.0, float(quantize_bytes(rows, cols, in_bytes)), hw.flops_fp32, hw.hbm_bw, rows)


def w8a16_bytes(m, n, k):
    """HBM bytes of y[m, n] = x[m, k] (bf16) . decode(codes[n, k]) * s[n]:
    codes, scales, the activation and the bf16 output."""
    return n * k + 4 * n + 2 * m * k + 2 * m * n


def w8a16_ceiling(hw, m, n, k):
    """The fp8-dequant GEMV / skinny GEMM: 2 m n k flops on bf16 MFMA against
    its bytes (HBM-bound for m <= 64)."""
    return ceiling_from(2.0 * m * n * k, float(w8a16_bytes(m, n, k)), Precision.BF16.compute_flops(hw),
                        hw.hbm_bw, m)


def fp8_gemm_ceiling(hw, m, n, k):
    """The fp8 x fp8 GEMM: 2 m n k flops on the fp8 MFMA rate against fp8
    operands, f32 scales and the bf16 output."""
    bytes_ = m * k + n * k + 4 * (m + n) + 2 * m * n
    return ceiling_from(2.0 * m * n * k, float(bytes_), Precision.FP8.compute_flops(hw), hw.hbm_bw, m)
