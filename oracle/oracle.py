"""ctypes view of the CPU oracle (oracle/build/libfp8_oracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP path and bench.py's CPU
baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
import this module; the product (libreng_hip.so and its bindings) never does.
Each function restates crates/reng-fp8/src/lib.rs; see fp8_oracle.c for the
line-by-line citations.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libfp8_oracle.so")

E4M3, E5M2 = 0, 1
PCS, HW, UNIT = 0, 1, 2
FORMATS = {"e4m3": E4M3, "e5m2": E5M2}
SCALINGS = {"pcs": PCS, "hw": HW, "unit": UNIT}

_lib = None

_P = ctypes.c_void_p
_SZ = ctypes.c_size_t


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_encode": (ctypes.c_uint8, [ctypes.c_float, ctypes.c_int]),
            "orc_decode": (ctypes.c_float, [ctypes.c_uint8, ctypes.c_int]),
            "orc_max_finite": (ctypes.c_float, [ctypes.c_int]),
            "orc_max_finite_code": (ctypes.c_uint8, [ctypes.c_int]),
            "orc_choose_exp_bias": (ctypes.c_uint32, [ctypes.c_float, ctypes.c_int]),
            "orc_split": (ctypes.c_int, [_SZ, _SZ]),
            "orc_encode_array": (None, [_P, _SZ, ctypes.c_int, _P, ctypes.c_int]),
            "orc_encode_bits_range": (None, [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, _P, ctypes.c_int]),
            "orc_decode_array": (None, [_P, _SZ, ctypes.c_int, _P]),
            "orc_row_absmax": (None, [_P, _SZ, _SZ, _P]),
            "orc_quantize_with": (ctypes.c_uint32, [_P, _SZ, _SZ, ctypes.c_int, ctypes.c_int, ctypes.c_float, _P, _P, ctypes.c_int]),
            "orc_quantize_f32_with": (ctypes.c_uint32, [_P, _SZ, _SZ, ctypes.c_int, ctypes.c_int, ctypes.c_float, _P, _P, ctypes.c_int]),
            "orc_dequantize": (None, [_P, _P, _SZ, _SZ, ctypes.c_int, _P]),
            "orc_row_errors": (None, [_P, _P, _P, _SZ, _SZ, ctypes.c_int, _P, _P]),
            "orc_sample_row_errors": (_SZ, [_P, _P, _P, _SZ, _SZ, ctypes.c_int, _SZ, _P, _P]),
            "orc_gemm": (None, [_P, _P, _SZ, _SZ, _SZ, _P, ctypes.c_int]),
            "orc_gemm_cols": (None, [_P, _P, _SZ, _SZ, _P, _SZ, _P, ctypes.c_int]),
            "orc_rel_l2": (ctypes.c_float, [_P, _P, _SZ]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def _fmt(f):
    return FORMATS[f] if isinstance(f, str) else int(f)


def _sc(s):
    return SCALINGS[s] if isinstance(s, str) else int(s)


def bf16_to_f32(x):
    return lib().orc_bf16_to_f32(int(x))


def f32_to_bf16(x):
    return lib().orc_f32_to_bf16(float(x))


def bf16_bits(x):
    """f32 array -> bf16 bit patterns with the reference's RNE (lib.rs:41-48)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + (0x7FFF + ((b >> 16) & 1))) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def encode(x, fmt):
    return lib().orc_encode(float(x), _fmt(fmt))


def decode(c, fmt):
    return lib().orc_decode(int(c), _fmt(fmt))


def max_finite(fmt):
    return lib().orc_max_finite(_fmt(fmt))


def choose_exp_bias(absmax, fmt):
    return lib().orc_choose_exp_bias(float(absmax), _fmt(fmt))


def split(rows, cols):
    return lib().orc_split(rows, cols)


def encode_array(x, fmt, threads=8):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().orc_encode_array(_ptr(x), x.size, _fmt(fmt), _ptr(out), threads)
    return out


def encode_bits_range(first, count, fmt, threads=8):
    out = np.empty(count, dtype=np.uint8)
    lib().orc_encode_bits_range(first, count, _fmt(fmt), _ptr(out), threads)
    return out


def decode_array(codes, fmt):
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(c.shape, dtype=np.float32)
    lib().orc_decode_array(_ptr(c), c.size, _fmt(fmt), _ptr(out))
    return out


def row_absmax(w_bits, rows, cols):
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    out = np.empty(rows, dtype=np.float32)
    lib().orc_row_absmax(_ptr(w), rows, cols, _ptr(out))
    return out


class Quantized:
    """Mirror of reng_fp8::Quantized (lib.rs:291-306)."""

    def __init__(self, fmt, scaling, rows, cols, codes, scales, exp_bias):
        self.format, self.scaling = fmt, scaling
        self.rows, self.cols = rows, cols
        self.codes, self.scales, self.exp_bias = codes, scales, exp_bias

    def dequantize(self):
        out = np.empty(self.rows * self.cols, dtype=np.float32)
        lib().orc_dequantize(_ptr(self.codes), _ptr(self.scales), self.rows, self.cols,
                             _fmt(self.format), _ptr(out))
        return out


def quantize_with(w, rows, cols, fmt, scaling, backoff=1.0, thread_cap=8):
    """bf16 bits (uint16) or f32 (float32) [rows, cols] -> Quantized."""
    w = np.ascontiguousarray(w)
    assert w.size == rows * cols
    codes = np.empty(rows * cols, dtype=np.uint8)
    scales = np.empty(rows, dtype=np.float32)
    if w.dtype == np.uint16:
        fn = lib().orc_quantize_with
    elif w.dtype == np.float32:
        fn = lib().orc_quantize_f32_with
    else:
        raise TypeError(w.dtype)
    b = fn(_ptr(w), rows, cols, _fmt(fmt), _sc(scaling), float(backoff), _ptr(codes),
           _ptr(scales), thread_cap)
    return Quantized(fmt, scaling, rows, cols, codes, scales, int(b))


def quantize(w, rows, cols, fmt, scaling):
    return quantize_with(w, rows, cols, fmt, scaling, 1.0)


def row_errors(w_bits, q):
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    mean = np.empty(q.rows, dtype=np.float32)
    mx = np.empty(q.rows, dtype=np.float32)
    lib().orc_row_errors(_ptr(w), _ptr(q.codes), _ptr(q.scales), q.rows, q.cols,
                         _fmt(q.format), _ptr(mean), _ptr(mx))
    return mean, mx


def sample_row_errors(w_bits, q, max_rows):
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    mean = np.empty(q.rows, dtype=np.float32)
    mx = np.empty(q.rows, dtype=np.float32)
    k = lib().orc_sample_row_errors(_ptr(w), _ptr(q.codes), _ptr(q.scales), q.rows, q.cols,
                                    _fmt(q.format), max_rows, _ptr(mean), _ptr(mx))
    return mean[:k].copy(), mx[:k].copy()


def gemm(a, b, m, k, n, threads=8):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    c = np.empty(m * n, dtype=np.float32)
    lib().orc_gemm(_ptr(a), _ptr(b), m, k, n, _ptr(c), threads)
    return c


def gemm_cols(a, b, m, k, cols_idx, threads=8):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    idx = np.ascontiguousarray(cols_idx, dtype=np.int64)
    c = np.empty(m * idx.size, dtype=np.float32)
    lib().orc_gemm_cols(_ptr(a), _ptr(b), m, k, _ptr(idx), idx.size, _ptr(c), threads)
    return c


def rel_l2(got, want):
    g = np.ascontiguousarray(got, dtype=np.float32)
    w = np.ascontiguousarray(want, dtype=np.float32)
    assert g.size == w.size
    return lib().orc_rel_l2(_ptr(g), _ptr(w), g.size)
