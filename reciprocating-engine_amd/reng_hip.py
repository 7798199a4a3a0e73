"""Python binding of libreng_hip.so (include/reng_hip.h) over ctypes.

The names follow the reference's reng-fp8 API (crates/reng-fp8/src/lib.rs):
`quantize_with`, `quantize`, `encode`, `decode`, `row_absmax`, `row_errors`,
`sample_row_errors`, `choose_exp_bias`, `Quantized.dequantize`, and the
consumer `gemm_w8a16` / `gemm_fp8_scaled` (crates/reng-synapse/src/fp8.rs).

Device work takes torch tensors that live on the GPU (torch is only the
allocator and the stream here) and runs on torch's current stream. There is no
CPU path: if the library is missing or a call fails, this module raises.
Argument errors that reng-fp8 turns into panics (lib.rs:527-532) raise
`ValueError` with the library's message.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libreng_hip.so")

OK, EINVAL, EDEVICE, ENOMEM, EUNSUPPORTED = 0, 1, 2, 3, 4
E4M3, E5M2 = 0, 1
PCS, HW, UNIT = 0, 1, 2
BF16, F32 = 0, 1
DEFAULT_BACKOFF = 1.0

FORMAT_NAMES = {"e4m3": E4M3, "fp8_143": E4M3, "hf8": E4M3, "e5m2": E5M2, "fp8_152": E5M2, "f8": E5M2}
SCALING_NAMES = {"pcs": PCS, "per-channel": PCS, "perchannel": PCS, "hw": HW, "hw-exp-bias": HW,
                 "expbias": HW, "unit": UNIT, "none": UNIT}
MAX_FINITE = {E4M3: 240.0, E5M2: 57344.0}
EXPONENT_BIAS = {E4M3: 7, E5M2: 15}


class RengHipError(RuntimeError):
    pass


class _Matrix(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("codes", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("exp_bias", ctypes.c_void_p), ("rows", ctypes.c_size_t), ("cols", ctypes.c_size_t),
                ("ld", ctypes.c_size_t)]


_lib = None
_P, _SZ, _I, _F, _U32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_uint32

SIGNATURES = {
    "reng_hip_version": (ctypes.c_char_p, []),
    "reng_hip_last_error": (ctypes.c_char_p, []),
    "reng_hip_device_info": (_I, [ctypes.c_char_p, _SZ]),
    "reng_hip_quantize": (_I, [_P, _I, _SZ, _SZ, _SZ, _I, _I, _F, _P, _P, _P, _P]),
    "reng_hip_quantize_host": (_I, [_P, _I, _SZ, _SZ, _I, _I, _F, _P, _P, _P]),
    "reng_hip_quantize_batch": (_I, [ctypes.POINTER(_Matrix), _SZ, _I, _I, _I, _F, _P]),
    "reng_hip_row_absmax": (_I, [_P, _I, _SZ, _SZ, _SZ, _P, _P]),
    "reng_hip_choose_exp_bias": (_U32, [_F, _I]),
    "reng_hip_encode": (_I, [_P, _SZ, _I, _P, _P]),
    "reng_hip_decode": (_I, [_P, _SZ, _I, _P, _P]),
    "reng_hip_dequantize": (_I, [_P, _P, _SZ, _SZ, _I, _I, _P, _P]),
    "reng_hip_row_errors": (_I, [_P, _P, _P, _SZ, _SZ, _I, _SZ, _P, _P, _P]),
    "reng_hip_gemm_w8a16": (_I, [_P, _P, _P, _SZ, _SZ, _SZ, _I, _P, _P]),
    "reng_hip_gemm_w8a16_noalloc": (_I, [_P, _P, _P, _SZ, _SZ, _SZ, _I, _P, _P]),
    "reng_hip_gemm_fp8_scaled": (_I, [_P, _I, _P, _SZ, _P, _I, _P, _SZ, _SZ, _SZ, _SZ, _P, _P]),
    "reng_hip_verify_hw_convert": (_I, [_I, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint32)]),
    "reng_hip_rms_norm_bf16": (_I, [_P, _P, _SZ, _SZ, _F, _P, _P]),
    "reng_hip_add_rms_norm_bf16": (_I, [_P, _P, _P, _SZ, _SZ, _F, _P, _P, _P]),
    "reng_hip_gemv_w8a16_residual": (_I, [_P, _P, _P, _SZ, _SZ, _I, _P, _P, _P]),
    "reng_hip_gemv_w8a16_swiglu": (_I, [_P, _P, _P, _SZ, _SZ, _I, _P, _P]),
    "reng_hip_gemv_w8a16_rmsnorm": (_I, [_P, _P, _F, _P, _P, _SZ, _SZ, _I, _P, _P]),
    "reng_hip_gemv_w8a16_rmsnorm_swiglu": (_I, [_P, _P, _F, _P, _P, _SZ, _SZ, _I, _P, _P]),
    "reng_hip_gemv_w8a16_rmsnorm_qkv_rope": (_I, [_P, _P, _F, _P, _P, _SZ, _SZ, _SZ, _SZ, _I, _P, _P, _P, _P, _P,
                                                   _P]),
    "reng_hip_rope_append": (_I, [_P, _P, _P, _SZ, _SZ, _SZ, _P, _P, _P, _P, _P]),
    "reng_hip_attention_decode": (_I, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _F, _P, _P]),
    "reng_hip_attention_workspace_bytes": (_SZ, [_SZ, _SZ, _SZ]),
    "reng_hip_attention_decode_split": (_I, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _F, _P, _SZ, _P, _P]),
    "reng_hip_silu_mul_bf16": (_I, [_P, _P, _SZ, _P, _P]),
    "reng_hip_add_bf16_f32": (_I, [_P, _P, _SZ, _P, _P]),
    "reng_hip_stream_read_sink_bytes": (_SZ, []),
    "reng_hip_stream_read": (_I, [_P, _SZ, _P, _P]),
    "reng_hip_stream_narrow": (_I, [_P, _SZ, _P, _P]),
    "reng_hip_stream_stage": (_I, [_P, _P, _SZ, _SZ, _SZ, _P, _P]),
}


def lib():
    """Load libreng_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        # torch ships its own HIP runtime under the same soname; loading torch
        # first makes libreng_hip.so bind to that one, so the process holds a
        # single runtime (two runtimes on one device: the second to initialise
        # finds no device).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RengHipError(f"{LIB_PATH} is missing: build it with `make -C reciprocating-engine_amd`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc != OK:
        msg = lib().reng_hip_last_error().decode()
        if rc == EINVAL:
            raise ValueError(msg)
        raise RengHipError(f"status {rc}: {msg}")


def _fmt(f):
    if isinstance(f, str):
        if f.strip().lower() not in FORMAT_NAMES:
            raise ValueError(f"unknown format {f}")
        return FORMAT_NAMES[f.strip().lower()]
    return int(f)


def _sc(s):
    if isinstance(s, str):
        if s.strip().lower() not in SCALING_NAMES:
            raise ValueError(f"unknown scaling {s}")
        return SCALING_NAMES[s.strip().lower()]
    return int(s)


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(t, what, nbytes=None):
    """The device address of a contiguous GPU tensor; with nbytes, refuse a
    tensor smaller than the bytes the C call will touch (the reference refuses
    a weight slice of the wrong length, crates/reng-fp8/src/lib.rs:528; here a
    short buffer would be read or written past its end on the device)."""
    if not t.is_cuda:
        raise ValueError(f"{what} must be a GPU tensor")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")
    if nbytes is not None:
        have = t.numel() * t.element_size()
        if have < nbytes:
            raise ValueError(f"{what} length against the shape: {have} bytes, the call touches {nbytes}")
    return ctypes.c_void_p(t.data_ptr())


def _opt(t, what, nbytes=None):
    return None if t is None else _dev(t, what, nbytes)


def _span(rows, cols, ld):
    """Elements a [rows, cols] window of row pitch ld spans."""
    return 0 if rows == 0 or cols == 0 else (rows - 1) * ld + cols


def _dtype_code(t):
    import torch

    if t.dtype in (torch.bfloat16, torch.int16, torch.uint16):
        return BF16
    if t.dtype == torch.float32:
        return F32
    raise ValueError(f"weights must be bf16 (or its bits as int16/uint16) or f32, not {t.dtype}")


def version():
    return lib().reng_hip_version().decode()


def device_info():
    buf = ctypes.create_string_buffer(512)
    _check(lib().reng_hip_device_info(buf, 512))
    return buf.value.decode()


def choose_exp_bias(absmax, fmt):
    return int(lib().reng_hip_choose_exp_bias(float(absmax), _fmt(fmt)))


class Quantized:
    """reng_fp8::Quantized (lib.rs:291-345), holding device tensors."""

    def __init__(self, format, scaling, rows, cols, codes, scales, exp_bias):
        self.format, self.scaling = format, scaling
        self.rows, self.cols = rows, cols
        self.codes, self.scales = codes, scales
        self.exp_bias = exp_bias

    def code_bytes(self):
        return self.rows * self.cols

    def scale_operand(self):
        return self.scales if _sc(self.scaling) == PCS else None

    def dequantize(self):
        import torch

        out = torch.empty(self.rows * self.cols, dtype=torch.float32, device=self.codes.device)
        _check(lib().reng_hip_dequantize(_dev(self.codes, "codes", self.rows * self.cols),
                                         _dev(self.scales, "scales", 4 * self.rows), self.rows,
                                         self.cols, _fmt(self.format), F32, _dev(out, "out"), _stream()))
        return out

    def dequantize_bf16(self):
        import torch

        out = torch.empty(self.rows * self.cols, dtype=torch.int16, device=self.codes.device)
        _check(lib().reng_hip_dequantize(_dev(self.codes, "codes", self.rows * self.cols),
                                         _dev(self.scales, "scales", 4 * self.rows), self.rows,
                                         self.cols, _fmt(self.format), BF16, _dev(out, "out"), _stream()))
        return out


def quantize_into(w, rows, cols, fmt, scaling, backoff, codes, scales, exp_bias=None, ld=None):
    """Device quantize into caller-owned tensors (no allocation)."""
    ld = cols if ld is None else ld
    dt = _dtype_code(w)
    _check(lib().reng_hip_quantize(_dev(w, "weight", _span(rows, cols, ld) * (2 if dt == BF16 else 4)), dt, rows,
                                   cols, ld, _fmt(fmt), _sc(scaling), float(backoff),
                                   _dev(codes, "codes", rows * cols), _dev(scales, "scales", 4 * rows),
                                   _opt(exp_bias, "exp_bias", 4), _stream()))


def quantize_with(w, rows, cols, fmt, scaling, backoff=DEFAULT_BACKOFF, ld=None):
    """reng_fp8::quantize_with (lib.rs:519-563) on the GPU: w is a device tensor
    of bf16 (or its int16 bits) or f32, [rows, ld] row-major."""
    import torch

    codes = torch.empty(rows * cols, dtype=torch.uint8, device=w.device)
    scales = torch.empty(rows, dtype=torch.float32, device=w.device)
    eb = torch.empty(1, dtype=torch.int32, device=w.device)
    quantize_into(w, rows, cols, fmt, scaling, backoff, codes, scales, eb, ld)
    return Quantized(fmt, scaling, rows, cols, codes, scales, int(eb.item()))


def quantize(w, rows, cols, fmt, scaling):
    return quantize_with(w, rows, cols, fmt, scaling, DEFAULT_BACKOFF)


def quantize_host(w, rows, cols, fmt, scaling, backoff=DEFAULT_BACKOFF):
    """The host-pointer entry (numpy in, numpy out), as Rust's quantize_with calls it."""
    import numpy as np

    w = np.ascontiguousarray(w)
    dt = BF16 if w.dtype == np.uint16 else F32 if w.dtype == np.float32 else None
    if dt is None:
        raise ValueError(f"weights must be uint16 (bf16 bits) or float32, not {w.dtype}")
    if rows > 0 and cols > 0 and w.size != rows * cols:   # lib.rs:528 (an empty shape is the library's refusal)
        raise ValueError(f"weight length against the shape: {w.size} elements for [{rows}, {cols}]")
    codes = np.empty(rows * cols, dtype=np.uint8)
    scales = np.empty(rows, dtype=np.float32)
    eb = ctypes.c_uint32(0)
    _check(lib().reng_hip_quantize_host(ctypes.c_void_p(w.ctypes.data), dt, rows, cols, _fmt(fmt), _sc(scaling),
                                        float(backoff), ctypes.c_void_p(codes.ctypes.data),
                                        ctypes.c_void_p(scales.ctypes.data), ctypes.byref(eb)))
    return codes, scales, int(eb.value)


def quantize_batch(mats, fmt, scaling, backoff=DEFAULT_BACKOFF):
    """mats: list of (w, rows, cols, codes, scales, exp_bias_or_None) device
    tensors, all bf16 (or its int16 bits) or all f32."""
    if not mats:
        raise ValueError("empty batch")
    dts = {_dtype_code(m[0]) for m in mats}
    if len(dts) != 1:
        raise ValueError("a batch holds one weight dtype (bf16 or f32), not a mix")
    dtype = dts.pop()
    esz = 2 if dtype == BF16 else 4
    arr = (_Matrix * len(mats))()
    for i, (w, rows, cols, codes, scales, eb) in enumerate(mats):
        arr[i] = _Matrix(_dev(w, f"weight {i}", rows * cols * esz).value, _dev(codes, f"codes {i}", rows * cols).value,
                         _dev(scales, f"scales {i}", 4 * rows).value,
                         0 if eb is None else _dev(eb, f"exp_bias {i}", 4).value, rows, cols, cols)
    _check(lib().reng_hip_quantize_batch(arr, len(mats), dtype, _fmt(fmt), _sc(scaling), float(backoff),
                                         _stream()))


def row_absmax(w, rows, cols, ld=None):
    import torch

    out = torch.empty(rows, dtype=torch.float32, device=w.device)
    ld = cols if ld is None else ld
    dt = _dtype_code(w)
    _check(lib().reng_hip_row_absmax(_dev(w, "weight", _span(rows, cols, ld) * (2 if dt == BF16 else 4)), dt, rows,
                                     cols, ld, _dev(out, "out"), _stream()))
    return out


def encode(x, fmt):
    """encode over a device f32 tensor -> uint8 codes."""
    import torch

    out = torch.empty(x.numel(), dtype=torch.uint8, device=x.device)
    _check(lib().reng_hip_encode(_dev(x, "x"), x.numel(), _fmt(fmt), _dev(out, "out"), _stream()))
    return out


def decode(codes, fmt):
    import torch

    out = torch.empty(codes.numel(), dtype=torch.float32, device=codes.device)
    _check(lib().reng_hip_decode(_dev(codes, "codes"), codes.numel(), _fmt(fmt), _dev(out, "out"), _stream()))
    return out


def _errors(w, q, max_rows):
    import torch

    n = q.rows if max_rows == 0 else min(max_rows, q.rows)
    step = -(-q.rows // n)
    k = -(-q.rows // step)
    mean = torch.empty(k, dtype=torch.float32, device=q.codes.device)
    mx = torch.empty(k, dtype=torch.float32, device=q.codes.device)
    _check(lib().reng_hip_row_errors(_dev(w, "weight", 2 * q.rows * q.cols), _dev(q.codes, "codes", q.rows * q.cols),
                                     _dev(q.scales, "scales", 4 * q.rows), q.rows,
                                     q.cols, _fmt(q.format), max_rows, _dev(mean, "mean"), _dev(mx, "max"),
                                     _stream()))
    return mean, mx


def row_errors(w, q):
    return _errors(w, q, 0)


def sample_row_errors(w, q, max_rows):
    if max_rows == 0:
        raise ValueError("max_rows must be positive")
    return _errors(w, q, max_rows)


def gemm_w8a16(x, codes, scales, M, N, K, fmt, y=None):
    """y[M, N] bf16 = x[M, K] bf16 . (decode(codes[N, K]) * scales[N])^T."""
    import torch

    if y is None:
        y = torch.empty(M * N, dtype=torch.bfloat16, device=x.device)
    _check(lib().reng_hip_gemm_w8a16(_dev(x, "x", 2 * M * K), _dev(codes, "codes", N * K),
                                     _opt(scales, "scales", 4 * N), M, N, K, _fmt(fmt),
                                     _dev(y, "y", 2 * M * N), _stream()))
    return y


def gemm_fp8_scaled(a, a_fmt, scale_a, b, b_fmt, scale_b, M, N, K, out=None):
    """gemm_fp8_scaled (crates/reng-synapse/src/fp8.rs:295-331): bf16 out[M, N]."""
    import torch

    if out is None:
        out = torch.empty(M * N, dtype=torch.bfloat16, device=a.device)
    na = 0 if scale_a is None else scale_a.numel()
    nb = 0 if scale_b is None else scale_b.numel()
    _check(lib().reng_hip_gemm_fp8_scaled(_dev(a, "a", M * K), _fmt(a_fmt), _opt(scale_a, "scale_a", 4 * na),
                                          na, _dev(b, "b", N * K), _fmt(b_fmt), _opt(scale_b, "scale_b", 4 * nb), nb,
                                          M, N, K, _dev(out, "out", 2 * M * N), _stream()))
    return out


# ---------------------------------------------------------------- decode step
# The non-GEMM steps of one Llama decoder layer at decode time (csrc/layer.hip);
# the C++ host path (host/fp8_decoder.hpp) strings them together with the GEMV.


def rms_norm_bf16(x, gamma, rows, cols, eps, out=None):
    """out[rows, cols] bf16 = x / sqrt(mean(x^2) + eps) * gamma, x f32 (ops.rs:49-72)."""
    import torch

    if out is None:
        out = torch.empty(rows * cols, dtype=torch.bfloat16, device=x.device)
    _check(lib().reng_hip_rms_norm_bf16(_dev(x, "x", 4 * rows * cols), _dev(gamma, "gamma", 4 * cols), rows, cols,
                                        eps, _dev(out, "out", 2 * rows * cols), _stream()))
    return out


def gemv_residual(x, codes, scales, n, k, fmt, residual, out=None):
    """f32 out[n] = residual + bf16(x . (decode(codes[n, k]) * scales)^T), x bf16 [k]."""
    import torch

    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=x.device)
    _check(lib().reng_hip_gemv_w8a16_residual(_dev(x, "x", 2 * k), _dev(codes, "codes", n * k),
                                              _opt(scales, "scales", 4 * n), n, k, _fmt(fmt),
                                              _dev(residual, "residual", 4 * n), _dev(out, "out", 4 * n), _stream()))
    return out


def gemv_swiglu(x, codes, scales, n, k, fmt, out=None):
    """bf16 out[n / 2] = silu(gate) * up over codes whose rows alternate gate,
    up (row 2i gate row i, row 2i + 1 up row i)."""
    import torch

    if out is None:
        out = torch.empty(n // 2, dtype=torch.bfloat16, device=x.device)
    _check(lib().reng_hip_gemv_w8a16_swiglu(_dev(x, "x", 2 * k), _dev(codes, "codes", n * k),
                                            _opt(scales, "scales", 4 * n), n, k, _fmt(fmt),
                                            _dev(out, "out", 2 * (n // 2)), _stream()))
    return out


def gemv_rmsnorm(x, gamma, eps, codes, scales, n, k, fmt, swiglu=False, out=None):
    """bf16 out = W . bf16(rms_norm(x) * gamma), x f32 [k]; with swiglu the rows
    of codes alternate gate, up and out[n / 2] = silu(gate) * up."""
    import torch

    if out is None:
        out = torch.empty(n // 2 if swiglu else n, dtype=torch.bfloat16, device=x.device)
    fn = lib().reng_hip_gemv_w8a16_rmsnorm_swiglu if swiglu else lib().reng_hip_gemv_w8a16_rmsnorm
    _check(fn(_dev(x, "x", 4 * k), _dev(gamma, "gamma", 4 * k), eps, _dev(codes, "codes", n * k),
              _opt(scales, "scales", 4 * n), n, k, _fmt(fmt), _dev(out, "out", 2 * (n // 2 if swiglu else n)),
              _stream()))
    return out


def qkv_rope_row_order(n_heads, n_kv_heads, head_dim):
    """Source row (in [Wq; Wk; Wv] order) of each row of the rotation-pair
    order gemv_rmsnorm_qkv_rope takes."""
    import numpy as np

    half = head_dim // 2
    order = []
    for heads, base in ((n_heads, 0), (n_kv_heads, n_heads * head_dim)):
        for h in range(heads):
            for d in range(half):
                order += [base + h * head_dim + d, base + h * head_dim + d + half]
    order += list(range((n_heads + n_kv_heads) * head_dim, (n_heads + 2 * n_kv_heads) * head_dim))
    return np.asarray(order, dtype=np.int64)


def gemv_rmsnorm_qkv_rope(x, gamma, eps, codes, scales, n_heads, n_kv_heads, head_dim, k, fmt, sin_row, cos_row,
                          q, k_row, v_row):
    """Norm + [q | k | v] projection + RoPE + cache-row writes in one pass over
    codes in qkv_rope_row_order."""
    n = (n_heads + 2 * n_kv_heads) * head_dim
    _check(lib().reng_hip_gemv_w8a16_rmsnorm_qkv_rope(
        _dev(x, "x", 4 * k), _dev(gamma, "gamma", 4 * k), eps, _dev(codes, "codes", n * k),
        _opt(scales, "scales", 4 * n), n_heads, n_kv_heads, head_dim, k, _fmt(fmt),
        _dev(sin_row, "sin_row", 4 * head_dim), _dev(cos_row, "cos_row", 4 * head_dim),
        _dev(q, "q", 2 * n_heads * head_dim), _dev(k_row, "k_row", 2 * n_kv_heads * head_dim),
        _dev(v_row, "v_row", 2 * n_kv_heads * head_dim), _stream()))


def add_rms_norm_bf16(x, d, gamma, rows, cols, eps, h=None, out=None):
    """h = x + d (f32) and out = bf16(rms_norm(h) * gamma); returns (h, out)."""
    import torch

    if h is None:
        h = torch.empty(rows * cols, dtype=torch.float32, device=x.device)
    if out is None:
        out = torch.empty(rows * cols, dtype=torch.bfloat16, device=x.device)
    n = rows * cols
    _check(lib().reng_hip_add_rms_norm_bf16(_dev(x, "x", 4 * n), _dev(d, "d", 2 * n), _dev(gamma, "gamma", 4 * cols),
                                            rows, cols, eps, _dev(h, "h", 4 * n), _dev(out, "out", 2 * n),
                                            _stream()))
    return h, out


def rope_append(q, k, v, n_heads, n_kv_heads, head_dim, sin_row, cos_row, k_row, v_row):
    """Rotate-half RoPE of one position: q in place, k into k_row, v copied to v_row."""
    nq, nk = 2 * n_heads * head_dim, 2 * n_kv_heads * head_dim
    _check(lib().reng_hip_rope_append(_dev(q, "q", nq), _dev(k, "k", nk), _dev(v, "v", nk), n_heads, n_kv_heads,
                                      head_dim, _dev(sin_row, "sin_row", 4 * head_dim),
                                      _dev(cos_row, "cos_row", 4 * head_dim), _dev(k_row, "k_row", nk),
                                      _dev(v_row, "v_row", nk), _stream()))


def attention_decode(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, length, scale, out=None):
    """One query per head over cache rows 0 .. length - 1, bf16 out [n_heads * head_dim]."""
    import torch

    if out is None:
        out = torch.empty(n_heads * head_dim, dtype=torch.bfloat16, device=q.device)
    nq, nc = 2 * n_heads * head_dim, 2 * length * n_kv_heads * head_dim
    _check(lib().reng_hip_attention_decode(_dev(q, "q", nq), _dev(k_cache, "k_cache", nc),
                                           _dev(v_cache, "v_cache", nc), n_heads, n_kv_heads, head_dim, length, scale,
                                           _dev(out, "out", nq), _stream()))
    return out


def attention_workspace_bytes(n_heads, head_dim, length):
    """Device workspace attention_decode_split needs for caches of 1 .. length rows."""
    return lib().reng_hip_attention_workspace_bytes(n_heads, head_dim, length)


def attention_decode_split(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, length, scale, workspace=None,
                           out=None):
    """attention_decode with the cache split over workgroups and merged; workspace
    a device tensor of at least attention_workspace_bytes(...) bytes (allocated
    here when None)."""
    import torch

    if out is None:
        out = torch.empty(n_heads * head_dim, dtype=torch.bfloat16, device=q.device)
    if workspace is None:
        workspace = torch.empty(max(1, attention_workspace_bytes(n_heads, head_dim, length)), dtype=torch.uint8,
                                device=q.device)
    nq, nc = 2 * n_heads * head_dim, 2 * length * n_kv_heads * head_dim
    _check(lib().reng_hip_attention_decode_split(_dev(q, "q", nq), _dev(k_cache, "k_cache", nc),
                                                 _dev(v_cache, "v_cache", nc), n_heads, n_kv_heads, head_dim, length,
                                                 scale,
                                                 _dev(workspace, "workspace"),
                                                 workspace.numel() * workspace.element_size(),
                                                 _dev(out, "out", nq), _stream()))
    return out


def silu_mul_bf16(gate, up, n, out=None):
    import torch

    if out is None:
        out = torch.empty(n, dtype=torch.bfloat16, device=gate.device)
    _check(lib().reng_hip_silu_mul_bf16(_dev(gate, "gate", 2 * n), _dev(up, "up", 2 * n), n, _dev(out, "out", 2 * n),
                                        _stream()))
    return out


def add_bf16_f32(x, d, n, out=None):
    import torch

    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=x.device)
    _check(lib().reng_hip_add_bf16_f32(_dev(x, "x", 4 * n), _dev(d, "d", 2 * n), n, _dev(out, "out", 4 * n),
                                       _stream()))
    return out


def stream_read(buf, nbytes, sink):
    """The read yardstick: read nbytes of buf once (a device tensor; sink a
    device tensor of at least stream_read_sink_bytes() bytes)."""
    _check(lib().reng_hip_stream_read(_dev(buf, "buf", nbytes), nbytes,
                                      _dev(sink, "sink", lib().reng_hip_stream_read_sink_bytes()), _stream()))


def stream_narrow(src, elems, dst):
    """The stream yardstick: the high byte of each of elems bf16 values of src
    into dst (device tensors)."""
    _check(lib().reng_hip_stream_narrow(_dev(src, "src", 2 * elems), elems, _dev(dst, "dst", elems), _stream()))


def stream_stage(x, codes, M, N, K, sink):
    """The copy yardstick of the 16 < M <= 64 skinny GEMM: its global -> LDS
    copy stream for x [M, K] and codes [N, K] with no arithmetic (device tensors;
    sink: a device tensor of at least 4 bytes)."""
    _check(lib().reng_hip_stream_stage(_dev(x, "x", 2 * M * K), _dev(codes, "codes", N * K), M, N, K,
                                       _dev(sink, "sink", 4), _stream()))


def stream_read_sink_bytes():
    return int(lib().reng_hip_stream_read_sink_bytes())


def verify_hw_convert(fmt):
    n = ctypes.c_uint64(0)
    first = ctypes.c_uint32(0)
    _check(lib().reng_hip_verify_hw_convert(_fmt(fmt), ctypes.byref(n), ctypes.byref(first)))
    return int(n.value), int(first.value)
