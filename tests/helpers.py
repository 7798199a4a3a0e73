"""Shared test helpers: the golden fixture reader and the independent checks.

The independent checks do not restate the reference's bit manipulation:

* `closed_form_decode` builds every fp8 value from sign, exponent and mantissa
  with exact rational arithmetic (the format definition, lib.rs:4-9, 206-225).
* `nearest_encode` rounds by searching the sorted table of finite values and
  comparing against the exact midpoint of the two neighbours (round to nearest,
  ties to the even code, saturation above the largest finite value).
* `torch_cast` is torch's own float8 cast with the fixture generator's
  saturation substitution (tools/fp8_fixtures.py:46-55).
"""
import json
from fractions import Fraction

import numpy as np

E4M3, E5M2 = 0, 1
FMT = {"e4m3": E4M3, "e5m2": E5M2}
MBITS = {E4M3: 3, E5M2: 2}
BIAS = {E4M3: 7, E5M2: 15}
MAXCODE = {E4M3: 0x77, E5M2: 0x7B}


def closed_form_decode(code, fmt):
    """Exact value of a code as a Fraction, or 'inf'/'nan' for the top exponent field."""
    m = MBITS[fmt]
    e_bits = 7 - m
    sign = -1 if code & 0x80 else 1
    mant = code & ((1 << m) - 1)
    ef = (code & 0x7F) >> m
    if ef == (1 << e_bits) - 1:
        return "inf" if mant == 0 else "nan"
    if ef == 0:
        return sign * Fraction(mant, 1 << m) * Fraction(2) ** (1 - BIAS[fmt])
    return sign * (1 + Fraction(mant, 1 << m)) * Fraction(2) ** (ef - BIAS[fmt])


def positive_table(fmt):
    """(codes, values) of every finite non-negative code, in increasing value."""
    codes = [c for c in range(0x80) if closed_form_decode(c, fmt) not in ("inf", "nan")]
    vals = [float(closed_form_decode(c, fmt)) for c in codes]
    order = np.argsort(vals, kind="stable")
    return np.array(codes, dtype=np.uint8)[order], np.array(vals, dtype=np.float64)[order]


def nearest_encode(x, fmt):
    """Round-to-nearest-even onto the finite grid, saturating; NaN -> sign|0x7f."""
    x = np.asarray(x, dtype=np.float32).ravel()
    codes, vals = positive_table(fmt)
    a = np.abs(x.astype(np.float64))
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    out = np.empty(x.size, dtype=np.uint8)
    nan = np.isnan(x)
    fin = ~nan
    af = np.where(fin, a, 0.0)
    # Saturate: anything at or beyond the largest finite value maps to it, and
    # everything between it and the next (absent) grid point rounds down too.
    hi_idx = np.searchsorted(vals, af, side="left")
    hi_idx = np.clip(hi_idx, 1, len(vals) - 1)
    lo = vals[hi_idx - 1]
    hi = vals[hi_idx]
    mid = (lo + hi) / 2.0  # exact in f64: both have a few significant bits
    pick_hi = af > mid
    tie = af == mid
    lo_code = codes[hi_idx - 1]
    hi_code = codes[hi_idx]
    even_hi = (hi_code & 1) == 0
    pick_hi = np.where(tie, even_hi, pick_hi)
    c = np.where(pick_hi, hi_code, lo_code)
    c = np.where(af >= vals[-1], codes[-1], c)
    c = np.where(af <= vals[0], codes[0], c)
    out[:] = c | sign
    out[nan] = sign[nan] | 0x7F
    return out


def torch_cast(x, fmt):
    """torch's fp8 bytes for f32 x, with Gaudi's saturation substituted."""
    import torch

    dt = torch.float8_e4m3fn if fmt == E4M3 else torch.float8_e5m2
    reserved = 0x78 if fmt == E4M3 else 0x7C
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    raw = t.to(dt).view(torch.uint8).numpy().copy()
    over = (raw & reserved) == reserved
    return np.where(over, (raw & 0x80) | MAXCODE[fmt], raw).astype(np.uint8), raw


def hex_u16(s):
    return np.frombuffer(bytes.fromhex(s), dtype=">u2").astype(np.uint16)


def hex_u8(s):
    return np.frombuffer(bytes.fromhex(s), dtype=np.uint8).copy()


class Case:
    pass


def load_cases(path):
    """The fixture cases with shared weights resolved (fixtures.rs:70-107)."""
    doc = json.load(open(path))
    out = []
    for c in doc["cases"]:
        k = Case()
        k.name = c["name"]
        src = c.get("bf16_from", "")
        if src:
            k.w = next(o for o in out if o.name == src).w.copy()
        else:
            k.w = hex_u16(c["bf16_hex"])
        k.fmt = c["format"]
        k.scaling = c["scaling"]
        k.rows, k.cols = c["rows"], c["cols"]
        k.exp_bias = c["exp_bias"]
        k.scale_bits = np.array(c["scale_bits"], dtype=np.uint32)
        k.codes = hex_u8(c["codes_hex"])
        k.torch_raw = hex_u8(c["torch_raw_hex"]) if "torch_raw_hex" in c else None
        k.mean_rel = np.array(c["mean_rel"], dtype=np.float64)
        k.max_rel = np.array(c["max_rel"], dtype=np.float64)
        out.append(k)
    return doc, out


def bf16_bits(x):
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((b + (0x7FFF + ((b >> 16) & 1))) >> 16).astype(np.uint16)


def bf16_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def probe_weights(rows, cols):
    """fp8_probe.rs:35-43, the deterministic Llama-like weight rows (bf16 bits)."""
    i = np.arange(rows * cols, dtype=np.uint64)
    x = ((i * np.uint64(2654435761)) % np.uint64(65536)).astype(np.float32) / np.float32(65536.0)
    x = (x - np.float32(0.5)) * np.float32(0.08)
    outlier = np.where(i % np.uint64(977) == 0, np.float32(12.0), np.float32(1.0))
    return bf16_bits((x * outlier).astype(np.float32))


def probe_activations(n):
    """fp8_probe.rs:46-50."""
    i = np.arange(n, dtype=np.int64)
    return (((i * 7919) % 2003).astype(np.float32) - np.float32(1000.0)) / np.float32(700.0)


def special_matrix_f32(rng, rows=24, cols=512):
    """f32 weights (the [2048, 2048] workload's input type): N(0, 0.02) rows with
    0.1% of entries x50, then rows that exercise every special case of the f32
    entry: +-inf and NaN of both signs inside per-channel rows, a row whose
    absmax is 2^-149 (so s = m / 240 underflows to 0: x / 0 saturates and
    0 / 0 is x86's negative default NaN), rows whose s is subnormal (normal and
    subnormal entries), an all-NaN row (absmax 0, s = 1), rows of zeros and of
    negative zeros, f32 max and out-of-range finite values, and the tie
    240 * 2^-150 (m = 120 * 2^-149) where s rounds to 0 by ties-to-even next to
    m = 121 * 2^-149 where it rounds up to 2^-149."""
    assert rows >= 24 and cols >= 16
    x = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    out = rng.random((rows, cols)) < 0.001
    x[out] *= np.float32(50.0)
    tiny = np.float32(2.0 ** -149)
    x[1, 5] = np.inf
    x[2, 7] = -np.inf
    x[3, 11] = np.array(0x7FC00001, dtype=np.uint32).view(np.float32)      # +NaN with a payload
    x[4, 0] = np.array(0xFFC00000, dtype=np.uint32).view(np.float32)       # -NaN
    x[4, 3] = np.inf                                                       # and +inf in the same row
    x[5] = rng.choice(np.array([0.0, -0.0, tiny, -tiny], dtype=np.float32), cols)
    x[5, 0] = tiny                                                         # absmax 2^-149: s = 0
    x[6] = (rng.standard_normal(cols) * 1e-37).astype(np.float32)          # s ~ 4e-40, subnormal
    x[7] = (rng.standard_normal(cols) * 1e-40).astype(np.float32)          # subnormal entries, subnormal s
    x[8] = 0.0
    x[9] = -0.0
    x[10] = np.array(0x7FC00000, dtype=np.uint32).view(np.float32)         # all NaN: absmax 0, s = 1
    x[10, ::3] = np.array(0xFFC00000, dtype=np.uint32).view(np.float32)
    x[11, :4] = np.float32(3.4028235e38)                                   # f32 max
    x[11, 4:8] = np.float32(-3.4028235e38)
    x[12, ::5] = np.float32(3e38)
    x[13] = rng.integers(-120, 121, cols).astype(np.float32) * tiny
    x[13, 0] = 120 * tiny                                                  # m / 240 = 2^-150: ties to 0
    x[14] = rng.integers(-121, 122, cols).astype(np.float32) * tiny
    x[14, 0] = 121 * tiny                                                  # m / 240 rounds up to 2^-149
    x[15] = rng.integers(-1000, 1001, cols).astype(np.float32) * tiny      # s = 1000 * 2^-149 / 240
    x[15, 0] = 1000 * tiny
    x[16, 1] = -np.inf
    x[16, 2] = np.inf
    return x


def quantize_f32_closed_form(x, fmt, scaling, backoff):
    """What quantize_with gives f32 weights, from numpy's own f32 arithmetic
    and the independent table search: per-channel s = RN(m / RN(max * backoff))
    (m the NaN-ignoring row absmax, 1 for m = 0), hw s = 2^(bias - b) for the
    largest allowed b whose range covers RN(tensor absmax / backoff), unit
    s = 1; codes = nearest_encode(RN(x / s))."""
    rows, cols = x.shape
    maxf = np.float32(240.0 if fmt == E4M3 else 57344.0)
    a = np.abs(x)
    m = np.where(np.isnan(a), np.float32(0), a).max(axis=1).astype(np.float32)
    bias = BIAS[fmt]
    if scaling == "pcs":
        full = np.float32(maxf * np.float32(backoff))
        with np.errstate(all="ignore"):
            s = np.where(m > 0, m / full, np.float32(1.0)).astype(np.float32)
    elif scaling == "hw":
        with np.errstate(all="ignore"):
            tm = np.float32(m.max() / np.float32(backoff))
        allowed = [15, 11, 7, 3] if fmt == E4M3 else [15]
        bias = next((bb for bb in allowed if tm <= maxf * np.float32(2.0 ** (BIAS[fmt] - bb))), allowed[-1])
        s = np.full(rows, np.float32(2.0 ** (BIAS[fmt] - bias)), dtype=np.float32)
    else:
        s = np.ones(rows, dtype=np.float32)
    with np.errstate(all="ignore"):
        quot = (x / s[:, None]).astype(np.float32)
    return nearest_encode(quot, fmt), s, bias
