"""The CPU oracle against the reference's own tests and against independent checks.

Which check pins which oracle function (oracle/fp8_oracle.c):

* encode      - fixture codes (12 cases, bytewise), the reference's KATs, the
                torch cast with saturation substitution, `nearest_encode` (an
                independent table search), the round trip over every code.
* decode      - `closed_form_decode` over all 256 codes of both formats.
* bf16 <-> f32 - numpy RNE formula over every bf16 pattern and random f32.
* row absmax, quantize_with, split/threads - fixture scale bits and codes,
                the reference KATs (per-channel, hw, unit, backoff, zero rows,
                parallel == serial, ragged last chunk), and the closed forms
                s = RN(m / RN(max * backoff)), s = 2^(bias - b), s = 1.
* choose_exp_bias - the reference KAT thresholds and a brute-force rule.
* row_errors / sample_row_errors - fixture statistics (1e-6 + 1e-5 * want) and
                a numpy restatement.
* dequantize  - closed-form decode times the scale.
* gemm / rel_l2 - numpy float64 products and formulas.
* the x86 division semantics (inf inside a per-channel row, NaN inputs) -
                numpy's own float32 division on the same host.
"""
import numpy as np
import pytest

import oracle as O
from helpers import (BIAS, E4M3, E5M2, FMT, MAXCODE, bf16_bits, bf16_f32, closed_form_decode,
                     load_cases, nearest_encode, torch_cast)


def b(x):
    return O.f32_to_bf16(x)


# ---------------------------------------------------------------- fixtures.rs


def test_the_fixture_is_the_one_the_generator_writes(golden_path):
    doc, cases = load_cases(golden_path)
    assert doc["generator"] == "tools/fp8_fixtures.py"
    assert len(cases) >= 12
    assert sum(c.name.startswith("ckpt_") for c in cases) >= 6


def _q(c):
    return O.quantize(c.w, c.rows, c.cols, c.fmt, c.scaling)


def test_scales_match_torchs_input_bit_for_bit(golden_path):
    for c in load_cases(golden_path)[1]:
        q = _q(c)
        assert q.rows == c.rows
        assert q.exp_bias == c.exp_bias, c.name
        assert np.array_equal(q.scales.view(np.uint32), c.scale_bits), c.name


def test_codes_match_the_torch_cast(golden_path):
    for c in load_cases(golden_path)[1]:
        q = _q(c)
        bad = np.nonzero(q.codes != c.codes)[0]
        assert bad.size == 0, f"{c.name}: {bad.size} codes differ, first {bad[:4]}"


def test_the_only_divergence_from_torch_is_the_saturation(golden_path):
    checked = 0
    for c in load_cases(golden_path)[1]:
        if c.torch_raw is None:
            continue
        checked += 1
        q = _q(c)
        reserved = 0x78 if c.fmt == "e4m3" else 0x7C
        over = (c.torch_raw & reserved) == reserved
        assert over.sum() > 0
        assert np.array_equal(q.codes[over], (c.torch_raw[over] & 0x80) | MAXCODE[FMT[c.fmt]])
        assert np.array_equal(q.codes[~over], c.torch_raw[~over])
    assert checked >= 2


def test_row_error_statistics_match_numpy(golden_path):
    for c in load_cases(golden_path)[1]:
        q = _q(c)
        mean, mx = O.row_errors(c.w, q)
        assert np.all(np.abs(mean.astype(np.float64) - c.mean_rel) <= 1e-6 + 1e-5 * c.mean_rel), c.name
        assert np.all(np.abs(mx.astype(np.float64) - c.max_rel) <= 1e-6 + 1e-5 * c.max_rel), c.name


def test_checkpoint_rows_quantize_within_the_formats_resolution(golden_path):
    seen = 0
    for c in load_cases(golden_path)[1]:
        if not c.name.startswith("ckpt_") or c.scaling != "pcs":
            continue
        seen += 1
        q = _q(c)
        mean, mx = O.row_errors(c.w, q)
        assert np.all(mean < 0.03) and np.all(mx <= 0.25)
        back = q.dequantize().reshape(c.rows, c.cols)
        w = bf16_f32(c.w).reshape(c.rows, c.cols)
        for r in range(c.rows):
            ai = int(np.argmax(np.abs(w[r])))
            assert abs(back[r, ai] - w[r, ai]) <= abs(w[r, ai]) * 1e-6
    assert seen >= 3


# ------------------------------------------------------------- lib.rs tests


def test_e4m3_codes_match_the_device_cast():
    cases = [(0.0, 0x00), (1.0, 0x38), (1.375, 0x3B), (-3.3, 0xC5), (100.0, 0x6C), (0.01, 0x05),
             (0.0625, 0x18), (17.0, 0x58), (240.0, 0x77), (-240.0, 0xF7), (250.0, 0x77),
             (300.0, 0x77), (0.001, 0x01), (1e-9, 0x00), (np.inf, 0x77), (-np.inf, 0xF7)]
    for x, code in cases:
        assert O.encode(np.float32(x), "e4m3") == code, x
    assert O.encode(np.float32("nan"), "e4m3") & 0x7F == 0x7F


def test_e5m2_codes_match_the_device_cast():
    for x, code in [(1.375, 0x3E), (250.0, 0x5C), (300.0, 0x5D), (-240.0, 0xDC), (1.0, 0x3C)]:
        assert O.encode(np.float32(x), "e5m2") == code, x
    assert O.decode(0x3E, "e5m2") == 1.5
    assert O.decode(0x5C, "e5m2") == 256.0
    assert O.decode(0x5D, "e5m2") == 320.0
    assert O.decode(0xDC, "e5m2") == -256.0


def test_format_constants():
    assert O.max_finite("e4m3") == 240.0
    assert O.lib().orc_max_finite_code(E4M3) == 0x77
    assert O.max_finite("e5m2") == 57344.0
    assert O.lib().orc_max_finite_code(E5M2) == 0x7B
    assert np.isinf(O.decode(0x78, "e4m3"))
    assert np.isnan(O.decode(0x7F, "e4m3"))


def test_every_code_round_trips_through_the_encoder():
    for fmt in (E4M3, E5M2):
        for code in range(256):
            v = O.decode(code, fmt)
            if not np.isfinite(v):
                continue
            assert O.encode(np.float32(v), fmt) == code, (fmt, hex(code))


def test_rounding_is_to_nearest_even():
    assert O.encode(np.float32(1.0625), "e4m3") == 0x38
    assert O.encode(np.float32(1.1875), "e4m3") == 0x3A
    assert O.encode(np.float32(1.0626), "e4m3") == 0x39


def test_per_channel_scales_stretch_each_row_to_full_scale():
    w = np.array([b(x) for x in [0.5, -1.0, 0.25, 0.0, 100.0, -50.0, 12.5, 0.0]], dtype=np.uint16)
    q = O.quantize(w, 2, 4, "e4m3", "pcs")
    assert q.scales[0] == np.float32(1.0) / np.float32(240.0)
    assert q.scales[1] == np.float32(100.0) / np.float32(240.0)
    assert q.exp_bias == 7
    assert q.codes[1] & 0x7F == 0x77 and q.codes[4] & 0x7F == 0x77
    d = q.dequantize()
    assert abs(d[0] - 0.5) < 0.5 * 0.07 and abs(d[4] - 100.0) < 100.0 * 0.07


def test_hw_exp_bias_picks_the_finest_range_that_fits():
    for a, want in [(0.5, 15), (0.9375, 15), (1.0, 11), (15.0, 11), (16.0, 7), (1000.0, 3), (1e9, 3)]:
        assert O.choose_exp_bias(a, "e4m3") == want, a
    assert O.choose_exp_bias(1e9, "e5m2") == 15
    w = bf16_bits((np.arange(64, dtype=np.float32) - 32.0) / 64.0)
    q = O.quantize(w, 4, 16, "e4m3", "hw")
    assert q.exp_bias == 15
    assert np.all(q.scales == np.float32(1.0 / 256.0))


def test_unit_scaling_leaves_the_codes_alone():
    w = np.array([b(x) for x in [1.0, 2.0, 0.5, 100.0]], dtype=np.uint16)
    q = O.quantize(w, 1, 4, "e4m3", "unit")
    assert list(q.scales) == [1.0]
    assert q.codes[0] == O.encode(1.0, "e4m3") and q.codes[3] == O.encode(100.0, "e4m3")


def _hashed(rows, cols):
    i = np.arange(rows * cols, dtype=np.uint64)
    x = ((i * np.uint64(2654435761)) % np.uint64(65536)).astype(np.float32) / np.float32(65536.0) - np.float32(0.5)
    return bf16_bits(x * (np.float32(1.0) + (i // np.uint64(cols)).astype(np.float32)))


def test_dequantize_of_quantize_is_within_the_format_resolution():
    rows, cols = 32, 128
    w = _hashed(rows, cols)
    q = O.quantize(w, rows, cols, "e4m3", "pcs")
    mean, mx = O.row_errors(w, q)
    assert np.all(mx <= 0.0626) and np.all(mean < 0.03)


def _mod_weights(rows, cols):
    i = np.arange(rows * cols, dtype=np.int64)
    return bf16_bits((((i * 7919) % 2003).astype(np.float32) - np.float32(1000.0)) / np.float32(977.0))


def test_the_parallel_path_agrees_with_the_serial_one():
    rows, cols = 512, 4096
    w = _mod_weights(rows, cols)
    assert O.split(rows, cols) > 1
    par = O.quantize_with(w, rows, cols, "e4m3", "pcs", 1.0, thread_cap=8)
    ser = O.quantize_with(w, rows, cols, "e4m3", "pcs", 1.0, thread_cap=1)
    absmax = O.row_absmax(w, rows, cols)
    assert np.array_equal(par.scales, absmax / np.float32(240.0))
    assert np.array_equal(par.codes, ser.codes)


def test_the_parallel_path_carries_a_ragged_last_chunk():
    rows, cols = 67, 16 * 1024
    w = _mod_weights(rows, cols)
    t = O.split(rows, cols)
    assert t > 1 and rows % t != 0
    for sc in ("pcs", "hw", "unit"):
        par = O.quantize_with(w, rows, cols, "e4m3", sc, 1.0, thread_cap=8)
        ser = O.quantize_with(w, rows, cols, "e4m3", sc, 1.0, thread_cap=1)
        assert np.array_equal(par.codes, ser.codes), sc
        assert np.any(par.codes[(rows - 1) * cols:] != 0), sc


def test_the_hardware_bias_scheme_is_the_identity_for_e5m2():
    i = np.arange(4 * 32, dtype=np.int64)
    w = bf16_bits((((i * 37) % 101).astype(np.float32) - 50.0) / np.float32(13.0))
    hw = O.quantize(w, 4, 32, "e5m2", "hw")
    unit = O.quantize(w, 4, 32, "e5m2", "unit")
    assert hw.exp_bias == 15 and np.all(hw.scales == 1.0)
    assert np.array_equal(hw.codes, unit.codes)


def test_sampling_agrees_with_the_full_error_pass():
    i = np.arange(16 * 64, dtype=np.int64)
    w = bf16_bits((((i * 37) % 101).astype(np.float32) - 50.0) / np.float32(50.0))
    q = O.quantize(w, 16, 64, "e4m3", "pcs")
    mean, mx = O.row_errors(w, q)
    sm, sx = O.sample_row_errors(w, q, 16)
    assert np.array_equal(sm, mean) and np.array_equal(sx, mx)
    sm, sx = O.sample_row_errors(w, q, 4)
    assert len(sm) == 4 and np.array_equal(sm, mean[::4]) and np.array_equal(sx, mx[::4])
    assert len(O.sample_row_errors(w, q, 1000)[0]) == 16


def test_zero_rows_keep_a_unit_scale():
    w = np.zeros(8, dtype=np.uint16)
    q = O.quantize(w, 2, 4, "e4m3", "pcs")
    assert list(q.scales) == [1.0, 1.0] and not q.codes.any()
    mean, mx = O.row_errors(w, q)
    assert mean[0] == 0.0 and mx[0] == 0.0


def test_a_backoff_leaves_headroom():
    w = np.array([b(x) for x in [1.0, -0.5, 0.25, 0.125]], dtype=np.uint16)
    q = O.quantize_with(w, 1, 4, "e4m3", "pcs", 0.5)
    assert q.scales[0] == np.float32(1.0) / np.float32(120.0)
    assert q.codes[0] == 0x6F and O.decode(q.codes[0], "e4m3") == 120.0


# ------------------------------------------------------ independent checks


def test_decode_is_the_closed_form_for_every_code():
    for fmt in (E4M3, E5M2):
        got = O.decode_array(np.arange(256, dtype=np.uint8), fmt)
        for c in range(256):
            want = closed_form_decode(c, fmt)
            if want == "nan":
                assert np.isnan(got[c])
            elif want == "inf":
                assert np.isinf(got[c]) and (got[c] < 0) == bool(c & 0x80)
            else:
                assert got[c] == float(want) and np.signbit(got[c]) == bool(c & 0x80), hex(c)


def test_bf16_conversions_follow_rne():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bf16_f32(bits)
    assert all(O.bf16_to_f32(int(x)) == f[x] or np.isnan(f[x]) for x in range(0, 65536, 257))
    rng = np.random.default_rng(1)
    xs = rng.standard_normal(2000).astype(np.float32) * np.float32(1e3)
    want = bf16_bits(xs)
    assert all(O.f32_to_bf16(float(x)) == w for x, w in zip(xs, want))
    assert O.f32_to_bf16(float("nan")) == 0x7FC0


def _sample_patterns(seed=7, n_random=1 << 20):
    """Every bf16 pattern, every f32 pattern on a coarse stride, random ones,
    and values within a few ulps of every midpoint of both formats."""
    rng = np.random.default_rng(seed)
    parts = [
        (np.arange(65536, dtype=np.uint32) << 16),
        np.arange(0, 1 << 32, 4093, dtype=np.uint64).astype(np.uint32),
        rng.integers(0, 1 << 32, n_random, dtype=np.uint64).astype(np.uint32),
    ]
    for fmt in (E4M3, E5M2):
        from helpers import positive_table
        _, vals = positive_table(fmt)
        mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32).view(np.uint32)
        for d in range(-4, 5):
            parts.append((mids.astype(np.int64) + d).astype(np.uint32))
            parts.append(((mids.astype(np.int64) + d) | 0x80000000).astype(np.uint32))
    return np.concatenate(parts).view(np.float32)


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_encode_is_round_to_nearest_even_onto_the_grid(fmt):
    x = _sample_patterns()
    x = x[~np.isnan(x)]
    got = O.encode_array(x, fmt)
    want = nearest_encode(x, fmt)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(x.view(np.uint32)[i]), got[i], want[i]) for i in bad[:5]]


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_encode_matches_torchs_cast_with_saturation(fmt):
    x = _sample_patterns(seed=11, n_random=1 << 19)
    x = x[~np.isnan(x)]
    want, _ = torch_cast(x, fmt)
    got = O.encode_array(x, fmt)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(x.view(np.uint32)[i]), got[i], want[i]) for i in bad[:5]]


def test_nan_keeps_its_sign():
    for fmt in (E4M3, E5M2):
        assert O.encode(np.float32("nan"), fmt) == 0x7F
        assert O.encode(-np.float32("nan"), fmt) == 0xFF


def test_a_planted_rounding_mistake_is_caught(golden_path):
    """Round-half-away-from-zero (a plausible encoder slip) must disagree with the
    fixture and with the oracle: the checks above can tell the two apart."""
    x = np.float32([1.0625, 17.0, 0.0009765625])
    away = []
    for v in x:
        from helpers import positive_table
        codes, vals = positive_table(E4M3)
        i = np.searchsorted(vals, abs(v))
        away.append(codes[i] if abs(v) - vals[i - 1] >= vals[i] - abs(v) else codes[i - 1])
    assert list(O.encode_array(x, E4M3)) != away


def test_scales_follow_their_closed_forms():
    rng = np.random.default_rng(3)
    rows, cols = 64, 96
    w = bf16_bits(rng.standard_normal((rows, cols)).astype(np.float32) * np.float32(0.02)
                  * np.exp2(rng.integers(-20, 20, (rows, 1))).astype(np.float32))
    wf = bf16_f32(w).reshape(rows, cols)
    m = np.abs(wf).max(axis=1)
    for fmt in (E4M3, E5M2):
        maxf = np.float32(240.0 if fmt == E4M3 else 57344.0)
        for backoff in (1.0, 0.5, 0.8, 0.3):
            q = O.quantize_with(w, rows, cols, fmt, "pcs", backoff)
            full = np.float32(maxf * np.float32(backoff))
            assert np.array_equal(q.scales, (m / full).astype(np.float32))
            assert q.exp_bias == BIAS[fmt]
        q = O.quantize_with(w, rows, cols, fmt, "hw", 0.7)
        tm = np.float32(m.max() / np.float32(0.7))
        allowed = [15, 11, 7, 3] if fmt == E4M3 else [15]
        bias = next((bb for bb in allowed if tm <= maxf * np.float32(2.0 ** (BIAS[fmt] - bb))), allowed[-1])
        assert q.exp_bias == bias
        assert np.all(q.scales == np.float32(2.0 ** (BIAS[fmt] - bias)))
        q = O.quantize_with(w, rows, cols, fmt, "unit", 0.7)
        assert np.all(q.scales == 1.0)


def test_quantize_codes_are_the_encoding_of_the_ieee_quotient():
    """codes = nearest_encode(f32(w) / s) with numpy's own f32 division, including
    the special values: a +inf inside a per-channel row makes s = inf, finite
    entries become signed zero and inf/inf is x86's negative default NaN."""
    rng = np.random.default_rng(5)
    rows, cols = 16, 256
    x = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x[2, 7] = np.inf
    x[3, 9] = -np.inf
    x[4, 1] = np.nan
    x[5, :] = 0.0
    x[6, 3] = np.float32(3e38)
    x[7, :] = bf16_f32(np.arange(1, cols + 1, dtype=np.uint16))  # bf16 subnormals only
    w = bf16_bits(x)
    w[4, 1] = 0xFFC1  # a negative NaN with a payload
    for fmt in (E4M3, E5M2):
        q = O.quantize(w.ravel(), rows, cols, fmt, "pcs")
        with np.errstate(all="ignore"):
            quot = (bf16_f32(w) / q.scales[:, None]).astype(np.float32)
        want = nearest_encode(quot, fmt)
        assert np.array_equal(q.codes, want)
        assert q.codes[2 * cols + 7] == 0xFF and q.codes[3 * cols + 9] == 0xFF
        assert q.codes[4 * cols + 1] == 0xFF
        assert np.isinf(q.scales[2])


def test_gemm_and_rel_l2_follow_numpy():
    rng = np.random.default_rng(9)
    m, k, n = 3, 200, 17
    a = rng.standard_normal(m * k).astype(np.float32)
    bm = rng.standard_normal(n * k).astype(np.float32)
    c = O.gemm(a, bm, m, k, n)
    ref = a.reshape(m, k).astype(np.float64) @ bm.reshape(n, k).astype(np.float64).T
    assert np.allclose(c.reshape(m, n), ref, rtol=1e-4, atol=1e-4)
    cc = O.gemm_cols(a, bm, m, k, [3, 0, 16])
    assert np.array_equal(cc.reshape(m, 3), c.reshape(m, n)[:, [3, 0, 16]])
    g = c + np.float32(0.01)
    want = np.sqrt(np.sum((g - c).astype(np.float64) ** 2)) / np.sqrt(np.sum(c.astype(np.float64) ** 2))
    assert abs(O.rel_l2(g, c) - want) <= 1e-6 * want


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_f32_quantize_follows_numpy_division_and_the_table_search(fmt):
    """orc_quantize_f32_with, the checker of the f32 [2048, 2048] workload,
    against numpy's f32 arithmetic and the nearest-value search, on every
    special case of f32 input (helpers.special_matrix_f32), for the three
    schemes and backoffs below, above and at 1."""
    from helpers import quantize_f32_closed_form, special_matrix_f32

    rng = np.random.default_rng(41 + fmt)
    x = special_matrix_f32(rng, 24, 512)
    for scaling in ("pcs", "hw", "unit"):
        for backoff in (1.0, 0.5, 2.0, 0.8):
            q = O.quantize_with(x.ravel(), 24, 512, fmt, scaling, backoff)
            codes, s, bias = quantize_f32_closed_form(x, fmt, scaling, backoff)
            assert np.array_equal(q.scales.view(np.uint32), s.view(np.uint32)), (scaling, backoff)
            assert q.exp_bias == bias, (scaling, backoff)
            bad = np.nonzero(q.codes != codes)[0]
            assert bad.size == 0, (scaling, backoff, bad[:5], q.codes[bad[:5]], codes[bad[:5]])
    # The special cases land where the reference's arithmetic puts them.
    q = O.quantize_with(x.ravel(), 24, 512, fmt, "pcs", 1.0)
    c = q.codes.reshape(24, 512)
    mx = MAXCODE[fmt]
    assert q.scales[5] == 0.0 and q.scales[13] == 0.0          # 2^-149 / max and the 2^-150 tie underflow
    if fmt == E4M3:
        assert q.scales[14] == np.float32(2.0 ** -149)         # 121 * 2^-149 / 240 rounds up
    assert 0 < q.scales[6] < np.finfo(np.float32).tiny and 0 < q.scales[7] < np.finfo(np.float32).tiny
    row5 = x[5]
    assert np.all(c[5][row5 == 0] == 0xFF)                     # 0 / 0: negative default NaN
    assert np.all(c[5][row5 > 0] == mx) and np.all(c[5][row5 < 0] == (0x80 | mx))
    assert np.isinf(q.scales[1]) and c[1, 5] == 0xFF           # inf / inf
    assert np.all(c[1][np.isfinite(x[1]) & ~np.signbit(x[1])] == 0x00)
    assert c[3, 11] == 0x7F and c[4, 0] == 0xFF                # NaN keeps its sign
    assert q.scales[10] == 1.0 and np.all((c[10] & 0x7F) == 0x7F)
    assert q.scales[8] == 1.0 and np.all(c[8] == 0) and np.all(c[9] == 0x80)
    assert c[11, 0] == mx and c[11, 4] == 0x80 | mx


def test_f32_quantize_a_planted_mistake_is_caught():
    """The closed form rejects an oracle that multiplies by the reciprocal of s
    instead of dividing (the slip an f32 fast path invites): on rows whose
    quotients sit next to fp8 midpoints the two round apart."""
    from helpers import quantize_f32_closed_form, positive_table

    rng = np.random.default_rng(43)
    _, vals = positive_table(E4M3)
    mids = (vals[1:] + vals[:-1]) / 2
    rows, cols = 64, 1024
    m = np.exp(rng.uniform(np.log(1e-3), np.log(1e2), rows)).astype(np.float32)
    s = (m / np.float32(240.0)).astype(np.float32)
    x = np.empty((rows, cols), dtype=np.float32)
    for r in range(rows):
        base = (mids * np.float64(s[r])).astype(np.float32).view(np.int32)
        cand = np.concatenate([base + d for d in (-1, 0, 1)]).view(np.float32)
        cand = cand[np.abs(cand) <= m[r]]
        x[r] = np.resize(rng.permutation(cand), cols)
        x[r, 0] = m[r]
    codes, s2, _ = quantize_f32_closed_form(x, E4M3, "pcs", 1.0)
    assert np.array_equal(O.quantize_with(x.ravel(), rows, cols, E4M3, "pcs").codes, codes)
    recip = nearest_encode((x * (np.float32(1.0) / s2)[:, None]).astype(np.float32), E4M3)
    assert not np.array_equal(recip, codes)


def test_rows_whose_scale_is_subnormal_saturate():
    """The closed form on bf16 rows of absmax 2^-133 .. 2^-127: E5M2's s rounds
    to a subnormal with few bits, the quotient passes 57344 and saturates."""
    rng = np.random.default_rng(67)
    rows, cols = 64, 256
    w = np.zeros((rows, cols), dtype=np.uint16)
    for r in range(rows):
        top = 1 + r
        w[r] = rng.integers(0, top + 1, cols).astype(np.uint16) | (rng.integers(0, 2, cols).astype(np.uint16) << 15)
        w[r, 0] = top
    x = bf16_f32(w)
    for fmt in (E4M3, E5M2):
        from helpers import quantize_f32_closed_form

        codes, s, _ = quantize_f32_closed_form(x.reshape(rows, cols), fmt, "pcs", 1.0)
        q = O.quantize(w.ravel(), rows, cols, fmt, "pcs")
        assert np.array_equal(q.scales.view(np.uint32), s.view(np.uint32))
        assert np.array_equal(q.codes, codes)
    q = O.quantize(w.ravel(), rows, cols, E5M2, "pcs")
    assert q.scales[0] == np.float32(2.0 ** -149) and q.codes[0] == 0x7B   # x / s = 2^16 saturates
