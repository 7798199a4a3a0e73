"""The HIP quantizer against the CPU oracle, bit for bit (codes, scales, exp_bias).

Runs through libreng_hip.so's C ABI (reng_hip.py is a ctypes view of it).
Covers: the hardware-conversion precondition of the fast path on every f32
pattern; encode over all 2^32 patterns and decode over all 256 codes; the
reference's golden fixture; its unit tests' cases; special values (NaN, +-inf,
zero rows, bf16 subnormals, out-of-range values) inside rows; every bf16
pattern against thousands of scales; f32 values within a few ulps of every
fp8 midpoint; generic shapes (cols not a multiple of 8, strided windows);
batches; full Llama-3.1-8B layer shapes; the stream yardstick bench.py measures with.
"""
import numpy as np
import pytest

import oracle as O
from helpers import BIAS, E4M3, E5M2, bf16_bits, bf16_f32, load_cases, positive_table

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def R():
    import reng_hip

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    reng_hip.lib()
    print("device:", reng_hip.device_info(), flush=True)
    return reng_hip


def dev(a):
    """numpy -> device tensor with the same bytes."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def host(t):
    return t.cpu().numpy()


def check_quantize(R, w, rows, cols, fmt, scaling, backoff=1.0, label=""):
    q = R.quantize_with(dev(w), rows, cols, fmt, scaling, backoff)
    ref = O.quantize_with(w, rows, cols, fmt, scaling, backoff)
    codes, scales = host(q.codes), host(q.scales)
    assert q.exp_bias == ref.exp_bias, label
    sb, rb = scales.view(np.uint32), ref.scales.view(np.uint32)
    bad_s = np.nonzero(sb != rb)[0]
    assert bad_s.size == 0, f"{label}: {bad_s.size} scales differ, row {bad_s[0]}: {sb[bad_s[0]]:#x} vs {rb[bad_s[0]]:#x}"
    bad = np.nonzero(codes != ref.codes)[0]
    assert bad.size == 0, (f"{label}: {bad.size} of {codes.size} codes differ; first at {bad[0]} "
                           f"(row {bad[0] // cols}): gpu {codes[bad[0]]:#04x} oracle {ref.codes[bad[0]]:#04x}, "
                           f"x bits {np.asarray(w).ravel()[bad[0]]!r}")
    return q, ref


# ------------------------------------------------------------ preconditions


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_hw_conversion_is_exact_wherever_the_fast_path_uses_it(R, fmt):
    n, first = R.verify_hw_convert(fmt)
    assert n == 0, f"{n} f32 patterns convert differently, first {first:#010x}"


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_encode_matches_the_oracle_on_every_f32_pattern(R, fmt):
    chunk = 1 << 28
    for c in range((1 << 32) // chunk):
        start = c * chunk
        u = torch.arange(start, start + chunk, dtype=torch.int64, device="cuda")
        u = torch.where(u >= (1 << 31), u - (1 << 32), u).to(torch.int32)
        got = host(R.encode(u.view(torch.float32), fmt))
        del u
        want = O.encode_bits_range(start, chunk, fmt, threads=16)
        if not np.array_equal(got, want):
            i = int(np.nonzero(got != want)[0][0])
            pytest.fail(f"pattern {start + i:#010x}: gpu {got[i]:#04x} oracle {want[i]:#04x}")


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_decode_matches_the_oracle_on_every_code(R, fmt):
    c = np.arange(256, dtype=np.uint8)
    got = host(R.decode(dev(c), fmt))
    want = O.decode_array(c, fmt)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ------------------------------------------------------------ golden fixture


def test_the_golden_fixture_bit_for_bit(R, golden_path):
    for c in load_cases(golden_path)[1]:
        q = R.quantize(dev(c.w), c.rows, c.cols, c.fmt, c.scaling)
        assert q.exp_bias == c.exp_bias, c.name
        assert np.array_equal(host(q.scales).view(np.uint32), c.scale_bits), c.name
        assert np.array_equal(host(q.codes), c.codes), c.name
        mean, mx = R.row_errors(dev(c.w), q)
        assert np.all(np.abs(host(mean).astype(np.float64) - c.mean_rel) <= 1e-6 + 1e-5 * c.mean_rel), c.name
        assert np.all(np.abs(host(mx).astype(np.float64) - c.max_rel) <= 1e-6 + 1e-5 * c.max_rel), c.name


def test_the_host_pointer_entry_matches_the_fixture(R, golden_path):
    for c in load_cases(golden_path)[1]:
        codes, scales, eb = R.quantize_host(c.w, c.rows, c.cols, c.fmt, c.scaling)
        assert eb == c.exp_bias and np.array_equal(scales.view(np.uint32), c.scale_bits)
        assert np.array_equal(codes, c.codes), c.name


# ------------------------------------------------------ the reference's cases


def test_reference_unit_cases(R):
    b = lambda xs: bf16_bits(np.float32(xs))
    check_quantize(R, b([0.5, -1.0, 0.25, 0.0, 100.0, -50.0, 12.5, 0.0]), 2, 4, E4M3, "pcs", label="pcs")
    w = bf16_bits((np.arange(64, dtype=np.float32) - 32.0) / 64.0)
    q, _ = check_quantize(R, w, 4, 16, E4M3, "hw", label="hw")
    assert q.exp_bias == 15
    check_quantize(R, b([1.0, 2.0, 0.5, 100.0]), 1, 4, E4M3, "unit", label="unit")
    q, _ = check_quantize(R, b([1.0, -0.5, 0.25, 0.125]), 1, 4, E4M3, "pcs", 0.5, label="backoff")
    assert host(q.codes)[0] == 0x6F
    q, _ = check_quantize(R, np.zeros(8, dtype=np.uint16), 2, 4, E4M3, "pcs", label="zero rows")
    assert list(host(q.scales)) == [1.0, 1.0]
    i = np.arange(4 * 32)
    w = bf16_bits((((i * 37) % 101).astype(np.float32) - 50.0) / np.float32(13.0))
    hw, _ = check_quantize(R, w, 4, 32, E5M2, "hw", label="e5m2 hw")
    unit, _ = check_quantize(R, w, 4, 32, E5M2, "unit", label="e5m2 unit")
    assert np.array_equal(host(hw.codes), host(unit.codes))
    for rows, cols in [(512, 4096), (67, 16 * 1024)]:
        i = np.arange(rows * cols, dtype=np.int64)
        w = bf16_bits((((i * 7919) % 2003).astype(np.float32) - np.float32(1000.0)) / np.float32(977.0))
        for sc in ("pcs", "hw", "unit"):
            check_quantize(R, w, rows, cols, E4M3, sc, label=f"{rows}x{cols} {sc}")


def test_argument_errors_are_refused(R):
    w = dev(np.zeros(16, dtype=np.uint16))
    with pytest.raises(ValueError, match="empty shape"):
        R.quantize_with(w, 0, 16, E4M3, "pcs")
    for bad in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="not positive and finite"):
            R.quantize_with(w, 1, 16, E4M3, "pcs", bad)
    with pytest.raises(ValueError, match="row pitch"):
        R.quantize_with(w, 1, 16, E4M3, "pcs", 1.0, ld=8)


# ------------------------------------------------------------ stress


def special_matrix(rng, rows, cols):
    """N(0, 0.02) bf16 with the injections the Llama-3.1-8B workload carries:
    all-zero rows, bf16 subnormals, out-of-range finite values, +-inf and NaN."""
    x = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w = bf16_bits(x)
    zr = rng.choice(rows, max(1, rows // 50), replace=False)
    w[zr] = 0
    sub = rng.integers(1, 0x80, (rows, cols)).astype(np.uint16) | (rng.integers(0, 2, (rows, cols)).astype(np.uint16) << 15)
    mask = rng.random((rows, cols)) < 0.01
    w[mask] = sub[mask]
    w[rows // 3] = sub[rows // 3]                           # a row whose absmax is subnormal
    big = bf16_bits(np.float32(rng.choice([1e4, -1e4, 3e38, -3e38], (rows, cols))))
    mask = rng.random((rows, cols)) < 0.001
    w[mask] = big[mask]
    w[1, 5] = 0x7F80                                        # +inf in a row
    w[2, 7] = 0xFF80                                        # -inf
    w[3, 11] = 0x7FC1                                       # NaN
    w[4, 0] = 0xFFC0                                        # negative NaN
    w[4, 3] = 0x7F80                                        # NaN and inf together
    w[5, :] = 0x8000                                        # a row of negative zeros
    return w


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
@pytest.mark.parametrize("scaling", ["pcs", "hw", "unit"])
def test_special_values_inside_rows(R, fmt, scaling):
    rng = np.random.default_rng(17 + fmt)
    for rows, cols in [(64, 4096), (33, 1536), (16, 14336), (9, 100)]:
        w = special_matrix(rng, rows, cols)
        for backoff in (1.0, 0.5, 2.0):
            check_quantize(R, w.ravel(), rows, cols, fmt, scaling, backoff, label=f"{rows}x{cols} b{backoff}")


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_every_bf16_value_against_many_scales(R, fmt):
    """Row r holds every non-NaN bf16 pattern of magnitude <= M_r (cyclically)
    plus M_r itself, so its per-channel scale is M_r / max_finite: 1024 scales
    drawn over the whole bf16 range, each against every representable input."""
    rng = np.random.default_rng(23)
    allp = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mag = allp & 0x7FFF
    allp = allp[mag <= 0x7F80]
    rows, cols = 1024, 65536
    tops = np.sort(rng.integers(0x0001, 0x7F7F, rows).astype(np.uint16))
    w = np.empty((rows, cols), dtype=np.uint16)
    for r, t in enumerate(tops):
        cand = allp[(allp & 0x7FFF) <= t]
        w[r] = np.resize(cand, cols)
        w[r, 0] = t
    check_quantize(R, w.ravel(), rows, cols, fmt, "pcs", label="all bf16 x 1024 scales")
    check_quantize(R, w.ravel(), rows, cols, fmt, "pcs", 0.37, label="all bf16 backoff 0.37")


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_f32_values_next_to_every_midpoint(R, fmt):
    """f32 input (the [2048, 2048] workload's type): elements within +-4 ulps of
    s * m for every fp8 midpoint m, for 256 scales: the cases where x * (1/s)
    and RN(x / s) can round to different codes."""
    rng = np.random.default_rng(29 + fmt)
    _, vals = positive_table(fmt)
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float64)
    rows = 256
    maxf = 240.0 if fmt == E4M3 else 57344.0
    m_row = (np.exp(rng.uniform(np.log(1e-6), np.log(1e4), rows))).astype(np.float32)
    s_row = (m_row / np.float32(maxf)).astype(np.float32)
    cols = 2048
    w = np.empty((rows, cols), dtype=np.float32)
    for r in range(rows):
        base = (mids * np.float64(s_row[r])).astype(np.float32).view(np.int32)
        cand = np.concatenate([base + d for d in range(-4, 5)]).view(np.float32)
        cand = np.concatenate([cand, -cand])
        cand = cand[np.abs(cand) <= m_row[r]]
        row = np.resize(rng.permutation(cand), cols)
        row[0] = m_row[r]
        w[r] = row
    check_quantize(R, w.ravel(), rows, cols, fmt, "pcs", label="midpoints f32")
    check_quantize(R, w.ravel(), rows, cols, fmt, "hw", label="midpoints f32 hw")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_random_shapes_and_paths(R, dtype):
    rng = np.random.default_rng(31)
    shapes = [(1, 8), (3, 4), (5, 12), (7, 100), (8, 64), (8, 576), (4, 1536), (2, 4104), (3, 4096),
              (2, 3584), (2, 18944), (2, 27648), (2, 5120), (1, 131072), (1, 65544)]
    for rows, cols in shapes:
        x = (rng.standard_normal((rows, cols)) * np.exp2(rng.integers(-30, 30, (rows, 1)))).astype(np.float32)
        w = bf16_bits(x).ravel() if dtype == "bf16" else x.ravel()
        for fmt in (E4M3, E5M2):
            for sc in ("pcs", "hw", "unit"):
                check_quantize(R, w, rows, cols, fmt, sc, label=f"{dtype} {rows}x{cols} {sc}")


def test_strided_windows(R):
    rng = np.random.default_rng(37)
    rows, cols, ld = 64, 4096, 4096 + 512
    full = bf16_bits((rng.standard_normal((rows, ld)) * 0.02).astype(np.float32))
    window = np.ascontiguousarray(full[:, 256:256 + cols])
    base = torch.from_numpy(full.view(np.int16).ravel()).cuda()
    view = base[256:]
    codes = torch.empty(rows * cols, dtype=torch.uint8, device="cuda")
    scales = torch.empty(rows, dtype=torch.float32, device="cuda")
    R.quantize_into(view, rows, cols, E4M3, "pcs", 1.0, codes, scales, ld=ld)
    ref = O.quantize_with(window.ravel(), rows, cols, E4M3, "pcs", 1.0)
    assert np.array_equal(host(codes), ref.codes)
    assert np.array_equal(host(scales), ref.scales)


def test_batches_match_per_matrix_quantization(R):
    rng = np.random.default_rng(41)
    shapes = [(256, 512), (64, 512), (64, 512), (256, 512), (448, 512), (448, 512), (256, 1792),
              (33, 100), (5, 4096)]
    mats, refs = [], []
    for i, (r, c) in enumerate(shapes):
        w = bf16_bits((rng.standard_normal((r, c)) * 0.02 * (1 + 10 * i)).astype(np.float32))
        if i == 3:
            w[7, 9] = 0x7FC0
        refs.append((w, r, c))
        mats.append((dev(w.ravel()), r, c, torch.empty(r * c, dtype=torch.uint8, device="cuda"),
                     torch.empty(r, dtype=torch.float32, device="cuda"),
                     torch.zeros(1, dtype=torch.int32, device="cuda")))
    for fmt in (E4M3, E5M2):
        for sc in ("pcs", "hw", "unit"):
            R.quantize_batch(mats, fmt, sc, 0.8)
            for (w, r, c), m in zip(refs, mats):
                ref = O.quantize_with(w.ravel(), r, c, fmt, sc, 0.8)
                assert np.array_equal(host(m[3]), ref.codes), (fmt, sc, r, c)
                assert np.array_equal(host(m[4]), ref.scales), (fmt, sc, r, c)
                assert int(m[5].item()) == ref.exp_bias, (fmt, sc, r, c)


LLAMA_8B = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
            ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_one_llama_8b_layer_at_full_size(R, fmt):
    rng = np.random.default_rng(43 + fmt)
    for name, rows, cols in LLAMA_8B:
        w = special_matrix(rng, rows, cols) if name == "down" else bf16_bits(
            (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))
        check_quantize(R, w.ravel(), rows, cols, fmt, "pcs", label=name)


def test_qwen_32b_mlp_matrices_at_full_size(R):
    """The C5 set's two row widths at full size: one [27648, 5120] gate/up and
    one [5120, 27648] down matrix (rows of 27648 take the 9-wave kernel), the
    down one with the bench's injections, bit for bit against the oracle."""
    rng = np.random.default_rng(2025)
    up = bf16_bits((rng.standard_normal((27648, 5120)) * 0.02).astype(np.float32))
    check_quantize(R, up.ravel(), 27648, 5120, E4M3, "pcs", label="gate/up")
    del up
    down = special_matrix(rng, 5120, 27648)
    check_quantize(R, down.ravel(), 5120, 27648, E4M3, "pcs", label="down")


# ------------------------------------------------------------ helpers of the API


def test_row_absmax_dequantize_and_error_sampling(R):
    rng = np.random.default_rng(47)
    rows, cols = 100, 576
    w = special_matrix(rng, rows, cols).ravel()
    got = host(R.row_absmax(dev(w), rows, cols))
    want = O.row_absmax(w, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    wf = bf16_bits((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)).ravel()
    for fmt in (E4M3, E5M2):
        q = R.quantize(dev(wf), rows, cols, fmt, "pcs")
        ref = O.quantize(wf, rows, cols, fmt, "pcs")
        assert np.array_equal(host(q.dequantize()).view(np.uint32), ref.dequantize().view(np.uint32))
        assert np.array_equal(host(q.dequantize_bf16()).view(np.uint16), O.bf16_bits(ref.dequantize()))
        for n in (0, 8, 7, 1000):
            mean, mx = R.row_errors(dev(wf), q) if n == 0 else R.sample_row_errors(dev(wf), q, n)
            wm, wx = O.row_errors(wf, ref) if n == 0 else O.sample_row_errors(wf, ref, n)
            assert len(mean) == len(wm)
            assert np.allclose(host(mean), wm, rtol=1e-6, atol=1e-9)
            assert np.array_equal(host(mx), wx)
    for a in (0.5, 0.9375, 1.0, 15.0, 16.0, 1000.0, 1e9):
        assert R.choose_exp_bias(a, E4M3) == O.choose_exp_bias(a, E4M3)
    assert R.choose_exp_bias(1e9, E5M2) == 15


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
@pytest.mark.parametrize("scaling", ["pcs", "hw", "unit"])
def test_f32_special_values_inside_rows(R, fmt, scaling):
    """f32 input with +-inf and NaN inside rows, s underflowing to 0, subnormal
    s, all-NaN and zero rows (helpers.special_matrix_f32), at the widths of the
    f32 exact-fit kernels (2048, 8192), a predicated width and the generic one."""
    from helpers import special_matrix_f32

    rng = np.random.default_rng(53 + fmt)
    for rows, cols in [(24, 2048), (40, 8192), (24, 4096), (24, 520), (30, 100)]:
        x = special_matrix_f32(rng, rows, cols)
        for backoff in (1.0, 0.5, 2.0):
            check_quantize(R, x.ravel(), rows, cols, fmt, scaling, backoff,
                           label=f"f32 {rows}x{cols} {scaling} b{backoff}")


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_the_f32_2048x2048_workload(R, fmt):
    """The reference's CPU-runnable case at its full size: one f32 [2048, 2048]
    matrix, N(0, 0.02) with 0.1% of entries (4194, drawn without replacement)
    x50, per-channel scales, backoff 1; and the same matrix under hw and unit."""
    rng = np.random.default_rng(2048)
    rows = cols = 2048
    x = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32).ravel()
    idx = rng.choice(rows * cols, 4194, replace=False)
    x[idx] *= np.float32(50.0)
    for sc in ("pcs", "hw", "unit"):
        check_quantize(R, x, rows, cols, fmt, sc, label=f"f32 2048x2048 {sc}")


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_rows_whose_scale_is_subnormal(R, fmt):
    """bf16 rows whose absmax is a bf16 subnormal (2^-133 .. 2^-127): s = m / max
    is an f32 subnormal with few significant bits (E5M2, m = 2^-133: s rounds
    to 2^-149 and x / s reaches 2^16, past 57344), so the quotient passes the
    range the clamp-free conversion covers; such rows must still saturate as
    the reference does. Both fast-path widths and a generic one."""
    rng = np.random.default_rng(61 + fmt)
    for rows, cols in [(64, 4096), (32, 14336), (16, 100)]:
        w = np.zeros((rows, cols), dtype=np.uint16)
        for r in range(rows):
            top = 1 + (r % 64)   # absmax bit pattern 0x0001 .. 0x0040
            vals = rng.integers(0, top + 1, cols).astype(np.uint16)
            vals |= (rng.integers(0, 2, cols).astype(np.uint16) << 15)
            vals[0] = top
            w[r] = vals
        for backoff in (1.0, 0.5):
            check_quantize(R, w.ravel(), rows, cols, fmt, "pcs", backoff, label=f"tiny bf16 {rows}x{cols} b{backoff}")


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_the_staged_host_entry_over_many_chunks(R, dtype):
    """reng_hip_quantize_host moves a matrix in 4 MB row chunks through three
    pinned slots and streams, with thread pools copying in and out: matrices of
    one chunk, of more chunks than slots with a ragged last one, of one row per
    chunk, and (f32) of rows larger than a slot (the unpipelined path); every
    scheme, bit for bit against the oracle, twice in a row (the staging buffers
    and threads are kept and reused)."""
    rng = np.random.default_rng(71)
    for rows, cols in [(64, 4096), (4100, 4096), (2304, 14336), (3, 1048592)]:
        x = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        w = bf16_bits(x).ravel() if dtype == "bf16" else x.ravel()
        for fmt, sc in ((E4M3, "pcs"), (E5M2, "hw"), (E4M3, "unit"), (E4M3, "hw")):
            for _ in range(2):
                codes, scales, eb = R.quantize_host(w, rows, cols, fmt, sc, 0.8)
                ref = O.quantize_with(w, rows, cols, fmt, sc, 0.8)
                assert eb == ref.exp_bias, (rows, cols, fmt, sc)
                assert np.array_equal(scales.view(np.uint32), ref.scales.view(np.uint32)), (rows, cols, fmt, sc)
                bad = np.nonzero(codes != ref.codes)[0]
                assert bad.size == 0, (rows, cols, fmt, sc, bad[:4])


def test_the_stream_yardstick_writes_the_high_bytes(R):
    """reng_hip_stream_narrow (the quantizer's 2:1 memory stream with no
    arithmetic, a measuring stick for bench.py): the high byte of every bf16
    value, on a length that exercises the unrolled loop and its remainder."""
    rng = np.random.default_rng(12)
    for n in (8, 8 * 1000003):
        w = rng.integers(0, 1 << 16, n, dtype=np.uint16)
        out = torch.empty(n, dtype=torch.uint8, device="cuda")
        R.stream_narrow(dev(w), n, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), (w >> 8).astype(np.uint8)), n
