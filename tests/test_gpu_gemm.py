"""The fused fp8-dequant GEMV / skinny GEMM and the fp8 x fp8 GEMM against the
oracle's f32 gemm_cpu over Quantized::dequantize (fp8_probe.rs:55-78).

Tolerance: relative L2 < 1e-2 over the bf16 outputs (twice as tight as the
reference probe's own acceptance of 0.02, fp8_probe.rs:327,344). For the
fp8 x fp8 path the reference product uses the dequantized fp8 activation, as
the reference probe does (fp8_probe.rs:242-248, 295-298). Exactness of the
in-register decode is checked on its own: a one-hot activation reads every
finite code back bit for bit.
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import E4M3, E5M2, bf16_bits, bf16_f32, probe_activations, probe_weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 1e-2


def assert_elementwise(got, a, b, K, what, acc=None):
    """Every output against float64 numpy (an independent product): with
    want = a b^T and s = |a| |b|^T in float64,
        |got - want| <= 2^-8 |want| + acc s,
    the bf16 rounding of the output plus the accumulation error, by default
    acc = 1.01 (K / 64 + 16) 2^-23: IEEE f32 additions, at most K / 32 + 32 in
    sequence (the VALU dot products and the bf16 MFMA). The fp8 MFMA adds each
    instruction's 64 products at a lower internal precision: its callers pass
    fp8_acc(K). A wrong scale on one output row, a dropped or repeated chunk,
    or a swapped tile edge breaks the bound on the outputs it touches, where an
    aggregate rel-L2 would not."""
    a = np.asarray(a, dtype=np.float64).reshape(-1, K)
    b = np.asarray(b, dtype=np.float64).reshape(-1, K)
    want = a @ b.T
    s = np.abs(a) @ np.abs(b).T
    got = np.asarray(got, dtype=np.float64).reshape(want.shape)
    if acc is None:
        acc = 1.01 * (K / 64 + 16) * 2.0 ** -23
    bound = 2.0 ** -8 * np.abs(want) + acc * s
    bad = np.abs(got - want) > bound
    if bad.any():
        i, j = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outputs outside the bound; first [{i}, {j}]: "
                             f"got {got[i, j]!r} want {want[i, j]!r} bound {bound[i, j]!r}")


def fp8_acc(K):
    """The accumulation term of the fp8 MFMA GEMM's per-element bound:
    2^-12 + 1.01 (K / 64 + 16) 2^-23. Each v_mfma_*_f8f6f4 sums its 64 exact
    fp8 products internally with an error of at most c s_i (s_i = that
    instruction's sum of |a b|), and the K / 64 instruction results go through
    f32 additions (the second term, as for the other kernels); since the s_i add
    up to s, the internal errors add up to at most c s. c is measured, not
    documented: over codes drawn uniformly from every finite code (the widest
    spread of magnitudes inside one instruction), K = 128 ... 27648, both
    formats, the largest excess seen is 2^-13.2 s at K = 128
    (test_fp8_mfma_accumulation_over_k); c = 2^-12 leaves a factor of 2."""
    return 2.0 ** -12 + 1.01 * (K / 64 + 16) * 2.0 ** -23


@pytest.fixture(scope="module")
def R():
    import reng_hip

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    reng_hip.lib()
    return reng_hip


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def bf16_out(t):
    return bf16_f32(t.view(torch.int16).cpu().numpy().view(np.uint16))


def quantized_weight(rng, n, k, fmt, sigma=0.02):
    w = bf16_bits((rng.standard_normal((n, k)) * sigma).astype(np.float32)).ravel()
    return O.quantize(w, n, k, fmt, "pcs")


def check_w8a16(R, rng, M, N, K, fmt, sample_cols=None):
    q = quantized_weight(rng, N, K, fmt)
    x = bf16_bits(rng.standard_normal((M, K)).astype(np.float32)).ravel()
    y = bf16_out(R.gemm_w8a16(dev(x), dev(q.codes), dev(q.scales), M, N, K, fmt)).reshape(M, N)
    deq = q.dequantize()
    if sample_cols is None:
        want = O.gemm(bf16_f32(x), deq, M, K, N, threads=16).reshape(M, N)
        got = y
    else:
        idx = np.unique(np.concatenate([rng.choice(N, sample_cols, replace=False), [0, N - 1]]))
        want = O.gemm_cols(bf16_f32(x), deq, M, K, idx, threads=16).reshape(M, idx.size)
        got = y[:, idx]
    rel = O.rel_l2(got.ravel(), want.ravel())
    assert rel < TOL, f"M={M} N={N} K={K} fmt={fmt}: rel_L2 {rel}"
    assert np.all(np.isfinite(y))
    rows = slice(None) if sample_cols is None else idx
    assert_elementwise(got, bf16_f32(x), deq.reshape(N, K)[rows], K, f"M={M} N={N} K={K} fmt={fmt}")
    return rel


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_in_register_decode_reads_every_finite_code_exactly(R, fmt):
    """Row n of the weight is code n (all finite codes), the activation is one-hot
    at k, so y[m, n] = decode(code) * s exactly (bf16 holds every fp8 value)."""
    maxc = 0x77 if fmt == E4M3 else 0x7B
    codes = np.array([c for c in range(256) if (c & 0x7F) <= maxc], dtype=np.uint8)
    N, K = codes.size, 64
    w = np.zeros((N, K), dtype=np.uint8)
    for kk in range(K):
        w[:, kk] = np.roll(codes, kk)
    scales = np.ones(N, dtype=np.float32)
    for M in (1, 4, 16):
        x = np.zeros((M, K), dtype=np.uint16)
        for m in range(M):
            x[m, (5 * m + 3) % K] = 0x3F80   # 1.0
        y = bf16_out(R.gemm_w8a16(dev(x.ravel()), dev(w.ravel()), dev(scales), M, N, K, fmt)).reshape(M, N)
        for m in range(M):
            kk = (5 * m + 3) % K
            want = O.decode_array(w[:, kk], fmt)
            # A sum of products cannot return -0.0 (-0 + 0 = +0), so compare values;
            # every non-zero value must match bit for bit.
            assert np.array_equal(y[m], want), (M, m)
            nz = want != 0
            assert np.array_equal(y[m][nz].view(np.uint32), want[nz].view(np.uint32)), (M, m)


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 14336)])
def test_gemv_batch1_llama_8b_shapes(R, fmt, shape):
    rng = np.random.default_rng(101 + fmt)
    N, K = shape
    check_w8a16(R, rng, 1, N, K, fmt)


@pytest.mark.parametrize("N,K", [(1, 16), (7, 1040), (1000, 3584), (7169, 18944), (300, 32768), (64, 33792),
                                 (20000, 512), (129, 14336), (333, 15008), (77, 16384), (5, 11264),
                                 (517, 27648), (9, 20000), (1031, 16400)])
def test_gemv_batch1_contiguous_rows(R, N, K):
    """M = 1 on the contiguous-rows GEMV: ragged last chunks (K % 1024 != 0),
    fewer rows than waves, a row count that leaves the last wave short, rows
    longer than the 10-chunk load window (11 to 32 chunks, ragged among them),
    the 32-chunk limit (a 64 KB activation copy in LDS) and one past it (the
    row-strided GEMV then), both formats, with and without the scale operand."""
    rng = np.random.default_rng(N + K)
    check_w8a16(R, rng, 1, N, K, E4M3 if N % 2 else E5M2)
    q = quantized_weight(rng, N, K, E4M3)
    x = bf16_bits(rng.standard_normal(K).astype(np.float32))
    y = bf16_out(R.gemm_w8a16(dev(x), dev(q.codes), None, 1, N, K, E4M3))
    assert_elementwise(y.reshape(1, N), bf16_f32(x), O.decode_array(q.codes, E4M3).reshape(N, K), K, "unit scale")


def test_gemv_refuses_an_unaligned_activation(R):
    """The activation and the codes are read in 16-byte pieces: a pointer off
    that alignment is refused before any launch."""
    K = 4096
    x = torch.zeros(K + 8, dtype=torch.int16, device="cuda")
    c = torch.zeros(8 * K, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError, match="16-byte aligned"):
        R.gemm_w8a16(x[1:K + 1], c, None, 1, 8, K, E4M3)


@pytest.mark.parametrize("M", [2, 3, 4])
def test_gemv_small_batches(R, M):
    """M = 2 with 1024 < K <= 8192 runs the one-wave-per-row GEMV with both
    activation rows in LDS; otherwise K % 128 != 0 keeps M <= 4 on the strided
    GEMV, and with K % 128 == 0, M = 3 and 4 (and M = 2 at a long K) take the
    MFMA kernel with padded rows."""
    rng = np.random.default_rng(103 + M)
    check_w8a16(R, rng, M, 1024, 4096, E4M3)
    check_w8a16(R, rng, M, 1024, 4112, E4M3)
    check_w8a16(R, rng, M, 100, 176, E5M2)
    check_w8a16(R, rng, M, 300, 18944, E5M2)


@pytest.mark.parametrize("N,K", [(1000, 4096), (333, 7184), (77, 8192), (5, 1040), (4101, 2048)])
def test_gemv_two_rows_equal_two_single_rows(R, N, K):
    """Two activation rows on the row GEMV (1024 < K <= 8192): each output row
    is bit for bit the single-row GEMV of that activation row (same lanes, order
    and accumulators per row), for ragged K, few rows, a partial last block, both
    formats; and within the per-element bound of the oracle."""
    rng = np.random.default_rng(N + 7 * K)
    fmt = E4M3 if N % 2 else E5M2
    q = quantized_weight(rng, N, K, fmt)
    x = bf16_bits(rng.standard_normal((2, K)).astype(np.float32)).ravel()
    y2 = bf16_out(R.gemm_w8a16(dev(x), dev(q.codes), dev(q.scales), 2, N, K, fmt)).reshape(2, N)
    for r in range(2):
        y1 = bf16_out(R.gemm_w8a16(dev(x[r * K:(r + 1) * K].copy()), dev(q.codes), dev(q.scales), 1, N, K, fmt))
        assert np.array_equal(y2[r].view(np.uint32), y1.view(np.uint32)), (N, K, r)
    assert_elementwise(y2, bf16_f32(x), q.dequantize().reshape(N, K), K, f"M=2 N={N} K={K}")


def random_w8a16_shapes(n=96, seed=20261202):
    """Seeded (M, N, K, fmt) cases across the batch-size dispatch: M on and
    around every boundary (1, 2, 3-4, 5-16, 17-64, > 64), K a multiple of 16
    (half of them of 128, some past 8 and 16 KB rows), N from 1 up, sized so
    the oracle finishes each in well under a second."""
    rng = np.random.default_rng(seed)
    ms = [1, 1, 2, 2, 3, 4, 5, 8, 9, 15, 16, 17, 24, 31, 32, 33, 48, 63, 64, 65, 96, 130]
    out = []
    while len(out) < n:
        M = ms[len(out) % len(ms)]   # every M at least twice
        K = int(rng.integers(1, 1250)) * 16
        if rng.random() < 0.5:
            K = max(128, K // 128 * 128)
        if M <= 2 and rng.random() < 0.3:
            K = int(rng.integers(1025, 2048)) * 16   # rows past 16 KB
        N = int(rng.integers(1, 4000)) if rng.random() < 0.8 else int(rng.integers(1, 64))
        if N * K > (16 << 20) or M * N * K > 1_000_000_000:
            continue
        out.append((M, N, K, E4M3 if rng.random() < 0.5 else E5M2))
    return out


@pytest.mark.parametrize("case", random_w8a16_shapes(), ids=lambda c: f"M{c[0]}-N{c[1]}-K{c[2]}-f{c[3]}")
def test_w8a16_random_shapes(R, case):
    """Every path of the batch-size dispatch on seeded random shapes, each
    against the oracle (rel-L2) and float64 (per element)."""
    M, N, K, fmt = case
    rng = np.random.default_rng(M * 1_000_003 + N * 101 + K)
    check_w8a16(R, rng, M, N, K, fmt, sample_cols=None if M * N <= 65536 else 512)


@pytest.mark.parametrize("M", [1, 3])
def test_gemv_many_rows_per_wave(R, M):
    """N = 300000 short rows: ~74 rows per wave, past the 64 per-row scales a
    wave holds at a time (the refill path), with a ragged chunk count."""
    rng = np.random.default_rng(211 + M)
    check_w8a16(R, rng, M, 300000, 48, E4M3, sample_cols=4096)


QWEN_7B = [(3584, 3584), (512, 3584), (18944, 3584), (3584, 18944)]


@pytest.mark.parametrize("M", [8, 64])
@pytest.mark.parametrize("shape", QWEN_7B)
def test_skinny_gemm_qwen_7b_shapes(R, M, shape):
    rng = np.random.default_rng(107 + M)
    N, K = shape
    check_w8a16(R, rng, M, N, K, E4M3, sample_cols=512)


@pytest.mark.parametrize("M", [5, 16, 17, 33, 65, 130])
def test_skinny_gemm_ragged_batches(R, M):
    rng = np.random.default_rng(109 + M)
    check_w8a16(R, rng, M, 200, 512, E4M3)
    check_w8a16(R, rng, M, 48, 4096, E5M2)


# K not a multiple of the 128-code chunk, M > 4: skinny_wide with a short last
# chunk (16 to 112 codes), zero-padded in registers, on 1 to 64 activation rows
# per launch (M = 100: a 64-row and a 36-row launch; the tiled kernel wants
# K % 64 == 0). Shapes with K splits (the short chunk in the last split), one
# chunk in all (K = 48, 80), one weight row tile, N % 4 != 0 and long rows.
@pytest.mark.parametrize("M", [5, 8, 17, 40, 64, 100])
@pytest.mark.parametrize("N,K", [(512, 3632), (1000, 1008), (77, 4000), (300, 5200), (64, 48), (17, 80),
                                 (130, 18960)])
def test_skinny_wide_short_last_chunk(R, M, N, K):
    rng = np.random.default_rng(4000 * M + N + K)
    fmt = E4M3 if (M + K // 16) % 2 else E5M2
    check_w8a16(R, rng, M, N, K, fmt, sample_cols=None if M * N * K <= 64 * 1024 * 4096 else 256)


@pytest.mark.parametrize("M,N,K", [(64, 512, 3632), (8, 1000, 1008), (33, 130, 18960)])
def test_short_last_chunk_is_deterministic(R, M, N, K):
    """The short chunk's padding adds exact zeros wherever it falls: repeated
    calls give the same bits, equal to the product over K zero-padded to a
    whole chunk (the same codes and activation with 128 - K % 128 zero columns
    appended)."""
    rng = np.random.default_rng(M * N + K)
    q = quantized_weight(rng, N, K, E4M3)
    xh = bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    x, c, s = dev(xh.ravel()), dev(q.codes), dev(q.scales)
    first = R.gemm_w8a16(x, c, s, M, N, K, E4M3).clone()
    for _ in range(2):
        assert torch.equal(R.gemm_w8a16(x, c, s, M, N, K, E4M3), first)
    Kp = (K + 127) // 128 * 128
    cp = np.zeros((N, Kp), dtype=np.uint8)
    cp[:, :K] = q.codes.reshape(N, K)
    xp = np.zeros((M, Kp), dtype=np.uint16)
    xp[:, :K] = xh.reshape(M, K)
    padded = R.gemm_w8a16(dev(xp.ravel()), dev(cp.ravel()), s, M, N, Kp, E4M3)
    torch.cuda.synchronize()
    if M > 16:
        # The same kernel and plan over whole chunks (the same chunk count):
        # the padding's products are the same zeros, so the same bits.
        assert torch.equal(first, padded)
    else:
        # Whole chunks at M <= 16 take the 16-row kernels: another order of sums.
        assert O.rel_l2(bf16_out(first).ravel(), bf16_out(padded).ravel()) < 4e-3


# 4 < M <= 16 (skinny_rows): every block shape the launcher picks (16, 32, 64,
# 80 or 128 rows per block by N; the 80-row form holds the activation in LDS
# for M <= 8 and K <= 4096: N = 20000, and 18950 at that K limit), K runs with
# a one-chunk last stage (K % 256 == 128), K shorter than the waves' split
# (some waves get no chunk), N not a multiple of 16 or of 4, and both
# staged-activation heights (8 and 16 rows); and long rows whose 16-row tiles
# fill the CUs (N = 4096 and 3900 at K = 14336 and 8192: whole-K at M <= 8).
@pytest.mark.parametrize("M", [5, 7, 8, 9, 12, 16])
@pytest.mark.parametrize("N,K", [(200, 128), (4101, 384), (8000, 256), (16000, 3712), (20000, 1152), (18950, 4096),
                                 (4096, 14336), (3900, 8192)])
def test_skinny_rows_block_shapes(R, M, N, K):
    rng = np.random.default_rng(1000 * M + N + K)
    fmt = E4M3 if (M + N) % 2 else E5M2
    check_w8a16(R, rng, M, N, K, fmt, sample_cols=None if N * K <= 4096 * 384 else 512)


# 16 < M <= 64 (skinny_wide): 32-, 64-, 96- and 128-row blocks (96 where
# 128-row blocks leave CUs idle: N = 18950, K = 1024, with a partial last
# block), one K split (N past a grid's worth of tiles) and many (the partials
# merged in the launch), the scalar paths for N % 4 != 0, N below one block,
# 2, 3 and 4 activation tiles.
@pytest.mark.parametrize("M", [17, 32, 40, 48, 63, 64])
@pytest.mark.parametrize("N,K", [(48, 4096), (3584, 1152), (4101, 384), (40000, 256), (6000, 2944),
                                 (18950, 1024)])
def test_skinny_wide_block_shapes(R, M, N, K):
    rng = np.random.default_rng(2000 * M + N + K)
    fmt = E5M2 if (M + N) % 2 else E4M3
    check_w8a16(R, rng, M, N, K, fmt, sample_cols=None if N * K <= 4096 * 384 else 512)


# The K splits merged inside the launch: M <= 16 products on the split form
# (K >= 8192; 8 < M <= 16 outside the band where 16-row tiles fill half to all
# of the CUs), 16 < M <= 64 with 32-row blocks (few tiles, and the tie where
# 64-row blocks would fill exactly half the CUs: [1024, 4096]), row tiles not
# a multiple of the 8 XCDs (padding blocks in the XCD-major grid), a short last
# split, N % 4 != 0, one row tile in all, and 2 <= M <= 4 on long rows.
@pytest.mark.parametrize("M", [2, 8, 12, 16, 24, 64])
@pytest.mark.parametrize("N,K", [(512, 3584), (1000, 8192), (77, 9344), (3000, 2944), (200, 16384), (1024, 4096)])
def test_split_merge_shapes(R, M, N, K):
    rng = np.random.default_rng(3000 * M + N + K)
    fmt = E4M3 if (M + K // 128) % 2 else E5M2
    check_w8a16(R, rng, M, N, K, fmt, sample_cols=None if N * K <= 1024 * 8192 else 384)


@pytest.mark.parametrize("M,N,K", [(64, 512, 3584), (16, 3584, 18944), (8, 1000, 8192), (40, 3584, 3584)])
def test_split_merge_is_deterministic_and_leaves_its_counters_zeroed(R, M, N, K):
    """The last block of a row tile adds the splits in split order whichever
    block it is, and resets the tile's counter: repeated calls, and calls after
    other split products on the same stream, give the same bits."""
    rng = np.random.default_rng(M + N + K)
    q = quantized_weight(rng, N, K, E4M3)
    x = dev(bf16_bits(rng.standard_normal((M, K)).astype(np.float32)).ravel())
    c, s = dev(q.codes), dev(q.scales)
    first = R.gemm_w8a16(x, c, s, M, N, K, E4M3).clone()
    for _ in range(3):
        assert torch.equal(R.gemm_w8a16(x, c, s, M, N, K, E4M3), first)
    q2 = quantized_weight(rng, 700, 4096, E5M2)
    x2 = dev(bf16_bits(rng.standard_normal((24, 4096)).astype(np.float32)).ravel())
    R.gemm_w8a16(x2, dev(q2.codes), dev(q2.scales), 24, 700, 4096, E5M2)
    assert torch.equal(R.gemm_w8a16(x, c, s, M, N, K, E4M3), first)
    torch.cuda.synchronize()


_FIRST_CALL_CHILD = r"""
import ctypes, os, sys
root = sys.argv[1]
for p in (os.path.join(root, "reciprocating-engine_amd"), os.path.join(root, "oracle"), os.path.join(root, "tests")):
    sys.path.insert(0, p)
import os

import numpy as np
import torch
import oracle as O
import reng_hip as R
from helpers import bf16_bits
torch.cuda.set_device(0)
L = R.lib()
rng = np.random.default_rng(7)
st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
outs = []
for (M, N, K) in ((64, 3584, 3584), (8, 1000, 8192), (24, 512, 3584)):
    w = bf16_bits((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).ravel()
    q = O.quantize(w, N, K, 0, "pcs")
    x = torch.from_numpy(bf16_bits(rng.standard_normal((M, K)).astype(np.float32)).ravel().view(np.int16)).cuda()
    c, s = torch.from_numpy(q.codes).cuda(), torch.from_numpy(q.scales).cuda()
    y = torch.empty(M * N, dtype=torch.int16, device="cuda")
    rc = L.reng_hip_gemm_w8a16_noalloc(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(c.data_ptr()),
                                       ctypes.c_void_p(s.data_ptr()), M, N, K, 0, ctypes.c_void_p(y.data_ptr()), st)
    assert rc == 0, L.reng_hip_last_error()
    outs.append((x, c, s, M, N, K, y))
torch.cuda.synchronize()
for x, c, s, M, N, K, y in outs:
    want = R.gemm_w8a16(x, c, s, M, N, K, "e4m3")
    torch.cuda.synchronize()
    assert torch.equal(y, want.view(torch.int16)), (M, N, K)
print("first-call products equal", flush=True)
"""


def test_split_merge_before_the_placement_check_matches_after_it():
    """The first split products of a process, through the allocation-free entry
    (which never runs the XCD placement check), merge their partials with
    agent-coherent accesses; the allocating entry then checks the placement
    and merges through the XCD's L2. Run in a fresh process so that nothing
    has checked the placement yet: both give the same bits."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CHILD, root], capture_output=True, text=True, timeout=180)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "first-call products equal" in r.stdout


@pytest.mark.parametrize("M", [8, 64])
def test_skinny_every_output_of_a_qwen_7b_gate_up(R, M):
    """Every output of the Qwen2.5-7B gate/up product [18944, 3584] at M = 8 and
    64, each element against float64 numpy within the bound above."""
    rng = np.random.default_rng(401 + M)
    check_w8a16(R, rng, M, 18944, 3584, E4M3)


@pytest.mark.parametrize("M, N, K, fmt", [
    (1000, 12288, 1024, E4M3),  # 256 x 256 tiles; ragged M
    (384, 20480, 1024, E5M2),   # 128 x 256 tiles
    (200, 20480, 768, E4M3),    # 128 x 160 tiles (4 waves, 128-code stages); ragged M
    (200, 20001, 768, E5M2),    # 128 x 160 tiles; ragged M and N (element stores)
    (768, 4097, 1536, E5M2),    # 128 x 128 tiles; ragged N (element stores)
    (200, 4097, 3072, E4M3),    # 64 x 128 tiles; ragged M and N
    (96, 8192, 64, E5M2),       # 64 x 64 tiles (4 waves); one stage
    (512, 8192, 192, E4M3),     # 64 x 64 tiles; K % 128 != 0
])
def test_w8a16_tiles_every_output(R, M, N, K, fmt):
    """More than 64 activation rows take the tiled bf16-MFMA kernel; one shape
    per tile form the launcher's cost model picks on a 256-CU MI355X, every
    output against the oracle and float64."""
    rng = np.random.default_rng(M * 7 + N + K)
    check_w8a16(R, rng, M, N, K, fmt)


@pytest.mark.parametrize("M, N, K, fmt", [
    (256, 2048, 8192, E4M3),    # 32 tiles of 128 x 128 over 64 stages each: stream-K
    (200, 1000, 8320, E5M2),    # ragged M and N under stream-K
])
def test_w8a16_stream_k_every_output(R, M, N, K, fmt):
    """Long K over few tiles runs stream-K: blocks take equal runs of
    (tile, stage) units across tile edges and the last block of each split tile
    adds the partials. Two products in a row with other weights check that the
    tile counters come back to zero."""
    rng = np.random.default_rng(M + N + K)
    check_w8a16(R, rng, M, N, K, fmt)
    check_w8a16(R, rng, M, N, K, fmt)


def test_w8a16_tiles_two_input_form(R):
    """No scale operand on the tiled kernel: the product over the raw codes."""
    rng = np.random.default_rng(5)
    M, N, K = 256, 8192, 64
    q = quantized_weight(rng, N, K, E4M3)
    x = bf16_bits(rng.standard_normal((M, K)).astype(np.float32)).ravel()
    y = bf16_out(R.gemm_w8a16(dev(x), dev(q.codes), None, M, N, K, E4M3)).reshape(M, N)
    raw = O.decode_array(q.codes, E4M3).reshape(N, K)
    assert_elementwise(y, bf16_f32(x), raw, K, "tiles, no scales")


def test_the_reference_probe_shapes(R):
    """fp8_probe.rs:478-505: weights(512, 256), m in {1, 256}, rel_L2 < 0.02."""
    N, K = 512, 256
    w = probe_weights(N, K)
    q = O.quantize(w, N, K, E4M3, "pcs")
    for m in (1, 256):
        a = bf16_bits(probe_activations(m * K))
        y = bf16_out(R.gemm_w8a16(dev(a), dev(q.codes), dev(q.scales), m, N, K, E4M3))
        want = O.gemm(bf16_f32(a), q.dequantize(), m, K, N)
        assert O.rel_l2(y, want) < TOL
        # The 2-input form: no scale operand, the product over the raw codes.
        y2 = bf16_out(R.gemm_w8a16(dev(a), dev(q.codes), None, m, N, K, E4M3))
        raw = O.decode_array(q.codes, E4M3)
        assert O.rel_l2(y2, O.gemm(bf16_f32(a), raw, m, K, N)) < TOL


def test_w8a16_refuses_bad_shapes(R):
    x = torch.zeros(64, dtype=torch.int16, device="cuda")
    c = torch.zeros(64 * 8, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError, match="multiple of 16"):
        R.gemm_w8a16(x, c, None, 1, 8, 40, E4M3)
    with pytest.raises(ValueError, match="empty product"):
        R.gemm_w8a16(x, c, None, 0, 8, 64, E4M3)


# ------------------------------------------------------------ fp8 x fp8


def check_fp8(R, rng, M, N, K, fa, fb, act="pcs", nsb="N", sample_cols=None):
    x = bf16_bits(rng.standard_normal((M, K)).astype(np.float32)).ravel()
    qa = O.quantize(x, M, K, fa, act)
    qw = quantized_weight(rng, N, K, fb)
    sa = None if act == "unit" else qa.scales
    sb = {"N": qw.scales, "1": qw.scales[:1].copy(), "0": None}[nsb]
    out = bf16_out(R.gemm_fp8_scaled(dev(qa.codes), fa, None if sa is None else dev(sa), dev(qw.codes), fb,
                                     None if sb is None else dev(sb), M, N, K)).reshape(M, N)
    a_deq = qa.dequantize()
    if sb is None:
        b_scale = np.float32(1.0)
    elif sb.size == 1:
        b_scale = sb[0]
    else:
        b_scale = np.repeat(sb, K)
    b_deq = (O.decode_array(qw.codes, fb) * b_scale).astype(np.float32)
    if sample_cols and sample_cols < N:
        idx = np.unique(np.concatenate([rng.choice(N, sample_cols, replace=False), [0, N - 1]]))
        want = O.gemm_cols(a_deq, b_deq, M, K, idx, threads=16).reshape(M, idx.size)
        got = out[:, idx]
    else:
        want = O.gemm(a_deq, b_deq, M, K, N, threads=16).reshape(M, N)
        got = out
    rel = O.rel_l2(got.ravel(), want.ravel())
    assert rel < TOL, f"M={M} N={N} K={K} {fa}x{fb} act={act} sb={nsb}: rel_L2 {rel}"
    rows = idx if sample_cols and sample_cols < N else slice(None)
    assert_elementwise(got, a_deq, b_deq.reshape(N, K)[rows], K, f"M={M} N={N} K={K} {fa}x{fb} act={act} sb={nsb}",
                       acc=fp8_acc(K))
    return rel


@pytest.mark.parametrize("fa,fb", [(E4M3, E4M3), (E5M2, E5M2), (E4M3, E5M2), (E5M2, E4M3)])
def test_fp8_gemm_formats_and_scale_forms(R, fa, fb):
    rng = np.random.default_rng(113 + 2 * fa + fb)
    for act, nsb in (("pcs", "N"), ("unit", "N"), ("pcs", "1"), ("unit", "0")):
        check_fp8(R, rng, 160, 200, 384, fa, fb, act, nsb)


# Ragged edges on each tile size the launcher picks (256 x 256, 128 x 128,
# 256 x 128 for long K, 64 x 64): M and N off the tile grid, N % 4 != 0 (the
# scalar output path) and N % 4 == 0 with a partial last tile.
@pytest.mark.parametrize("M,N,K", [(1000, 16390, 256), (1000, 4100, 384), (520, 8300, 8320), (100, 70, 128)])
def test_fp8_gemm_ragged_tiles(R, M, N, K):
    rng = np.random.default_rng(M + N + K)
    check_fp8(R, rng, M, N, K, E4M3, E4M3, sample_cols=160)


# Whole-tile shapes take the wide forms, one shape per tile the launcher's
# cost model picks on a 256-CU MI355X: 256 x 256 (1024 x 16384), 256 x 128
# (512 x 16384), 128 x 160 (1024 x 5120), 128 x 128 (1024 x 4096), 64 x 64
# (256 x 32768), and the mixed grid (1024 x 27648: 252 tiles of 256 x 256 over
# the first 16128 columns, 240 of 256 x 192 over the rest); K of one to eight
# 128-code stages, every format pair and scale form.
@pytest.mark.parametrize("M,N,K", [(1024, 16384, 256), (512, 16384, 384), (1024, 5120, 1024), (1024, 4096, 1024),
                                   (256, 32768, 128), (1024, 27648, 256)])
@pytest.mark.parametrize("fa,fb", [(E4M3, E4M3), (E5M2, E5M2), (E4M3, E5M2), (E5M2, E4M3)])
def test_fp8_gemm_wide_tiles(R, M, N, K, fa, fb):
    rng = np.random.default_rng(M + N + K + 4 * fa + fb)
    for act, nsb in (("pcs", "N"), ("unit", "1"), ("pcs", "0")):
        check_fp8(R, rng, M, N, K, fa, fb, act, nsb, sample_cols=96)


def test_fp8_gemm_every_output_of_a_qwen_32b_projection(R):
    """Every output of the M = 1024 prefill product on Qwen2.5-32B's q/o shape
    [5120, 5120], each element against float64 numpy."""
    rng = np.random.default_rng(131)
    check_fp8(R, rng, 1024, 5120, 5120, E4M3, E4M3)


@pytest.mark.parametrize("shape", [(5120, 5120), (1024, 5120), (27648, 5120), (5120, 27648)])
def test_fp8_gemm_prefill_qwen_32b_shapes(R, shape):
    rng = np.random.default_rng(127)
    N, K = shape
    check_fp8(R, rng, 1024, N, K, E4M3, E4M3, sample_cols=192)


def random_fp8_shapes(n=48, seed=20261203):
    """Seeded fp8 x fp8 cases: M and N on and off every tile grid (whole tiles
    take the wide forms, the rest the ragged kernel; 1024-row products with many
    256-wide column tiles the mixed grid), K in 128-code stages, every format
    pair and scale form."""
    rng = np.random.default_rng(seed)
    ms = [1, 7, 64, 100, 128, 256, 300, 512, 1000, 1024]
    forms = [("pcs", "N"), ("unit", "N"), ("pcs", "1"), ("unit", "0"), ("pcs", "0")]
    pairs = [(E4M3, E4M3), (E5M2, E5M2), (E4M3, E5M2), (E5M2, E4M3)]
    out = []
    while len(out) < n:
        M = ms[len(out) % len(ms)]
        K = 128 * int(rng.integers(1, 48))
        r = rng.random()
        N = 64 * int(rng.integers(1, 400)) if r < 0.4 else 256 * int(rng.integers(64, 112)) if r < 0.5 \
            else int(rng.integers(1, 6000))
        if M * N * K > 1_500_000_000:
            continue
        fa, fb = pairs[int(rng.integers(0, 4))]
        act, nsb = forms[int(rng.integers(0, 5))]
        out.append((M, N, K, fa, fb, act, nsb))
    return out


@pytest.mark.parametrize("case", random_fp8_shapes(), ids=lambda c: "M{}-N{}-K{}-{}x{}-{}-{}".format(*c))
def test_fp8_gemm_random_shapes(R, case):
    """The fp8 GEMM's dispatch on seeded random shapes, each against the oracle
    (rel-L2) and float64 (per element, the fp8 bound)."""
    M, N, K, fa, fb, act, nsb = case
    rng = np.random.default_rng(M * 7919 + N * 31 + K)
    check_fp8(R, rng, M, N, K, fa, fb, act, nsb, sample_cols=None if M * N <= 65536 else 256)


@pytest.mark.parametrize("fmt", [E4M3, E5M2])
def test_fp8_mfma_accumulation_over_k(R, fmt):
    """The fp8 MFMA's accumulation error against fp8_acc(K): codes drawn
    uniformly from every finite code of the format with random signs (values
    from 2^-9 to 240 for e4m3, 2^-16 to 57344 for e5m2 in one instruction's 64
    products), unit scales, a wide-form and a ragged-form shape, K = 128 ...
    27648; every output against float64."""
    rng = np.random.default_rng(7 + fmt)
    maxc = 0x77 if fmt == E4M3 else 0x7B
    for M, N in ((256, 256), (250, 300)):
        for K in (128, 384, 1024, 5120, 27648):
            a = rng.integers(0, maxc + 1, (M, K), dtype=np.uint8) | (rng.integers(0, 2, (M, K), dtype=np.uint8) << 7)
            b = rng.integers(0, maxc + 1, (N, K), dtype=np.uint8) | (rng.integers(0, 2, (N, K), dtype=np.uint8) << 7)
            out = bf16_out(R.gemm_fp8_scaled(dev(a.ravel()), fmt, None, dev(b.ravel()), fmt, None, M, N, K))
            ad = O.decode_array(a.ravel(), fmt).reshape(M, K)
            bd = O.decode_array(b.ravel(), fmt).reshape(N, K)
            assert_elementwise(out.reshape(M, N), ad, bd, K, f"uniform codes {fmt} M={M} N={N} K={K}", acc=fp8_acc(K))


@pytest.mark.parametrize("shape", [(27648, 5120), (5120, 27648)])
def test_fp8_gemm_every_output_of_the_qwen_32b_long_shapes(R, shape):
    """Every output of the M = 1024 prefill product on Qwen2.5-32B's gate/up
    (the 256 x 256 form) and down (the 128 x 160 form, K = 27648) shapes,
    each element against float64 numpy within the fp8 bound."""
    rng = np.random.default_rng(137)
    N, K = shape
    M = 1024
    x = bf16_bits(rng.standard_normal((M, K)).astype(np.float32)).ravel()
    qa = O.quantize(x, M, K, E4M3, "pcs")
    qw = quantized_weight(rng, N, K, E4M3)
    out = bf16_out(R.gemm_fp8_scaled(dev(qa.codes), E4M3, dev(qa.scales), dev(qw.codes), E4M3, dev(qw.scales),
                                     M, N, K)).reshape(M, N)
    assert np.all(np.isfinite(out))
    assert_elementwise(out, qa.dequantize(), qw.dequantize(), K, f"M={M} N={N} K={K}", acc=fp8_acc(K))


@pytest.mark.parametrize("M,N,K", [(17, 512, 3584), (40, 3584, 3584), (64, 18944, 3584), (64, 3584, 18944)])
def test_the_stage_copy_yardstick_runs_the_skinny_grid(R, M, N, K):
    """reng_hip_stream_stage (skinny_wide's copy stream with no arithmetic, a
    measuring stick for bench.py) on each block shape the wide kernel takes:
    it completes, and with all-zero operands never writes its sink."""
    x = torch.zeros(M * K, dtype=torch.int16, device="cuda")
    c = torch.zeros(N * K, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    R.stream_stage(x, c, M, N, K, sink)
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
