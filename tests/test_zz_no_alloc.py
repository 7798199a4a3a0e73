"""reng_hip_gemm_w8a16_noalloc, the entry point that allocates nothing: through
the C ABI it must give what reng_hip_gemm_w8a16 gives, bit for bit, on two
calls in a row (the second smaller, so it runs on what the first left in the
shared static scratch), on products that use the split-K scratch (16 < M <= 64
with K splits, M > 64 in 64-row tiles), the stream-K partials and tile
counters (long-K M > 64 over few tiles) and on ones that do not; and captured
into a hipGraph on a fresh stream, where the allocating entry refuses to grow
its per-stream buffers, with every replay equal to the eager result."""
import ctypes
import warnings

import numpy as np
import pytest

import oracle as O
from helpers import E4M3, E5M2, bf16_bits

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def R():
    import reng_hip

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    reng_hip.lib()
    return reng_hip


def operands(rng, M, N, K, fmt):
    w = bf16_bits((rng.standard_normal((N, K)) * 0.02).astype(np.float32)).ravel()
    q = O.quantize(w, N, K, fmt, "pcs")
    x = bf16_bits(rng.standard_normal((M, K)).astype(np.float32)).ravel()
    return (torch.from_numpy(x.view(np.int16)).cuda(), torch.from_numpy(q.codes).cuda(),
            torch.from_numpy(q.scales).cuda())


def call(R, name, x, codes, scales, M, N, K, fmt):
    y = torch.full((M * N,), -1, dtype=torch.int16, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = getattr(R.lib(), name)(ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(codes.data_ptr()),
                                ctypes.c_void_p(scales.data_ptr()), M, N, K, fmt, ctypes.c_void_p(y.data_ptr()), st)
    assert rc == 0, R.lib().reng_hip_last_error()
    return y


@pytest.mark.parametrize("first,second", [
    ((64, 3584, 3584), (40, 512, 3584)),      # K-split partials both times, the second plan smaller
    ((64, 3584, 18944), (17, 1000, 1024)),    # the largest Qwen2.5-7B plan, then a 2-tile one
    ((130, 2048, 1024), (65, 700, 512)),      # M > 64: 64-row tiles share the scratch in stream order
    ((8, 18944, 3584), (1, 4096, 4096)),      # no split: skinny_rows, then the GEMV
    ((256, 2048, 8192), (100, 1000, 8192)),   # stream-K partials and counters, then a smaller stream-K plan
    ((64, 512, 3632), (9, 1000, 1008)),       # K % 128 != 0: a short last chunk, K splits both times
])
def test_noalloc_matches_the_allocating_entry_twice(R, first, second):
    rng = np.random.default_rng(sum(first) + sum(second))
    for (M, N, K), fmt in ((first, E4M3), (second, E5M2)):
        x, codes, scales = operands(rng, M, N, K, fmt)
        got = call(R, "reng_hip_gemm_w8a16_noalloc", x, codes, scales, M, N, K, fmt)
        torch.cuda.synchronize()
        want = call(R, "reng_hip_gemm_w8a16", x, codes, scales, M, N, K, fmt)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (M, N, K, fmt)


def test_noalloc_refuses_what_the_allocating_entry_refuses(R):
    L = R.lib()
    p = ctypes.c_void_p(256)   # never dereferenced: the checks come first
    assert L.reng_hip_gemm_w8a16_noalloc(p, p, None, 1, 8, 40, E4M3, p, None) == R.EINVAL
    assert b"multiple of 16" in L.reng_hip_last_error()
    assert L.reng_hip_gemm_w8a16_noalloc(p, p, None, 0, 8, 64, E4M3, p, None) == R.EINVAL


@pytest.mark.parametrize("M,N,K", [(64, 3584, 3584), (256, 2048, 8192)])   # K-split partials; stream-K
def test_noalloc_under_graph_capture_on_a_fresh_stream(R, M, N, K):
    """What the entry point is for: captured into a hipGraph on a stream that has
    never run a split-K or stream-K product (so the allocating entry would have
    to grow its per-stream buffers, which it refuses while the stream is
    captured), replayed three times with eager work and synchronizations in
    between; every replay equals the allocating entry's eager result."""
    rng = np.random.default_rng(M + N + K)
    x, codes, scales = operands(rng, M, N, K, E4M3)
    want = call(R, "reng_hip_gemm_w8a16", x, codes, scales, M, N, K, E4M3)
    torch.cuda.synchronize()
    L = R.lib()
    args = lambda y: (ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(codes.data_ptr()),
                      ctypes.c_void_p(scales.data_ptr()), M, N, K, E4M3, ctypes.c_void_p(y.data_ptr()))

    # The allocating entry on a fresh stream under capture: refused, nothing
    # queued (so torch's warning that this graph is empty is the expected
    # outcome here).
    side = torch.cuda.Stream()
    y0 = torch.full((M * N,), -1, dtype=torch.int16, device="cuda")
    g0 = torch.cuda.CUDAGraph()
    with warnings.catch_warnings():
        warnings.filterwarnings("ignore", message="The CUDA Graph is empty")
        with torch.cuda.graph(g0, stream=side):
            rc = L.reng_hip_gemm_w8a16(*args(y0), ctypes.c_void_p(side.cuda_stream))
    assert rc == R.EINVAL and b"captured" in L.reng_hip_last_error()

    fresh = torch.cuda.Stream()
    y = torch.full((M * N,), -1, dtype=torch.int16, device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=fresh):
        rc = L.reng_hip_gemm_w8a16_noalloc(*args(y), ctypes.c_void_p(fresh.cuda_stream))
    assert rc == 0, L.reng_hip_last_error()
    for rep in range(3):
        y.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), (M, N, K, rep)
