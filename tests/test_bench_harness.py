"""bench.py's measurement mechanics on the CPU, with a fake clock standing in for
the device: the quantize step's launch grouping and per-launch accounting (one
event before a step and one after each launch, launch i spanning the events
either side of it), the dominant-kernel selection the roofline object uses,
and the buffer rotation that keeps timed launches out of the Infinity Cache.
The device timing itself is the reference harness's shape (time_launches,
crates/reng-synapse/src/fp8.rs:419-429: warm-ups, then launches between two
clock reads), run on the GPU by bench.py and reng-fp8-probe `time`."""
import pytest

import bench


class Clock:
    def __init__(self):
        self.t = 0.0


class FakeEvent:
    def __init__(self, clock):
        self.clock, self.t = clock, None

    def record(self):
        self.t = self.clock.t

    def elapsed_time(self, other):   # milliseconds, as torch.cuda.Event
        return (other.t - self.t) * 1e3


class FakeTorch:
    def __init__(self, clock):
        clock_ = clock

        class Cuda:
            @staticmethod
            def Event(enable_timing=False):
                return FakeEvent(clock_)

            @staticmethod
            def synchronize():
                pass

        self.cuda = Cuda


class FakeLib:
    """quantize_batch advances the clock by 1 us per matrix of <= 4096 columns and
    3 us per wider matrix, plus a 0.5 us gap after the launch."""

    def __init__(self, clock):
        self.clock, self.calls = clock, []

    def quantize_batch(self, b, fmt, scheme, backoff):
        assert len(b) <= 32 and len({m[2] for m in b}) == 1   # one row width per launch
        self.calls.append(len(b))
        self.clock.t += sum(1e-6 if m[2] <= 4096 else 3e-6 for m in b)
        self.clock.t += 0.5e-6


def weight_set(layers):
    ws = bench.WeightSet.__new__(bench.WeightSet)
    ws.mats = [(li, name, rows, cols, None, None, None, None)
               for li in range(layers) for name, rows, cols in bench.LLAMA_8B]
    ws.bytes = sum(bench.quant_bytes(m[2], m[3]) for m in ws.mats)
    return ws


def test_launch_grouping_is_by_width_and_32_per_launch():
    ws = weight_set(32)
    launches = ws.launches()
    assert [c for c, _, _ in launches] == [4096] * 6 + [14336]
    assert [len(ch) for _, ch, _ in launches] == [32] * 7
    assert sum(b for _, _, b in launches) == ws.bytes == 20_943_470_592
    # every matrix exactly once
    assert sum(len(ch) for _, ch, _ in launches) == len(ws.mats) == 224


def test_time_quantize_accounts_each_launch_between_its_events():
    clock = Clock()
    ws = weight_set(32)
    lib = FakeLib(clock)
    res = bench.time_quantize(FakeTorch(clock), lib, ws, "e4m3", steps=4, warmup=2)
    assert lib.calls == [32] * 7 * 6   # 2 warm-up + 4 timed steps of 7 launches
    dom = res["dominant"]
    assert dom["cols"] == 4096 and dom["launches_per_step"] == 6
    # each 4096-wide launch: 32 us of kernel + the 0.5 us gap before the next event
    assert dom["secs_per_launch"] == pytest.approx(32.5e-6)
    assert res["configs"]["14336"]["launches_per_step"] == 1
    assert res["kernel_sum_s"] == pytest.approx(6 * 32.5e-6 + 96.5e-6)
    assert dom["bytes_per_launch"] == sum(b for c, _, b in ws.launches() if c == 4096) / 6


def test_rotation_exceeds_the_infinity_cache():
    for nbytes in (1 << 20, 13 << 20, 58_720_256, 117 << 20, 1 << 30):
        n = bench.rotation(nbytes)
        assert n >= 4
        assert n * nbytes >= 2 * bench.MALL_BYTES or n == 1024
    assert bench.MALL_BYTES == 256 << 20


class FakeOracle:
    """quantize_with returns a token per matrix; split follows reng-fp8's rule
    (one thread per 2^20 elements, capped at 8 and at rows)."""

    def __init__(self):
        self.calls = 0

    def quantize_with(self, w, rows, cols, fmt, scheme, backoff, thread_cap=8):
        self.calls += 1
        return ("q", rows, cols, self.calls)

    @staticmethod
    def split(rows, cols):
        return max(1, min(8, (rows * cols) >> 20, rows))


def test_cpu_baseline_is_the_median_of_three_runs(monkeypatch):
    O = FakeOracle()
    host = [(4096, 4096, None), (1024, 4096, None)]
    ticks = iter([0.0, 5.0, 5.0, 7.0, 7.0, 13.0])   # runs of 5, 2 and 6 s
    monkeypatch.setattr(bench.time, "perf_counter", lambda: next(ticks))
    refs, secs = bench.time_oracle_sample(O, host, "e4m3")
    assert secs == [5.0, 2.0, 6.0]
    assert [r[3] for r in refs] == [1, 2]           # the first run's results are the ones kept
    rec = bench.cpu_record(O, host, secs, "two matrices")
    nbytes = bench.quant_bytes(4096, 4096) + bench.quant_bytes(1024, 4096)
    assert rec["value"] == pytest.approx(round(nbytes / 5.0 / 1e9, 3))   # median 5 s
    assert rec["cores"] == 8 and rec["kind"] == "port" and rec["unit"] == "GB/s"
    assert "median of 3 runs" in rec["sample"]
