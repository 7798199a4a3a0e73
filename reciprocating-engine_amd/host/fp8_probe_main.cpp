// reng-fp8-probe - the device acceptance probes of
// crates/reng-model/src/bin/fp8_probe.rs, retargeted to libreng_hip.so.
//
//   reng-fp8-probe [check] [time] [--format e4m3|e5m2] [--iters <n>] [--min-speedup <x>]
//
// check (the default): the device's reading of every code and its clipping
// cast against the host references, the mixed bf16 x fp8 pair (the decode
// path here; the reference's stack refuses it), the fp8 x fp8 product with
// an exponent-bias weight, and the scaled form with and without its scale
// operands, at 1 and 256 rows. time: the fp8 paths against a bf16 GEMM
// (rocBLAS) at K = 4096, N = 4096 and 14336, m = 1 and 256, with the
// N = 14336, m = 1 ratio checked against --min-speedup (default 1.2x).
// Every check prints one line ending in PASS or FAIL; the exit status is
// non-zero if any failed.
#include <hip/hip_runtime_api.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/reng_hip.h"
#include "fp8_probe.hpp"

using namespace reng_probe;
using reng_fp8::Scaling;

namespace {

constexpr double DEFAULT_SPEEDUP_FLOOR = 1.2;

struct Fail : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Fail(std::string(what) + ": " + hipGetErrorString(e));
}

template <typename T>
T *upload(const std::vector<T> &v) {
    void *p = nullptr;
    hip_ok(hipMalloc(&p, v.size() * sizeof(T)), "hipMalloc");
    hip_ok(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
    return static_cast<T *>(p);
}

// Seconds per launch over `iters` back-to-back launches after 3 warm-ups.
template <typename F>
double time_launches(F launch, int iters) {
    for (int i = 0; i < 3; ++i) launch();
    hipEvent_t e0, e1;
    hip_ok(hipEventCreate(&e0), "hipEventCreate");
    hip_ok(hipEventCreate(&e1), "hipEventCreate");
    hip_ok(hipEventRecord(e0, nullptr), "hipEventRecord");
    for (int i = 0; i < iters; ++i) launch();
    hip_ok(hipEventRecord(e1, nullptr), "hipEventRecord");
    hip_ok(hipEventSynchronize(e1), "hipEventSynchronize");
    float ms = 0.0f;
    hip_ok(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return ms / 1e3 / iters;
}

void abi_ok(int rc) {
    if (rc != RENG_HIP_OK) throw Fail(std::string("reng-hip: ") + reng_hip_last_error());
}

void timings(Checks &c, int iters, Fp8Format fmt, double floor) {
    rocblas_handle handle;
    if (rocblas_create_handle(&handle) != rocblas_status_success) throw Fail("rocblas_create_handle failed");
    std::printf("%-8s %6s %10s %10s %10s %8s\n", "form", "m", "K x N", "ms/launch", "weight MB", "GB/s");
    for (auto kn : {std::pair<size_t, size_t>{4096, 4096}, {4096, 14336}}) {
        const size_t k = kn.first, n = kn.second;
        const std::vector<uint16_t> w = weights(n, k);
        const Quantized q = reng_fp8::quantize(w, n, k, fmt, Scaling::PerChannel);
        uint16_t *dw = upload(w);
        uint8_t *dc = upload(q.codes);
        float *ds = upload(q.scales);
        for (size_t m : {size_t(1), size_t(256)}) {
            std::vector<uint16_t> a(m * k);
            const std::vector<float> af = activations(m * k);
            for (size_t i = 0; i < a.size(); ++i) a[i] = reng_fp8::f32_to_bf16(af[i]);
            const Quantized aq = reng_fp8::quantize(a, m, k, fmt, Scaling::PerChannel);
            uint16_t *da = upload(a);
            uint8_t *dac = upload(aq.codes);
            float *das = upload(aq.scales);
            uint16_t *dy = nullptr;
            hip_ok(hipMalloc((void **)&dy, m * n * 2), "hipMalloc");
            const double t_mixed = time_launches(
                [&] { abi_ok(reng_hip_gemm_w8a16(da, dc, ds, m, n, k, (int)fmt, dy, nullptr)); }, iters);
            const double t_fp8 = time_launches(
                [&] {
                    abi_ok(reng_hip_gemm_fp8_scaled(dac, (int)fmt, das, m, dc, (int)fmt, ds, n, m, n, k, dy, nullptr));
                },
                iters);
            const float one = 1.0f, zero = 0.0f;
            const double t_bf16 = time_launches(
                [&] {
                    // y [m, N] row-major = (W [N, K] row-major) . (x [m, K] row-major)^T, column-major view.
                    if (rocblas_gemm_ex(handle, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)n,
                                        (rocblas_int)m, (rocblas_int)k, &one, dw, rocblas_datatype_bf16_r,
                                        (rocblas_int)k, da, rocblas_datatype_bf16_r, (rocblas_int)k, &zero, dy,
                                        rocblas_datatype_bf16_r, (rocblas_int)n, dy, rocblas_datatype_bf16_r,
                                        (rocblas_int)n, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0,
                                        0) != rocblas_status_success)
                        throw Fail("rocblas_gemm_ex failed");
                },
                iters);
            const double mb8 = (double)(k * n) / 1e6, mb16 = 2.0 * mb8;
            const std::string shape = std::to_string(k) + "x" + std::to_string(n);
            std::printf("%-8s %6zu %10s %10.4f %10.0f %8.0f\n", "w8a16", m, shape.c_str(), t_mixed * 1e3, mb8,
                        mb8 / 1e3 / t_mixed);
            std::printf("%-8s %6zu %10s %10.4f %10.0f %8.0f\n", reng_fp8::name(fmt), m, shape.c_str(), t_fp8 * 1e3,
                        mb8, mb8 / 1e3 / t_fp8);
            std::printf("%-8s %6zu %10s %10.4f %10.0f %8.0f\n", "bf16", m, shape.c_str(), t_bf16 * 1e3, mb16,
                        mb16 / 1e3 / t_bf16);
            const double best = std::min(t_mixed, t_fp8);
            std::printf("  speedup bf16 -> fp8: %.2fx\n", t_bf16 / best);
            if (k == 4096 && n == 14336 && m == 1) {
                const double ratio = t_bf16 / best;
                char d[160];
                std::snprintf(d, sizeof d, "%.2fx bf16 -> %s against a %.2fx floor:", ratio, reng_fp8::name(fmt), floor);
                c.line("speedup-" + shape + "-m1", d, ratio >= floor);
            }
            (void)hipFree(da);
            (void)hipFree(dac);
            (void)hipFree(das);
            (void)hipFree(dy);
        }
        (void)hipFree(dw);
        (void)hipFree(dc);
        (void)hipFree(ds);
    }
    rocblas_destroy_handle(handle);
}

int run(int argc, char **argv) {
    std::vector<std::string> a(argv + 1, argv + argc);
    Fp8Format fmt = Fp8Format::E4M3;
    int iters = 20;
    double floor = DEFAULT_SPEEDUP_FLOOR;
    bool do_time = false, do_check = true;
    for (const auto &s : a) do_time |= s == "time";
    do_check = !do_time;
    for (const auto &s : a) do_check |= s == "check";
    for (size_t i = 0; i < a.size();) {
        if (a[i] == "--format") {
            if (i + 1 >= a.size()) throw Fail("--format needs a value");
            auto f = reng_fp8::format_from_name(a[i + 1]);
            if (!f) throw Fail("unknown format " + a[i + 1]);
            fmt = *f;
            i += 2;
        } else if (a[i] == "--iters") {
            if (i + 1 >= a.size()) throw Fail("--iters needs a value");
            iters = std::atoi(a[i + 1].c_str());
            if (iters <= 0) throw Fail("--iters: invalid digit found in string");
            i += 2;
        } else if (a[i] == "--min-speedup") {
            if (i + 1 >= a.size()) throw Fail("--min-speedup needs a value");
            char *end = nullptr;
            floor = std::strtod(a[i + 1].c_str(), &end);
            if (!end || *end) throw Fail("--min-speedup: invalid float literal");
            i += 2;
        } else {
            i += 1;
        }
    }
    Checks c;
    if (do_check) {
        const size_t k = 256, n = 512;
        const std::vector<uint16_t> w = weights(n, k);
        const Quantized q = reng_fp8::quantize(w, n, k, fmt, Scaling::PerChannel);
        const Quantized q_hw = reng_fp8::quantize(w, n, k, fmt, Scaling::HwExpBias);
        std::printf("weight [%zu, %zu] %s: %s exp_bias %u, %s exp_bias %u (scale %.3e)\n", n, k, reng_fp8::name(fmt),
                    reng_fp8::name(q.scaling), q.exp_bias, reng_fp8::name(q_hw.scaling), q_hw.exp_bias,
                    (double)q_hw.scales[0]);
        check_decode(c, fmt);
        check_cast(c, fmt);
        for (size_t m : {size_t(1), size_t(256)}) {
            check_mixed(c, q, m, k, n);
            check_gemm(c, q_hw, m, k, n, fmt);
            check_gemm_scaled(c, q, m, k, n, fmt);
        }
    }
    if (do_time) timings(c, iters, fmt, floor);
    if (c.failed > 0) throw Fail(std::to_string(c.failed) + " of " + std::to_string(c.ran) + " checks failed");
    if (c.ran == 0) throw Fail("nothing to do: pass `check`, `time` or both");
    std::printf("reng-fp8-probe: %d checks passed\n", c.ran);
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception &e) {
        std::fprintf(stderr, "Error: %s\n", e.what());
        return 1;
    }
}
