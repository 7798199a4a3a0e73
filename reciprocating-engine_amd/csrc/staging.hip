// staging.hip - the pipeline behind reng_hip_quantize_host: a bf16 / f32
// matrix in (pageable) host memory -> pinned chunks -> device -> quantize ->
// pinned chunks -> host codes, the path reng-fp8's host `quantize_with`
// (crates/reng-fp8/src/lib.rs:519-563) and reng-model's quantize pass
// (crates/reng-model/src/lib.rs:1882-1937) take when the weights live in host
// memory.
//
// A matrix moves in row chunks of about CHUNK bytes through NS pinned input and
// NS pinned output slots, one HIP stream per slot. Per chunk i (slot i % NS):
//   1. the calling thread and the input copy pool copy the rows into the
//      pinned input slot (once that slot's previous upload has read it);
//   2. the upload, the quantize of the chunk's rows and the download of its
//      codes into the pinned output slot are queued on the slot's stream;
//   3. the drainer thread waits for the download and copies the codes out to
//      the caller's buffer with the output copy pool, then frees the slot.
// So the host copies in, the PCIe uploads and downloads (both directions at
// once) and the host copies out of neighbouring chunks all overlap. The HW
// scheme needs the whole matrix's absmax before any code: every chunk goes up
// first, one quantize runs, then the chunks come down through the drainer.
//
// The pools and the drainer are started on the first call on a device and
// live, idle between calls, until the process ends (they are never joined, so
// no thread outlives the HIP runtime's teardown in a destructor).
#include <string.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "common.h"
#include "staging.h"

namespace reng {
namespace {

// Input bytes per chunk. 8 MB chunks of two Llama-3.1-8B layers (bf16) ran a
// pass in 24-25 ms against 32-40 ms for 4 MB ones (half the per-chunk hand-offs,
// and pieces big enough for every copy thread); 16 MB ones no faster, the
// drainer waiting longer for each download.
constexpr size_t CHUNK = (size_t)8 << 20;
constexpr int NS = 3;                        // pinned slots (and streams)

// Worker threads that run pieces of large memcpys. copy() splits a copy over
// the workers and the calling thread and returns when every piece is done.
class CopyPool {
  public:
    explicit CopyPool(int workers) {
        for (int i = 0; i < workers; ++i) th_.emplace_back([this] { run(); });
    }
    int workers() const { return (int)th_.size(); }

    void copy(void *dst, const void *src, size_t n) {
        constexpr size_t MIN_PIECE = (size_t)256 << 10;   // smaller pieces cost more hand-offs than they save
        const size_t parts = std::max<size_t>(1, std::min<size_t>(th_.size() + 1, n / MIN_PIECE));
        if (parts == 1) {
            memcpy(dst, src, n);
            return;
        }
        const size_t piece = (n + parts - 1) / parts;
        Group g;
        g.left = (int)parts - 1;
        {
            std::lock_guard<std::mutex> lk(mu_);
            for (size_t p = 1; p < parts; ++p) {
                const size_t a = p * piece, b = std::min(n, a + piece);
                q_.push_back(Piece{static_cast<char *>(dst) + a, static_cast<const char *>(src) + a, b - a, &g});
            }
        }
        cv_.notify_all();
        memcpy(dst, src, std::min(n, piece));
        std::unique_lock<std::mutex> lk(g.mu);
        g.cv.wait(lk, [&] { return g.left == 0; });
    }

  private:
    struct Group {
        std::mutex mu;
        std::condition_variable cv;
        int left = 0;
    };
    struct Piece {
        char *d;
        const char *s;
        size_t n;
        Group *g;
    };
    void run() {
        for (;;) {
            Piece p;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return !q_.empty(); });
                p = q_.front();
                q_.pop_front();
            }
            memcpy(p.d, p.s, p.n);
            std::lock_guard<std::mutex> lk(p.g->mu);
            if (--p.g->left == 0) p.g->cv.notify_all();
        }
    }
    std::mutex mu_;
    std::condition_variable cv_;
    std::deque<Piece> q_;
    std::vector<std::thread> th_;
};

// Copies downloaded chunks out of their pinned slots, in order, on its own
// thread: wait for the download's event, copy (with the output pool), free the slot.
class Drainer {
  public:
    explicit Drainer(CopyPool *pool) : pool_(pool) { th_ = std::thread([this] { run(); }); }

    void push(hipEvent_t ev, void *dst, const void *src, size_t n, int slot) {
        {
            std::lock_guard<std::mutex> lk(mu_);
            busy_[slot] = true;
            q_.push_back(Job{ev, dst, src, n, slot});
        }
        cv_.notify_all();
    }
    // Waits until slot's last copy-out is done (or everything, slot < 0).
    void wait(int slot) {
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] {
            if (slot >= 0) return !busy_[slot];
            for (bool b : busy_)
                if (b) return false;
            return true;
        });
    }
    // The first device error a copy-out saw since the last call (then cleared).
    hipError_t take_error() {
        std::lock_guard<std::mutex> lk(mu_);
        const hipError_t e = err_;
        err_ = hipSuccess;
        return e;
    }

  private:
    struct Job {
        hipEvent_t ev;
        void *dst;
        const void *src;
        size_t n;
        int slot;
    };
    void run() {
        for (;;) {
            Job j;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return !q_.empty(); });
                j = q_.front();
                q_.pop_front();
            }
            const hipError_t e = hipEventSynchronize(j.ev);
            if (e == hipSuccess) pool_->copy(j.dst, j.src, j.n);
            {
                std::lock_guard<std::mutex> lk(mu_);
                if (e != hipSuccess && err_ == hipSuccess) err_ = e;
                busy_[j.slot] = false;
            }
            done_cv_.notify_all();
        }
    }
    CopyPool *pool_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    std::deque<Job> q_;
    bool busy_[NS] = {};
    hipError_t err_ = hipSuccess;
    std::thread th_;
};

struct HostStage {
    std::mutex mu;   // one staged call per device at a time
    bool ready = false;
    hipStream_t st[NS] = {};
    hipEvent_t up[NS] = {};     // slot's pinned input has been read by its upload
    hipEvent_t down[NS] = {};   // slot's pinned output holds its chunk's codes
    hipEvent_t all_up = nullptr, quantized = nullptr;
    void *pin_in[NS] = {};
    void *pin_out[NS] = {};
    void *dw = nullptr;
    size_t dw_cap = 0;
    uint8_t *dc = nullptr;
    size_t dc_cap = 0;
    float *ds = nullptr;   // the rows' scales, then the exponent bias (one u32)
    size_t ds_cap = 0;
    CopyPool *in_pool = nullptr, *out_pool = nullptr;   // started once, never destroyed
    Drainer *drainer = nullptr;
};

HostStage &host_stage(int dev) {
    static std::mutex mu;
    static std::map<int, HostStage *> stages;   // kept until the process ends
    std::lock_guard<std::mutex> lk(mu);
    HostStage *&p = stages[dev];
    if (!p) p = new HostStage();
    return *p;
}

int grow(void **p, size_t *cap, size_t bytes) {
    if (*cap >= bytes) return RENG_HIP_OK;
    if (*p) RENG_CHECK_HIP(hipFree(*p));
    *p = nullptr;
    *cap = 0;
    RENG_CHECK_HIP(hipMalloc(p, bytes));
    *cap = bytes;
    return RENG_HIP_OK;
}

int stage_init(HostStage &S) {
    if (S.ready) return RENG_HIP_OK;
    for (int i = 0; i < NS; ++i) {
        if (!S.st[i]) RENG_CHECK_HIP(hipStreamCreateWithFlags(&S.st[i], hipStreamNonBlocking));
        if (!S.up[i]) RENG_CHECK_HIP(hipEventCreateWithFlags(&S.up[i], hipEventDisableTiming));
        if (!S.down[i]) RENG_CHECK_HIP(hipEventCreateWithFlags(&S.down[i], hipEventDisableTiming));
        if (!S.pin_in[i]) RENG_CHECK_HIP(hipHostMalloc(&S.pin_in[i], CHUNK, hipHostMallocDefault));
        if (!S.pin_out[i]) RENG_CHECK_HIP(hipHostMalloc(&S.pin_out[i], CHUNK, hipHostMallocDefault));
    }
    if (!S.all_up) RENG_CHECK_HIP(hipEventCreateWithFlags(&S.all_up, hipEventDisableTiming));
    if (!S.quantized) RENG_CHECK_HIP(hipEventCreateWithFlags(&S.quantized, hipEventDisableTiming));
    if (!S.in_pool) {
        // Copy-in carries twice (bf16) or four times (f32) the bytes of the
        // copy-out, but the copy-out writes into the caller's freshly
        // allocated pages, whose first-touch faults make it the slower
        // stream per byte (12 GB/s per thread against 25 for the copy-in on
        // an EPYC host), so both get several threads; the calling thread and
        // the drainer each copy a piece too.
        const unsigned hw = std::max(4u, std::thread::hardware_concurrency());
        const int in_workers = (int)std::min(5u, hw / 3), out_workers = (int)std::min(4u, hw / 4);
        S.in_pool = new CopyPool(in_workers);
        S.out_pool = new CopyPool(out_workers);
        S.drainer = new Drainer(S.out_pool);
    }
    S.ready = true;
    return RENG_HIP_OK;
}

// The staged quantize of one host matrix (arguments already checked).
int quantize_staged(HostStage &S, const void *w, int dtype, size_t rows, size_t cols, int format, int scaling,
                    float backoff, uint8_t *codes, float *scales, uint32_t *exp_bias) {
    if (int rc = stage_init(S)) return rc;
    const size_t esz = dtype == RENG_HIP_BF16 ? 2 : 4;
    const size_t row_bytes = cols * esz;
    if (int rc = grow(&S.dw, &S.dw_cap, rows * row_bytes)) return rc;
    if (int rc = grow(reinterpret_cast<void **>(&S.dc), &S.dc_cap, rows * cols)) return rc;
    if (int rc = grow(reinterpret_cast<void **>(&S.ds), &S.ds_cap, (rows + 1) * sizeof(float))) return rc;
    uint32_t *dbias = reinterpret_cast<uint32_t *>(S.ds + rows);
    const bool per_row = scaling != RENG_HIP_HW;   // PCS and UNIT quantize rows independently
    if (row_bytes > CHUNK) {
        // A single row larger than a pinned slot: unpipelined copies.
        RENG_CHECK_HIP(hipMemcpy(S.dw, w, rows * row_bytes, hipMemcpyHostToDevice));
        int rc = reng_hip_quantize(S.dw, dtype, rows, cols, cols, format, scaling, backoff, S.dc, S.ds, dbias,
                                   S.st[0]);
        if (rc) return rc;
        RENG_CHECK_HIP(hipStreamSynchronize(S.st[0]));
        RENG_CHECK_HIP(hipMemcpy(codes, S.dc, rows * cols, hipMemcpyDeviceToHost));
        RENG_CHECK_HIP(hipMemcpy(scales, S.ds, rows * sizeof(float), hipMemcpyDeviceToHost));
        if (exp_bias) RENG_CHECK_HIP(hipMemcpy(exp_bias, dbias, sizeof(uint32_t), hipMemcpyDeviceToHost));
        return RENG_HIP_OK;
    }
    const size_t rpc = std::max<size_t>(1, CHUNK / row_bytes);   // rows per chunk
    const size_t chunks = (rows + rpc - 1) / rpc;
    auto range = [&](size_t i, size_t &r0, size_t &nr) {
        r0 = i * rpc;
        nr = std::min(rpc, rows - r0);
    };
    // Chunk i's codes: downloaded into slot i % NS once its previous
    // copy-out is done, then handed to the drainer.
    auto download = [&](size_t i) -> int {
        size_t r0, nr;
        range(i, r0, nr);
        const int k = (int)(i % NS);
        S.drainer->wait(k);
        RENG_CHECK_HIP(hipMemcpyAsync(S.pin_out[k], S.dc + r0 * cols, nr * cols, hipMemcpyDeviceToHost, S.st[k]));
        RENG_CHECK_HIP(hipEventRecord(S.down[k], S.st[k]));
        S.drainer->push(S.down[k], codes + r0 * cols, S.pin_out[k], nr * cols, k);
        return RENG_HIP_OK;
    };
    for (size_t i = 0; i < chunks; ++i) {
        size_t r0, nr;
        range(i, r0, nr);
        const int k = (int)(i % NS);
        if (i >= NS) RENG_CHECK_HIP(hipEventSynchronize(S.up[k]));   // the slot's pinned input is free
        S.in_pool->copy(S.pin_in[k], static_cast<const char *>(w) + r0 * row_bytes, nr * row_bytes);
        char *dst = static_cast<char *>(S.dw) + r0 * row_bytes;
        RENG_CHECK_HIP(hipMemcpyAsync(dst, S.pin_in[k], nr * row_bytes, hipMemcpyHostToDevice, S.st[k]));
        RENG_CHECK_HIP(hipEventRecord(S.up[k], S.st[k]));
        if (per_row) {
            int rc = reng_hip_quantize(dst, dtype, nr, cols, cols, format, scaling, backoff, S.dc + r0 * cols,
                                       S.ds + r0, nullptr, S.st[k]);
            if (rc) return rc;
            if ((rc = download(i))) return rc;
        }
    }
    if (!per_row) {
        // HW: one exponent bias from the whole matrix, so every chunk is on the
        // device before the quantize; then the chunks come down through the slots.
        for (int k = 1; k < NS; ++k) {
            RENG_CHECK_HIP(hipEventRecord(S.all_up, S.st[k]));
            RENG_CHECK_HIP(hipStreamWaitEvent(S.st[0], S.all_up, 0));
        }
        int rc = reng_hip_quantize(S.dw, dtype, rows, cols, cols, format, scaling, backoff, S.dc, S.ds, dbias,
                                   S.st[0]);
        if (rc) return rc;
        RENG_CHECK_HIP(hipEventRecord(S.quantized, S.st[0]));
        for (int k = 1; k < NS; ++k) RENG_CHECK_HIP(hipStreamWaitEvent(S.st[k], S.quantized, 0));
        for (size_t i = 0; i < chunks; ++i)
            if ((rc = download(i))) return rc;
    }
    // The scales (and the bias) ride behind the last chunk's quantize on every stream.
    for (int k = 0; k < NS; ++k) RENG_CHECK_HIP(hipStreamSynchronize(S.st[k]));
    RENG_CHECK_HIP(hipMemcpy(scales, S.ds, rows * sizeof(float), hipMemcpyDeviceToHost));
    if (exp_bias) {
        if (per_row) *exp_bias = format == RENG_HIP_E4M3 ? 7u : 15u;   // the format's own bias (lib.rs:544, 550)
        else RENG_CHECK_HIP(hipMemcpy(exp_bias, dbias, sizeof(uint32_t), hipMemcpyDeviceToHost));
    }
    S.drainer->wait(-1);
    const hipError_t de = S.drainer->take_error();
    if (de != hipSuccess) {
        set_error("copying codes out of a staging slot: %s", hipGetErrorString(de));
        return RENG_HIP_EDEVICE;
    }
    return RENG_HIP_OK;
}

}  // namespace

int quantize_host_staged(const void *w, int dtype, size_t rows, size_t cols, int format, int scaling, float backoff,
                         uint8_t *codes, float *scales, uint32_t *exp_bias) {
    int dev = 0;
    RENG_CHECK_HIP(hipGetDevice(&dev));
    HostStage &S = host_stage(dev);
    std::lock_guard<std::mutex> lk(S.mu);
    const int rc = quantize_staged(S, w, dtype, rows, cols, format, scaling, backoff, codes, scales, exp_bias);
    if (rc && S.ready) {
        // Nothing may still write the caller's buffers once the call returns:
        // let the queued work and the copy-outs finish, then forget their errors.
        for (int k = 0; k < NS; ++k) (void)hipStreamSynchronize(S.st[k]);
        S.drainer->wait(-1);
        (void)S.drainer->take_error();
    }
    return rc;
}

}  // namespace reng
