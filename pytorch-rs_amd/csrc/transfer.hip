// transfer.hip -- host <-> device copies for libtrs_hip.so.
//
// Ingest and egress of whole buffers (the reference converts Python buffers
// element by element, src/python.rs:10329-10403, and egresses through Python
// lists, :4031-4052).  Page-locked memory from trs_host_alloc goes straight to
// the DMA engine.  Large copies from or to pageable memory are pipelined
// through two page-locked chunks per device: while the DMA engine moves one
// chunk over PCIe, host threads copy the next one between the caller's pages
// and the other chunk.  One host thread copies ~30 GB/s between cold pages,
// about half the PCIe rate, so the host side is split over a small pool.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "trs_internal.h"

namespace trs {

namespace {

constexpr size_t kStageChunk = 16u << 20;  // bytes per page-locked chunk
// Smaller copies go direct.  The runtime's own pageable path runs ~35 GB/s
// host-to-device but ~18 GB/s device-to-host, so egress is staged earlier.
constexpr size_t kStageMinH2D = 16u << 20;
constexpr size_t kStageMinD2H = 4u << 20;
constexpr size_t kSplitMin = 1u << 20;     // smallest share of one copy thread

// Pipeline step for a copy of `bytes`: at least four steps, so the host copy
// and the DMA overlap for most of the copy, and at most one chunk.
size_t stage_step(size_t bytes) {
    const size_t quarter = ((bytes + 3) / 4 + 65535) & ~(size_t)65535;
    return std::max<size_t>(1u << 20, std::min(kStageChunk, quarter));
}

// Splits a host memcpy over a fixed set of worker threads.  One copy runs at
// a time; a second caller waits for the pool.  The pool lives until the
// process ends (never destroyed, so no thread is joined during exit).
class CopyPool {
public:
    explicit CopyPool(int threads) : threads_(std::max(threads, 1)) {
        for (int i = 1; i < threads_; i++) std::thread([this, i] { worker(i); }).detach();
    }

    void copy(void *dst, const void *src, size_t bytes) {
        const int parts = (int)std::min<size_t>((size_t)threads_, std::max<size_t>(bytes / kSplitMin, 1));
        if (parts == 1) {
            std::memcpy(dst, src, bytes);
            return;
        }
        std::lock_guard<std::mutex> call(call_mu_);
        {
            std::lock_guard<std::mutex> lock(mu_);
            dst_ = (char *)dst;
            src_ = (const char *)src;
            bytes_ = bytes;
            parts_ = parts;
            pending_ = parts - 1;
            gen_++;
        }
        work_cv_.notify_all();
        part(0);
        std::unique_lock<std::mutex> lock(mu_);
        done_cv_.wait(lock, [this] { return pending_ == 0; });
    }

private:
    // Part i of the current job: 4 KiB-aligned slices of nearly equal size.
    void part(int i) {
        const size_t per = (bytes_ / parts_ + 4095) & ~(size_t)4095;
        const size_t lo = std::min(bytes_, per * (size_t)i);
        const size_t hi = i + 1 == parts_ ? bytes_ : std::min(bytes_, lo + per);
        if (hi > lo) std::memcpy(dst_ + lo, src_ + lo, hi - lo);
    }

    void worker(int i) {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lock(mu_);
                work_cv_.wait(lock, [&] { return gen_ != seen; });
                seen = gen_;
                if (i >= parts_) continue;
            }
            part(i);
            std::lock_guard<std::mutex> lock(mu_);
            if (--pending_ == 0) done_cv_.notify_one();
        }
    }

    const int threads_;
    std::mutex call_mu_, mu_;
    std::condition_variable work_cv_, done_cv_;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t bytes_ = 0;
    int parts_ = 1, pending_ = 0;
    uint64_t gen_ = 0;
};

// TRS_COPY_THREADS overrides the pool size (default: 8, or fewer cores).
CopyPool &copy_pool() {
    static CopyPool *pool = [] {
        int n = (int)std::min(8u, std::max(1u, std::thread::hardware_concurrency()));
        if (const char *env = std::getenv("TRS_COPY_THREADS")) n = std::max(1, std::min(64, std::atoi(env)));
        return new CopyPool(n);
    }();
    return *pool;
}

// True when `p` lies in page-locked memory the runtime knows (hipHostMalloc).
bool is_page_locked(const void *p) {
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeHost;
}

// Allocates the device's two staging chunks on first use; `dev->stage_mu`
// is held by the caller.
int ensure_staging(DeviceState *dev) {
    if (dev->stage[0]) return TRS_OK;
    for (int s = 0; s < 2; s++) {
        TRS_HIP_CHECK(hipHostMalloc(&dev->stage[s], kStageChunk, hipHostMallocDefault), "staging hipHostMalloc");
        TRS_HIP_CHECK(hipEventCreateWithFlags(&dev->stage_done[s], hipEventDisableTiming), "staging event");
    }
    return TRS_OK;
}

int staged_h2d(DeviceState *dev, char *dst, const char *src, size_t bytes) {
    std::lock_guard<std::mutex> lock(dev->stage_mu);
    TRS_CHECK(ensure_staging(dev));
    CopyPool &pool = copy_pool();
    const size_t step = stage_step(bytes);
    int slot = 0;
    for (size_t off = 0; off < bytes; off += step, slot ^= 1) {
        const size_t len = std::min(step, bytes - off);
        // The DMA that last read this chunk must be done before it is refilled.
        TRS_HIP_CHECK(hipEventSynchronize(dev->stage_done[slot]), "staging wait");
        pool.copy(dev->stage[slot], src + off, len);
        TRS_HIP_CHECK(hipMemcpyAsync(dst + off, dev->stage[slot], len, hipMemcpyHostToDevice, dev->stream), "h2d chunk");
        TRS_HIP_CHECK(hipEventRecord(dev->stage_done[slot], dev->stream), "staging record");
    }
    TRS_HIP_CHECK(hipStreamSynchronize(dev->stream), "h2d sync");
    return TRS_OK;
}

int staged_d2h(DeviceState *dev, char *dst, const char *src, size_t bytes) {
    std::lock_guard<std::mutex> lock(dev->stage_mu);
    TRS_CHECK(ensure_staging(dev));
    CopyPool &pool = copy_pool();
    const size_t step = stage_step(bytes);
    const size_t chunks = (bytes + step - 1) / step;
    auto issue = [&](size_t c) -> int {
        const size_t off = c * step, len = std::min(step, bytes - off);
        TRS_HIP_CHECK(hipMemcpyAsync(dev->stage[c & 1], src + off, len, hipMemcpyDeviceToHost, dev->stream), "d2h chunk");
        TRS_HIP_CHECK(hipEventRecord(dev->stage_done[c & 1], dev->stream), "staging record");
        return TRS_OK;
    };
    TRS_CHECK(issue(0));
    for (size_t c = 0; c < chunks; c++) {
        // Chunk c+1 reuses the buffer of chunk c-1, already copied out below.
        if (c + 1 < chunks) TRS_CHECK(issue(c + 1));
        TRS_HIP_CHECK(hipEventSynchronize(dev->stage_done[c & 1]), "staging wait");
        const size_t off = c * step;
        pool.copy(dst + off, dev->stage[c & 1], std::min(step, bytes - off));
    }
    return TRS_OK;
}

}  // namespace

}  // namespace trs

using namespace trs;

extern "C" {

int trs_host_alloc(size_t bytes, void **ptr) {
    return abi_guard([&]() -> int {
        if (!ptr) return set_error(TRS_E_INVALID_ARGUMENT, "null out pointer");
        *ptr = nullptr;
        if (bytes == 0) return TRS_OK;
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        hipError_t e = hipHostMalloc(ptr, bytes, hipHostMallocDefault);
        if (e != hipSuccess) {
            *ptr = nullptr;
            (void)hipGetLastError();
            return set_error(TRS_E_ALLOCATION_FAILED, "hipHostMalloc of %zu bytes failed: %s", bytes, hipGetErrorString(e));
        }
        return TRS_OK;
    });
}

int trs_host_free(void *ptr) {
    return abi_guard([&]() -> int {
        if (!ptr) return TRS_OK;
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        // Copies queued from or to this buffer must finish before it is released.
        TRS_HIP_CHECK(hipStreamSynchronize(dev->stream), "host free sync");
        TRS_HIP_CHECK(hipHostFree(ptr), "hipHostFree");
        return TRS_OK;
    });
}

int trs_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    return abi_guard([&]() -> int {
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        if (bytes == 0) return TRS_OK;
        if (!dst || !src) return set_error(TRS_E_INVALID_ARGUMENT, "null pointer in h2d copy");
        if (bytes >= kStageMinH2D && !is_page_locked(src)) return staged_h2d(dev, (char *)dst, (const char *)src, bytes);
        // Small or page-locked: one DMA.  Returning after the sync means `src`
        // has been consumed and may be reused by the caller.
        TRS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream), "h2d copy");
        TRS_HIP_CHECK(hipStreamSynchronize(dev->stream), "h2d sync");
        return TRS_OK;
    });
}

int trs_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    return abi_guard([&]() -> int {
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        if (bytes == 0) return TRS_OK;
        if (!dst || !src) return set_error(TRS_E_INVALID_ARGUMENT, "null pointer in d2h copy");
        if (bytes >= kStageMinD2H && !is_page_locked(dst)) return staged_d2h(dev, (char *)dst, (const char *)src, bytes);
        TRS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, dev->stream), "d2h copy");
        TRS_HIP_CHECK(hipStreamSynchronize(dev->stream), "d2h sync");
        return TRS_OK;
    });
}

}  // extern "C"
