// trs_internal.h -- host-side internals shared by the libtrs_hip.so sources.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <map>
#include <mutex>
#include <unordered_map>

#include "trs_hip.h"

namespace trs {

// Per-device state: one in-order stream carries every entry point's work, so
// stream order gives the reference's eager semantics.
struct DeviceState {
    int index = -1;
    bool ready = false;
    hipStream_t stream = nullptr;
    int cu_count = 0;
    int clock_khz = 0;
    char name[256] = {0};
    std::mutex mu;
    // Block cache behind trs_alloc/trs_free: freed blocks are kept by rounded
    // size and handed out again without a hipFree/hipMalloc pair.  Reuse is
    // safe without a sync because every kernel and copy of this library runs
    // in order on `stream`.
    std::mutex cache_mu;
    std::multimap<size_t, void *> free_blocks;
    std::unordered_map<void *, size_t> live_blocks;
    size_t cached_bytes = 0;
    // Two page-locked chunks that pipeline copies from or to pageable host
    // memory, each with the event of the last DMA that used it.
    std::mutex stage_mu;
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t stage_done[2] = {nullptr, nullptr};
};

// Returns the current device's state, initialising it on first use.
// On failure returns nullptr with the error recorded.
DeviceState *device_state();


// Records a thread-local error message and returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a HIP failure to TRS_E_HIP with the runtime's message.
int hip_fail(hipError_t e, const char *what);

// Validates rank (0..8), non-negative shape/stride/offset.
int check_layout(const trs_layout *l, const char *what);
int64_t layout_numel(const trs_layout *l);
bool layout_is_contiguous(const trs_layout *l);

#define TRS_HIP_CHECK(expr, what)                 \
    do {                                          \
        hipError_t trs_e_ = (expr);               \
        if (trs_e_ != hipSuccess) return ::trs::hip_fail(trs_e_, what); \
    } while (0)

// Returns a non-OK status of a call of this library to the caller.
#define TRS_CHECK(expr)               \
    do {                              \
        const int trs_rc_ = (expr);   \
        if (trs_rc_ != TRS_OK) return trs_rc_; \
    } while (0)

// A launch's error surfaces from hipGetLastError right after the launch.
#define TRS_LAUNCH_CHECK(what) TRS_HIP_CHECK(hipGetLastError(), what)

}  // namespace trs
