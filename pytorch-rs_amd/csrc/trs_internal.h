// trs_internal.h -- host-side internals shared by the libtrs_hip.so sources.
#pragma once

#include <atomic>
#include <exception>
#include <new>

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <map>
#include <mutex>
#include <unordered_map>

#include "trs_hip.h"

namespace trs {

// Pointwise grid cap set by trs_debug_pointwise_grid_cap (0: kMaxGrid).
extern std::atomic<int64_t> g_pw_grid_cap;

// Lanes per block of the one-dimensional helper kernels (fills, slice and
// split-K sums, the per-element reduction).  Their bodies index with this
// constant rather than blockDim: reading blockDim costs each wave a memory
// load and a wait before its first load, one more memory latency in a pass
// whose time is load latency.
constexpr int kHelperLanes = 256;

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
    // Device address of this device's copy of the sum's static scratch array
    // (pointwise.hip), looked up once at set-up; null if the lookup failed,
    // with the failure's message kept for trs_sum_f32_noalloc to report.
    float *sum_scratch = nullptr;
    char sum_scratch_error[160] = {0};
};

// Looks up the device address of the static sum scratch array for `dev`
// (the device must be current); called once per device at set-up.
void setup_sum_scratch(DeviceState *dev);

// Returns the current device's state, initialising it on first use.
// On failure returns nullptr with the error recorded.
DeviceState *device_state();


// Records a thread-local error message and returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));

// Runs an entry point's body and turns any C++ exception (a failed host
// allocation in a container, a thread that cannot start) into an error code,
// so that none crosses the C ABI.
template <class Fn>
int abi_guard(Fn &&fn) noexcept {
    try {
        return fn();
    } catch (const std::bad_alloc &) {
        return set_error(TRS_E_ALLOCATION_FAILED, "host memory allocation failed");
    } catch (const std::exception &e) {
        return set_error(TRS_E_INVALID_ARGUMENT, "internal error: %s", e.what());
    } catch (...) {
        return set_error(TRS_E_INVALID_ARGUMENT, "internal error");
    }
}
// Maps a HIP failure to TRS_E_HIP with the runtime's message.
int hip_fail(hipError_t e, const char *what);

// Validates rank (0..TRS_MAX_RANK), non-negative shape/stride/offset.
int check_layout(const trs_layout *l, const char *what);
int64_t layout_numel(const trs_layout *l);
bool layout_is_contiguous(const trs_layout *l);
// Drops size-1 dims and merges each dim into its inner neighbour where
// stride[d] == stride[d+1] * shape[d+1]: the same elements in the same
// row-major order, in as few dims as the view allows (at least one).
void merge_layout_dims(const trs_layout *in, trs_layout *out);

// Contiguous layout of `l`'s shape (for gradients, which are logical-order).
inline trs_layout contiguous_like(const trs_layout *l) {
    trs_layout c{};
    c.rank = l->rank;
    int64_t s = 1;
    for (int d = l->rank - 1; d >= 0; d--) {
        c.shape[d] = l->shape[d];
        c.stride[d] = s;
        s *= l->shape[d];
    }
    c.offset = 0;
    return c;
}

// The bytes a non-empty view can touch: [begin, end) from its base pointer.
struct ByteRange {
    uintptr_t begin = 0, end = 0;
};
inline ByteRange byte_range(const void *base, const trs_layout *l, int elem_bytes) {
    int64_t last = l->offset;
    for (int d = 0; d < l->rank; d++) last += (l->shape[d] - 1) * l->stride[d];
    const uintptr_t b = (uintptr_t)base;
    return ByteRange{b + (uintptr_t)(l->offset * elem_bytes), b + (uintptr_t)((last + 1) * elem_bytes)};
}
inline bool ranges_overlap(const ByteRange &a, const ByteRange &b) { return a.begin < b.end && b.begin < a.end; }
// Same rank, shape and strides (the offsets are compared as byte addresses).
inline bool same_view_shape(const trs_layout *a, const trs_layout *b) {
    if (a->rank != b->rank) return false;
    for (int d = 0; d < a->rank; d++)
        if (a->shape[d] != b->shape[d] || a->stride[d] != b->stride[d]) return false;
    return true;
}

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
