// runtime.hip -- device selection, memory and streams for libtrs_hip.so.
//
// Replaces the reference's storage/device layer (src/storage.rs:7-18,
// src/device.rs:5-9), which only knows a CPU Vec<f32>: here storage is HBM
// owned by the caller through trs_alloc/trs_free, and all work is ordered on
// one stream per device.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>

#include "trs_internal.h"

namespace trs {

namespace {

thread_local char g_last_error[1024];
thread_local int g_device = 0;

constexpr int kMaxDevices = 16;
// Never destroyed: tensors released during interpreter shutdown may still
// return blocks to the cache after static destructors would have run.
DeviceState *const g_devices = new DeviceState[kMaxDevices];
std::mutex g_init_mu;
int g_device_count = -1;

__global__ void __launch_bounds__(kHelperLanes) fill_u32_kernel(uint32_t *dst, size_t n, uint32_t value) {
    const size_t stride = (size_t)gridDim.x * kHelperLanes;
    for (size_t i = (size_t)blockIdx.x * kHelperLanes + threadIdx.x; i < n; i += stride) dst[i] = value;
}

__global__ void __launch_bounds__(kHelperLanes) fill_u8_kernel(uint8_t *dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * kHelperLanes;
    for (size_t i = (size_t)blockIdx.x * kHelperLanes + threadIdx.x; i < n; i += stride) dst[i] = 0;
}

int count_devices() {
    std::lock_guard<std::mutex> lock(g_init_mu);
    if (g_device_count < 0) {
        int n = 0;
        hipError_t e = hipGetDeviceCount(&n);
        if (e != hipSuccess) {
            g_device_count = 0;
            return set_error(TRS_E_NO_DEVICE, "hipGetDeviceCount failed: %s", hipGetErrorString(e));
        }
        g_device_count = n < kMaxDevices ? n : kMaxDevices;
    }
    return TRS_OK;
}

// Block sizes: 512 B granules below 1 MiB, 2 MiB granules above (HBM pages).
size_t round_block(size_t bytes) {
    const size_t g = bytes < (1u << 20) ? 512 : (2u << 20);
    return (bytes + g - 1) / g * g;
}

// Returns every cached block to HIP after the device stream has drained.
int release_cache(DeviceState *dev) {
    std::multimap<size_t, void *> blocks;
    {
        std::lock_guard<std::mutex> lock(dev->cache_mu);
        blocks.swap(dev->free_blocks);
        dev->cached_bytes = 0;
    }
    if (blocks.empty()) return TRS_OK;
    TRS_HIP_CHECK(hipStreamSynchronize(dev->stream), "cache release sync");
    for (auto &kv : blocks) TRS_HIP_CHECK(hipFree(kv.second), "hipFree");
    return TRS_OK;
}

}  // namespace

int set_error(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    std::memcpy(g_last_error, buf, sizeof buf);
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return set_error(TRS_E_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

int check_layout(const trs_layout *l, const char *what) {
    if (l == nullptr) return set_error(TRS_E_INVALID_ARGUMENT, "%s layout is null", what);
    if (l->rank < 0 || l->rank > TRS_MAX_RANK)
        return set_error(TRS_E_INVALID_ARGUMENT, "%s rank %d outside [0, %d]", what, l->rank, TRS_MAX_RANK);
    if (l->offset < 0) return set_error(TRS_E_INVALID_ARGUMENT, "%s offset is negative", what);
    int64_t numel = 1;
    for (int d = 0; d < l->rank; d++) {
        if (l->shape[d] < 0 || l->stride[d] < 0)
            return set_error(TRS_E_INVALID_ARGUMENT, "%s dim %d has a negative size or stride", what, d);
        if (__builtin_mul_overflow(numel, l->shape[d], &numel))
            return set_error(TRS_E_INDEX_OVERFLOW, "%s element count overflows 64 bits", what);
    }
    if (numel == 0) return TRS_OK;  // nothing is addressed
    // The last element's offset, and its byte offset, must fit in 64 bits
    // (IndexCalculationOverflow, src/tensor.rs:3815-3841).
    int64_t last = l->offset;
    for (int d = 0; d < l->rank; d++) {
        int64_t step;
        if (__builtin_mul_overflow(l->shape[d] - 1, l->stride[d], &step) || __builtin_add_overflow(last, step, &last))
            return set_error(TRS_E_INDEX_OVERFLOW, "%s offsets overflow 64 bits", what);
    }
    if (last > (INT64_MAX >> 3)) return set_error(TRS_E_INDEX_OVERFLOW, "%s byte offsets overflow 64 bits", what);
    return TRS_OK;
}

int64_t layout_numel(const trs_layout *l) {
    int64_t n = 1;
    for (int d = 0; d < l->rank; d++) n *= l->shape[d];
    return n;
}

bool layout_is_contiguous(const trs_layout *l) {
    if (layout_numel(l) == 0) return true;
    int64_t expected = 1;
    for (int d = l->rank - 1; d >= 0; d--) {
        if (l->shape[d] == 1) continue;
        if (l->stride[d] != expected) return false;
        expected *= l->shape[d];
    }
    return true;
}

void merge_layout_dims(const trs_layout *in, trs_layout *out) {
    trs_layout m{};
    m.offset = in->offset;
    int r = 0;
    for (int d = 0; d < in->rank; d++) {
        if (in->shape[d] == 1) continue;
        if (r > 0 && m.stride[r - 1] == in->stride[d] * in->shape[d]) {
            m.shape[r - 1] *= in->shape[d];
            m.stride[r - 1] = in->stride[d];
            continue;
        }
        m.shape[r] = in->shape[d];
        m.stride[r] = in->stride[d];
        r++;
    }
    if (r == 0) {
        m.shape[0] = 1;
        m.stride[0] = 1;
        r = 1;
    }
    m.rank = r;
    *out = m;
}

DeviceState *device_state() {
    if (count_devices() != TRS_OK) return nullptr;
    if (g_device_count == 0) {
        set_error(TRS_E_NO_DEVICE, "no HIP device is visible");
        return nullptr;
    }
    if (g_device < 0 || g_device >= g_device_count) {
        set_error(TRS_E_INVALID_ARGUMENT, "device %d out of range", g_device);
        return nullptr;
    }
    DeviceState *dev = &g_devices[g_device];
    std::lock_guard<std::mutex> lock(dev->mu);
    if (dev->ready) {
        if (hipSetDevice(g_device) != hipSuccess) {
            set_error(TRS_E_HIP, "hipSetDevice(%d) failed", g_device);
            return nullptr;
        }
        return dev;
    }
    hipError_t e = hipSetDevice(g_device);
    if (e != hipSuccess) {
        hip_fail(e, "hipSetDevice");
        return nullptr;
    }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, g_device);
    if (e != hipSuccess) {
        hip_fail(e, "hipGetDeviceProperties");
        return nullptr;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error(TRS_E_NO_DEVICE, "device %d is %s; this library is built for gfx950 only", g_device,
                  prop.gcnArchName);
        return nullptr;
    }
    // Default-priority stream (never a prioritised one).
    e = hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        hip_fail(e, "hipStreamCreate");
        return nullptr;
    }
    dev->index = g_device;
    dev->cu_count = prop.multiProcessorCount;
    dev->clock_khz = prop.clockRate;
    std::snprintf(dev->name, sizeof dev->name, "%s (%s)", prop.name[0] ? prop.name : "AMD GPU", prop.gcnArchName);
    setup_sum_scratch(dev);
    dev->ready = true;
    return dev;
}

}  // namespace trs

using namespace trs;

namespace trs {
// Allocations trs_alloc grants before it refuses every one (-1: no limit).
std::atomic<int64_t> g_allocs_before_failure{-1};
std::atomic<int64_t> g_pw_grid_cap{0};
}  // namespace trs

extern "C" {

const char *trs_last_error(void) { return g_last_error; }

int trs_init(void) {
    return abi_guard([&]() -> int {
        DeviceState *dev = device_state();
        return dev ? TRS_OK : TRS_E_NO_DEVICE;
    });
}

int trs_device_count(int *count) {
    if (!count) return set_error(TRS_E_INVALID_ARGUMENT, "null count");
    int rc = count_devices();
    *count = g_device_count < 0 ? 0 : g_device_count;
    return rc;
}

int trs_set_device(int device) {
    return abi_guard([&]() -> int {
        int rc = count_devices();
        if (rc) return rc;
        if (device < 0 || device >= g_device_count)
            return set_error(TRS_E_INVALID_ARGUMENT, "device %d out of range [0, %d)", device, g_device_count);
        g_device = device;
        return device_state() ? TRS_OK : TRS_E_HIP;
    });
}

int trs_get_device(int *device) {
    if (!device) return set_error(TRS_E_INVALID_ARGUMENT, "null device");
    *device = g_device;
    return TRS_OK;
}

int trs_device_info(char *name, size_t name_len, int *cu_count, int *clock_khz) {
    return abi_guard([&]() -> int {
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        if (name && name_len) std::snprintf(name, name_len, "%s", dev->name);
        if (cu_count) *cu_count = dev->cu_count;
        if (clock_khz) *clock_khz = dev->clock_khz;
        return TRS_OK;
    });
}

int trs_debug_fail_allocs_after(int64_t n) {
    trs::g_allocs_before_failure.store(n < 0 ? -1 : n);
    return TRS_OK;
}

int trs_debug_pointwise_grid_cap(int64_t blocks) {
    if (blocks < 0) return set_error(TRS_E_INVALID_ARGUMENT, "negative grid cap");
    trs::g_pw_grid_cap.store(blocks);
    return TRS_OK;
}

int trs_alloc(size_t bytes, void **ptr) {
    return abi_guard([&]() -> int {
        if (!ptr) return set_error(TRS_E_INVALID_ARGUMENT, "null out pointer");
        *ptr = nullptr;
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        if (bytes == 0) return TRS_OK;
        // The test hook (trs_debug_fail_allocs_after): count down, then refuse.
        for (int64_t left = trs::g_allocs_before_failure.load(); left >= 0;) {
            if (left == 0)
                return set_error(TRS_E_ALLOCATION_FAILED, "allocation refused (trs_debug_fail_allocs_after)");
            if (trs::g_allocs_before_failure.compare_exchange_weak(left, left - 1)) break;
        }
        const size_t rounded = round_block(bytes);
        {
            std::lock_guard<std::mutex> lock(dev->cache_mu);
            auto it = dev->free_blocks.find(rounded);
            if (it != dev->free_blocks.end()) {
                *ptr = it->second;
                dev->free_blocks.erase(it);
                dev->cached_bytes -= rounded;
                dev->live_blocks[*ptr] = rounded;
                return TRS_OK;
            }
        }
        hipError_t e = hipMalloc(ptr, rounded);
        if (e != hipSuccess) {
            // Out of memory with blocks parked in the cache: release them and retry once.
            (void)hipGetLastError();
            int rc = release_cache(dev);
            if (rc) return rc;
            e = hipMalloc(ptr, rounded);
        }
        if (e != hipSuccess) {
            *ptr = nullptr;
            (void)hipGetLastError();
            return set_error(TRS_E_ALLOCATION_FAILED, "hipMalloc of %zu bytes failed: %s", bytes,
                             hipGetErrorString(e));
        }
        std::lock_guard<std::mutex> lock(dev->cache_mu);
        dev->live_blocks[*ptr] = rounded;
        return TRS_OK;
    });
}

int trs_free(void *ptr) {
    return abi_guard([&]() -> int {
        if (!ptr) return TRS_OK;
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        {
            std::lock_guard<std::mutex> lock(dev->cache_mu);
            auto it = dev->live_blocks.find(ptr);
            if (it != dev->live_blocks.end()) {
                // Stream-ordered release: work already queued on the device
                // stream may still read the block; anything that reuses it is
                // queued behind that work.
                dev->free_blocks.emplace(it->second, ptr);
                dev->cached_bytes += it->second;
                dev->live_blocks.erase(it);
                return TRS_OK;
            }
        }
        // Not a block of this cache: drain queued readers, then hand it back.
        TRS_HIP_CHECK(hipStreamSynchronize(dev->stream), "free sync");
        TRS_HIP_CHECK(hipFree(ptr), "hipFree");
        return TRS_OK;
    });
}

int trs_empty_cache(void) {
    return abi_guard([&]() -> int {
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        return release_cache(dev);
    });
}

int trs_memory_stats(size_t *live_bytes, size_t *cached_bytes) {
    return abi_guard([&]() -> int {
        DeviceState *dev = device_state();
        if (!dev) return TRS_E_NO_DEVICE;
        std::lock_guard<std::mutex> lock(dev->cache_mu);
        size_t live = 0;
        for (auto &kv : dev->live_blocks) live += kv.second;
        if (live_bytes) *live_bytes = live;
        if (cached_bytes) *cached_bytes = dev->cached_bytes;
        return TRS_OK;
    });
}

int trs_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    if (bytes == 0) return TRS_OK;
    if (!dst || !src) return set_error(TRS_E_INVALID_ARGUMENT, "null pointer in d2d copy");
    TRS_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, dev->stream), "d2d copy");
    return TRS_OK;
}

int trs_memset_zero(void *dst, size_t bytes) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    if (bytes == 0) return TRS_OK;
    if (!dst) return set_error(TRS_E_INVALID_ARGUMENT, "null pointer in memset");
    const int64_t want = (int64_t)dev->cu_count * 8;
    if (bytes % 4 == 0 && ((uintptr_t)dst % 4) == 0) {
        const size_t n = bytes / 4;
        const int64_t grid = std::min<int64_t>(std::max<int64_t>(1, (int64_t)((n + 255) / 256)), want);
        hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)grid), dim3(kHelperLanes), 0, dev->stream,
                           (uint32_t *)dst, n, 0u);
    } else {
        const int64_t grid = std::min<int64_t>(std::max<int64_t>(1, (int64_t)((bytes + 255) / 256)), want);
        hipLaunchKernelGGL(fill_u8_kernel, dim3((unsigned)grid), dim3(kHelperLanes), 0, dev->stream,
                           (uint8_t *)dst, bytes);
    }
    TRS_LAUNCH_CHECK("memset kernel");
    return TRS_OK;
}

int trs_synchronize(void) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    TRS_HIP_CHECK(hipStreamSynchronize(dev->stream), "synchronize");
    return TRS_OK;
}

int trs_stream(void **stream) {
    if (!stream) return set_error(TRS_E_INVALID_ARGUMENT, "null stream out pointer");
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    *stream = (void *)dev->stream;
    return TRS_OK;
}

}  // extern "C"
