// lds_dma.h -- loading global memory straight into LDS
// (global_load_lds_dwordx4), shared by the GEMM and skinny-product kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace trs {

typedef __attribute__((address_space(3))) float lds_float;

// The LDS byte address of a __shared__ float.
__device__ __forceinline__ uint32_t lds_address(const float *p) { return (uint32_t)(uintptr_t)(const lds_float *)p; }

// 16 bytes per lane from sbase + voff (bytes) to LDS at m0 + 16 * lane: a
// wave's instruction fills one contiguous KiB of LDS, with no registers in
// between.  sbase must be wave-uniform.  The address needs only dword
// alignment (a probe on the box read every float right at each of the four
// float offsets within 16 bytes).  As asm the compiler adds no waits of its
// own around it: it cannot tell these LDS bytes from the ones being read, and
// through its builtin it waited for the loads before every LDS read.  Callers
// wait for the loads themselves (s_waitcnt vmcnt) before the barrier that
// makes them visible to the other waves.
__device__ __forceinline__ void lds_dma16(const float *sbase, uint32_t voff, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(m0)
                 : "memory", "m0");
}

// s_waitcnt immediate that waits until at most `n` vector-memory operations
// of this wave are outstanding (n < 64), leaving the other counters alone.
constexpr int vmcnt_at_most(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

}  // namespace trs
