// pw_ops.h -- the ahead-of-time pointwise ops: functors with the reference's
// scalar semantics, the kernel wrappers over the engine in pw_core.h, and the
// host launcher that plans a launch (pw_host.h) and picks the compiled
// variant.  Each family of entry points (pw_binary.hip, pw_scalar.hip,
// pw_unary.hip, pw_mask.hip) includes it and instantiates only its own ops, so
// the families compile in parallel.  Compiled with -ffp-contract=off, so
// `a * b + c` is never fused.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>

#include "pw_core.h"
#include "pw_host.h"
#include "trs_internal.h"

namespace trs {

// ---- op functors ----------------------------------------------------------

template <int OP>
struct BinaryF {
    static constexpr int NIN = 2;
    __device__ __forceinline__ float operator()(const float *a) const {
        if constexpr (OP == TRS_ADD) return a[0] + a[1];
        else if constexpr (OP == TRS_SUB) return a[0] - a[1];
        else if constexpr (OP == TRS_MUL) return a[0] * a[1];
        else return a[0] / a[1];
    }
};

template <int OP>
struct ScalarF {
    static constexpr int NIN = 1;
    float s;
    __device__ __forceinline__ float operator()(const float *a) const {
        if constexpr (OP == TRS_S_ADD) return a[0] + s;
        else if constexpr (OP == TRS_S_SUB) return a[0] - s;
        else if constexpr (OP == TRS_S_MUL) return a[0] * s;
        else if constexpr (OP == TRS_S_DIV) return a[0] / s;
        else if constexpr (OP == TRS_S_RSUB) return s - a[0];
        else return s * (1.0f / a[0]);  // scalar_div: reciprocal multiplication
    }
};

template <int OP>
struct UnaryF {
    static constexpr int NIN = 1;
    __device__ __forceinline__ float operator()(const float *a) const {
        if constexpr (OP == TRS_EXP) return exp_value(a[0]);
        else if constexpr (OP == TRS_RELU) return relu_value(a[0]);
        else if constexpr (OP == TRS_NEG) return negate_value(a[0]);
        else return a[0];
    }
};

// (h * mask) * scale with the mask read as uint8 (input 1).
struct MaskApplyF {
    static constexpr int NIN = 2;
    float scale;
    __device__ __forceinline__ float operator()(const float *a) const {
        const float t = a[0] * a[1];
        return t * scale;
    }
};

// Backward of dropout-apply (h * mask) * scale, in the order the reference's
// graph runs it: the MultiplyScalar VJP (up * scale) and then the Multiply VJP
// (* mask) -- two roundings, one pass.
struct MaskBackwardF {
    static constexpr int NIN = 2;  // (upstream, mask as u8)
    float scale;
    __device__ __forceinline__ float operator()(const float *a) const {
        const float t = a[0] * scale;
        return t * a[1];
    }
};

struct ReluBackwardF {
    static constexpr int NIN = 2;  // (saved input, upstream)
    __device__ __forceinline__ float operator()(const float *a) const {
        return relu_backward_value(a[0], a[1]);
    }
};

// ---- AOT wrappers -----------------------------------------------------------
// S: inputs read once (loaded non-temporally), a compile-time mask.

// The geometry is every wrapper's first argument: the bodies read it in place
// (kernarg_geom); the functor, which may carry a scalar, comes last.
template <class F, unsigned M, bool V, unsigned S>
__global__ void __launch_bounds__(kFlatBlock) k_flat(PwGeom, PwPtrs p, F f) {
    pw_flat_body<F, M, V, S>(f, kernarg_geom(), p);
}
template <class F, unsigned M>
__global__ void __launch_bounds__(kFlatBlock) k_flat_contig(PwGeom, PwPtrs p, F f) {
    pw_flat_contig_body<F, M>(f, kernarg_geom(), p);
}
template <class F, unsigned M, bool V, unsigned S, int RK = 0>
__global__ void __launch_bounds__(kRowLanesMax) k_rows(PwGeom, PwPtrs p, F f) {
    pw_rows_body<F, M, V, S, RK>(f, kernarg_geom(), p);
}
template <class F, unsigned M, bool V, unsigned TR, unsigned S>
__global__ void __launch_bounds__(64 * kXposeWT * kXposeWX) k_xpose(PwGeom, PwPtrs p, F f) {
    pw_xpose_body<F, M, V, kXposeWT, kXposeWX, TR, 0u, 0u, 1, S>(f, kernarg_geom(), p);
}
template <class F, unsigned M>
__global__ void __launch_bounds__(kGenericBlock) k_generic(PwGeom, PwPtrs p, F f) { pw_generic_body<F, M>(f, kernarg_geom(), p); }

// Calls fn.template operator()<K>() with K the compile-time value of the
// run-time mask `m` over NIN bits (NIN is 1 or 2 here).
template <int NIN, class Fn>
void with_mask(unsigned m, Fn &&fn) {
    static_assert(NIN >= 1 && NIN <= 2, "AOT functors take one or two inputs");
    if constexpr (NIN == 1) {
        if (m & 1u) fn.template operator()<1u>();
        else fn.template operator()<0u>();
    } else {
        switch (m & 3u) {
        case 0u: fn.template operator()<0u>(); break;
        case 1u: fn.template operator()<1u>(); break;
        case 2u: fn.template operator()<2u>(); break;
        default: fn.template operator()<3u>(); break;
        }
    }
}

// One launch of the plan's kernel on geometry `g` (the plan's own, or one
// part of a split plan).
template <class F, unsigned M>
int launch_part(const F &f, const PwPlan &pl, const PwGeom &g, hipStream_t s) {
    constexpr int NIN = F::NIN;
    const dim3 grid((unsigned)pl.grid), block((unsigned)pl.block);
    const unsigned sm = g.streamed & ((1u << NIN) - 1u);
    switch (pl.variant) {
    case PwVariant::Empty:
        return TRS_OK;
    case PwVariant::Flat:
        if (pl.contig) hipLaunchKernelGGL((k_flat_contig<F, M>), grid, block, 0, s, g, pl.p, f);
        else if (pl.vec)
            with_mask<NIN>(sm, [&]<unsigned S>() { hipLaunchKernelGGL((k_flat<F, M, true, S>), grid, block, 0, s, g, pl.p, f); });
        else hipLaunchKernelGGL((k_flat<F, M, false, 0u>), grid, block, 0, s, g, pl.p, f);
        break;
    case PwVariant::Rows:
        if (pl.vec)
            with_mask<NIN>(sm, [&]<unsigned S>() {
                if (pl.rk == 2) hipLaunchKernelGGL((k_rows<F, M, true, S, 2>), grid, block, 0, s, g, pl.p, f);
                else if (pl.rk == 3) hipLaunchKernelGGL((k_rows<F, M, true, S, 3>), grid, block, 0, s, g, pl.p, f);
                else if (pl.rk == 4) hipLaunchKernelGGL((k_rows<F, M, true, S, 4>), grid, block, 0, s, g, pl.p, f);
                else hipLaunchKernelGGL((k_rows<F, M, true, S, 0>), grid, block, 0, s, g, pl.p, f);
            });
        else hipLaunchKernelGGL((k_rows<F, M, false, 0u>), grid, block, 0, s, g, pl.p, f);
        break;
    case PwVariant::Xpose:
        // One outer tuple per block (no roles): every transposed-operand mask.
        with_mask<NIN>(pl.trans, [&]<unsigned TR>() {
            if constexpr (TR != 0u) {
                if (pl.vec)
                    with_mask<NIN>(sm, [&]<unsigned S>() {
                        hipLaunchKernelGGL((k_xpose<F, M, true, TR, S>), grid, block, 0, s, g, pl.p, f);
                    });
                else hipLaunchKernelGGL((k_xpose<F, M, false, TR, 0u>), grid, block, 0, s, g, pl.p, f);
            }
        });
        break;
    case PwVariant::Generic:
        hipLaunchKernelGGL((k_generic<F, M>), grid, block, 0, s, g, pl.p, f);
        break;
    }
    TRS_LAUNCH_CHECK("pointwise kernel launch");
    return TRS_OK;
}

template <class F, unsigned M>
int launch_planned(const F &f, const PwPlan &pl, hipStream_t s) {
    if (pl.variant == PwVariant::Empty) return TRS_OK;
    return for_each_part(pl, [&](const PwGeom &g) { return launch_part<F, M>(f, pl, g, s); });
}

template <class F, unsigned M = 0u>
int run_pointwise(const F &f, const trs_layout *lo, float *out, int nin, const void *const *bases,
                  const trs_layout *const *lins, const int *eb) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    PwPlan pl;
    int rc = plan_pointwise(lo, out, nin, bases, lins, eb, dev->cu_count, &pl);
    if (rc) return rc;
    return launch_planned<F, M>(f, pl, dev->stream);
}

}  // namespace trs
