// pw_core.h -- device-side pointwise engine for gfx950 (CDNA4).
//
// Shared verbatim by the ahead-of-time kernels (pw_ops.h) and by the
// runtime fusion compiler (fusion.hip embeds this file and compiles it with
// hipRTC), so an eager op and a fused chain run the same index machinery.
//
// The host normalises every launch first (pw_host.h): operands are aligned
// to the output rank with zero strides on broadcast dims, size-1 dims are
// dropped, dims are ordered by decreasing output stride and adjacent dims
// that are contiguous for every operand are merged.  The kernels below then
// cover four cases:
//   pw_flat  -- rank 1, every operand unit-stride or broadcast: one 16-byte
//               vector per lane, one-wave blocks, one-shot grid.
//   pw_rows  -- innermost dim unit-stride or broadcast for every operand:
//               one (outer row, column chunk) tile per block, one 16-byte
//               vector per lane;
//               the outer-row decode is wave-uniform (scalar registers), the
//               lanes stream 16-byte vectors along the row.
//   pw_xpose -- an operand is unit-stride along another dim (a transposed or
//               permuted view such as c.mT): each lane transposes a 4x4
//               block in registers, so reads and writes are both 16-byte
//               vectors; blocks walk the remaining dims, keeping operands
//               that do not move along them in registers.
//   pw_generic -- any strides: per-element decode with magic-number division.
//
// Every op is written so that hipcc and hipRTC (both run with
// -ffp-contract=off) emit exactly one IEEE binary32 rounding per reference op.
#pragma once
#ifndef TRS_RTC
#include <hip/hip_runtime.h>
#include <stdint.h>
#else
// hipRTC provides the fixed-width integer types in __hip_internal.
using __hip_internal::int32_t;
using __hip_internal::int64_t;
using __hip_internal::uint32_t;
using __hip_internal::uint64_t;
using __hip_internal::uint8_t;
#endif

#pragma clang fp contract(off)

namespace trs {

constexpr int kMaxRank = 8;
constexpr int kMaxIn = 8;
constexpr int kMaxOut = 8;  // outputs of one program (all share one layout)
constexpr int kRowChunk = 1024;  // columns per scalar pw_rows tile (256 lanes x 4)
// Vector pw_rows tiles: one float4 per lane, g.chunkcols = 4 x lanes
// columns, the lanes per block (64, 128 or 256) chosen per launch by
// rows_lanes() in pw_host.h.  At most this many:
constexpr int kRowLanesMax = 256;
// Largest grid a launch uses, in blocks.  Launches are one-shot -- one tile
// per block -- up to this many blocks; beyond it the bodies loop.  A
// dispatch counts at most 2^32 - 1 lanes per dimension, and the widest
// block here has 512 lanes, so 2^22 blocks always fit.  On gfx950 the
// three-input chain over 2^30 elements (16 GiB per launch, one-wave blocks)
// took 2,536 us one-shot against 2,830 us capped at 2^20 blocks, each lane
// then taking 4 groups in a grid-stride loop.
constexpr int64_t kMaxGrid = 1 << 22;
// Lanes per block of the flat kernels: one wave, one float4 per lane per
// operand, so a block reads 1 KiB of each operand and retires as soon as its
// one store is issued.  On gfx950 a standalone three-input chain over 2^28
// elements took 642 us with 64-lane blocks against 654 (128), 667 (256) and
// 685 (512) in interleaved runs on two boards; two or four float4 per lane
// were slower at every block size (670-707 us).  The bodies index with this
// constant, not blockDim: reading blockDim costs each wave a memory load and
// a wait before its first data load.
constexpr int kFlatBlock = 64;

// Unsigned 32-bit division by a runtime-invariant divisor (Granlund-Montgomery
// round-up method): q = (umulhi(n, mul) + n) >> shift, exact for all n < 2^32.
struct FastDiv {
    uint32_t div;
    uint32_t mul;
    uint32_t shift;
    uint32_t pad;
};

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv &d) {
    uint32_t t = __umulhi(n, d.mul);
    return (uint32_t)(((uint64_t)t + n) >> d.shift);
}

// Element offsets: 32-bit where the host planned every offset of a launch
// below 2^32 (strides are non-negative, so no partial sum of an in-range
// offset wraps), else 64-bit.
template <bool O32> struct OffsetT { using type = int64_t; };
template <> struct OffsetT<true> { using type = uint32_t; };

struct PwGeom {
    int32_t rank;   // >= 1 after normalisation
    int32_t tdim;   // pw_xpose: dim along which transposed operands are unit-stride
    int32_t wide;   // a dim exceeds 32 bits: always decode with 64-bit division
    int32_t skew;   // pw_xpose: a tuple's tiles are taken in diagonal order (x tile += t tile)
    int64_t numel;
    int64_t size[kMaxRank];
    FastDiv fd[kMaxRank];
    int64_t ostride[kMaxRank];
    int64_t istride[kMaxIn][kMaxRank];
    int64_t ooff;
    int64_t ioff[kMaxIn];
    uint32_t transposed;  // pw_xpose: bit i set when input i is unit-stride along tdim
    uint32_t streamed;    // bit i set when input i is read once (no broadcast dim)
    int64_t rows;         // pw_rows / pw_xpose: number of outer index tuples
    int64_t chunks;       // pw_rows: column chunks per row; pw_xpose: tiles per outer tuple
    FastDiv fdchunks;     // pw_rows / pw_xpose: divides a tile index below 2^32 by chunks
    FastDiv fdttiles;     // pw_xpose: divides by ttiles
    FastDiv fdxtiles;     // pw_xpose: divides by the x tiles of a tuple (skewed order)
    int64_t ttiles;       // pw_xpose: tiles along tdim
    int64_t groups;       // pw_xpose: block groups G; a block walks outer tuples c, c+G, c+2G, ...
    int64_t chunkcols;    // pw_rows (vector): columns per tile, 4 per lane
};

// The launch geometry, read in place in the kernel-argument segment: every
// kernel of this engine takes its PwGeom as the first argument, at offset 0
// of the segment.  Bound to the by-value parameter instead, the body's
// reference made the compiler copy the parameter, and wherever the body
// indexes the geometry at run time (dims chosen at run time) the copy stayed:
// 936 bytes per lane written to scratch memory and read back, in the
// transposing kernel's run-time-rank path, and SGPR spills elsewhere.
__device__ __forceinline__ const PwGeom &kernarg_geom() {
    return *(const PwGeom *)__builtin_amdgcn_kernarg_segment_ptr();
}

typedef float vf4 __attribute__((ext_vector_type(4)));
typedef uint8_t vu8x4 __attribute__((ext_vector_type(4)));

// Output 0 and the inputs; `more` holds outputs 1.. of a multi-output
// program.  Every output has the output layout (same offset and strides).
struct PwPtrs {
    float *out;
    const void *in[kMaxIn];
    float *more[kMaxOut - 1];
};

// ---- element loads --------------------------------------------------------

template <unsigned U8MASK, int I>
__device__ __forceinline__ float ld1(const PwPtrs &p, int64_t off) {
    if constexpr (((U8MASK >> I) & 1u) != 0u) {
        return (float)(((const uint8_t *)p.in[I])[off]);
    } else {
        return ((const float *)p.in[I])[off];
    }
}

// Four consecutive elements (unit stride) or one broadcast element (stride 0).
// STREAM: the operand is read once, so it is loaded non-temporally; re-read
// (broadcast) operands keep normal caching.  The choice is a template
// parameter because a function holding both kinds of load to one address is
// optimised, before it is inlined, into a single plain load: a run-time flag
// would silently lose the non-temporal hint.
template <unsigned U8MASK, int I, bool STREAM = false>
__device__ __forceinline__ void ld4(const PwPtrs &p, int64_t off, bool unit, float *v) {
    if (!unit) {
        float s = ld1<U8MASK, I>(p, off);
        v[0] = s; v[1] = s; v[2] = s; v[3] = s;
        return;
    }
    if constexpr (((U8MASK >> I) & 1u) != 0u) {
        const vu8x4 *src = (const vu8x4 *)(((const uint8_t *)p.in[I]) + off);
        vu8x4 q;
        if constexpr (STREAM) q = __builtin_nontemporal_load(src);
        else q = *src;
        v[0] = (float)q.x; v[1] = (float)q.y; v[2] = (float)q.z; v[3] = (float)q.w;
    } else {
        const vf4 *src = (const vf4 *)(((const float *)p.in[I]) + off);
        vf4 q;
        if constexpr (STREAM) q = __builtin_nontemporal_load(src);
        else q = *src;
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    }
}

__device__ __forceinline__ void st4(float *dst, const float *v) {
    vf4 q = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(q, (vf4 *)dst);
}

// Compile-time loop over inputs.
template <int N, int I = 0, class Fn>
__device__ __forceinline__ void static_for(Fn &&fn) {
    if constexpr (I < N) {
        fn.template operator()<I>();
        static_for<N, I + 1>(fn);
    }
}

// ---- functor outputs --------------------------------------------------------
// A functor computes one value (float operator()(const float *args)) or, when
// it declares `static constexpr int NOUT` > 1, NOUT values
// (void operator()(const float *args, float *results)).

template <class F>
constexpr int nout_of() {
    if constexpr (requires { F::NOUT; }) {
        return F::NOUT;
    } else {
        return 1;
    }
}

template <class F>
__device__ __forceinline__ void eval1(const F &f, const float *a, float *r) {
    if constexpr (nout_of<F>() == 1) {
        r[0] = f(a);
    } else {
        f(a, r);
    }
}

// r[o][k]: output o of element k of a four-element group v[input][k].
template <class F, int NI, int NO>
__device__ __forceinline__ void eval4(const F &f, const float (&v)[NI][4], float (&r)[NO][4]) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        float a[NI];
#pragma unroll
        for (int i = 0; i < NI; i++) a[i] = v[i][k];
        float o[NO];
        eval1(f, a, o);
#pragma unroll
        for (int q = 0; q < NO; q++) r[q][k] = o[q];
    }
}

template <int O>
__device__ __forceinline__ float *out_base(const PwPtrs &p) {
    if constexpr (O == 0) {
        return p.out;
    } else {
        return p.more[O - 1];
    }
}

template <int NO>
__device__ __forceinline__ void store4(const PwPtrs &p, int64_t off, const float (&r)[NO][4]) {
    static_for<NO>([&]<int O>() { st4(out_base<O>(p) + off, r[O]); });
}

template <int NO>
__device__ __forceinline__ void store1(const PwPtrs &p, int64_t off, const float *o) {
    static_for<NO>([&]<int O>() { out_base<O>(p)[off] = o[O]; });
}

// Offsets of output and inputs for a logical index tuple given by the first
// `ndims` dims of the decomposition of `outer` (row-major over dims
// [0, ndims)).  Uses 32-bit magic division when `outer` fits in 32 bits.
// ROLLED: the 32-bit path loops over the ndims dims at run time instead of
// unrolling over every possible one (fewer geometry fields live in scalar
// registers at once, for bodies that would otherwise spill them).
template <int NIN, bool ROLLED = false>
__device__ __forceinline__ void decode_outer(const PwGeom &g, int ndims, int64_t outer,
                                             int64_t &oo, int64_t *io) {
    oo = g.ooff;
    for (int i = 0; i < NIN; i++) io[i] = g.ioff[i];
    if (ROLLED && !g.wide && outer < 0x100000000LL) {
        uint32_t rem = (uint32_t)outer;
        for (int d = ndims - 1; d >= 0; d--) {
            const uint32_t q = fast_div(rem, g.fd[d]);
            const uint32_t c = rem - q * g.fd[d].div;
            rem = q;
            oo += (int64_t)c * g.ostride[d];
            for (int i = 0; i < NIN; i++) io[i] += (int64_t)c * g.istride[i][d];
        }
    } else if (!g.wide && outer < 0x100000000LL) {
        // Unrolled over every possible dim so each geometry field has a
        // constant index (loads the compiler can issue up front); dims at or
        // above ndims are skipped by a uniform branch.  The rows kernels
        // decode at most kMaxRank - 1 outer dims, the generic kernel and the
        // strided sum all kMaxRank.
        uint32_t rem = (uint32_t)outer;
#pragma unroll
        for (int d = kMaxRank - 1; d >= 0; d--) {
            if (d >= ndims) continue;
            uint32_t q = fast_div(rem, g.fd[d]);
            uint32_t c = rem - q * g.fd[d].div;
            rem = q;
            oo += (int64_t)c * g.ostride[d];
            for (int i = 0; i < NIN; i++) io[i] += (int64_t)c * g.istride[i][d];
        }
    } else {
        int64_t rem = outer;
        for (int d = ndims - 1; d >= 0; d--) {
            int64_t q = rem / g.size[d];
            int64_t c = rem - q * g.size[d];
            rem = q;
            oo += c * g.ostride[d];
            for (int i = 0; i < NIN; i++) io[i] += c * g.istride[i][d];
        }
    }
}

// Kernel bodies are __device__ functions so that the ahead-of-time wrappers
// (templates) and the hipRTC-generated wrappers (extern "C") share them.

// ---- pw_flat --------------------------------------------------------------
// rank 1; ostride 1; istride in {0, 1}.  VEC requires numel % 4 == 0 is NOT
// assumed: the vector body covers floor(numel/4) groups and a scalar tail the
// rest.  VEC is chosen by the host only when every unit-stride operand and
// the output are 16-byte aligned (4-byte for u8).  STRM: bit i set when input
// i is read once (g.streamed), loaded non-temporally.
template <class F, unsigned U8MASK, bool VEC, unsigned STRM = 0u>
__device__ __forceinline__ void pw_flat_body(const F &f, const PwGeom &g, const PwPtrs &p) {
    constexpr int NIN = F::NIN;
    constexpr int NOUT = nout_of<F>();
    const int64_t n = g.numel;
    const int64_t tid = (int64_t)blockIdx.x * kFlatBlock + threadIdx.x;
    const int64_t nthreads = (int64_t)gridDim.x * kFlatBlock;
    bool unit[NIN > 0 ? NIN : 1];
    for (int i = 0; i < NIN; i++) unit[i] = g.istride[i][0] != 0;
    int64_t tail_start = 0;
    if constexpr (VEC) {
        // One float4 group per lane.  The host sizes the grid to cover every
        // group in one pass (the loop only runs again past kMaxGrid blocks):
        // one-shot blocks keep the set of open DRAM pages compact, which
        // measured ~6.5 TB/s on gfx950 against ~4.3 TB/s for a persistent
        // grid-stride loop with 4 groups in flight per lane.
        const int64_t groups = n >> 2;
        for (int64_t gi = tid; gi < groups; gi += nthreads) {
            const int64_t e = gi << 2;
            float v[NIN > 0 ? NIN : 1][4];
            static_for<NIN>([&]<int I>() {
                ld4<U8MASK, I, ((STRM >> I) & 1u) != 0u>(p, g.ioff[I] + (unit[I] ? e : 0), unit[I], v[I]);
            });
            float r[NOUT][4];
            eval4(f, v, r);
            store4(p, g.ooff + e, r);
        }
        tail_start = groups << 2;
    }
    for (int64_t e = tail_start + tid; e < n; e += nthreads) {
        float a[NIN > 0 ? NIN : 1];
        static_for<NIN>([&]<int I>() { a[I] = ld1<U8MASK, I>(p, g.ioff[I] + (unit[I] ? e : 0)); });
        float o[NOUT];
        eval1(f, a, o);
        store1<NOUT>(p, g.ooff + e, o);
    }
}

// pw_flat with every operand unit-stride and read once (no broadcast), the
// 16-byte-aligned case: operand kinds are fixed at compile time, so each lane
// issues its NIN non-temporal vector loads back to back with no uniform
// branches between them (the general body above measured ~10% slower on
// three-input chains for that reason).
template <unsigned U8MASK, int I>
__device__ __forceinline__ void ld4_stream(const PwPtrs &p, int64_t off, float *v) {
    if constexpr (((U8MASK >> I) & 1u) != 0u) {
        vu8x4 q = __builtin_nontemporal_load((const vu8x4 *)(((const uint8_t *)p.in[I]) + off));
        v[0] = (float)q.x; v[1] = (float)q.y; v[2] = (float)q.z; v[3] = (float)q.w;
    } else {
        vf4 q = __builtin_nontemporal_load((const vf4 *)(((const float *)p.in[I]) + off));
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    }
}

template <class F, unsigned U8MASK>
__device__ __forceinline__ void pw_flat_contig_body(const F &f, const PwGeom &g, const PwPtrs &p) {
    constexpr int NIN = F::NIN;
    constexpr int NOUT = nout_of<F>();
    const int64_t n = g.numel;
    const int64_t tid = (int64_t)blockIdx.x * kFlatBlock + threadIdx.x;
    const int64_t nthreads = (int64_t)gridDim.x * kFlatBlock;
    const int64_t groups = n >> 2;
    for (int64_t gi = tid; gi < groups; gi += nthreads) {
        const int64_t e = gi << 2;
        float v[NIN > 0 ? NIN : 1][4];
        static_for<NIN>([&]<int I>() { ld4_stream<U8MASK, I>(p, g.ioff[I] + e, v[I]); });
        float r[NOUT][4];
        eval4(f, v, r);
        store4(p, g.ooff + e, r);
    }
    for (int64_t e = (groups << 2) + tid; e < n; e += nthreads) {
        float a[NIN > 0 ? NIN : 1];
        static_for<NIN>([&]<int I>() { a[I] = ld1<U8MASK, I>(p, g.ioff[I] + e); });
        float o[NOUT];
        eval1(f, a, o);
        store1<NOUT>(p, g.ooff + e, o);
    }
}

// ---- pw_rows --------------------------------------------------------------
// Innermost dim (size[rank-1] columns) has ostride 1 and istride in {0, 1}.
// g.rows = product of the outer dims, g.chunks = ceil(cols / chunk) with
// chunk = g.chunkcols under VEC, else kRowChunk.
// VEC: cols % 4 == 0 and every unit-stride row start 16-byte aligned.  A lane
// takes one float4 of the row; the block's lanes (g.chunkcols / 4) are
// chosen per launch for the HBM bytes a block moves (rows_lanes()).
// STRM: as for pw_flat.
// RANK = 2, 3 or 4: the rank is fixed, so the row splits into its outer
// indices by RANK - 2 multiply-shifts with every geometry field at a constant
// index (no decode loop, no run-time branch).  RANK = 0: any rank, through
// decode_outer.  O32 (a fixed RANK): every element offset of the launch is
// below 2^32, so the row's offsets are 32-bit products.  SMALL: fewer than
// 2^32 tiles, so a tile index splits into (row, chunk) by multiply-shift
// instead of a 64-bit division.  All of this runs before the first load of
// every block: the decode loop's dependent scalar loads cost about 5% of a
// [4096, 4096] launch, and on a [64, 512, 1024] one whose blocks each write
// one 4 KiB row, the decode loop took half the time and 64-bit stride
// products a further sixth.  A loop unrolled over all 8 possible dims (rank
// 4 to 8 in one variant) held too many fields for the scalar registers and
// reloaded them dim by dim: 32 us where the fixed rank 4 takes 24.5 (rank
// 3: 22; the 64-bit run-time path: 41.5).
template <class F, unsigned U8MASK, bool VEC, unsigned STRM, int RANK, bool O32, bool SMALL>
__device__ __forceinline__ void pw_rows_loop(const F &f, const PwGeom &g, const PwPtrs &p) {
    static_assert(RANK == 0 || (RANK >= 2 && RANK <= 4 && SMALL), "a fixed rank is 2, 3 or 4, below 2^32 tiles");
    static_assert(!O32 || RANK != 0, "32-bit offsets need a fixed rank");
    constexpr int NIN = F::NIN;
    constexpr int NOUT = nout_of<F>();
    const int inner = RANK != 0 ? RANK - 1 : g.rank - 1;
    const int64_t cols = g.size[inner];
    const int64_t ntiles = g.rows * g.chunks;
    bool unit[NIN > 0 ? NIN : 1];
    for (int i = 0; i < NIN; i++) unit[i] = g.istride[i][inner] != 0;
    // One tile per block in every launch below 2^20 tiles: the first tile
    // runs outside the loop, so a block with no second tile ends without
    // the wait for its own stores that the loop's back edge needs (the
    // next tile's loads reuse the registers the stores read).
    auto do_tile = [&](int64_t tile) {
        // Wave-uniform decode of the outer tuple (held in scalar registers).
        int64_t row, chunk;
        if constexpr (SMALL) {
            const uint32_t r = fast_div((uint32_t)tile, g.fdchunks);
            row = r;
            chunk = (uint32_t)tile - r * g.fdchunks.div;
        } else {
            row = tile / g.chunks;
            chunk = tile - row * g.chunks;
        }
        int64_t oo, io[NIN > 0 ? NIN : 1];
        if constexpr (RANK != 0) {
            // outer dims RANK-2 .. 0, innermost first; row < 2^32 (SMALL).
            // With O32 every offset is below 2^32 and every term
            // non-negative, so no partial sum wraps in 32 bits.
            using Off = typename OffsetT<O32>::type;
            uint32_t rem = (uint32_t)row;
            Off o = (Off)g.ooff, ii[NIN > 0 ? NIN : 1];
            for (int i = 0; i < NIN; i++) ii[i] = (Off)g.ioff[i];
#pragma unroll
            for (int d = RANK - 2; d >= 0; d--) {
                const uint32_t q = d == 0 ? 0u : fast_div(rem, g.fd[d]);
                const Off c = (Off)(rem - q * g.fd[d].div);
                rem = q;
                o += c * (Off)g.ostride[d];
                for (int i = 0; i < NIN; i++) ii[i] += c * (Off)g.istride[i][d];
            }
            oo = (int64_t)o;
            for (int i = 0; i < NIN; i++) io[i] = (int64_t)ii[i];
        } else {
            // The scalar fallback (rows not float4-aligned) decodes in a
            // rolled loop: unrolled, this body spilled 46 scalar registers
            // and reserved a private segment.
            decode_outer<NIN, !VEC>(g, inner, row, oo, io);
        }
        if constexpr (VEC) {
            const int64_t c0 = chunk * g.chunkcols;
            const int64_t c = c0 + (int64_t)threadIdx.x * 4;
            // cols % 4 == 0, so a lane's float4 lies wholly inside or past
            // the row.  Lanes past it load the row's last float4 and store
            // nothing: no branch around the loads, which would hold back the
            // geometry reads they depend on until the lane test.  A streamed
            // operand (read once, no broadcast dim) is unit-stride here, so
            // its load kind is fixed at compile time, and the streamed loads
            // are issued first, ahead of the other operands' run-time choice
            // between a vector and a broadcast load.
            const int64_t cl = c < cols ? c : cols - 4;
            float v[NIN > 0 ? NIN : 1][4];
            static_for<NIN>([&]<int I>() {
                if constexpr (((STRM >> I) & 1u) != 0u) ld4<U8MASK, I, true>(p, io[I] + cl, true, v[I]);
            });
            static_for<NIN>([&]<int I>() {
                if constexpr (((STRM >> I) & 1u) == 0u) ld4<U8MASK, I, false>(p, io[I] + (unit[I] ? cl : 0), unit[I], v[I]);
            });
            float r[NOUT][4];
            eval4(f, v, r);
            if (c < cols) store4(p, oo + c, r);
        } else {
            const int64_t c0 = chunk * kRowChunk;
            for (int k = 0; k < 4; k++) {
                const int64_t c = c0 + (int64_t)k * 256 + threadIdx.x;
                if (c < cols) {
                    float a[NIN > 0 ? NIN : 1];
                    static_for<NIN>([&]<int I>() {
                        a[I] = ld1<U8MASK, I>(p, io[I] + (unit[I] ? c : 0));
                    });
                    float o[NOUT];
                    eval1(f, a, o);
                    store1<NOUT>(p, oo + c, o);
                }
            }
        }
    };
    // The host launches at most ntiles blocks (grid = min(tiles, kMaxGrid),
    // checked before every launch), so the first tile needs no bounds check.
    // With one, every geometry load behind it waited for the tile count: four
    // dependent rounds of scalar loads before a block's first data load.
    do_tile(blockIdx.x);
    for (int64_t tile = (int64_t)blockIdx.x + gridDim.x; tile < ntiles; tile += gridDim.x) do_tile(tile);
}

// RK = 2, 3 or 4: the host planned a launch of that rank, fewer than 2^32
// tiles and every element offset below 2^32 (the common cases, compiled with
// no run-time geometry branches and 32-bit offsets); RK = 0: any rows launch,
// dispatched at run time with 64-bit offsets.
template <class F, unsigned U8MASK, bool VEC, unsigned STRM = 0u, int RK = 0>
__device__ __forceinline__ void pw_rows_body(const F &f, const PwGeom &g, const PwPtrs &p) {
    if constexpr (RK != 0) {
        pw_rows_loop<F, U8MASK, VEC, STRM, RK, true, true>(f, g, p);
    } else {
        if (g.rows * g.chunks > 0xFFFFFFFFll) pw_rows_loop<F, U8MASK, VEC, STRM, 0, false, false>(f, g, p);
        else if (g.rank == 2) pw_rows_loop<F, U8MASK, VEC, STRM, 2, false, true>(f, g, p);
        else if (g.rank == 3) pw_rows_loop<F, U8MASK, VEC, STRM, 3, false, true>(f, g, p);
        else pw_rows_loop<F, U8MASK, VEC, STRM, 0, false, true>(f, g, p);
    }
}

// ---- pw_xpose -------------------------------------------------------------
// Output unit-stride along x = dim rank-1; operands in TRANS are unit-stride
// along t = g.tdim, every other operand has stride 0 or 1 along x (the
// planner's Xpose layouts).  A lane owns a 4(t) x 4(x) block: it reads a
// TRANS operand as four 16-byte vectors along t (one per x) and any other
// operand, and writes the output, as four vectors along x (one per t), so the
// transpose happens in registers with no LDS and no barrier.  A wave is 8 x 8
// lanes covering 32 t x 32 x, so each of its vector accesses is 8 runs of
// 128 B; a block of WT x WX waves covers a (32 WT) x (32 WX) tile.  Measured
// on (a + b) * c.mT over [64, 512, 1024], the 128 x 64 tile's transpose alone
// runs at the speed of the same access pattern without any data exchange.
// The other dims ("outer" tuples, g.rows of them) are walked: block
// (c, tile) takes the NW tuples c, c + G, ..., c + (NW-1) G with
// G = g.groups = g.rows / NW, so
//   HELD operands (stride 0 over every outer dim) are loaded once per block,
//   ONCE operands (stride 0 along t) once per outer tuple,
// and each tuple's loads are issued before the previous tuple's stores.
// NW = 1 walks nothing (one tuple per block).  g.ttiles = t tiles,
// g.chunks = t tiles * x tiles.  Consecutive blocks take consecutive t tiles
// of one x tile.  When a tuple has more tiles than the GPU holds at once
// (g.skew), block (tt, xt) takes x tile (xt + tt) mod x tiles instead: in the
// plain order the resident blocks then share a few x tiles, so their output
// rows are written at the same few offsets within each row, which with a
// large power-of-two row stride fall on the same memory channels.  x + y.mT
// over [8192, 8192] measured 205 us plain and 141 us skewed (0.49 -> 0.71 of
// HBM); a tuple of config 2's [64, 512, 1024] (4 x 16 tiles) gains nothing.
template <unsigned M, int I>
constexpr int mask_rank() {  // set bits of M below bit I
    return __builtin_popcount(M & ((1u << I) - 1u));
}

// XBC (inputs with stride 0 along x) equal to kRuntimeMask is read from the
// geometry at run time; otherwise it is fixed at compile time.
constexpr unsigned kRuntimeMask = 0xffffffffu;

// RK = 3: the host planned a rank-3 launch of fewer than 2^32 tiles and every
// element offset below 2^32, compiled with no run-time geometry branches, a
// direct offset for the one outer dim and 32-bit offsets; RK = 0: any launch,
// dispatched at run time with 64-bit offsets.  Tile indices below 2^32 split
// into (tuple, t tile, x tile) by multiply-shift either way.  TD (0 or 1,
// with RK = 3): the t dim fixed at compile time, so the geometry fields a
// block reads sit at constant offsets.  PLAIN (with RK = 3 and VEC): every
// tile is interior and the tiles are taken in plain order, so no block tests
// either.  Without both, the scalar loads of the geometry waited behind the
// run-time t dim and the two tests: five rounds of them before a walking
// block's first data load.
template <class F, unsigned U8MASK, bool VEC, int WT, int WX, unsigned TRANS, unsigned HELD, unsigned ONCE, int NW,
          unsigned STRM, unsigned XBC = kRuntimeMask, int RK = 0, int TD = -1, bool PLAIN = false>
__device__ __forceinline__ void pw_xpose_body(const F &f, const PwGeom &g, const PwPtrs &p) {
    static_assert(TD < 0 || (RK == 3 && TD <= 1), "a fixed t dim is 0 or 1 of a rank-3 launch");
    static_assert(!PLAIN || (RK == 3 && VEC), "plain tiles are a vector rank-3 case");
    constexpr int NIN = F::NIN;
    constexpr int NIN1 = NIN > 0 ? NIN : 1;
    constexpr int NOUT = nout_of<F>();
    constexpr int NH = __builtin_popcount(HELD);
    constexpr int BT = 32 * WT, BX = 32 * WX;
    using Off = typename OffsetT<RK == 3>::type;
    const int xd = RK == 3 ? 2 : g.rank - 1, td = TD >= 0 ? TD : g.tdim;
    const int64_t xs = g.size[xd], ts = g.size[td];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t ntiles = g.groups * g.chunks;
    // Operand I moves along x with unit stride (else stride 0): compile-time
    // unless XBC is kRuntimeMask.  STRM: inputs read once (non-temporal).
    auto unit_x = [&]<int I>() -> bool {
        if constexpr (XBC == kRuntimeMask) return g.istride[I][xd] != 0;
        else return ((XBC >> I) & 1u) == 0u;
    };
    // Offsets of outer tuple `o`: a wave-uniform decode over the dims other
    // than t and x (32-bit magic-number division when o fits).
    auto decode = [&](int64_t o, Off &oo, Off *io) {
        oo = (Off)g.ooff;
        for (int i = 0; i < NIN; i++) io[i] = (Off)g.ioff[i];
        if constexpr (RK == 3) {
            // the one outer dim is the dim of 0 and 1 that is not t
            const int wd = td == 0 ? 1 : 0;
            oo += (Off)o * (Off)g.ostride[wd];
            for (int i = 0; i < NIN; i++) io[i] += (Off)o * (Off)g.istride[i][wd];
        } else if (!g.wide && o < 0x100000000LL) {
            uint32_t rem = (uint32_t)o;
            for (int d = xd - 1; d >= 0; d--) {
                if (d == td) continue;
                const uint32_t q = fast_div(rem, g.fd[d]);
                const int64_t c = (int64_t)(rem - q * g.fd[d].div);
                rem = q;
                oo += c * g.ostride[d];
                for (int i = 0; i < NIN; i++) io[i] += c * g.istride[i][d];
            }
        } else {
            for (int d = xd - 1; d >= 0; d--) {
                if (d == td) continue;
                const int64_t q = o / g.size[d];
                const int64_t c = o - q * g.size[d];
                o = q;
                oo += c * g.ostride[d];
                for (int i = 0; i < NIN; i++) io[i] += c * g.istride[i][d];
            }
        }
    };
    const bool small = RK == 3 || ntiles <= 0xFFFFFFFFll;
    auto do_tile = [&](int64_t tile) {
        int64_t c, tt, xt;
        if (small) {
            const uint32_t q = fast_div((uint32_t)tile, g.fdchunks);
            const uint32_t rest = (uint32_t)tile - q * g.fdchunks.div;
            const uint32_t q2 = fast_div(rest, g.fdttiles);
            c = q;
            xt = q2;
            tt = rest - q2 * g.fdttiles.div;
            if (!PLAIN && g.skew) {  // xt + tt < xtiles * ttiles < 2^32
                const uint32_t sk = q2 + (uint32_t)tt;
                xt = sk - fast_div(sk, g.fdxtiles) * g.fdxtiles.div;
            }
        } else {
            c = tile / g.chunks;
            const int64_t rest = tile - c * g.chunks;
            tt = rest % g.ttiles;
            xt = rest / g.ttiles;
            if (g.skew) xt = (xt + tt) % (g.chunks / g.ttiles);
        }
        const int64_t t0 = tt * BT, x0 = xt * BX;
        const int64_t t = t0 + (wave % WT) * 32 + 4 * (lane & 7);
        const int64_t x = x0 + (wave / WT) * 32 + 4 * (lane >> 3);
        // Per-operand lane offset within an outer tuple and the step between
        // its four vectors: along x for TRANS operands (each vector runs along
        // t), along t for the others (each vector runs along x).
        // (A lane past the tensor's edge forms offsets past its end, which
        // may wrap in 32 bits; the edge path never loads or stores them.)
        Off loff[NIN1], lstep[NIN1];
        static_for<NIN>([&]<int I>() {
            if constexpr ((TRANS >> I) & 1u) {
                loff[I] = (Off)x * (Off)g.istride[I][xd] + (Off)t;
                lstep[I] = (Off)g.istride[I][xd];
            } else {
                loff[I] = (Off)t * (Off)g.istride[I][td] + (unit_x.template operator()<I>() ? (Off)x : (Off)0);
                lstep[I] = (Off)g.istride[I][td];
            }
        });
        const Off ooff_lane = (Off)t * (Off)g.ostride[td] + (Off)x;
        // The block runs its whole tile with 16-byte vectors when the tile
        // is interior and the operands aligned (a wave-uniform test), else
        // every access is scalar and bounds-checked.
        auto run = [&]<bool FAST, bool ONE_OUTER>() {
            // Operand I's four vectors (raw[j][e]: vector j, element e) at
            // tuple base b.  Element (t+k, x+i) is raw[i][k] for TRANS
            // operands and raw[k][i] for the others.
            // Every loop over a block's 4 vectors or 4 elements is unrolled:
            // a register array indexed at run time is moved to LDS or
            // scratch by the compiler (this cost a fifth of the transposed
            // copy's time).
            auto load_block = [&]<int I, int NV>(Off b, float (&raw)[4][4]) {
                const Off base = b + loff[I];
                constexpr bool tr = ((TRANS >> I) & 1u) != 0;
                const bool unit = tr || unit_x.template operator()<I>();
                if constexpr (FAST) {
                    constexpr bool stream = ((HELD >> I) & 1u) == 0u && ((STRM >> I) & 1u) != 0u;
#pragma unroll
                    for (int j = 0; j < NV; j++) ld4<U8MASK, I, stream>(p, base + (Off)j * lstep[I], unit, raw[j]);
                } else {
#pragma unroll
                    for (int j = 0; j < NV; j++)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const bool in = tr ? (t + e < ts && x + j < xs) : (t + j < ts && x + e < xs);
                            raw[j][e] = in ? ld1<U8MASK, I>(p, base + (Off)j * lstep[I] + (unit ? (Off)e : (Off)0)) : 0.0f;
                        }
                }
            };
            float held[NH > 0 ? NH : 1][4][4];
            static_for<NIN>([&]<int I>() {
                if constexpr ((HELD >> I) & 1u) load_block.template operator()<I, 4>((Off)g.ioff[I], held[mask_rank<HELD, I>()]);
            });
            // One outer tuple's loads (all operands but HELD) into `dst`.
            auto loads = [&](const Off *io, float (&dst)[NIN1][4][4]) {
                static_for<NIN>([&]<int I>() {
                    if constexpr (!((HELD >> I) & 1u))
                        load_block.template operator()<I, ((ONCE >> I) & 1u) ? 1 : 4>(io[I], dst[I]);
                });
            };
            // Compute and store one outer tuple from its loaded values.
            auto compute = [&](const float (&v)[NIN1][4][4], Off oo) {
                const Off ob0 = oo + ooff_lane;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    // Element (t+k, x+i), one functor call per element with
                    // each argument picked straight from the loaded blocks:
                    // gathering them into a [NIN][4] array first led the
                    // compiler to rebuild the transpose through a stack array
                    // (moved to LDS), a fifth of the transposed copy's time.
                    float r[NOUT][4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        float args[NIN1];
                        static_for<NIN>([&]<int I>() {
                            if constexpr ((HELD >> I) & 1u) {
                                constexpr int h = mask_rank<HELD, I>();
                                if constexpr ((TRANS >> I) & 1u) args[I] = held[h][i][k];
                                else args[I] = held[h][k][i];
                            } else if constexpr ((ONCE >> I) & 1u) {
                                args[I] = v[I][0][i];
                            } else if constexpr ((TRANS >> I) & 1u) {
                                args[I] = v[I][i][k];
                            } else {
                                args[I] = v[I][k][i];
                            }
                        });
                        float o[NOUT];
                        eval1(f, args, o);
#pragma unroll
                        for (int q = 0; q < NOUT; q++) r[q][i] = o[q];
                    }
                    const Off ob = ob0 + (Off)k * (Off)g.ostride[td];
                    if constexpr (FAST) {
                        store4(p, ob, r);
                    } else if (t + k < ts) {
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            if (x + i < xs) {
                                float ov[NOUT];
                                for (int q = 0; q < NOUT; q++) ov[q] = r[q][i];
                                store1<NOUT>(p, ob + (Off)i, ov);
                            }
                        }
                    }
                }
            };
            // Tuple offsets: with one outer dim (rank 3) tuple o + groups is
            // tuple o advanced by constant per-operand steps; otherwise each
            // tuple is decoded.
            Off dstep[NIN1], ostep = 0;
            if constexpr (ONE_OUTER) {
                const int wd = (td == 0) ? 1 : 0;
                for (int i = 0; i < NIN; i++) dstep[i] = (Off)g.groups * (Off)g.istride[i][wd];
                ostep = (Off)g.groups * (Off)g.ostride[wd];
            }
            Off io[NIN1], oo = 0;
            // Exactly NW tuples per block (the host sets g.rows = g.groups *
            // NW).  The walk is unrolled at compile time: tuple s+1's loads
            // are issued before tuple s computes and stores, with no branch
            // between them, so each compute waits only for its own loads.
            float nv[NIN1][4][4];
            decode(c, oo, io);
            loads(io, nv);
#pragma unroll
            for (int s = 0; s < NW; s++) {
                float v[NIN1][4][4];
#pragma unroll
                for (int i = 0; i < NIN; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
#pragma unroll
                        for (int e = 0; e < 4; e++) v[i][j][e] = nv[i][j][e];
                const Off ocur = oo;
                if (s + 1 < NW) {
                    if constexpr (ONE_OUTER) {
                        oo += ostep;
                        for (int i = 0; i < NIN; i++) io[i] += dstep[i];
                    } else {
                        decode(c + (int64_t)(s + 1) * g.groups, oo, io);
                    }
                    loads(io, nv);
                }
                compute(v, ocur);
            }
        };
        const bool fast = PLAIN || (VEC && t0 + BT <= ts && x0 + BX <= xs);
        if (RK == 3 || g.rank == 3) {
            if (fast) run.template operator()<true, true>();
            else run.template operator()<false, true>();
        } else {
            if constexpr (RK != 3) {
                if (fast) run.template operator()<true, false>();
                else run.template operator()<false, false>();
            }
        }
    };
    // The first tile runs outside the loop: a block with one tile ends
    // without waiting at the loop's back edge for its own stores.  As in
    // pw_rows, the host launches at most ntiles blocks, so it is unchecked.
    do_tile(blockIdx.x);
    for (int64_t tile = (int64_t)blockIdx.x + gridDim.x; tile < ntiles; tile += gridDim.x) do_tile(tile);
}

// ---- pw_generic -----------------------------------------------------------
// Any strides: every element decoded on its own by magic-number division.  A
// block takes kGenericUnroll * kGenericBlock consecutive elements per step,
// lane t the elements t, t + kGenericBlock, ... of them, so each load still
// covers consecutive elements; the lane issues all its loads before any
// arithmetic.  With one element per lane, x[::2] + y[::2] over 2^25 elements
// took 171 us, each lane waiting for its loads before the next element.
constexpr int kGenericUnroll = 4;
constexpr int kGenericBlock = 256;  // lanes per block of pw_generic

template <class F, unsigned U8MASK>
__device__ __forceinline__ void pw_generic_body(const F &f, const PwGeom &g, const PwPtrs &p) {
    constexpr int NIN = F::NIN;
    constexpr int NIN1 = NIN > 0 ? NIN : 1;
    constexpr int NOUT = nout_of<F>();
    constexpr int U = kGenericUnroll;
    constexpr int B = kGenericBlock;
    const int64_t step = (int64_t)gridDim.x * B * U;
    for (int64_t base = (int64_t)blockIdx.x * B * U; base < g.numel; base += step) {
        int64_t oo[U], io[U][NIN1];
        float a[U][NIN1];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t e = base + (int64_t)u * B + threadIdx.x;
            if (e < g.numel) {
                decode_outer<NIN>(g, g.rank, e, oo[u], io[u]);
                static_for<NIN>([&]<int I>() { a[u][I] = ld1<U8MASK, I>(p, io[u][I]); });
            }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t e = base + (int64_t)u * B + threadIdx.x;
            if (e < g.numel) {
                float o[NOUT];
                eval1(f, a[u], o);
                store1<NOUT>(p, oo[u], o);
            }
        }
    }
}

// ---- scalar semantics of the reference ------------------------------------

// relu_value (src/tensor.rs:4392-4400): exact zeros (either sign) pass
// through; otherwise max(v, 0) with NaN -> +0.0.
__device__ __forceinline__ float relu_value(float v) {
    if ((__float_as_uint(v) & 0x7fffffffu) == 0u) return v;
    return v > 0.0f ? v : 0.0f;
}

// relu_backward_value (src/tensor.rs:4422-4432).
__device__ __forceinline__ float relu_backward_value(float input, float up) {
    const uint32_t bits = __float_as_uint(input);
    const uint32_t mag = bits & 0x7fffffffu;
    const bool pass = mag > 0x7f800000u || ((bits & 0x80000000u) == 0u && mag != 0u);
    return pass ? up : 0.0f;
}

// negate_value (src/tensor.rs:4388-4390): sign-bit flip.
__device__ __forceinline__ float negate_value(float v) {
    return __uint_as_float(__float_as_uint(v) ^ 0x80000000u);
}

// exp: the device libm expf (ocml, about 1 ulp, denormal outputs kept).
__device__ __forceinline__ float exp_value(float v) { return expf(v); }

}  // namespace trs
