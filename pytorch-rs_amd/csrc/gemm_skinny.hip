// gemm_skinny.hip -- fp32 products with a short output side on FP32 MFMA.
//
// Replaces Tensor::matmul (src/tensor.rs:2453-2533, 3872-3994) for outputs
// of at most 32 rows or columns: matrix-vector products and small-batch
// linear layers.  These read one long operand Y once and do little
// arithmetic per byte, so the bound is HBM.  On the square-tile kernel
// (gemm.hip) a [1, 4096] x [4096, 4096] product ran as 32 blocks, each
// walking all of K, and took ~350 us for 64 MiB.
//
// Layout of the work: the short operand X (R <= 32 rows) is the MFMA's A
// operand, padded with zero rows to 16 or 32; Y supplies the B operand.  A
// block owns 64 output columns and one slice of K; its 4 waves take
// consecutive quarters of that slice and their accumulators are added in
// wave order through LDS at the end.  K is split into slices so the grid
// holds ~4 blocks per CU; the slices' partial products go to a workspace
// and one more pass adds them in slice order (slice_sum).  Adding them in
// the kernel instead, the last block of each column group to arrive summing
// its group's partials (stored and reloaded as tagged relaxed agent-scope
// atomics, so no release fence is needed), measured slower on the box:
// 20.3 against 16.6 us for x[1,4096] @ W, 43.7 against 24.8 us for
// x[32,4096] @ W.mT (and the separate pass has since become faster).
//
// Fragments straight from global memory, no LDS staging (each Y element is
// used by one lane of one MFMA):
//   - Y unit-stride along k ("dot" form, e.g. W.mT): lane (fi, fk) loads
//     float4 k = kg + 4fk .. +3 of row j = 16t + fi, and MFMA step e of the
//     16-k group takes its component e (the MFMA sums k in any order);
//   - Y unit-stride along j: lane (fi, fk) loads float4 columns 4fi .. 4fi+3
//     of row k = kg + 4fk + e, and component c feeds column sub-tile c, so
//     output column 4fi + c comes from lane fi of sub-tile c.
// Either way one float4 of Y feeds four MFMAs per 16-row group of X.
//
// The sum is fp32 in MFMA order, then wave order, then slice order; like
// gemm.hip it is checked against the reference's sequential sum within
// |dC| <= 1e-5*sqrt(K)*(|A||B|).  Zero padding (rows of X past R, columns
// of Y past L, k past the slice) only meets outputs that are not stored, so
// an infinity in X or Y cannot turn a stored output into NaN through it.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "gemm_skinny.h"
#include "lds_dma.h"
#include "trs_internal.h"

namespace trs {

namespace {

typedef float vf4 __attribute__((ext_vector_type(4)));
// A float4 at any float: global_load_dwordx4 needs only dword alignment, so
// operands at any offset and rows of any length load as vectors (each load
// below lies inside its row).
typedef float vf4u __attribute__((ext_vector_type(4), aligned(4)));

struct SkinnyArgs {
    const float *x;
    const float *y;
    float *o;
    int64_t xi, xk, yl;
    int64_t oi, oj, bo, os;  // output strides: (i, j), batch, slice
    int64_t bx, by;
    int64_t R, L, K, kc;
    int32_t S, jblocks;
};

// A block's column block, slice and batch: block = (b*S + s)*jblocks + jb.
// In 32 bits (the planner keeps the grid below 2^31): a 64-bit division is a
// long VALU sequence, and these kernels run a few microseconds.
struct BlockCoords {
    uint32_t jb, s, b;
};
__device__ __forceinline__ BlockCoords block_coords(const SkinnyArgs &g) {
    const uint32_t bid = blockIdx.x, jbs = (uint32_t)g.jblocks, ss = (uint32_t)g.S;
    const uint32_t q = bid / jbs;
    return {bid - q * jbs, q % ss, q / ss};
}

constexpr int kWaves = 4;
constexpr int kStepK = 32;  // k per wave step

template <bool VEC>
__device__ __forceinline__ vf4 load4(const float *p) {
    if constexpr (VEC) return *(const vf4u *)p;
    else return (vf4){p[0], p[1], p[2], p[3]};
}

// The long operand, read once: a non-temporal load, so it does not displace
// the short operand, which every block re-reads, from the caches.
__device__ __forceinline__ vf4 load4_stream(const float *p) { return __builtin_nontemporal_load((const vf4u *)p); }

// Four waves per SIMD (128 registers).  YVEC is always set since float4
// loads need only dword alignment; the scalar form stays for the ragged k
// groups (GUARD below).
template <bool DOT, bool YVEC, bool XVEC, int RG>
__global__ void __launch_bounds__(256, 4) gemm_f32_skinny(SkinnyArgs g) {
    // 16-k groups a wave loads before its MFMAs: two where they fit in the
    // 128 registers of 4 waves per SIMD without spilling, else one (then
    // a step is two load-then-MFMA rounds).
    constexpr int kGroups = (RG == 1 && YVEC) ? 2 : 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int fi = lane & 15, fk = lane >> 4;
    const BlockCoords bc = block_coords(g);
    const int64_t jb = bc.jb, s = bc.s, b = bc.b;
    const int64_t j0 = jb * kSkinnyCols;
    const int64_t kbeg = s * g.kc, kend = std::min(g.K, kbeg + g.kc);
    // Wave w takes the w-th quarter of the slice, in 32-k steps, so each of
    // its rows is read as one contiguous run.
    const int64_t kw = ((kend - kbeg + kWaves - 1) / kWaves + kStepK - 1) / kStepK * kStepK;
    const int64_t wbeg = kbeg + wave * kw, wend = std::min(kend, wbeg + kw);
    const float *X = g.x + b * g.bx;
    const float *Y = g.y + b * g.by;

    // This lane's X row in each 16-row group (zero past R).
    const float *xrow[RG];
    bool xin[RG];
#pragma unroll
    for (int rg = 0; rg < RG; rg++) {
        const int64_t i = 16 * rg + fi;
        xin[rg] = i < g.R;
        xrow[rg] = X + (xin[rg] ? i : 0) * g.xi;
    }
    // Dot form: this lane's Y row in each column sub-tile.  Otherwise: how
    // many of its four columns lie below L.
    const float *yrow[4];
    bool yin[4];
    int ncols = 0;
    if constexpr (DOT) {
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int64_t j = j0 + 16 * t + fi;
            yin[t] = j < g.L;
            yrow[t] = Y + (yin[t] ? j : 0) * g.yl;
        }
    } else {
        ncols = (int)std::max<int64_t>(0, std::min<int64_t>(4, g.L - (j0 + 4 * fi)));
    }

    vf4 acc[RG][4];
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
        for (int t = 0; t < 4; t++) acc[rg][t] = (vf4){0.f, 0.f, 0.f, 0.f};

    // Loads one 16-k group starting at kg.  GUARD: k may reach wend.
    auto load_group = [&]<bool GUARD>(int64_t kg, vf4 (&ya)[4], vf4 (&xa)[RG]) {
        const int64_t k4 = kg + 4 * fk;
        if constexpr (DOT) {
#pragma unroll
            for (int t = 0; t < 4; t++) {
                if (!GUARD) {
                    // Plain loads: non-temporal ones measured 7% slower here
                    // (32 rows), against 4% faster in the other form.
                    ya[t] = yin[t] ? load4<YVEC>(yrow[t] + k4) : (vf4){0.f, 0.f, 0.f, 0.f};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) ya[t][e] = (yin[t] && k4 + e < wend) ? yrow[t][k4 + e] : 0.f;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t k = k4 + e;
                const float *p = Y + k * g.yl + j0 + 4 * fi;
                const bool kin = !GUARD || k < wend;
                if (YVEC && kin && ncols == 4) {
                    ya[e] = load4_stream(p);
                } else {
#pragma unroll
                    for (int c = 0; c < 4; c++) ya[e][c] = (kin && c < ncols) ? p[c] : 0.f;
                }
            }
        }
#pragma unroll
        for (int rg = 0; rg < RG; rg++) {
            if (!GUARD && XVEC) {
                xa[rg] = load4<true>(xrow[rg] + k4);  // rows past R: row 0, into rows never stored
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    xa[rg][e] = (xin[rg] && (!GUARD || k4 + e < wend)) ? xrow[rg][(k4 + e) * g.xk] : 0.f;
            }
        }
    };

    auto mma_group = [&](const vf4 (&ya)[4], const vf4 (&xa)[RG]) {
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
            for (int rg = 0; rg < RG; rg++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    acc[rg][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[rg][e], DOT ? ya[t][e] : ya[e][t],
                                                                      acc[rg][t], 0, 0, 0);
    };

    for (int64_t k0 = wbeg; k0 < wend; k0 += kStepK) {
        const bool whole = k0 + kStepK <= wend;
#pragma unroll
        for (int h = 0; h < kStepK / 16; h += kGroups) {
            vf4 ya[kGroups][4], xa[kGroups][RG];
            if (whole) {
#pragma unroll
                for (int u = 0; u < kGroups; u++)
                    load_group.template operator()<false>(k0 + 16 * (h + u), ya[u], xa[u]);
            } else {
#pragma unroll
                for (int u = 0; u < kGroups; u++)
                    load_group.template operator()<true>(k0 + 16 * (h + u), ya[u], xa[u]);
            }
#pragma unroll
            for (int u = 0; u < kGroups; u++) mma_group(ya[u], xa[u]);
        }
    }

    // Waves' accumulators added in wave order; wave w finishes sub-tile w.
    // Lane (fi, fk) holds output rows 16rg + 4fk + r of sub-tile t's column
    // for lane slot fi.
    __shared__ float red[kWaves][RG * 16][64];
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[wave][rg * 16 + t * 4 + r][lane] = acc[rg][t][r];
    __syncthreads();
    const int t = wave;
    const int64_t j = DOT ? j0 + 16 * t + fi : j0 + 4 * fi + t;
    float *O = g.o + b * g.bo + s * g.os;
#pragma unroll
    for (int rg = 0; rg < RG; rg++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int q = rg * 16 + t * 4 + r;
            float v = red[0][q][lane];
#pragma unroll
            for (int w = 1; w < kWaves; w++) v += red[w][q][lane];
            const int64_t i = 16 * rg + 4 * fk + r;
            if (i < g.R && j < g.L) O[i * g.oi + j * g.oj] = v;
        }
    }
}

// Dot-form products with at most 4 short rows, on the VALU: padded to 16
// rows, each float4 of Y would cost four 32-cycle MFMAs, and the MFMA
// fragments read each row of Y in 64-byte pieces.  Here a block owns
// kGemvRows rows of Y (output columns) over the whole of K, its 4 waves take
// consecutive quarters of K, and a lane reads 16 bytes of a row per
// instruction, so one instruction reads 1 KiB of one row.  Each lane sums its
// k in order, the lanes' sums are added by a fixed shuffle tree and the
// waves' in wave order.  No split of K across blocks, so no slice pass.
constexpr int kGemvRows = 4;

template <int RR, bool XVEC>
__global__ void __launch_bounds__(256) gemv_f32_dot(SkinnyArgs g) {
    constexpr int U = (RR == 4 || !XVEC) ? 2 : 4;  // 256-k steps loaded before the FMAs
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t nb = (uint32_t)((g.L + kGemvRows - 1) / kGemvRows);  // blocks <= INT32_MAX: 32-bit division
    const uint32_t bq = blockIdx.x / nb;
    const int64_t b = bq, j0 = (int64_t)(blockIdx.x - bq * nb) * kGemvRows;
    const float *X = g.x + b * g.bx;
    const float *Y = g.y + b * g.by;
    const int64_t kq = (g.K + 4 * 256 - 1) / (4 * 256) * 256;
    const int64_t kb = wave * kq, ke = std::min(g.K, kb + kq);

    const float *yrow[kGemvRows];
    bool yin[kGemvRows];
#pragma unroll
    for (int t = 0; t < kGemvRows; t++) {
        yin[t] = j0 + t < g.L;
        yrow[t] = Y + (yin[t] ? j0 + t : 0) * g.yl;
    }
    const float *xrow[RR];
    bool xin[RR];
#pragma unroll
    for (int i = 0; i < RR; i++) {
        xin[i] = i < g.R;
        xrow[i] = X + (xin[i] ? i : 0) * g.xi;
    }
    float acc[kGemvRows][RR];
#pragma unroll
    for (int t = 0; t < kGemvRows; t++)
#pragma unroll
        for (int i = 0; i < RR; i++) acc[t][i] = 0.f;

    auto fma4 = [&](const vf4 (&y)[kGemvRows], const vf4 (&x)[RR]) {
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int t = 0; t < kGemvRows; t++)
#pragma unroll
                for (int i = 0; i < RR; i++) acc[t][i] += x[i][c] * y[t][c];
    };
    // Whole steps load with no condition: a row of Y past L, or of X past R,
    // reads row 0 (the pointers are clamped) into sums that are never stored,
    // so there is no branch per load.
    auto load_step = [&](int64_t k, vf4 (&y)[kGemvRows], vf4 (&x)[RR]) {
#pragma unroll
        for (int t = 0; t < kGemvRows; t++) y[t] = load4_stream(yrow[t] + k);
#pragma unroll
        for (int i = 0; i < RR; i++) {
            if (XVEC) x[i] = load4<true>(xrow[i] + k);
            else x[i] = (vf4){xrow[i][k * g.xk], xrow[i][(k + 1) * g.xk], xrow[i][(k + 2) * g.xk], xrow[i][(k + 3) * g.xk]};
        }
    };

    int64_t k0 = kb;
    if (k0 + 256 * U <= ke && k0 + 2 * 256 * U > ke) {
        // A range of one batch (K = 4096 at U = 4, the common case): every
        // load goes out before the first FMA.  Left to the compiler, the
        // loop below is software-pipelined and issues only part of a batch's
        // loads up front: [1,4096] @ W.mT took 16.5 us that way, 14.0 us
        // this way (15.4 with a branch around each load).  Several batches
        // keep the compiler's pipelined loop; a barrier in every batch
        // measured 2-6% slower there with 2 or 4 short rows.
        vf4 y[U][kGemvRows], x[U][RR];
#pragma unroll
        for (int u = 0; u < U; u++) load_step(k0 + 256 * u + 4 * lane, y[u], x[u]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; u++) fma4(y[u], x[u]);
        k0 += 256 * U;
    }
    for (; k0 + 256 * U <= ke; k0 += 256 * U) {
        vf4 y[U][kGemvRows], x[U][RR];
#pragma unroll
        for (int u = 0; u < U; u++) load_step(k0 + 256 * u + 4 * lane, y[u], x[u]);
#pragma unroll
        for (int u = 0; u < U; u++) fma4(y[u], x[u]);
    }
    for (; k0 + 256 <= ke; k0 += 256) {
        vf4 y[kGemvRows], x[RR];
        load_step(k0 + 4 * lane, y, x);
        fma4(y, x);
    }
    if (k0 < ke) {  // ragged end of the wave's range: element by element
        vf4 y[kGemvRows], x[RR];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int64_t k = k0 + 4 * lane + c;
            const bool kin = k < ke;
#pragma unroll
            for (int t = 0; t < kGemvRows; t++) y[t][c] = (kin && yin[t]) ? yrow[t][k] : 0.f;
#pragma unroll
            for (int i = 0; i < RR; i++) x[i][c] = (kin && xin[i]) ? xrow[i][k * g.xk] : 0.f;
        }
        fma4(y, x);
    }

    __shared__ float red[4][kGemvRows * RR];
#pragma unroll
    for (int t = 0; t < kGemvRows; t++)
#pragma unroll
        for (int i = 0; i < RR; i++) {
            float v = acc[t][i];
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0) red[wave][t * RR + i] = v;
        }
    __syncthreads();
    if (threadIdx.x < kGemvRows * RR) {
        const int q = threadIdx.x, t = q / RR, i = q % RR;
        if (j0 + t < g.L && i < g.R) {
            float v = red[0][q];
#pragma unroll
            for (int w = 1; w < 4; w++) v += red[w][q];
            g.o[b * g.bo + i * g.oi + (j0 + t) * g.oj] = v;
        }
    }
}

// The other form (Y unit-stride along the output columns j, e.g. x @ W)
// with at most 8 short rows, on the VALU: padded to 16 MFMA rows it does 2
// to 16 times the arithmetic it needs, and the MFMA fragments read each row
// of Y in 256-byte pieces.  A block of kAxpyWaves waves owns kAxpyCols
// columns (one float4 per lane, so one load instruction reads 1 KiB of a row
// of Y) and one slice of kc rows of Y, which its waves split into
// consecutive parts.  A wave loads kAxpyInFlight rows of Y before their
// FMAs.  The X elements those rows need are the same for every lane of the
// wave, so they come through scalar loads and cost no vector-memory
// instruction.  Each lane adds its rows in increasing k with one fused
// multiply-add per element, the waves' sums are added in wave order through
// LDS, and the slices in slice order.  Measured on the box (a standalone
// probe of this form with the inputs rotated past the cache, main pass
// only): x[8,4096] @ W 12.5 us against 15.8 us for the MFMA form's 16 x 64
// tiles; x[1,4096] @ W 11.2 us against 13.6 us for the former VALU form
// (32-lane groups each reading one row's X through vector loads, at most 2
// rows); 16 rows 15.8 us, no gain over the MFMA form, so it takes at most 8.
// 8 waves per block and one block per CU measured fastest (256 blocks of
// 4 waves, 512 blocks and 16 waves per block: 13.3-15.6 us).
constexpr int kAxpyMaxRows = 8;
constexpr int kAxpyWaves = 8;
constexpr int kAxpyInFlight = 8;  // rows of Y loaded before their FMAs per lane

// RR: the rows compiled for (1, 2, 4 or 8, at least R).  X's offsets within
// a batch are 32-bit (the host takes this kernel only when they fit), and
// XK1 (X unit-stride along k) lets a row's U values come in one scalar load:
// with 64-bit offsets and a run-time k stride the 8-row kernel spilled 24
// scalar registers to VGPR lanes.
template <int RR, bool XK1>
__global__ void __launch_bounds__(64 * kAxpyWaves) gemv_f32_axpy(SkinnyArgs g) {
    constexpr int U = kAxpyInFlight;
    // X values held in scalar registers at once: 8 rows x 8 steps (64) left
    // too few for the addresses and spilled 17 to VGPR lanes.
    constexpr int UH = RR * U > 32 ? U / 2 : U;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const BlockCoords bc = block_coords(g);
    const int64_t jb = bc.jb, s = bc.s, b = bc.b;
    const int64_t j0 = jb * kAxpyCols;
    const int64_t j = j0 + 4 * lane;
    const bool jin = j < g.L;  // L is a multiple of 4: a lane's float4 is all in or all out
    // The slice's rows, split among the waves in parts of a whole number of
    // U-row steps (kc is a multiple of kAxpyWaves * U when K is split; an
    // unsplit product has kc = K, any length, and its last parts are short
    // or empty).
    const int64_t kbeg = s * g.kc, kend = std::min(g.K, kbeg + g.kc);
    const int64_t kw = ((g.kc + kAxpyWaves - 1) / kAxpyWaves + U - 1) / U * U;
    const int64_t wbeg = std::min(kend, kbeg + wave * kw), wend = std::min(kend, wbeg + kw);
    const float *yp = g.y + b * g.by + (jin ? j : 0);
    const float *xb = g.x + b * g.bx;
    // Row i's X at xb[xrow[i] + k * xk]; rows past R read row 0 into sums
    // that are never stored.
    const uint32_t xk = XK1 ? 1u : (uint32_t)g.xk;
    uint32_t xrow[RR];
#pragma unroll
    for (int i = 0; i < RR; i++) xrow[i] = (uint32_t)((i < g.R ? i : 0) * g.xi);

    vf4 acc[RR];
#pragma unroll
    for (int i = 0; i < RR; i++) acc[i] = (vf4){0.f, 0.f, 0.f, 0.f};
    // A step: U rows of Y (lanes past L read column 0 of each, into sums
    // that are never stored, so no load waits on a lane test), then every
    // row's X values in one scalar load each, then the FMAs in increasing k,
    // each row of Y used as soon as it lands.
    int64_t k = wbeg;
    for (; k + U <= wend; k += U) {
        vf4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = load4_stream(yp + (k + u) * g.yl);
        const uint32_t xo = (uint32_t)k * xk;
#pragma unroll
        for (int h = 0; h < U; h += UH) {
            float xv[RR][UH];
#pragma unroll
            for (int i = 0; i < RR; i++) {
                // Indexed from the row's pointer, so that with XK1 the
                // values are known to be adjacent and come in one scalar
                // load (offsets summed in 32 bits could wrap, which kept
                // them apart).
                const float *xr = xb + (xrow[i] + xo);
#pragma unroll
                for (int u = 0; u < UH; u++) xv[i][u] = xr[XK1 ? h + u : (int64_t)(h + u) * xk];
            }
#pragma unroll
            for (int u = 0; u < UH; u++)
#pragma unroll
                for (int i = 0; i < RR; i++)
#pragma unroll
                    for (int c = 0; c < 4; c++) acc[i][c] = __builtin_fmaf(xv[i][u], v[h + u][c], acc[i][c]);
            // Keeps the scheduler from hoisting the next half's scalar loads.
            if constexpr (UH < U) __builtin_amdgcn_sched_barrier(0);
        }
    }
    for (; k < wend; k++) {
        const vf4 v = load4_stream(yp + k * g.yl);
#pragma unroll
        for (int i = 0; i < RR; i++) {
            const float xv = xb[xrow[i] + (uint32_t)k * xk];
#pragma unroll
            for (int c = 0; c < 4; c++) acc[i][c] = __builtin_fmaf(xv, v[c], acc[i][c]);
        }
    }

    __shared__ float red[kAxpyWaves][RR][kAxpyCols];
#pragma unroll
    for (int i = 0; i < RR; i++)
#pragma unroll
        for (int c = 0; c < 4; c++) red[wave][i][4 * lane + c] = acc[i][c];
    __syncthreads();
    float *O = g.o + b * g.bo + s * g.os;
    for (int q = threadIdx.x; q < RR * kAxpyCols; q += 64 * kAxpyWaves) {
        const int i = q / kAxpyCols, cc = q - i * kAxpyCols;
        float r = red[0][i][cc];
#pragma unroll
        for (int w = 1; w < kAxpyWaves; w++) r += red[w][i][cc];
        if (i < g.R && j0 + cc < g.L) O[i * g.oi + (j0 + cc) * g.oj] = r;
    }
}

// Dot-form products with 5..32 short rows (x[32,K] @ W.mT): the same MFMA
// arithmetic, with Y streamed through LDS.  Here X's fragment loads
// (16 rows 16 KiB apart per instruction, twice Y's) set the time when each
// lane reads its fragments from global memory; instead every slice of 32 k
// -- 64 rows of Y and the 32 rows of X -- goes to LDS by
// global_load_lds_dwordx4 through a 4-stage pipeline (three slices in
// flight), and the fragments are read from LDS.  A block owns 64 output
// columns and one K slice; its 4 waves own 16 columns each.  Rows of X past
// R and of Y past L read row 0 / L-1 into sums that are never stored.  Tiles
// in LDS keep their 16-byte chunks XOR-swizzled by row (chunk c of row r at
// c ^ (r & 7)).  Measured on the box for x[32,4096] @ W.mT: 18.0-18.8 us per
// call against 23.6 us for the register-fed kernel above (8, 12 and 16
// rows: 16.7-17.4 against 21.0-22.6 us); 8 waves, 128 columns per block, 2
// or 6 stages, or 4 or 16 slices were slower.
constexpr int kLdsSkinnyStages = 4;

template <int RG>
__global__ void __launch_bounds__(256) gemm_f32_skinny_lds(SkinnyArgs g) {
    constexpr int BK = 32, NST = kLdsSkinnyStages, P = NST - 1;
    constexpr int WSZ = kLdsSkinnyCols * BK, XSZ = 32 * BK, STG = WSZ + XSZ;
    __shared__ __attribute__((aligned(16))) float lds[NST * STG];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int fi = lane & 15, fk = lane >> 4;
    const BlockCoords bc = block_coords(g);
    const int64_t jb = bc.jb, s = bc.s, b = bc.b;
    const int64_t j0 = jb * kLdsSkinnyCols;
    const int64_t kbeg = s * g.kc, kend = std::min(g.K, kbeg + g.kc);
    const int nsl = (int)((kend - kbeg) / BK);  // K and kc are multiples of 32
    const float *ybase = g.y + b * g.by + j0 * g.yl + kbeg;
    const float *xbase = g.x + b * g.bx + kbeg;
    // Y: 8 segments of 8 rows per slice, two per wave.  X: 4 segments, one
    // for each wave.  Byte offsets from the slice bases.
    uint32_t yoff[2], yseg[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int sg = wave + 4 * q;
        const int r = sg * 8 + (lane >> 3);
        const int64_t jr = std::min<int64_t>(r, g.L - 1 - j0);
        const int c = (lane & 7) ^ (r & 7);
        yoff[q] = (uint32_t)((jr * g.yl + 4 * c) * 4);
        yseg[q] = sg * 1024;
    }
    const int xr = wave * 8 + (lane >> 3);
    const uint32_t xoff = (uint32_t)(((xr < g.R ? xr : 0) * g.xi + 4 * ((lane & 7) ^ (xr & 7))) * 4);
    const uint32_t xseg = WSZ * 4 + wave * 1024;
    auto issue = [&](int sl) {
        const uint32_t at = lds_address(lds + (sl % NST) * STG);
#pragma unroll
        for (int q = 0; q < 2; q++) lds_dma16(ybase + sl * BK, yoff[q], at + yseg[q]);
        lds_dma16(xbase + sl * BK, xoff, at + xseg);
    };
    typedef float vf4acc __attribute__((ext_vector_type(4)));
    vf4acc acc[RG];
#pragma unroll
    for (int i = 0; i < RG; i++) acc[i] = (vf4acc){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < P; q++)
        if (q < nsl) issue(q);
    const int sw = fi & 7;     // rows 16i + fi of X and wn0 + fi of Y
    const int wn0 = wave * 16;
    for (int sl = 0; sl < nsl; sl++) {
        // Slice sl must have landed; slices sl+1 .. sl+P-1 (3 loads each) may
        // still be in flight, except near the end, where fewer were issued.
        if (sl + P <= nsl) __builtin_amdgcn_s_waitcnt(vmcnt_at_most((P - 1) * 3));
        else __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // every wave's loads of slice sl; every read of slice sl-1
        if (sl + P < nsl) issue(sl + P);  // into the buffer slice sl-1 used
        const float *Ys = lds + (sl % NST) * STG, *Xs = Ys + WSZ;
#pragma unroll
        for (int kg = 0; kg < BK; kg += 16) {
            const int c = ((kg / 4 + fk) ^ sw) << 2;
            const vf4 w4 = *(const vf4 *)(Ys + (wn0 + fi) * BK + c);
            vf4 x4[RG];
#pragma unroll
            for (int i = 0; i < RG; i++) x4[i] = *(const vf4 *)(Xs + (i * 16 + fi) * BK + c);
#pragma unroll
            for (int e = 0; e < 4; e++)
#pragma unroll
                for (int i = 0; i < RG; i++) acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(x4[i][e], w4[e], acc[i], 0, 0, 0);
        }
    }
    float *O = g.o + b * g.bo + s * g.os;
    const int64_t j = j0 + wn0 + fi;
#pragma unroll
    for (int i = 0; i < RG; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int64_t row = 16 * i + 4 * fk + r;
            if (row < g.R && j < g.L) O[row * g.oi + j * g.oj] = acc[i][r];
        }
}

// c[e] = ((p0 + p1) + p2) + ... over the S slices of e's batch, in slice
// order.  Slice s of batch b starts at ws + (b*S + s)*mn.  The element
// index e = b*mn + r (and r = i*L + j when scattering) is split in 32-bit
// arithmetic unless WIDE (outputs of 2^32 elements or more): one 64-bit
// division per lane, a long VALU sequence ahead of the loads, made this pass
// 1.4 us slower, and both widths in one kernel compile to both divisions.
// NS is S when 2 <= S <= 16, else 0 (S read at run time).  The sum of a
// matrix-vector product is a few KB, so its time is load latency: with NS
// all loads go out before the first add, with no branch between them (a
// copy at a branch join waits for every load issued before it; conditional
// loads made this pass 1.2 us slower).
template <bool WIDE, int NS>
__global__ void __launch_bounds__(kHelperLanes) slice_sum(const float *__restrict__ ws, float *__restrict__ c, int64_t mn,
                                                  int64_t total, int S, SliceOut out) {
    typedef std::conditional_t<WIDE, int64_t, uint32_t> Index;
    const int64_t e = (int64_t)blockIdx.x * kHelperLanes + threadIdx.x;
    if (e >= total) return;
    const Index b = total > mn ? (Index)e / (Index)mn : 0;
    const Index r = (Index)e - b * (Index)mn;
    const float *p = ws + (int64_t)b * S * mn + (int64_t)r;
    float v;
    if constexpr (NS > 0) {
        float part[NS];
        const float *pq = p;
#pragma unroll
        for (int q = 0; q < NS; q++) {
            part[q] = *pq;
            if (q + 1 < NS) pq += mn;
        }
        v = part[0];
#pragma unroll
        for (int q = 1; q < NS; q++) v += part[q];
    } else {
        v = p[0];
        for (int q = 1; q < S; q++) v += p[(int64_t)q * mn];
    }
    if (!out.scatter) {
        c[e] = v;
    } else {
        const Index i = r / (Index)out.L, j = r - i * (Index)out.L;
        c[(int64_t)b * out.bo + (int64_t)i * out.oi + (int64_t)j * out.oj] = v;
    }
}

template <bool WIDE, int NS = 2>
void launch_slices(int S, dim3 grid, hipStream_t s, const float *ws, float *c, int64_t mn, int64_t total,
                   const SliceOut &out) {
    if constexpr (NS > 16) hipLaunchKernelGGL((slice_sum<WIDE, 0>), grid, dim3(kHelperLanes), 0, s, ws, c, mn, total, S, out);
    else if (S == NS) hipLaunchKernelGGL((slice_sum<WIDE, NS>), grid, dim3(kHelperLanes), 0, s, ws, c, mn, total, S, out);
    else launch_slices<WIDE, NS + 1>(S, grid, s, ws, c, mn, total, out);
}

template <bool DOT, bool YVEC, bool XVEC>
int launch_rg(int rg, dim3 grid, hipStream_t s, const SkinnyArgs &g) {
    if (rg == 1) hipLaunchKernelGGL((gemm_f32_skinny<DOT, YVEC, XVEC, 1>), grid, dim3(256), 0, s, g);
    else hipLaunchKernelGGL((gemm_f32_skinny<DOT, YVEC, XVEC, 2>), grid, dim3(256), 0, s, g);
    TRS_LAUNCH_CHECK("skinny gemm launch");
    return TRS_OK;
}

template <bool DOT>
int launch_form(bool xvec, int rg, dim3 grid, hipStream_t s, const SkinnyArgs &g) {
    return xvec ? launch_rg<DOT, true, true>(rg, grid, s, g) : launch_rg<DOT, true, false>(rg, grid, s, g);
}


}  // namespace

bool plan_skinny(const SkinnyProblem &p, int cu_count, SkinnyPlan *plan) {
    if (p.R < 1 || p.R > kSkinnyMaxRows || p.L < 1 || p.K < 1 || p.batch < 1 || cu_count < 1) return false;
    SkinnyPlan pl;
    pl.row_groups = p.R <= 16 ? 1 : 2;
    // Float4 loads need only dword alignment (vf4u): Y is always read as
    // float4 where a whole float4 lies in its row, X when unit-stride along k.
    pl.yvec = true;
    pl.xvec = p.xk == 1;
    // The VALU matrix-vector kernel: dot form, at most 4 short rows, a K long
    // enough that each wave's quarter covers its 64 lanes, and enough rows
    // for two blocks per CU.  Every block reads all of X, element by element
    // when it is strided along k: a long stride (a GEMM's column rim, one
    // cache line per element) goes to the MFMA kernel, which reads X once
    // per 64 columns (27.5 us against 20.4 on the 4097^3 rim).
    const int64_t gemv_blocks = (p.L + kGemvRows - 1) / kGemvRows * p.batch;
    if (p.dot && pl.yvec && p.R <= 4 && p.xk <= 4 && p.K >= 1024 && gemv_blocks >= 2 * (int64_t)cu_count &&
        gemv_blocks <= INT32_MAX) {
        pl.gemv = true;
        pl.row_groups = p.R == 1 ? 1 : p.R == 2 ? 2 : 4;
        pl.kc = (p.K + 4 * 256 - 1) / (4 * 256) * 256;
        pl.splits = 1;
        pl.blocks = gemv_blocks;
        *plan = pl;
        return true;
    }
    // The VALU axpy kernel: Y unit-stride along j and read as float4, at most
    // kAxpyMaxRows short rows, and K deep enough for a 64-row slice per
    // block, X unit-stride along k when it has more than 2 rows (a strided
    // X's values load one by one, and 4 or 8 rows of them spilled scalar
    // registers), and X's offsets within a batch below 2^31.  About one block (8
    // waves) per CU, slices of a multiple of kAxpyWaves * kAxpyInFlight
    // rows, and the partial products' traffic (written and read back) at
    // most 1/8 of Y's.  Compiled for 1, 2, 4 or 8 rows; R rounds up to the
    // next.
    if (!p.dot && pl.yvec && p.R <= kAxpyMaxRows && p.L % 4 == 0 && p.K >= 64 && (p.xk == 1 || p.R <= 2) &&
        (p.R - 1) * p.xi + (p.K - 1) * p.xk < ((int64_t)1 << 31)) {
        constexpr int64_t kStep = kAxpyWaves * kAxpyInFlight;
        const int64_t jb = (p.L + kAxpyCols - 1) / kAxpyCols;
        const int64_t ab = jb * p.batch;
        const int64_t want = ((int64_t)cu_count + ab - 1) / ab;
        const int64_t cap = std::max<int64_t>(1, std::min(p.K / kStep, p.K / (16 * p.R)));
        int64_t S = std::clamp<int64_t>(want, 1, cap);
        int64_t kc = (p.K + S - 1) / S;
        kc = (kc + kStep - 1) / kStep * kStep;
        S = (p.K + kc - 1) / kc;
        if (ab * S <= INT32_MAX && jb <= INT32_MAX) {
            pl.axpy = true;
            pl.row_groups = p.R <= 1 ? 1 : p.R <= 2 ? 2 : p.R <= 4 ? 4 : 8;
            pl.kc = kc;
            pl.splits = S;
            pl.blocks = ab * S;
            *plan = pl;
            return true;
        }
    }
    // The LDS-streaming kernel: dot form, 5..32 short rows, X unit-stride
    // along k, K a multiple of 32, 64 rows of Y (and 32 of X) within 2^31
    // bytes of a slice's base.  About 2 blocks per CU, slices of whole
    // 32-k steps, and the partial products' traffic at most 1/8 of Y's.
    if (p.dot && p.R > 4 && p.xk == 1 && p.K % 32 == 0 && 64 * p.yl * 4 < ((int64_t)1 << 31) &&
        32 * p.xi * 4 < ((int64_t)1 << 31)) {
        const int64_t jb = (p.L + kLdsSkinnyCols - 1) / kLdsSkinnyCols;
        const int64_t ab = jb * p.batch;
        const int64_t want = (2 * (int64_t)cu_count + ab - 1) / ab;
        const int64_t cap = std::max<int64_t>(1, std::min(p.K / 256, p.K / (16 * p.R)));
        int64_t S = std::clamp<int64_t>(want, 1, cap);
        int64_t kc = (p.K + S - 1) / S;
        kc = (kc + 31) / 32 * 32;
        S = (p.K + kc - 1) / kc;
        if (ab * S <= INT32_MAX && jb <= INT32_MAX) {
            pl.lds = true;
            pl.row_groups = p.R <= 16 ? 1 : 2;
            pl.kc = kc;
            pl.splits = S;
            pl.blocks = ab * S;
            *plan = pl;
            return true;
        }
    }
    const int64_t jblocks = (p.L + kSkinnyCols - 1) / kSkinnyCols;
    const int64_t base = jblocks * p.batch;
    // ~4 blocks per CU; each slice at least 128 deep (one step per wave), and
    // the partial products' traffic (written and read back) at most 1/8 of Y's.
    const int64_t want = (4 * (int64_t)cu_count + base - 1) / base;
    const int64_t cap = std::max<int64_t>(1, std::min(p.K / 128, p.K / (16 * p.R)));
    int64_t S = std::clamp<int64_t>(want, 1, cap);
    int64_t kc = (p.K + S - 1) / S;
    kc = (kc + 127) / 128 * 128;
    S = (p.K + kc - 1) / kc;
    if (base * S > INT32_MAX || jblocks > INT32_MAX) return false;
    pl.kc = kc;
    pl.splits = S;
    pl.blocks = base * S;
    *plan = pl;
    return true;
}

int launch_slice_sum(const float *ws, float *c, int64_t mn, int64_t batch, int64_t S, hipStream_t s,
                     const SliceOut &out) {
    const int64_t total = mn * batch;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (total > (int64_t)UINT32_MAX) launch_slices<true>((int)S, grid, s, ws, c, mn, total, out);
    else launch_slices<false>((int)S, grid, s, ws, c, mn, total, out);
    TRS_LAUNCH_CHECK("gemm slice sum launch");
    return TRS_OK;
}

int run_skinny(const SkinnyProblem &p, const SkinnyPlan &plan, hipStream_t s) {
    SkinnyArgs g{};
    if (plan.gemv) {
        g.x = p.x, g.y = p.y, g.o = p.out;
        g.xi = p.xi, g.xk = p.xk, g.yl = p.yl;
        g.oi = p.oi, g.oj = p.oj, g.bo = p.bo ? p.bo : p.R * p.L;
        g.bx = p.bx, g.by = p.by;
        g.R = p.R, g.L = p.L, g.K = p.K;
        const dim3 grid((unsigned)plan.blocks);
        const int rr = plan.row_groups;
        if (plan.xvec) {
            if (rr == 1) hipLaunchKernelGGL((gemv_f32_dot<1, true>), grid, dim3(256), 0, s, g);
            else if (rr == 2) hipLaunchKernelGGL((gemv_f32_dot<2, true>), grid, dim3(256), 0, s, g);
            else hipLaunchKernelGGL((gemv_f32_dot<4, true>), grid, dim3(256), 0, s, g);
        } else {
            if (rr == 1) hipLaunchKernelGGL((gemv_f32_dot<1, false>), grid, dim3(256), 0, s, g);
            else if (rr == 2) hipLaunchKernelGGL((gemv_f32_dot<2, false>), grid, dim3(256), 0, s, g);
            else hipLaunchKernelGGL((gemv_f32_dot<4, false>), grid, dim3(256), 0, s, g);
        }
        TRS_LAUNCH_CHECK("gemv launch");
        return TRS_OK;
    }
    g.x = p.x;
    g.y = p.y;
    g.xi = p.xi;
    g.xk = p.xk;
    g.yl = p.yl;
    g.oi = p.oi;
    g.oj = p.oj;
    g.bx = p.bx;
    g.by = p.by;
    g.R = p.R;
    g.L = p.L;
    g.K = p.K;
    const int64_t cols = plan.axpy ? kAxpyCols : plan.lds ? kLdsSkinnyCols : kSkinnyCols;
    g.jblocks = (int32_t)((p.L + cols - 1) / cols);
    const int64_t mn = p.R * p.L;
    int64_t S = plan.splits, kc = plan.kc;
    void *ws = nullptr;
    // The split only adds blocks: without a workspace the product runs unsplit.
    if (S > 1 && trs_alloc((size_t)(S * mn * p.batch) * sizeof(float), &ws) != TRS_OK) {
        ws = nullptr;
        S = 1;
    }
    if (S == 1) kc = p.K;
    g.S = (int32_t)S;
    g.kc = kc;
    // The workspace holds each slice in the output's own element order when
    // the output is one contiguous product, else row-major (i, j), and the
    // slice pass scatters the sums to the output's strides.
    const int64_t bo = p.bo ? p.bo : mn;
    const bool compact = bo == mn && ((p.oi == p.L && p.oj == 1) || (p.oi == 1 && p.oj == p.R));
    SliceOut so;
    if (ws) {
        g.o = (float *)ws;
        g.os = mn;
        g.bo = S * mn;
        if (!compact) {
            g.oi = p.L;
            g.oj = 1;
            so.scatter = true;
            so.L = p.L, so.oi = p.oi, so.oj = p.oj, so.bo = bo;
        }
    } else {
        g.o = p.out;
        g.os = 0;
        g.bo = bo;
    }
    const dim3 grid((unsigned)((int64_t)g.jblocks * S * p.batch));
    int rc = TRS_OK;
    if (plan.axpy) {
        const dim3 block(64 * kAxpyWaves);
        // X with a k stride other than 1 is planned here only for R <= 2, so
        // only those row counts are compiled without XK1.
        if (p.xk != 1 && plan.row_groups > 2) return TRS_E_INVALID_ARGUMENT;
        auto axpy = [&]<bool XK1>() {
            if (plan.row_groups == 1) hipLaunchKernelGGL((gemv_f32_axpy<1, XK1>), grid, block, 0, s, g);
            else if (!XK1 || plan.row_groups == 2) hipLaunchKernelGGL((gemv_f32_axpy<2, XK1>), grid, block, 0, s, g);
            else if constexpr (XK1) {
                if (plan.row_groups == 4) hipLaunchKernelGGL((gemv_f32_axpy<4, true>), grid, block, 0, s, g);
                else hipLaunchKernelGGL((gemv_f32_axpy<8, true>), grid, block, 0, s, g);
            }
        };
        if (p.xk == 1) axpy.template operator()<true>();
        else axpy.template operator()<false>();
        TRS_LAUNCH_CHECK("axpy gemv launch");
    } else if (plan.lds) {
        if (plan.row_groups == 1) hipLaunchKernelGGL((gemm_f32_skinny_lds<1>), grid, dim3(256), 0, s, g);
        else hipLaunchKernelGGL((gemm_f32_skinny_lds<2>), grid, dim3(256), 0, s, g);
        TRS_LAUNCH_CHECK("skinny lds launch");
    } else {
        rc = p.dot ? launch_form<true>(plan.xvec, plan.row_groups, grid, s, g)
                   : launch_form<false>(plan.xvec, plan.row_groups, grid, s, g);
    }
    if (rc == TRS_OK && ws) rc = launch_slice_sum((const float *)ws, p.out, mn, p.batch, S, s, so);
    if (ws) {
        const int frc = trs_free(ws);
        if (!rc) rc = frc;
    }
    return rc;
}

}  // namespace trs
