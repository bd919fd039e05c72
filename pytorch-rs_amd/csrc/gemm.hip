// gemm.hip -- fp32 matmul on CDNA4 FP32 MFMA (v_mfma_f32_16x16x4_f32).
//
// Replaces Tensor::matmul's three CPU paths (src/tensor.rs:2453-2533,
// 3872-3994).  The reference computes each C[i,j] as a sequential sum
// (+0.0, then k ascending, mul and add rounded separately); this kernel keeps
// fp32 inputs and fp32 accumulation ("highest" precision,
// python/torch_rs/__init__.py:81-85) but sums in MFMA order, so it is checked
// against the reference within |dC| <= 1e-5*sqrt(K)*(|A||B|).
//
// Tiling: a block of WGM x WGN waves owns a BM x BN tile of C; each wave owns
// (BM/WGM) x (BN/WGN) as a grid of 16x16 MFMA tiles held in accumulators.
// Three shapes are used: 256x256 with 16 waves (one block per CU, 4 waves
// per SIMD, 140 KB of LDS) when the output has at least one such tile per CU
// (ragged M, N and K included: edge tiles clamp their loads, and rims of at
// most 32 rows or columns run as skinny products); else
// 128x128x32 with 8 waves (two blocks per CU), or 64x128x32 when 128x128
// would give fewer than two blocks per CU.  Measured on the MI355X at 4096^3:
// 84-88% of the FP32 MFMA peak for the large shape in every operand layout,
// against 71-80% for the small one.
// K advances in BK slices staged through LDS, double-buffered: the next
// slice's global loads are issued into registers before the MFMAs of the
// current slice and written to the other LDS buffer afterwards, so one
// barrier per slice suffices.  Each operand tile is copied to LDS in its
// memory order ([rows][contiguous cols] + padding), which serves both plain
// and transposed (.mT) operands; padding keeps fragment reads conflict-free,
// and the large tile reads k-contiguous tiles as one float4 per lane per 16 k.
// Blocks are remapped so that consecutive tiles share an XCD (each XCD has
// its own L2), and tiles are walked in groups of GROUP_M tile-rows.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "gemm_skinny.h"
#include "lds_dma.h"
#include "trs_internal.h"

namespace trs {

namespace {

typedef float vf4 __attribute__((ext_vector_type(4)));
// A float4 that may start at any float: global_load_dwordx4 needs only dword
// alignment, so rows of any length (4095, 2047 floats) load as vectors.
typedef float vf4u __attribute__((ext_vector_type(4), aligned(4)));

struct GemmArgs {
    const float *a;
    const float *b;
    float *c;
    int64_t M, N, K;
    int64_t lda;  // stride of A's non-unit dim (rows if !TA, k if TA)
    int64_t ldb;  // stride of B's non-unit dim (k if !TB, cols if TB)
    int64_t ldc;
    int64_t bsa, bsb, bsc;  // batch strides (elements)
    int64_t batch;
    // Split K (batches are K slices of depth K): the full depth, so the last
    // slice stops at ktotal; 0 when every batch has depth K.
    int64_t ktotal;
    int32_t tiles_m, tiles_n;
    int32_t xcd_remap;
    // Stream-K (gemm_f32_mfma_lds_sk and its fix-up pass): blocks, slices
    // per tile, (tile, slice) units, and the workspace of two partial tiles
    // per block.
    int64_t sk_blocks, sk_q, sk_units;
    float *sk_ws;
};

constexpr int kGroupM = 8;
constexpr int kXcds = 8;

// Load an R x C tile whose C dim is contiguous in memory (row stride ld),
// starting at (r0, c0) of an Rv x Cv matrix, into registers: NT lanes, one
// float4 each per step.  The float4 need only be dword-aligned.
//   kLoadFull: the tile lies inside the matrix.
//   kLoadClamp: the tile may cross the matrix's edge in its M or N dim
//     (never in k): rows past the edge read the last row, and a float4 that
//     crosses or passes the last column reads the row's last four floats,
//     shifted so that its columns inside the matrix hold their own values.
//     The values past the edge are real elements of the matrix: they meet
//     only outputs past M or N, which are not stored.  Needs Cv >= 4.
//   kLoadChecked: every element bounds-checked and zero outside (the ragged
//     k tail, where zeros are needed, and matrices narrower than 4).
constexpr int kLoadFull = 0, kLoadClamp = 1, kLoadChecked = 2;

template <int R, int C, int NT>
struct TileLoader {
    static constexpr int kVec = R * C / 4;          // float4 per tile
    static constexpr int kPerThread = kVec / NT;    // float4 per lane
    static_assert(kVec % NT == 0 && kPerThread >= 1, "tile must split evenly over the block");
    vf4 v[kPerThread];

    template <int MODE>
    __device__ __forceinline__ void load(const float *src, int64_t ld, int64_t r0, int64_t c0, int64_t Rv,
                                         int64_t Cv) {
#pragma unroll
        for (int i = 0; i < kPerThread; i++) {
            const int q = threadIdx.x + NT * i;
            const int r = q / (C / 4);
            const int c = (q % (C / 4)) * 4;
            const int64_t gr = r0 + r, gc = c0 + c;
            if constexpr (MODE == kLoadFull) {
                v[i] = *(const vf4u *)(src + gr * ld + gc);
            } else if constexpr (MODE == kLoadClamp) {
                // The shift of a float4 that crosses the edge is applied when
                // storing (store_shifted): selecting on the loaded values here
                // would wait for the prefetch before the slice's MFMAs.
                const int64_t cb = gc < Cv - 4 ? gc : Cv - 4;
                v[i] = *(const vf4u *)(src + (gr < Rv ? gr : Rv - 1) * ld + cb);
            } else {
                // Branch-free: an element outside the matrix loads the
                // matrix's first element instead and is replaced by 0, so
                // every load of the slice is issued before any is waited for.
                const bool rin = gr < Rv;
                const float *p = src + (rin ? gr : 0) * ld;
                vf4 t;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const bool in = rin && gc + e < Cv;
                    const float x = p[in ? gc + e : 0];
                    t[e] = in ? x : 0.f;
                }
                v[i] = t;
            }
        }
    }

    template <int PITCH>
    __device__ __forceinline__ void store(float *lds) const {
#pragma unroll
        for (int i = 0; i < kPerThread; i++) {
            const int q = threadIdx.x + NT * i;
            const int r = q / (C / 4);
            const int c = (q % (C / 4)) * 4;
            *(vf4 *)(lds + r * PITCH + c) = v[i];
        }
    }

    // store() of a kLoadClamp tile whose contiguous dim is M or N, starting
    // at c0 of Cv columns: a float4 that crossed the last column was read
    // from the row's last four floats, so its element e is that read's
    // element e + (column - (Cv - 4)) (capped at 3; the elements past the
    // edge meet no stored output).
    template <int PITCH>
    __device__ __forceinline__ void store_shifted(float *lds, int64_t c0, int64_t Cv) const {
#pragma unroll
        for (int i = 0; i < kPerThread; i++) {
            const int q = threadIdx.x + NT * i;
            const int r = q / (C / 4);
            const int c = (q % (C / 4)) * 4;
            const int64_t d = c0 + c - (Cv - 4);
            const int sh = d <= 0 ? 0 : d < 3 ? (int)d : 3;
            // Shift down by 1, then by 2, each a per-element select (nested
            // selects on a computed index compiled to branches).
            const bool s1 = (sh & 1) != 0, s2 = (sh & 2) != 0;
            const vf4 x = v[i];
            const float y0 = s1 ? x[1] : x[0], y1 = s1 ? x[2] : x[1], y2 = s1 ? x[3] : x[2], y3 = x[3];
            vf4 t;
            t[0] = s2 ? y2 : y0;
            t[1] = s2 ? y3 : y1;
            t[2] = s2 ? y3 : y2;
            t[3] = y3;
            *(vf4 *)(lds + r * PITCH + c) = t;
        }
    }
};

template <int BM, int BN, int BK, int WGM, int WGN, int MINB, bool VK, bool TA, bool TB, bool FULL>
__global__ void __launch_bounds__(WGM *WGN * 64, MINB) gemm_f32_mfma(GemmArgs args) {
    constexpr int NT = WGM * WGN * 64;          // lanes per block
    constexpr int WM = BM / WGM, WN = BN / WGN; // wave tile
    constexpr int TM = WM / 16, TN = WN / 16;   // MFMA tiles per wave
    // LDS tile shapes in memory order.
    constexpr int AR = TA ? BK : BM, AC = TA ? BM : BK;  // A: [m][k] or [k][m]
    constexpr int BR = TB ? BN : BK, BC = TB ? BK : BN;  // B: [k][n] or [n][k]
    static_assert(BK % 16 == 0, "fragments are read in 16-wide k groups");
    // Pitches (floats), all multiples of 4 so float4 rows stay aligned.
    // k-contiguous tiles ([m][k], [n][k]) take +4: 8 lanes' float4 reads of
    // rows m..m+7 cover all 32 banks.  k-row tiles ([k][m], [k][n]) take +4
    // under VK, where lanes fk and fk+1 read rows k and k+4 (16 banks apart),
    // and +16 otherwise, where they read rows k and k+1.
    constexpr int APITCH = AC + ((TA && !VK) ? 16 : 4);
    constexpr int BPITCH = BC + ((!TB && !VK) ? 16 : 4);
    constexpr int ASIZE = AR * APITCH, BSIZE = BR * BPITCH;
    __shared__ __attribute__((aligned(16))) float lds[2 * (ASIZE + BSIZE)];

    // ---- tile selection (XCD-aware, grouped) ----
    const int64_t tiles = (int64_t)args.tiles_m * args.tiles_n;
    int64_t bid = blockIdx.x;
    if (args.xcd_remap) {
        const int64_t total = tiles * args.batch;
        const int64_t per_xcd = total / kXcds;
        bid = (bid % kXcds) * per_xcd + bid / kXcds;
    }
    const int64_t batch_idx = bid / tiles;
    int64_t t = bid - batch_idx * tiles;
    const int64_t group_span = (int64_t)kGroupM * args.tiles_n;
    const int64_t group = t / group_span;
    const int64_t first_m = group * kGroupM;
    const int64_t gm = std::min<int64_t>(args.tiles_m - first_m, kGroupM);
    const int64_t within = t - group * group_span;
    const int64_t tile_m = first_m + within % gm;
    const int64_t tile_n = within / gm;

    const int64_t Kb = args.ktotal ? std::min<int64_t>(args.K, args.ktotal - batch_idx * args.K) : args.K;
    const float *A = args.a + batch_idx * args.bsa;
    const float *B = args.b + batch_idx * args.bsb;
    float *Cp = args.c + batch_idx * args.bsc;
    const int64_t m0 = tile_m * BM, n0 = tile_n * BN;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;

    TileLoader<AR, AC, NT> la;
    TileLoader<BR, BC, NT> lb;

    typedef float vf4acc __attribute__((ext_vector_type(4)));
    vf4acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (vf4acc){0.f, 0.f, 0.f, 0.f};

    // MODE: how a slice loads (kLoadFull, kLoadClamp, kLoadChecked above).
    auto load_tiles = [&]<int MODE>(int64_t k0) {
        if constexpr (TA) la.template load<MODE>(A, args.lda, k0, m0, Kb, args.M);
        else la.template load<MODE>(A, args.lda, m0, k0, args.M, Kb);
        if constexpr (TB) lb.template load<MODE>(B, args.ldb, n0, k0, args.N, Kb);
        else lb.template load<MODE>(B, args.ldb, k0, n0, Kb, args.N);
    };
    // The edge-guarded kernel loads every slice of whole k as float4,
    // clamped at M and N (kLoadClamp: inside the matrix it reads exactly what
    // kLoadFull does), and checks bounds only in the ragged last slice -- or
    // in every slice when a contiguous dim is shorter than 4 (no float4
    // fits).  With every element of an edge tile bounds-checked, 4095^3 took
    // 1.26 ms (all its blocks run at once, so the edge tiles set the pace);
    // clamped, 1.02 ms, and 2047^3 on the 128x128 tile 195 -> 154 us.
    const int64_t kslices = (Kb + BK - 1) / BK;
    const bool clampable = (TA ? args.M : Kb) >= 4 && (TB ? Kb : args.N) >= 4;
    const int64_t kvec = FULL ? kslices : (clampable ? Kb / BK : 0);
    // Only a tile that crosses M (A read as [k][m]) or N (B as [k][n]) has
    // float4 to shift; the test is block-uniform (the shifts' selects cost
    // the 4096 x 4096 x 4097 product 10% when every tile ran them).
    const bool a_edge = TA && m0 + BM > args.M, b_edge = !TB && n0 + BN > args.N;
    auto store_tiles = [&]<int MODE>(float *dst) {
        if (MODE == kLoadClamp && a_edge) la.template store_shifted<APITCH>(dst, m0, args.M);
        else la.template store<APITCH>(dst);
        if (MODE == kLoadClamp && b_edge) lb.template store_shifted<BPITCH>(dst + ASIZE, n0, args.N);
        else lb.template store<BPITCH>(dst + ASIZE);
    };
    constexpr int kWhole = FULL ? kLoadFull : kLoadClamp;  // slices of whole k
    if (FULL || kvec > 0) {
        load_tiles.template operator()<kWhole>(0);
        store_tiles.template operator()<kWhole>(lds);
    } else {
        load_tiles.template operator()<kLoadChecked>(0);
        store_tiles.template operator()<kLoadChecked>(lds);
    }
    __syncthreads();

    // Fragments: lane (fi, fk) supplies row/col fi of its 16x16 tile.  With
    // VK, MFMA step e of each group of 16 k takes k = 4*fk + e from lane fk
    // (the four steps together cover the 16 k once; MFMA sums k in any order),
    // so a lane's k values for the group are contiguous: one float4 LDS read
    // for a k-contiguous tile instead of four scalar reads.  Without VK, step
    // kk takes k = kk + fk, one scalar read per operand per step.
    const int fi = lane & 15;
    const int fk = lane >> 4;

    // One slice: prefetch slice s+1 (loaded in MODE) into registers, run
    // slice s's MFMAs from LDS, then store the prefetch to the other buffer.
    auto step = [&]<int MODE>(int64_t s) {
        const int cur = (int)(s & 1);
        const float *As = lds + cur * (ASIZE + BSIZE);
        const float *Bs = As + ASIZE;
        const bool more = s + 1 < kslices;
        if (more) load_tiles.template operator()<MODE>((s + 1) * BK);
        // The next slice goes to the other buffer, which no wave reads in this
        // slice (the barrier ending the previous slice saw its last reads).
        auto store_next = [&]() { store_tiles.template operator()<MODE>(lds + (cur ^ 1) * (ASIZE + BSIZE)); };
        if constexpr (VK) {
            // Kept rolled: unrolled, the groups' fragment reads are all
            // hoisted and BK=32 spills at 16 waves; rolled, one barrier per
            // 32 k measured ~1% faster than BK=16 at 4096^3.
#pragma unroll 1
            for (int kg = 0; kg < BK; kg += 16) {
                const int k4 = kg + 4 * fk;  // first of this lane's 4 k in the group
                vf4 a4[TM], b4[TN];
                if constexpr (!TA) {
#pragma unroll
                    for (int i = 0; i < TM; i++) a4[i] = *(const vf4 *)(As + (wm0 + i * 16 + fi) * APITCH + k4);
                }
                if constexpr (TB) {
#pragma unroll
                    for (int j = 0; j < TN; j++) b4[j] = *(const vf4 *)(Bs + (wn0 + j * 16 + fi) * BPITCH + k4);
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float af[TM], bf[TN];
#pragma unroll
                    for (int i = 0; i < TM; i++) af[i] = TA ? As[(k4 + e) * APITCH + wm0 + i * 16 + fi] : a4[i][e];
#pragma unroll
                    for (int j = 0; j < TN; j++) bf[j] = TB ? b4[j][e] : Bs[(k4 + e) * BPITCH + wn0 + j * 16 + fi];
#pragma unroll
                    for (int i = 0; i < TM; i++)
#pragma unroll
                        for (int j = 0; j < TN; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
                // After the first 16 k: the stores' LDS writes then complete
                // under the next group's MFMAs instead of before the barrier.
                if (kg == 0 && more) store_next();
            }
        } else {
            // The slice's MFMAs at raised wave priority: with two blocks per
            // CU, a wave in this section wins issue over the other block's
            // waves loading and storing tiles (batched 32x512^3: 1.8% faster;
            // the large tile's float4 path above measured no gain).
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int kk = 0; kk < BK; kk += 4) {
                float af[TM], bf[TN];
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const int m = wm0 + i * 16 + fi, k = kk + fk;
                    af[i] = TA ? As[k * APITCH + m] : As[m * APITCH + k];
                }
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int n = wn0 + j * 16 + fi, k = kk + fk;
                    bf[j] = TB ? Bs[n * BPITCH + k] : Bs[k * BPITCH + n];
                }
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
            __builtin_amdgcn_s_setprio(0);
            if (more) store_next();
        }
        __syncthreads();
    };
    // Two loops, each with one kind of load: a load under a per-slice
    // condition makes the compiler wait for it before the MFMAs, which
    // undoes the prefetch.
    if constexpr (FULL) {
        for (int64_t s = 0; s < kslices; s++) step.template operator()<kLoadFull>(s);
    } else {
        int64_t s = 0;
        for (; s + 1 < kvec; s++) step.template operator()<kLoadClamp>(s);
        for (; s < kslices; s++) step.template operator()<kLoadChecked>(s);
    }

    // ---- epilogue: lane holds C[4*(lane/16)+r][lane%16] of each 16x16 tile ----
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int64_t n = n0 + wn0 + j * 16 + fi;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t m = m0 + wm0 + i * 16 + 4 * fk + r;
                if (FULL || (m < args.M && n < args.N)) Cp[m * args.ldc + n] = acc[i][j][r];
            }
        }
    }
}

// ---- The large tile with its slices loaded straight into LDS ----
//
// global_load_lds_dwordx4: each lane's 16 bytes go from global memory to
// LDS at m0 + 16*lane, so a wave's load instruction fills one contiguous
// KiB of LDS with no registers in between.  Against the register-staged
// kernel above this drops the slice's four float4 LDS stores per lane and
// the registers that hold the prefetch; the result bits are the same (each
// lane's MFMA sequence is unchanged).  256x256 tile, 16 waves (a k that
// ends inside a slice ends with a partial slice loaded through registers),
// row offsets within 2^31 bytes.
//
// Ragged M or N (the EDGE form, M and N at least 256): the last tile row
// and column are moved back to end at the matrix's edge (rows M - 256 .. M,
// columns N - 256 .. N), so that every tile is whole and runs the same loads
// and loop; a moved tile stores only the outputs past the tile before it
// (those of its own row and column index).  Each output has one tile that
// stores it, with the k steps of any other tile, so the result bits are
// those of the zero-padded product.  (Clamping the edge tiles' loads
// instead took a per-lane shift of the chunks that straddle the edge, which
// cost the stream-K form registers or each slice an LDS round trip.)
//
// LDS layouts, per operand and buffer:
//   - a tile read along k (A not transposed, B transposed): 256 rows of BK
//     floats, unpadded; a KiB segment holds 256/BK whole rows, and row r
//     keeps its 16-byte chunk c at c ^ swz(r), which spreads the rows a
//     fragment read touches over the banks as the +4 pitch does above;
//   - a tile of k rows (A transposed, B plain): BK rows of 256 floats, one
//     segment each, at a pitch of 260 floats (padding between segments is
//     free).
constexpr int kLdsRowPitch = 260;  // floats per k row of 256 (+4: rows 4 apart sit 16 banks apart)

template <int BK>
__device__ __forceinline__ int lds_swizzle(int r) {
    static_assert(BK == 16 || BK == 32, "two slice depths");
    // 8 chunks of 16 B per row: chunk ^ (r & 7).  4 chunks per row (64-byte
    // rows, two to a 128-byte bank line): chunk ^ ((r >> 1) & 3).
    return BK == 32 ? (r & 7) : ((r >> 1) & 3);
}

// One operand's share of a slice: where each of this lane's loads reads
// (bytes from the slice's base) and where its wave's segment goes (bytes
// within the operand's LDS region).
template <int BK, bool KROWS>
struct LdsOperand {
    static constexpr int kSegs = BK / 16;  // segments per wave per slice
    static constexpr int kFloats = KROWS ? BK * kLdsRowPitch : 256 * BK;
    uint32_t voff[kSegs], seg[kSegs];
    int k0[kSegs];  // the slice k of this lane's first float in each segment

    // ld: the operand's row stride (elements).
    __device__ __forceinline__ void plan(int64_t ld, int lane, int wave) {
#pragma unroll
        for (int q = 0; q < kSegs; q++) {
            const int sg = wave + 16 * q;
            if constexpr (KROWS) {
                voff[q] = (uint32_t)((sg * ld + 4 * lane) * 4);
                seg[q] = sg * kLdsRowPitch * 4;
                k0[q] = sg;
            } else {
                constexpr int kChunks = BK / 4, kRowsPerSeg = 256 / BK;
                const int r = sg * kRowsPerSeg + lane / kChunks;
                const int c = (lane % kChunks) ^ lds_swizzle<BK>(r);
                voff[q] = (uint32_t)((r * ld + 4 * c) * 4);
                seg[q] = sg * 1024;
                k0[q] = 4 * c;
            }
        }
    }
    __device__ __forceinline__ void load(const float *base, const float *lds) const {
        const uint32_t at = lds_address(lds);
#pragma unroll
        for (int q = 0; q < kSegs; q++) lds_dma16(base, voff[q], at + seg[q]);
    }
    // The last, partial slice (its first `tail` k only), through registers
    // into the same LDS places, zero past the tail (so padded steps add
    // 0 * 0, as the register-staged kernel's checked slice does).  Reads
    // only elements inside the matrix.
    __device__ __forceinline__ void load_tail(const float *base, float *lds, int tail, int lane) const {
#pragma unroll
        for (int q = 0; q < kSegs; q++) {
            const float *p = base + voff[q] / 4;
            vf4 v;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const bool in = KROWS ? k0[q] < tail : k0[q] + e < tail;
                v[e] = in ? p[e] : 0.f;
            }
            *(vf4 *)(lds + seg[q] / 4 + 4 * lane) = v;
        }
    }
};

// The slice depth gemm_f32_mfma_lds runs a product at, or 0 when it cannot:
// the loads' byte offsets from a slice's base (256 rows of the row stride)
// must stay below 2^31.  The 16-byte loads need only dword alignment (a
// probe on the box read every float right at each of the four float offsets
// within 16 bytes), so rows of any length qualify.  g.K is the depth
// of one product (of one slice of a split K).  Measured at 4096^3: BK = 32
// runs 0.925-0.934 of the FP32 MFMA peak with A not transposed, against
// 0.919-0.924 at 16; with A transposed 16 is better (0.909-0.913 against
// 0.904-0.911), and so it is at K = 1024 (0.889 against 0.864).  Ragged M
// or N (the EDGE form) need M and N of at least 256.
inline int lds_tile_depth(const GemmArgs &g, bool a_trans) {
    const bool aligned = (uintptr_t)g.a % 4 == 0 && (uintptr_t)g.b % 4 == 0;
    const bool fits = g.lda >= 0 && g.ldb >= 0 && 256 * g.lda * 4 < ((int64_t)1 << 31) &&
                      256 * g.ldb * 4 < ((int64_t)1 << 31);
    if (!aligned || !fits) return 0;
    // Ragged M or N: the edge tiles move back inside the matrix.
    if ((g.M % 256 != 0 || g.N % 256 != 0) && (g.M < 256 || g.N < 256)) return 0;
    // Depth 32 only where every product's k is whole slices of 32: where k
    // ends inside a slice, the last slice is padded with zeros to 16, as in
    // the register-staged kernel, so that the steps (and any -0.0 sum) match.
    const bool whole32 = g.K % 32 == 0 && (g.ktotal == 0 || g.ktotal % 32 == 0);
    return (!a_trans && whole32 && g.K >= 2048) ? 32 : 16;
}

// Tile t of a launch (t over batch * tiles_m * tiles_n): tiles in groups of
// kGroupM tile rows, the group's tiles taken down its columns.
// min by value: std::min of a kernel argument and a temporary returns a
// reference the compiler may have to keep in scratch memory.
__device__ __forceinline__ int64_t imin(int64_t a, int64_t b) { return a < b ? a : b; }

struct TileCoord {
    int64_t batch, m, n;
};
__device__ __forceinline__ TileCoord decode_tile(const GemmArgs &args, int64_t t) {
    const int64_t tiles = (int64_t)args.tiles_m * args.tiles_n;
    TileCoord c;
    c.batch = t / tiles;
    t -= c.batch * tiles;
    const int64_t group_span = (int64_t)kGroupM * args.tiles_n;
    const int64_t group = t / group_span;
    const int64_t first_m = group * kGroupM;
    const int64_t gm = imin(args.tiles_m - first_m, kGroupM);
    const int64_t within = t - group * group_span;
    c.m = first_m + within % gm;
    c.n = within / gm;
    return c;
}

// decode_tile in 32 bits (t and the tile counts below 2^31): the stream-K
// loop decodes a tile per segment, and the 64-bit divisions' loop-invariant
// parts, kept in VGPRs across segments, spilled.
__device__ __forceinline__ TileCoord decode_tile32(const GemmArgs &args, uint32_t t) {
    const uint32_t tm = (uint32_t)args.tiles_m, tn = (uint32_t)args.tiles_n, tiles = tm * tn;
    TileCoord c;
    const uint32_t batch = t / tiles;
    t -= batch * tiles;
    const uint32_t group_span = (uint32_t)kGroupM * tn;
    const uint32_t group = t / group_span;
    const uint32_t first_m = group * kGroupM;
    const uint32_t gm = tm - first_m < (uint32_t)kGroupM ? tm - first_m : (uint32_t)kGroupM;
    const uint32_t within = t - group * group_span;
    c.batch = batch;
    c.m = first_m + within % gm;
    c.n = within / gm;
    return c;
}

constexpr int64_t kLargeTileFloats = 256 * 256;

// One 256x256 tile of the LDS-loading kernel over its slices [q0, q1) (q1
// past the last slice: to the end).  Stores the tile into C (masked on the
// edge, EDGE), or with `ws` set its partial sums into ws[r * 256 + c], all
// 256 x 256 of them.  tid: threadIdx.x (the stream-K loop passes a copy the
// compiler cannot see through, so that the lane values derived from it are
// not kept live across segments: they spilled there).
//
// TAIL: some product's k ends inside a slice (compiled apart: the branch in
// the slice loop cost 1% at 4096^3 and on the MLP step).  EDGE: M or N is
// not a multiple of 256 (compiled apart too, so that whole-tile products
// keep the loop they had).
template <int BK, bool TA, bool TB, bool TAIL, bool EDGE>
__device__ __forceinline__ void lds_tile_slices(const GemmArgs &args, float *lds, TileCoord tc, int64_t q0,
                                                int64_t q1, float *ws, unsigned tid) {
    constexpr int BM = 256, BN = 256, WGN = 4, WM = 64, WN = 64, TM = WM / 16, TN = WN / 16;
    using LA = LdsOperand<BK, TA>;
    using LB = LdsOperand<BK, !TB>;
    constexpr int ASIZE = LA::kFloats, BSIZE = LB::kFloats;

    const int64_t batch_idx = tc.batch;
    const int64_t Kb = args.ktotal ? imin(args.K, args.ktotal - batch_idx * args.K) : args.K;
    const float *A = args.a + batch_idx * args.bsa;
    const float *B = args.b + batch_idx * args.bsb;
    float *Cp = args.c + batch_idx * args.bsc;
    // The tile's own first row and column, and its origin: on the edge,
    // moved back to end at the matrix's (EDGE: M, N >= 256).
    const int64_t own_m = tc.m * BM, own_n = tc.n * BN;
    const int64_t m0 = EDGE ? imin(own_m, args.M - BM) : own_m;
    const int64_t n0 = EDGE ? imin(own_n, args.N - BN) : own_n;

    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
    const int fi = lane & 15, fk = lane >> 4;

    LA la;
    LB lb;
    la.plan(args.lda, lane, wave);
    lb.plan(args.ldb, lane, wave);
    // Slice s starts at abase + s * astep and bbase + s * bstep.
    const float *abase = TA ? A + m0 : A + m0 * args.lda;
    const float *bbase = TB ? B + n0 * args.ldb : B + n0;
    const int64_t astep = TA ? BK * args.lda : BK, bstep = TB ? BK : BK * args.ldb;

    typedef float vf4acc __attribute__((ext_vector_type(4)));
    vf4acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (vf4acc){0.f, 0.f, 0.f, 0.f};

    // Row wm0 + 16i + fi (or wn0 + 16j + fi) has the swizzle of fi.
    const int aswz = lds_swizzle<BK>(fi), bswz = aswz;
    // Slices of BK MFMA steps from one LDS buffer.
    auto slice_mfma = [&](const float *As) {
        const float *Bs = As + ASIZE;
        auto kgroup = [&](int kg) {
            const int k4 = kg + 4 * fk;
            const int chunk = kg / 4 + fk;
            vf4 a4[TM], b4[TN];
            if constexpr (!TA) {
                const float *ap = As + (wm0 + fi) * BK + ((chunk ^ aswz) << 2);
#pragma unroll
                for (int i = 0; i < TM; i++) a4[i] = *(const vf4 *)(ap + i * 16 * BK);
            }
            if constexpr (TB) {
                const float *bp = Bs + (wn0 + fi) * BK + ((chunk ^ bswz) << 2);
#pragma unroll
                for (int j = 0; j < TN; j++) b4[j] = *(const vf4 *)(bp + j * 16 * BK);
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float af[TM], bf[TN];
#pragma unroll
                for (int i = 0; i < TM; i++)
                    af[i] = TA ? As[(k4 + e) * kLdsRowPitch + wm0 + i * 16 + fi] : a4[i][e];
#pragma unroll
                for (int j = 0; j < TN; j++)
                    bf[j] = TB ? b4[j][e] : Bs[(k4 + e) * kLdsRowPitch + wn0 + j * 16 + fi];
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        };
        // The k groups of a slice unrolled, so the next group's fragment reads
        // can be issued among this group's MFMAs (0.3% on the MLP step and at
        // 4096^3); the stream-K form with B transposed and ragged M or N then
        // spills, so it keeps the rolled loop.
        if constexpr (TB && EDGE) {
#pragma unroll 1
            for (int kg = 0; kg < BK; kg += 16) kgroup(kg);
        } else {
#pragma unroll
            for (int kg = 0; kg < BK; kg += 16) kgroup(kg);
        }
    };
    // Whole slices load straight into LDS, each prefetched during the one
    // before.  A k that ends inside a slice ends with one more, partial
    // slice, loaded through registers once the last whole slice is done
    // (prefetched with the others, its loads' wait fell among the MFMAs:
    // stream-K at 5000^3 ran 0.75 of peak against 0.84 at K = 4992).
    const int64_t kwhole = Kb / BK;
    const int tail = TAIL ? (int)(Kb - kwhole * BK) : 0;
    const int64_t kend = imin(q1, kwhole + (tail ? 1 : 0));
    const int64_t kmain = TAIL ? imin(kend, kwhole) : kend;
    auto fetch = [&](int64_t s, float *dst) {
        la.load(abase + s * astep, dst);
        lb.load(bbase + s * bstep, dst + ASIZE);
    };
    auto fetch_tail = [&](float *dst) {
        la.load_tail(abase + kwhole * astep, dst, tail, lane);
        lb.load_tail(bbase + kwhole * bstep, dst + ASIZE, tail, lane);
    };
    if (TAIL && q0 == kwhole) fetch_tail(lds);
    else fetch(q0, lds);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int64_t s = q0; s < kend; s++) {
        const float *As = lds + ((s - q0) & 1) * (ASIZE + BSIZE);
        float *next = lds + ((s - q0 + 1) & 1) * (ASIZE + BSIZE);
        if (s + 1 < kmain) fetch(s + 1, next);
        slice_mfma(As);
        __builtin_amdgcn_s_waitcnt(0);  // this slice's loads into the other buffer have landed
        __syncthreads();
        if (TAIL && s + 1 == kwhole && s + 1 < kend) {
            fetch_tail(next);
            __syncthreads();
        }
    }

    if (ws) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 4; r++) ws[(wm0 + i * 16 + 4 * fk + r) * 256 + wn0 + j * 16 + fi] = acc[i][j][r];
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int64_t n = n0 + wn0 + j * 16 + fi;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t m = m0 + wm0 + i * 16 + 4 * fk + r;
                if (!EDGE || (m >= own_m && n >= own_n)) Cp[m * args.ldc + n] = acc[i][j][r];
            }
        }
    }
}

template <int BK, bool TA, bool TB>
constexpr int lds_tile_floats() {
    return 2 * (LdsOperand<BK, TA>::kFloats + LdsOperand<BK, !TB>::kFloats);
}

// One block per tile.
template <int BK, bool TA, bool TB, bool TAIL, bool EDGE>
__global__ void __launch_bounds__(1024, 1) gemm_f32_mfma_lds(GemmArgs args) {
    __shared__ __attribute__((aligned(16))) float lds[lds_tile_floats<BK, TA, TB>()];
    int64_t bid = blockIdx.x;
    if (args.xcd_remap) {
        const int64_t total = (int64_t)args.tiles_m * args.tiles_n * args.batch;
        const int64_t per_xcd = total / kXcds;
        bid = (bid % kXcds) * per_xcd + bid / kXcds;
    }
    lds_tile_slices<BK, TA, TB, TAIL, EDGE>(args, lds, decode_tile(args, bid), 0, INT64_MAX, nullptr, threadIdx.x);
}

// Stream-K: one persistent block per CU, block b taking the (tile, slice)
// units [b*U/G, (b+1)*U/G) of the U = tiles * Q of the product (G blocks, Q
// slices per tile, tile-major).  A tile whose units fall to one block is
// stored into C; a block's first and last segments that cover only part of
// a tile's slices go to its two workspace slots (slot 0 the first segment,
// slot 1 the last), which gemm_streamk_fixup adds in k order.  No block waits
// for another.  Logical block b runs as blockIdx (b % (G/8)) * 8 + b / (G/8),
// so each XCD takes one contiguous eighth of the units.
template <int BK, bool TA, bool TB, bool TAIL, bool EDGE>
__global__ void __launch_bounds__(1024, 1) gemm_f32_mfma_lds_sk(GemmArgs args) {
    __shared__ __attribute__((aligned(16))) float lds[lds_tile_floats<BK, TA, TB>()];
    const int64_t G = args.sk_blocks, U = args.sk_units, Q = args.sk_q;
    const int64_t b = args.xcd_remap ? (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds : blockIdx.x;
    const int64_t u0 = b * U / G, u1 = (b + 1) * U / G;
    // Segment: slices [qb, qe) of tile t; the next starts the next tile.
    int64_t t = u0 / Q, qb = u0 - t * Q;
    for (int64_t u = u0; u < u1; t++, qb = 0) {
        const int64_t qe = imin(Q, qb + (u1 - u));
        float *ws = (qb == 0 && qe == Q) ? nullptr : args.sk_ws + (2 * b + (u == u0 ? 0 : 1)) * kLargeTileFloats;
        unsigned tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        lds_tile_slices<BK, TA, TB, TAIL, EDGE>(args, lds, decode_tile32(args, (uint32_t)t), qb, qe, ws, tid);
        u += qe - qb;
    }
}

// The pieces of the tiles stream-K split between blocks, added in k order
// (block order) into C.  Block (t, y) takes rows 16y..16y+15 of tile t; a
// tile that one block ran whole was stored by it and is skipped.
__global__ void __launch_bounds__(256) gemm_streamk_fixup(GemmArgs args) {
    const int64_t G = args.sk_blocks, U = args.sk_units, Q = args.sk_q;
    const int64_t t = blockIdx.x;
    // The block whose units hold unit u: the largest b with b*U/G <= u.
    const auto block_of = [&](int64_t u) { return imin(G - 1, ((u + 1) * G - 1) / U); };
    const int64_t bf = block_of(t * Q), bl = block_of((t + 1) * Q - 1);
    if (bf == bl) return;
    const TileCoord tc = decode_tile32(args, (uint32_t)t);
    float *Cp = args.c + tc.batch * args.bsc;
    // The tile's origin, moved back on the edge as in lds_tile_slices, and
    // the outputs it owns: rows and columns from its own index on.
    const int64_t own_m = tc.m * 256, own_n = tc.n * 256;
    const int64_t m0 = imin(own_m, args.M - 256), n0 = imin(own_n, args.N - 256);
    const int r = (int)blockIdx.y * 16 + (int)(threadIdx.x >> 4);
    const int64_t m = m0 + r;
    if (m < own_m) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = 4 * ((int)(threadIdx.x & 15) + 16 * i);
        vf4 v;
        for (int64_t p = bf; p <= bl; p++) {
            // Slot 0 when the tile holds block p's first unit, else slot 1.
            const int64_t slot = p * U / G >= t * Q ? 0 : 1;
            const vf4 x = *(const vf4 *)(args.sk_ws + (2 * p + slot) * kLargeTileFloats + r * 256 + c);
            v = p == bf ? x : v + x;
        }
        const int64_t n = n0 + c;
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (n + e >= own_n) Cp[m * args.ldc + n + e] = v[e];
    }
}

// The 128x128x32 tile (8 waves of 32x64, two blocks per CU) with its slices
// loaded straight into LDS, for whole tiles.  Same fragment order as the
// register-staged small tile (MFMA step kk takes k = kk + fk), so the same
// result bits.  An operand tile is 16 KiB in 16 segments, two per wave:
//   - read along k (A not transposed, B transposed): 128 rows of 32 floats,
//     8 rows to a segment, chunk c of row r at c ^ (r & 7);
//   - k rows (A transposed, B plain): 32 rows of 128 floats, two to a
//     segment, segments at a pitch of kSmallSegPitch floats (rows k and k+2
//     then sit 16 banks apart, as the +16 pitch does above).
// Measured against the register-staged tile in one run, bit-identical:
// batched 32x512^3 0.0768 -> 0.0691 ms, batched 16 x 1024x1024x256
// 0.081 -> 0.072 ms, 2048^3 0.144 -> 0.141 ms.
constexpr int kSmallSegPitch = 272;

// ROWS: the tile's rows when read along k (128, or 64 for A of the 64x128
// tile); a k-row tile is always 128 wide.  NW: the block's waves.
template <bool KROWS, int ROWS, int NW>
struct LdsOperandSmall {
    static_assert(!KROWS || ROWS == 128, "k rows of 128 floats only");
    static constexpr int kFloats = KROWS ? 16 * kSmallSegPitch : ROWS * 32;
    static constexpr int kSegs = (KROWS ? 16 : ROWS / 8) / NW;  // per wave
    uint32_t voff[kSegs], seg[kSegs];

    __device__ __forceinline__ void plan(int64_t ld, int lane, int wave) {
#pragma unroll
        for (int q = 0; q < kSegs; q++) {
            const int sg = wave + NW * q;
            if constexpr (KROWS) {
                const int k = 2 * sg + (lane >> 5);
                voff[q] = (uint32_t)((k * ld + 4 * (lane & 31)) * 4);
                seg[q] = sg * kSmallSegPitch * 4;
            } else {
                const int r = sg * 8 + (lane >> 3);
                const int c = (lane & 7) ^ (r & 7);
                voff[q] = (uint32_t)((r * ld + 4 * c) * 4);
                seg[q] = sg * 1024;
            }
        }
    }
    __device__ __forceinline__ void load(const float *base, const float *lds) const {
        const uint32_t at = lds_address(lds);
#pragma unroll
        for (int q = 0; q < kSegs; q++) lds_dma16(base, voff[q], at + seg[q]);
    }
    // Element (row, k) of a k-contiguous tile for a lane whose row has
    // swizzle sw (its row's r & 7), at k step kk (k = kk + fk).
    __device__ __forceinline__ static int kcontig(int row, int kk, int fk, int sw) {
        return row * 32 + (((kk >> 2) ^ sw) << 2) + fk;
    }
    // Element (k, col) of a k-row tile.
    __device__ __forceinline__ static int krow(int k, int col) {
        return (k >> 1) * kSmallSegPitch + (k & 1) * 128 + col;
    }
};

// The 128x128 and 64x128 tiles qualify when 128 rows of a row stride stay
// below 2^31 bytes (their loads need only dword alignment, as the large
// tile's).
inline bool lds_small_ok(const GemmArgs &g) {
    const bool aligned = (uintptr_t)g.a % 4 == 0 && (uintptr_t)g.b % 4 == 0;
    const bool fits = g.lda >= 0 && g.ldb >= 0 && 128 * g.lda * 4 < ((int64_t)1 << 31) &&
                      128 * g.ldb * 4 < ((int64_t)1 << 31);
    return aligned && fits && g.K % 32 == 0;
}

// BM 128: 8 waves (4x2); BM 64 (the 64x128 tile, A not transposed): 4
// waves (2x2).  Each wave owns 32x64 either way.
template <int BM, bool TA, bool TB>
__global__ void __launch_bounds__(BM * 4, 2) gemm_f32_mfma_lds_small(GemmArgs args) {
    constexpr int NW = BM / 16, BN = 128, BK = 32, WGN = 2, WM = 32, WN = 64, TM = WM / 16, TN = WN / 16;
    using LA = LdsOperandSmall<TA, BM, NW>;
    using LB = LdsOperandSmall<!TB, 128, NW>;
    constexpr int ASIZE = LA::kFloats, BSIZE = LB::kFloats;
    __shared__ __attribute__((aligned(16))) float lds[2 * (ASIZE + BSIZE)];

    // The block's tile, decoded in 32 bits: the grid is one block per tile
    // and below 2^23 blocks (a dispatch counts under 2^32 lanes), so every
    // count fits.  In 64 bits the four divisions by run-time counts were
    // software loops, some 600 instructions before a block's first load.
    uint32_t bid = blockIdx.x;
    if (args.xcd_remap) {
        const uint32_t per_xcd = (uint32_t)args.tiles_m * (uint32_t)args.tiles_n * (uint32_t)args.batch / kXcds;
        bid = (bid % kXcds) * per_xcd + bid / kXcds;
    }
    const TileCoord tc = decode_tile32(args, bid);
    const int64_t batch_idx = tc.batch, tile_m = tc.m, tile_n = tc.n;

    const int64_t Kb = args.ktotal ? std::min<int64_t>(args.K, args.ktotal - batch_idx * args.K) : args.K;
    const float *A = args.a + batch_idx * args.bsa;
    const float *B = args.b + batch_idx * args.bsb;
    float *Cp = args.c + batch_idx * args.bsc;
    const int64_t m0 = tile_m * BM, n0 = tile_n * BN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;
    const int fi = lane & 15, fk = lane >> 4;

    LA la;
    LB lb;
    la.plan(args.lda, lane, wave);
    lb.plan(args.ldb, lane, wave);
    const float *abase = TA ? A + m0 : A + m0 * args.lda;
    const float *bbase = TB ? B + n0 * args.ldb : B + n0;
    const int64_t astep = TA ? BK * args.lda : BK, bstep = TB ? BK : BK * args.ldb;

    typedef float vf4acc __attribute__((ext_vector_type(4)));
    vf4acc acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = (vf4acc){0.f, 0.f, 0.f, 0.f};

    const int sw = fi & 7;  // rows wm0 + 16i + fi and wn0 + 16j + fi
    const int64_t kslices = Kb / BK;
    la.load(abase, lds);
    lb.load(bbase, lds + ASIZE);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int64_t s = 0; s < kslices; s++) {
        const float *As = lds + (s & 1) * (ASIZE + BSIZE);
        const float *Bs = As + ASIZE;
        if (s + 1 < kslices) {
            const float *nxt = lds + ((s + 1) & 1) * (ASIZE + BSIZE);
            la.load(abase + (s + 1) * astep, nxt);
            lb.load(bbase + (s + 1) * bstep, nxt + ASIZE);
        }
        // The slice's MFMAs at raised wave priority, as in the
        // register-staged small tile (two blocks share a CU).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 4) {
            const int k = kk + fk;
            float af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int m = wm0 + i * 16 + fi;
                af[i] = TA ? As[LA::krow(k, m)] : As[LA::kcontig(m, kk, fk, sw)];
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = wn0 + j * 16 + fi;
                bf[j] = TB ? Bs[LB::kcontig(n, kk, fk, sw)] : Bs[LB::krow(k, n)];
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_s_waitcnt(0);  // the next slice's loads have landed
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < TM; i++) {
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int64_t n = n0 + wn0 + j * 16 + fi;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int64_t m = m0 + wm0 + i * 16 + 4 * fk + r;
                Cp[m * args.ldc + n] = acc[i][j][r];
            }
        }
    }
}

// Split-K epilogue: c = ((p0 + p1) + p2) + ... over the S partial products,
// in slice order, four floats per lane.  NS is S when 2 <= S <= 16 (all S
// loads issued before the first add: one memory latency instead of one per
// slice, with no branch between the loads, where a copy at a branch join
// waits for every load issued before it), else 0 and S is read at run time.
template <int NS>
__global__ void __launch_bounds__(kHelperLanes) splitk_sum(const float4 *__restrict__ parts, float4 *__restrict__ c,
                                                  int64_t n4, int S) {
    const int64_t i = (int64_t)blockIdx.x * kHelperLanes + threadIdx.x;
    if (i >= n4) return;
    auto add = [](float4 &acc, const float4 &v) {
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    };
    float4 acc;
    if constexpr (NS > 0) {
        float4 part[NS];
        const float4 *pq = parts + i;
#pragma unroll
        for (int q = 0; q < NS; q++) {
            part[q] = *pq;
            if (q + 1 < NS) pq += n4;
        }
        acc = part[0];
#pragma unroll
        for (int q = 1; q < NS; q++) add(acc, part[q]);
    } else {
        acc = parts[i];
        for (int q = 1; q < S; q++) add(acc, parts[(int64_t)q * n4 + i]);
    }
    c[i] = acc;
}

template <int NS = 2>
void launch_splitk_sum(int S, dim3 grid, hipStream_t s, const float4 *parts, float4 *c, int64_t n4) {
    if constexpr (NS > 16) hipLaunchKernelGGL(splitk_sum<0>, grid, dim3(kHelperLanes), 0, s, parts, c, n4, S);
    else if (S == NS) hipLaunchKernelGGL(splitk_sum<NS>, grid, dim3(kHelperLanes), 0, s, parts, c, n4, S);
    else launch_splitk_sum<NS + 1>(S, grid, s, parts, c, n4);
}

// Simple fallback for operands with no unit stride: one thread per output,
// sequential k (the reference's own order).
__global__ void __launch_bounds__(kHelperLanes) gemm_f32_strided(const float *a, const float *b, float *c, int64_t M,
                                                        int64_t N, int64_t K, int64_t sam, int64_t sak,
                                                        int64_t sbk, int64_t sbn, int64_t bsa, int64_t bsb,
                                                        int64_t batch) {
    const int64_t total = M * N * batch;
    const int64_t stride = (int64_t)gridDim.x * kHelperLanes;
    for (int64_t e = (int64_t)blockIdx.x * kHelperLanes + threadIdx.x; e < total; e += stride) {
        const int64_t t = e / (M * N), rem = e - t * M * N, i = rem / N, j = rem - i * N;
        const float *A = a + t * bsa, *B = b + t * bsb;
        float acc = 0.0f;
        for (int64_t k = 0; k < K; k++) {
            const float p = A[i * sam + k * sak] * B[k * sbk + j * sbn];
            acc = acc + p;
        }
        c[e] = acc;
    }
}

// A tile configuration: BM x BN x BK, a WGM x WGN grid of waves, MINB
// blocks per CU requested from the compiler; VK reads k-contiguous fragments
// as float4; EDGE instantiates the bounds-guarded variant for shapes the tile
// does not divide.
template <int BM_, int BN_, int BK_, int WGM_, int WGN_, int MINB_, bool VK_, bool EDGE_>
struct Tiles {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_, MINB = MINB_;
    static constexpr bool VK = VK_, EDGE = EDGE_;
    static constexpr int NT = WGM * WGN * 64;
};
// The medium tile runs only on shapes it divides; the large and small tiles
// also on ragged ones (the large one since 4095^3 and 2047^3 ran 0.55 of
// peak on the small tile).  Float4 fragment reads measured +0.9% (NT) to -0.1% on the large tile and -2 to -3%
// on the 4-wave tiles, so only the large tile uses them.
// BK=32 pays only in the plain layout: 138.8 against 137.3 TFLOP/s at
// 8192x4096x4096, while a transposed A runs 1.6-1.9% slower at BK=32 than at
// BK=16 (134.6 against 137.2 TFLOP/s at 4096x4096x8192) and a transposed B
// holds more fragment registers and spills at BK=32 with 16 waves.  The k
// order, and so every result bit, is the same at both depths.
// Shapes the large tile does not divide run its BK=16 form in every layout:
// the BK=32 plain form's edge-guarded variant spills at 16 waves.
using LargeTiles = Tiles<256, 256, 32, 4, 4, 1, true, false>;
using LargeTilesK16 = Tiles<256, 256, 16, 4, 4, 1, true, true>;
// The 128x128 tile runs 8 waves of 32x64 each (4 per SIMD with two blocks per
// CU): batched 32x512^3 117.3 -> 121 TFLOP/s, 2047^3 214 -> 199 us against 4
// waves of 64x64; 8 waves of 64x32 and 16 waves of 32x32 measured between.
using SmallTiles = Tiles<128, 128, 32, 4, 2, 2, false, true>;
using MediumTiles = Tiles<64, 128, 32, 2, 2, 2, false, false>;  // halves M per block when 128x128 leaves CUs idle

template <class T, bool TA, bool TB>
int launch_tiled(GemmArgs g, bool full, hipStream_t s) {
    g.tiles_m = (int32_t)((g.M + T::BM - 1) / T::BM);
    g.tiles_n = (int32_t)((g.N + T::BN - 1) / T::BN);
    const int64_t blocks = (int64_t)g.tiles_m * g.tiles_n * g.batch;
    g.xcd_remap = blocks % kXcds == 0 ? 1 : 0;
    const dim3 grid((unsigned)blocks), block(T::NT);
    if constexpr (T::EDGE) {
        if (!full) {
            hipLaunchKernelGGL((gemm_f32_mfma<T::BM, T::BN, T::BK, T::WGM, T::WGN, T::MINB, T::VK, TA, TB, false>), grid,
                               block, 0, s, g);
            TRS_LAUNCH_CHECK("gemm kernel launch");
            return TRS_OK;
        }
    } else if (!full) {
        return set_error(TRS_E_INVALID_ARGUMENT, "gemm tile %dx%dx%d needs a shape it divides", T::BM, T::BN, T::BK);
    }
    hipLaunchKernelGGL((gemm_f32_mfma<T::BM, T::BN, T::BK, T::WGM, T::WGN, T::MINB, T::VK, TA, TB, true>), grid, block, 0,
                       s, g);
    TRS_LAUNCH_CHECK("gemm kernel launch");
    return TRS_OK;
}

template <int BM, bool TA, bool TB>
int launch_lds_small(GemmArgs g, hipStream_t s) {
    g.tiles_m = (int32_t)(g.M / BM);
    g.tiles_n = (int32_t)(g.N / 128);
    const int64_t blocks = (int64_t)g.tiles_m * g.tiles_n * g.batch;
    g.xcd_remap = blocks % kXcds == 0 ? 1 : 0;
    hipLaunchKernelGGL((gemm_f32_mfma_lds_small<BM, TA, TB>), dim3((unsigned)blocks), dim3(BM * 4), 0, s, g);
    TRS_LAUNCH_CHECK("gemm kernel launch");
    return TRS_OK;
}

template <class T>
int launch_layout(const GemmArgs &g, bool a_plain, bool b_plain, bool full, hipStream_t s);

// The 128x128 tile; whole tiles load their slices straight into LDS where
// lds_small_ok allows.
int launch_small(const GemmArgs &g, bool a_plain, bool b_plain, bool full, hipStream_t s) {
    if (full && lds_small_ok(g)) {
        if (a_plain && b_plain) return launch_lds_small<128, false, false>(g, s);
        if (a_plain) return launch_lds_small<128, false, true>(g, s);
        if (b_plain) return launch_lds_small<128, true, false>(g, s);
        return launch_lds_small<128, true, true>(g, s);
    }
    return launch_layout<SmallTiles>(g, a_plain, b_plain, full, s);
}

// The 64x128 tile (whole tiles only); with A not transposed its slices load
// straight into LDS where lds_small_ok allows.
int launch_medium(const GemmArgs &g, bool a_plain, bool b_plain, hipStream_t s) {
    if (a_plain && lds_small_ok(g))
        return b_plain ? launch_lds_small<64, false, false>(g, s) : launch_lds_small<64, false, true>(g, s);
    return launch_layout<MediumTiles>(g, a_plain, b_plain, true, s);
}

template <class T>
int launch_layout(const GemmArgs &g, bool a_plain, bool b_plain, bool full, hipStream_t s) {
    if (a_plain && b_plain) return launch_tiled<T, false, false>(g, full, s);
    if (a_plain) return launch_tiled<T, false, true>(g, full, s);
    if (b_plain) return launch_tiled<T, true, false>(g, full, s);
    return launch_tiled<T, true, true>(g, full, s);
}

// The LDS-loading large tile: one block per tile, or with g.sk_ws set the
// stream-K form (g.sk_blocks blocks) followed by its fix-up pass.
template <int BK, bool TA, bool TB>
int launch_lds_tile(GemmArgs g, hipStream_t s) {
    g.tiles_m = (int32_t)((g.M + 255) / 256);
    g.tiles_n = (int32_t)((g.N + 255) / 256);
    const int64_t tiles = (int64_t)g.tiles_m * g.tiles_n * g.batch;
    const bool sk = g.sk_ws != nullptr;
    if (sk) {
        g.sk_q = (g.K + BK - 1) / BK;
        g.sk_units = tiles * g.sk_q;
    }
    const int64_t blocks = sk ? g.sk_blocks : tiles;
    g.xcd_remap = blocks % kXcds == 0 ? 1 : 0;
    const bool tail = g.K % BK != 0 || (g.ktotal != 0 && g.ktotal % BK != 0);
    const bool edge = g.M % 256 != 0 || g.N % 256 != 0;
    const dim3 grid((unsigned)blocks), block(1024);
    auto go = [&]<bool TL, bool ED>() {
        if (sk) hipLaunchKernelGGL((gemm_f32_mfma_lds_sk<BK, TA, TB, TL, ED>), grid, block, 0, s, g);
        else hipLaunchKernelGGL((gemm_f32_mfma_lds<BK, TA, TB, TL, ED>), grid, block, 0, s, g);
    };
    // lds_tile_depth gives depth 32 to whole slices only.
    if constexpr (BK == 32) {
        if (tail) return set_error(TRS_E_INVALID_ARGUMENT, "gemm tile depth 32 needs whole slices");
        if (edge) go.template operator()<false, true>();
        else go.template operator()<false, false>();
    } else if (edge) {
        if (tail) go.template operator()<true, true>();
        else go.template operator()<false, true>();
    } else if (tail) {
        go.template operator()<true, false>();
    } else {
        go.template operator()<false, false>();
    }
    TRS_LAUNCH_CHECK("gemm kernel launch");
    if (sk) {
        hipLaunchKernelGGL(gemm_streamk_fixup, dim3((unsigned)tiles, 16), dim3(256), 0, s, g);
        TRS_LAUNCH_CHECK("stream-k fix-up launch");
    }
    return TRS_OK;
}

template <bool TA, bool TB>
int launch_lds_layout(const GemmArgs &g, int bk, hipStream_t s) {
    return bk == 32 ? launch_lds_tile<32, TA, TB>(g, s) : launch_lds_tile<16, TA, TB>(g, s);
}

// The large tile in each layout; `full` when it divides M, N and K.  Slices
// load straight into LDS where lds_tile_depth allows (any K, ragged M and N
// too), else through registers.
int launch_large(const GemmArgs &g, bool a_plain, bool b_plain, bool full, hipStream_t s) {
    if (const int bk = lds_tile_depth(g, !a_plain)) {
        if (a_plain && b_plain) return launch_lds_layout<false, false>(g, bk, s);
        if (a_plain) return launch_lds_layout<false, true>(g, bk, s);
        if (b_plain) return launch_lds_layout<true, false>(g, bk, s);
        return launch_lds_layout<true, true>(g, bk, s);
    }
    if (a_plain && b_plain)
        return full ? launch_tiled<LargeTiles, false, false>(g, true, s)
                    : launch_tiled<LargeTilesK16, false, false>(g, false, s);
    if (a_plain) return launch_tiled<LargeTilesK16, false, true>(g, full, s);
    if (b_plain) return launch_tiled<LargeTilesK16, true, false>(g, full, s);
    return launch_tiled<LargeTilesK16, true, true>(g, full, s);
}

// Split K: an output with fewer tiles than CUs runs its K in S slices as S
// batches of its tile, into a workspace of S partial products that one more
// pass sums in slice order.  The workspace comes from the block cache and
// returns to it in stream order.  The last slice may be shorter (the kernel
// bounds each batch's k by the full depth).
//   - The large tile (the MLP's 8192x1024 and 4096x1024 GEMMs): S a power of
//     two up to 8, slices of at least kMinSplitDepth.
//   - The 128x128 and 64x128 tiles, when they give at most one block per CU
//     (1000^3 ran as 64 blocks, a 64x4096x4096 product as 32): S up to 16,
//     for about two blocks per CU, slices of at least 128 k, and at most
//     65,536 floats of partial products per CU.
constexpr int64_t kMaxSplitK = 8;
constexpr int64_t kMinSplitDepth = 1024;
constexpr int64_t kMaxTileSplit = 16;
constexpr int64_t kMinTileSplitDepth = 128;
constexpr int64_t kSplitFloatsPerCu = 65536;
// Time of two 128x128 blocks sharing a CU against one 256x256 block on it,
// from the measured rates (0.77 and 0.887 of peak): a ragged output takes the
// large tile when its rounds of blocks, so weighted, are no more.
constexpr double kSmallPairOverLarge = 0.575;

// Which kernel a product runs.  Tile choice:
//   - the 256x256 tile when it divides M and N and gives every CU a block;
//     on ragged M or N (edge tiles bounds-checked, interior ones not) when
//     its rounds of blocks take no longer than the 128x128 tile's;
//   - a single matrix whose M or N exceeds such an output by at most 32 rows
//     or columns: the 256x256 tile on the rest, and the thin rims as skinny
//     products (4097^3 would otherwise run 17 x 17 large tiles, two rounds);
//   - else, for a single matrix with fewer large tiles than CUs, those
//     tiles at least 90% covered, and a long K, the 256x256 tile over S
//     K-slices, when S*tiles reaches half the CUs or at least the block
//     count of the tile it replaces;
//   - else 64x128 when 128x128 would give fewer than two blocks per CU and
//     64x128 divides the shape (76% against 69% of peak measured at
//     4096x1024x8192), else 128x128 (full or edge-guarded);
//   - a single matrix whose tile gives at most one block per CU splits K
//     over that tile (above);
//   - then stream-K on the 256x256 tile (below) replaces the plan where it
//     is estimated at least kStreamKGain faster.
enum class GemmKind { Strided, Large, SplitK, Medium, Small, StreamK };
struct GemmPlan {
    GemmKind kind = GemmKind::Strided;
    int bm = 0, bn = 0, bk = 0;
    int64_t splits = 1;
    int64_t blocks = 0;
    bool full = false;
    // SplitK only: the tile each slice runs on and the k per slice.
    // SplitK and StreamK: the plan run when no workspace can be allocated.
    GemmKind split_tile = GemmKind::Large;
    int64_t ks = 0;
    GemmKind fallback = GemmKind::Small;
    bool fallback_full = false;
    // Large with rims: the tile runs on rows [0, main_m) and columns
    // [0, main_n); the rest is peeled off as skinny products (0: nothing).
    int64_t main_m = 0, main_n = 0;
};

GemmPlan plan_gemm_tiles(const GemmArgs &g, bool a_plain, bool a_trans, bool b_plain, bool b_trans, int cu_count) {
    GemmPlan p;
    const int64_t M = g.M, N = g.N, K = g.K, batch = g.batch;
    if (!(a_plain || a_trans) || !(b_plain || b_trans)) {
        p.kind = GemmKind::Strided;
        p.blocks = std::min<int64_t>((M * N * batch + 255) / 256, (int64_t)cu_count * 16);
        return p;
    }
    constexpr int64_t L = LargeTiles::BM;  // 256, both dims
    const int64_t large_bk = (a_plain && b_plain) ? LargeTiles::BK : LargeTilesK16::BK;
    const auto ceil_div = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
    // The depth the large tile runs an mm x nn product of depth k at (ktotal:
    // the full depth of a split K, else 0): the LDS-loading kernel's where
    // it applies, else the register-staged tile's (BK = 32 only for whole
    // tiles and slices).
    const auto large_depth = [&](int64_t mm, int64_t nn, int64_t k, int64_t ktotal, bool full) -> int {
        GemmArgs t = g;
        t.M = mm, t.N = nn, t.K = k, t.ktotal = ktotal;
        const int d = lds_tile_depth(t, !a_plain);
        return d ? d : full ? (int)large_bk : LargeTilesK16::BK;
    };
    const int64_t large_tiles = ceil_div(M, L) * ceil_div(N, L) * batch;
    const int64_t small_tiles = ceil_div(M, 128) * ceil_div(N, 128) * batch;
    const bool large_div = M % L == 0 && N % L == 0;
    const auto use_large = [&](int64_t mm, int64_t nn, int64_t tiles) {
        p.kind = GemmKind::Large;
        p.bm = L, p.bn = L;
        p.blocks = tiles;
        p.full = mm % L == 0 && nn % L == 0 && K % large_bk == 0;
        p.bk = large_depth(mm, nn, K, 0, p.full);
    };
    if (large_div && large_tiles >= cu_count) {
        use_large(M, N, large_tiles);
        return p;
    }
    // Thin rims peeled off a single matrix.
    if (batch == 1) {
        const int64_t mr = M % L, nr = N % L;
        const bool pm = M > L && mr >= 1 && mr <= kSkinnyMaxRows;
        const bool pn = N > L && nr >= 1 && nr <= kSkinnyMaxRows;
        const int64_t mm = pm ? M - mr : M, nn = pn ? N - nr : N;
        const int64_t tiles = ceil_div(mm, L) * ceil_div(nn, L);
        if ((pm || pn) && tiles >= cu_count) {
            use_large(mm, nn, tiles);
            p.main_m = mm;
            p.main_n = nn;
            return p;
        }
    }
    if (!large_div && large_tiles >= cu_count &&
        (double)ceil_div(large_tiles, cu_count) <= kSmallPairOverLarge * (double)ceil_div(small_tiles, 2 * cu_count)) {
        use_large(M, N, large_tiles);
        return p;
    }
    const bool full = M % SmallTiles::BM == 0 && N % SmallTiles::BN == 0 && K % SmallTiles::BK == 0;
    const bool medium_full = M % MediumTiles::BM == 0 && N % MediumTiles::BN == 0 && K % MediumTiles::BK == 0;
    if (medium_full && small_tiles < 2 * (int64_t)cu_count) {
        p.kind = GemmKind::Medium;
        p.bm = MediumTiles::BM, p.bn = MediumTiles::BN, p.bk = MediumTiles::BK;
        p.blocks = (M / 64) * (N / 128) * batch;
        p.full = true;
    } else {
        p.kind = GemmKind::Small;
        p.bm = SmallTiles::BM, p.bn = SmallTiles::BN, p.bk = SmallTiles::BK;
        p.blocks = small_tiles;
        p.full = full;
    }
    // The large split needs the 256x256 tiles nearly full (a 64-row output
    // would compute four times its rows): at least 90% of their area.
    const bool large_dense = (double)(M * N * batch) >= 0.9 * (double)(large_tiles * L * L);
    if (batch == 1 && large_dense && large_tiles > 0 && large_tiles < cu_count) {
        int64_t S = 1;
        while (S < kMaxSplitK && large_tiles * S * 2 <= cu_count && K / (S * 2) >= kMinSplitDepth) S *= 2;
        if (S > 1 && (2 * large_tiles * S >= cu_count || large_tiles * S >= p.blocks)) {
            const int64_t ks = ceil_div(ceil_div(K, S), large_bk) * large_bk;
            p.fallback = p.kind;
            p.fallback_full = p.full;
            p.kind = GemmKind::SplitK;
            p.split_tile = GemmKind::Large;
            p.bm = L, p.bn = L;
            p.splits = ceil_div(K, ks);
            p.ks = ks;
            p.blocks = large_tiles * p.splits;
            p.full = large_div && K % ks == 0;
            p.bk = large_depth(M, N, ks, K, p.full);
            return p;
        }
    }
    if (batch == 1 && p.blocks <= cu_count) {
        int64_t S = std::min<int64_t>(kMaxTileSplit, 2 * (int64_t)cu_count / p.blocks);
        S = std::min<int64_t>(S, K / kMinTileSplitDepth);
        S = std::min<int64_t>(S, kSplitFloatsPerCu * cu_count / (M * N));
        if (S >= 2) {
            const int64_t ks = ((K + S - 1) / S + p.bk - 1) / p.bk * p.bk;
            S = (K + ks - 1) / ks;
            if (S >= 2) {
                p.fallback = p.kind;
                p.fallback_full = p.full;
                p.split_tile = p.kind;
                p.kind = GemmKind::SplitK;
                p.splits = S;
                p.ks = ks;
                p.blocks *= S;
            }
        }
    }
    return p;
}

// Stream-K on the LDS-loading 256x256 tile: one block per CU, each taking
// an equal share of the product's (tile, slice) units, then one pass adding
// the pieces of the tiles split between blocks (gemm_f32_mfma_lds_sk).  It
// removes the idle CUs of a last, partial round of tiles (6144^3: 576
// tiles, three rounds of 256 for 2.25 rounds of work) and of outputs with
// fewer tiles than CUs that no power-of-two K split fills (3072^3: 144).
//
// The choice compares estimated times in k steps of one 256x256 tile on one
// CU (0.21 us at the measured 0.92 of peak): the plan above by its rounds of
// blocks, and stream-K by its even share plus kStreamKCost for the pieces'
// extra traffic (two 256 KiB pieces per split tile written, read back and
// added, at most one split tile per block), the fix-up launch and a block's
// extra segment starts.  The 128x128 and 64x128 tiles cost 0.30 and 0.175
// of a large k step per k (their measured rates and areas).  Stream-K needs
// tiles at least 85% covered, no K split of its own (ktotal), and at least
// kStreamKMinWork k steps per CU.
constexpr double kStreamKCost = 150.0;
constexpr double kStreamKMinWork = 192.0;
constexpr double kStreamKGain = 1.15;
constexpr double kSmallStep = 0.30, kMediumStep = 0.175;

double plan_k_steps(const GemmPlan &p, int64_t K, int cu_count) {
    const auto rounds = [&](int64_t blocks) { return (double)((blocks + cu_count - 1) / cu_count); };
    switch (p.kind) {
    case GemmKind::Large: return rounds(p.blocks) * (double)K;
    case GemmKind::SplitK: {
        const double step = p.split_tile == GemmKind::Large ? 1.0 : p.split_tile == GemmKind::Medium ? kMediumStep : kSmallStep;
        return rounds(p.blocks) * (double)p.ks * step + 50.0;
    }
    case GemmKind::Medium: return rounds(p.blocks) * (double)K * kMediumStep;
    case GemmKind::Small: return rounds(p.blocks) * (double)K * kSmallStep;
    default: return 0.0;
    }
}

GemmPlan plan_gemm(const GemmArgs &g, bool a_plain, bool a_trans, bool b_plain, bool b_trans, int cu_count) {
    GemmPlan p = plan_gemm_tiles(g, a_plain, a_trans, b_plain, b_trans, cu_count);
    if (p.kind == GemmKind::Strided || p.main_m || g.ktotal) return p;
    const int bk = lds_tile_depth(g, !a_plain);
    if (!bk) return p;
    const int64_t tiles = ((g.M + 255) / 256) * ((g.N + 255) / 256) * g.batch;
    if ((double)(g.M * g.N * g.batch) < 0.85 * (double)(tiles * kLargeTileFloats)) return p;
    const double work = (double)tiles * (double)g.K / cu_count;
    if (work < kStreamKMinWork || plan_k_steps(p, g.K, cu_count) < kStreamKGain * (work + kStreamKCost)) return p;
    GemmPlan sk;
    sk.kind = GemmKind::StreamK;
    sk.bm = 256, sk.bn = 256, sk.bk = bk;
    sk.splits = 0;
    sk.blocks = cu_count;
    sk.fallback = p.kind == GemmKind::SplitK ? p.fallback : p.kind;
    sk.fallback_full = p.kind == GemmKind::SplitK ? p.fallback_full : p.full;
    return sk;
}

// Runs a stream-K plan; TRS_E_ALLOCATION_FAILED, with nothing launched, when
// the workspace (two partial tiles per block, 512 KiB per CU) cannot be had.
int launch_stream_k(const GemmPlan &p, GemmArgs g, bool a_plain, bool b_plain, int cu_count, hipStream_t s) {
    void *ws = nullptr;
    int rc = trs_alloc((size_t)(2 * (int64_t)cu_count * kLargeTileFloats) * sizeof(float), &ws);
    if (rc) return rc;
    g.sk_blocks = cu_count;
    g.sk_ws = (float *)ws;
    if (a_plain && b_plain) rc = launch_lds_layout<false, false>(g, p.bk, s);
    else if (a_plain) rc = launch_lds_layout<false, true>(g, p.bk, s);
    else if (b_plain) rc = launch_lds_layout<true, false>(g, p.bk, s);
    else rc = launch_lds_layout<true, true>(g, p.bk, s);
    const int frc = trs_free(ws);
    return rc ? rc : frc;
}

// Runs a split plan; returns TRS_E_ALLOCATION_FAILED without launching
// anything when the workspace cannot be had (the caller then runs the
// unsplit tile).  `sak`/`sbk` are the operands' k strides.
int launch_split_k(const GemmPlan &p, GemmArgs g, bool a_plain, bool b_plain, int64_t sak, int64_t sbk,
                   int cu_count, hipStream_t s) {
    float *const C = g.c;
    const int64_t mn = g.M * g.N, S = p.splits, Ks = p.ks;
    void *ws = nullptr;
    int rc = trs_alloc((size_t)(S * mn) * sizeof(float), &ws);
    if (rc) return rc;
    g.c = (float *)ws;
    g.ktotal = g.K;
    g.K = Ks;
    g.bsa = Ks * sak;
    g.bsb = Ks * sbk;
    g.bsc = mn;
    g.batch = S;
    switch (p.split_tile) {
    case GemmKind::Large: rc = launch_large(g, a_plain, b_plain, p.full, s); break;
    case GemmKind::Medium: rc = launch_medium(g, a_plain, b_plain, s); break;
    default: rc = launch_small(g, a_plain, b_plain, p.full, s); break;
    }
    if (rc == TRS_OK) {
        if (mn % 4 == 0 && (uintptr_t)C % 16 == 0) {
            const int64_t n4 = mn / 4;
            // A sum of at most two blocks per CU is load-latency bound: its
            // lanes issue every slice's load at once.  A larger one keeps one
            // load per lane in flight and leaves the latency to the many
            // resident waves (all at once measured 0.3 us slower at 1000^3
            // and 0.5% on the [8192,4096] -> 4096 -> 1024 MLP step).
            const dim3 grid((unsigned)((n4 + 255) / 256));
            if (n4 <= 2 * 256 * (int64_t)cu_count)
                launch_splitk_sum((int)S, grid, s, (const float4 *)ws, (float4 *)C, n4);
            else
                hipLaunchKernelGGL(splitk_sum<0>, grid, dim3(kHelperLanes), 0, s, (const float4 *)ws, (float4 *)C, n4, (int)S);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) rc = hip_fail(e, "split-k sum launch");
        } else {
            rc = launch_slice_sum((const float *)ws, C, mn, 1, S, s);
        }
    }
    const int frc = trs_free(ws);
    return rc ? rc : frc;
}

// Operand analysis shared by trs_matmul_f32 and trs_matmul_plan_f32: checks
// the layouts and fills the GEMM arguments.  *empty is set when nothing is
// to be computed (an empty output, or K = 0).
struct GemmSetup {
    GemmArgs g{};
    bool a_plain = false, a_trans = false, b_plain = false, b_trans = false;
    int64_t sam = 0, sak = 0, sbk = 0, sbn = 0;
    bool empty_output = false, zero_k = false;
};

int setup_gemm(const float *a, const trs_layout *la, const float *b, const trs_layout *lb, float *c,
               const trs_layout *lc, bool check_pointers, GemmSetup *st) {
    int rc = check_layout(la, "left");
    if (!rc) rc = check_layout(lb, "right");
    if (!rc) rc = check_layout(lc, "output");
    if (rc) return rc;
    if (la->rank != lb->rank || (la->rank != 2 && la->rank != 3))
        return set_error(TRS_E_MATMUL_REQUIRES_MATRICES,
                         "matmul currently requires two rank-2 tensors (or two rank-3 batches), got ranks %d and %d",
                         la->rank, lb->rank);
    const int r = la->rank;
    const int64_t batch = r == 3 ? la->shape[0] : 1;
    if (r == 3 && (lb->shape[0] != batch))
        return set_error(TRS_E_SHAPE_MISMATCH, "batch sizes differ (%lld and %lld)", (long long)batch,
                         (long long)lb->shape[0]);
    const int64_t M = la->shape[r - 2], K = la->shape[r - 1], K2 = lb->shape[r - 2], N = lb->shape[r - 1];
    if (K != K2)
        return set_error(TRS_E_MATMUL_INNER_MISMATCH, "mat1 and mat2 shapes cannot be multiplied (%lldx%lld and %lldx%lld)",
                         (long long)M, (long long)K, (long long)K2, (long long)N);
    if (lc->rank != r || lc->shape[r - 2] != M || lc->shape[r - 1] != N || (r == 3 && lc->shape[0] != batch))
        return set_error(TRS_E_SHAPE_MISMATCH, "matmul output layout has the wrong shape");
    if (!layout_is_contiguous(lc)) return set_error(TRS_E_INVALID_ARGUMENT, "matmul output must be contiguous");
    st->empty_output = M == 0 || N == 0 || batch == 0;
    st->zero_k = K == 0;
    if (st->empty_output) return TRS_OK;
    if (check_pointers) {
        // With K = 0 the operands are empty (no storage is needed) and C is +0.0.
        if (!c || (K > 0 && (!a || !b))) return set_error(TRS_E_INVALID_ARGUMENT, "null matmul operand");
        // C is written while A and B are still being read: no shared memory.
        const ByteRange out_bytes = byte_range(c, lc, 4);
        if (K > 0 && (ranges_overlap(out_bytes, byte_range(a, la, 4)) || ranges_overlap(out_bytes, byte_range(b, lb, 4))))
            return set_error(TRS_E_INVALID_ARGUMENT, "matmul output overlaps an operand");
    }
    st->sam = la->stride[r - 2], st->sak = la->stride[r - 1];
    st->sbk = lb->stride[r - 2], st->sbn = lb->stride[r - 1];
    const int64_t bsa = r == 3 ? la->stride[0] : 0, bsb = r == 3 ? lb->stride[0] : 0;
    // A unit-stride along k (plain) or along m (transposed view); same for B.
    st->a_plain = st->sak == 1 || K == 1;
    st->a_trans = !st->a_plain && (st->sam == 1 || M == 1);
    st->b_plain = st->sbn == 1 || N == 1;
    st->b_trans = !st->b_plain && (st->sbk == 1 || K == 1);
    GemmArgs &g = st->g;
    g.a = a ? a + la->offset : nullptr;
    g.b = b ? b + lb->offset : nullptr;
    g.c = c ? c + lc->offset : nullptr;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = st->a_plain ? st->sam : st->sak;
    g.ldb = st->b_plain ? st->sbk : st->sbn;
    g.ldc = N;
    g.bsa = bsa;
    g.bsb = bsb;
    g.bsc = M * N;
    g.batch = batch;
    return TRS_OK;
}

// The skinny form of a product whose operands each have a unit stride and
// whose output has at most kSkinnyMaxRows rows or columns: the short side
// is X's rows (A's rows, or B's columns read as B^T) and the other operand
// is Y.  Returns false otherwise.
bool skinny_problem(const GemmSetup &st, SkinnyProblem *sp) {
    const GemmArgs &g = st.g;
    if (!(st.a_plain || st.a_trans) || !(st.b_plain || st.b_trans)) return false;
    const bool short_m = g.M <= g.N;
    if ((short_m ? g.M : g.N) > kSkinnyMaxRows) return false;
    SkinnyProblem p;
    p.K = g.K;
    p.batch = g.batch;
    p.out = g.c;
    if (short_m) {
        // X(i, k) = A(i, k); Y(k, j) = B(k, j); C(i, j) at i*N + j.
        p.x = g.a, p.y = g.b;
        p.R = g.M, p.L = g.N;
        p.xi = st.a_plain ? g.lda : 1;
        p.xk = st.a_plain ? 1 : g.lda;
        p.dot = !st.b_plain;
        p.yl = g.ldb;
        p.oi = g.N, p.oj = 1;
        p.bx = g.bsa, p.by = g.bsb;
    } else {
        // X(i, k) = B(k, i); Y(k, j) = A(j, k); C(j, i) at j*N + i.
        p.x = g.b, p.y = g.a;
        p.R = g.N, p.L = g.M;
        p.xi = st.b_plain ? 1 : g.ldb;
        p.xk = st.b_plain ? g.ldb : 1;
        p.dot = st.a_plain;
        p.yl = g.lda;
        p.oi = 1, p.oj = g.N;
        p.bx = g.bsb, p.by = g.bsa;
    }
    *sp = p;
    return true;
}

int run_unsplit(const GemmPlan &p, const GemmArgs &g, bool a_plain, bool b_plain, hipStream_t s) {
    switch (p.kind) {
    case GemmKind::Large:
    case GemmKind::SplitK: return launch_large(g, a_plain, b_plain, p.full, s);
    case GemmKind::Medium: return launch_medium(g, a_plain, b_plain, s);
    default: return launch_small(g, a_plain, b_plain, p.full, s);
    }
}

// A Large plan with rims: the tile on C[0:main_m, 0:main_n], then the rows
// below as one skinny product (X = those rows of A, Y = B, full width) and
// the columns to the right of the tile's rows as another (X = those columns
// of B read as B^T, Y = A's first main_m rows), each writing its part of C
// in place.
int run_peeled(const GemmPlan &p, const GemmSetup &st, int cu_count, hipStream_t s) {
    const GemmArgs &g = st.g;
    GemmArgs gm = g;
    gm.M = p.main_m;
    gm.N = p.main_n;
    TRS_CHECK(launch_large(gm, st.a_plain, st.b_plain, p.full, s));
    if (p.main_m < g.M) {
        SkinnyProblem r;
        r.R = g.M - p.main_m, r.L = g.N, r.K = g.K, r.batch = 1;
        r.x = st.a_plain ? g.a + p.main_m * g.lda : g.a + p.main_m;
        r.xi = st.a_plain ? g.lda : 1;
        r.xk = st.a_plain ? 1 : g.lda;
        r.y = g.b, r.dot = !st.b_plain, r.yl = g.ldb;
        r.out = g.c + p.main_m * g.ldc, r.oi = g.ldc, r.oj = 1;
        SkinnyPlan rp;
        if (!plan_skinny(r, cu_count, &rp)) return set_error(TRS_E_INVALID_ARGUMENT, "gemm row rim has no plan");
        TRS_CHECK(run_skinny(r, rp, s));
    }
    if (p.main_n < g.N) {
        SkinnyProblem c;
        c.R = g.N - p.main_n, c.L = p.main_m, c.K = g.K, c.batch = 1;
        c.x = st.b_plain ? g.b + p.main_n : g.b + p.main_n * g.ldb;
        c.xi = st.b_plain ? 1 : g.ldb;
        c.xk = st.b_plain ? g.ldb : 1;
        c.y = g.a, c.dot = st.a_plain, c.yl = g.lda;
        c.out = g.c + p.main_n, c.oi = 1, c.oj = g.ldc;
        SkinnyPlan cp;
        if (!plan_skinny(c, cu_count, &cp)) return set_error(TRS_E_INVALID_ARGUMENT, "gemm column rim has no plan");
        TRS_CHECK(run_skinny(c, cp, s));
    }
    return TRS_OK;
}

}  // namespace

}  // namespace trs

using namespace trs;

extern "C" int trs_matmul_f32(const float *a, const trs_layout *la, const float *b, const trs_layout *lb,
                              float *c, const trs_layout *lc) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    GemmSetup st;
    int rc = setup_gemm(a, la, b, lb, c, lc, true, &st);
    if (rc || st.empty_output) return rc;
    const GemmArgs &g = st.g;
    if (st.zero_k) return trs_memset_zero(g.c, (size_t)(g.M * g.N * g.batch) * sizeof(float));
    SkinnyProblem sp;
    SkinnyPlan spl;
    if (skinny_problem(st, &sp) && plan_skinny(sp, dev->cu_count, &spl)) return run_skinny(sp, spl, dev->stream);
    const GemmPlan p = plan_gemm(g, st.a_plain, st.a_trans, st.b_plain, st.b_trans, dev->cu_count);
    if (p.main_m) return run_peeled(p, st, dev->cu_count, dev->stream);
    if (p.kind == GemmKind::Strided) {
        // An operand with no unit stride is gathered into a contiguous buffer
        // from the block cache (the library's copy kernel, bit for bit), and
        // the product runs on the MFMA tiles: 1024^3 over stride-2 views took
        // 0.589 ms in the one-lane-per-output kernel below, against 0.049 ms
        // for contiguous operands.  The buffers go back to the cache in stream
        // order.  Without memory for them, that kernel runs instead.
        const bool ga = !(st.a_plain || st.a_trans), gb = !(st.b_plain || st.b_trans);
        const trs_layout ca = contiguous_like(la), cb = contiguous_like(lb);
        void *ta = nullptr, *tb = nullptr;
        if (ga) rc = trs_alloc((size_t)layout_numel(la) * sizeof(float), &ta);
        if (!rc && gb) rc = trs_alloc((size_t)layout_numel(lb) * sizeof(float), &tb);
        if (!rc && ga) rc = trs_unary_f32(TRS_COPY, a, la, (float *)ta, &ca);
        if (!rc && gb) rc = trs_unary_f32(TRS_COPY, b, lb, (float *)tb, &cb);
        if (!rc)
            rc = trs_matmul_f32(ga ? (const float *)ta : a, ga ? &ca : la, gb ? (const float *)tb : b, gb ? &cb : lb,
                                c, lc);
        const bool no_memory = rc == TRS_E_ALLOCATION_FAILED;
        if (ta) trs_free(ta);
        if (tb) trs_free(tb);
        if (!no_memory) return rc;
        hipLaunchKernelGGL(gemm_f32_strided, dim3((unsigned)p.blocks), dim3(kHelperLanes), 0, dev->stream, g.a, g.b, g.c, g.M,
                           g.N, g.K, st.sam, st.sak, st.sbk, st.sbn, g.bsa, g.bsb, g.batch);
        TRS_LAUNCH_CHECK("strided gemm launch");
        return TRS_OK;
    }
    if (p.kind == GemmKind::StreamK) {
        rc = launch_stream_k(p, g, st.a_plain, st.b_plain, dev->cu_count, dev->stream);
        if (rc != TRS_E_ALLOCATION_FAILED) return rc;
        // No workspace: run the plan stream-K replaced, unsplit.
        GemmPlan fb;
        fb.kind = p.fallback;
        fb.full = p.fallback_full;
        return run_unsplit(fb, g, st.a_plain, st.b_plain, dev->stream);
    }
    if (p.kind == GemmKind::SplitK) {
        rc = launch_split_k(p, g, st.a_plain, st.b_plain, st.sak, st.sbk, dev->cu_count, dev->stream);
        if (rc != TRS_E_ALLOCATION_FAILED) return rc;
        // No workspace: the split is only an optimisation, so run the tile the
        // plan would otherwise have chosen (nothing was launched).
        GemmPlan fb;
        fb.kind = p.fallback;
        fb.full = p.fallback_full;
        return run_unsplit(fb, g, st.a_plain, st.b_plain, dev->stream);
    }
    return run_unsplit(p, g, st.a_plain, st.b_plain, dev->stream);
}

extern "C" int trs_matmul_plan_f32(const float *a, const trs_layout *la, const float *b, const trs_layout *lb,
                                   const float *c, const trs_layout *lc, int *tile_m, int *tile_n, int *tile_k,
                                   int64_t *splits, int64_t *blocks) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    GemmSetup st;
    int rc = setup_gemm(a, la, b, lb, const_cast<float *>(c), lc, false, &st);
    if (rc) return rc;
    GemmPlan p;
    const bool work = !st.empty_output && !st.zero_k;
    if (work) p = plan_gemm(st.g, st.a_plain, st.a_trans, st.b_plain, st.b_trans, dev->cu_count);
    GemmSetup sg;
    const GemmSetup *ran = &st;
    if (p.kind == GemmKind::Strided) {
        // What trs_matmul_f32 runs: the plan of the gathered, contiguous
        // operands (their buffers come from the block cache, 256-byte aligned).
        const bool ga = !(st.a_plain || st.a_trans), gb = !(st.b_plain || st.b_trans);
        const trs_layout ca = contiguous_like(la), cb = contiguous_like(lb);
        rc = setup_gemm(ga ? nullptr : a, ga ? &ca : la, gb ? nullptr : b, gb ? &cb : lb, const_cast<float *>(c), lc,
                        false, &sg);
        if (rc) return rc;
        p = plan_gemm(sg.g, sg.a_plain, sg.a_trans, sg.b_plain, sg.b_trans, dev->cu_count);
        ran = &sg;
    }
    SkinnyProblem sp;
    SkinnyPlan spl;
    if (work && skinny_problem(*ran, &sp) && plan_skinny(sp, dev->cu_count, &spl)) {
        // The short side's padded MFMA rows by the 64 columns of a block, or
        // for the matrix-vector kernel its 1, 2 or 4 rows by the 4 rows of
        // the long operand a block takes.
        const bool short_m = ran->g.M <= ran->g.N;
        const int rows = (spl.gemv || spl.axpy) ? spl.row_groups : 16 * spl.row_groups;
        const int cols = spl.gemv ? 4 : spl.axpy ? kAxpyCols : spl.lds ? kLdsSkinnyCols : kSkinnyCols;
        p.bm = short_m ? rows : cols;
        p.bn = short_m ? cols : rows;
        p.bk = (int)spl.kc;
        p.splits = spl.splits;
        p.blocks = spl.blocks;
    }
    if (tile_m) *tile_m = p.bm;
    if (tile_n) *tile_n = p.bn;
    if (tile_k) *tile_k = p.bk;
    if (splits) *splits = p.splits;
    if (blocks) *blocks = p.blocks;
    return TRS_OK;
}
