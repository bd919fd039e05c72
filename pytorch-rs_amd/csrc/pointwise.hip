// pointwise.hip -- reductions and the backward helpers built on them: the
// device sum, the ordered broadcast-reduction VJPs (add and mul unbroadcast),
// fills and in-place accumulation.  The pointwise op families live in
// pw_binary.hip, pw_scalar.hip, pw_unary.hip and pw_mask.hip over pw_ops.h.
// Each entry point replaces the loop of one reference function, cited at the
// entry point.  Compiled with -ffp-contract=off.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>

#include "pw_core.h"
#include "pw_host.h"
#include "trs_internal.h"

namespace trs {

// ---- reductions -------------------------------------------------------------

constexpr int kSumBlocks = 1024;
constexpr int64_t kSumOneBlock = 32768;  // at most 128 elements per lane in one block

// Fixed-order two-level sum.  Pass 1: block b sums the contiguous element
// range [b*chunk, (b+1)*chunk) -- lane l adds elements l, l+256, ... in order,
// then a fixed LDS tree over the 256 lanes.  Pass 2 sums the block partials
// in the same way.  Up to kSumOneBlock elements, pass 1 runs as one block
// over the whole range.  The order depends only on the element count.
// Every lane starts from -0.0, the additive identity (x + -0.0 == x for every
// x, +0.0 included), as Rust's f32 Sum does: an all-(-0.0) input sums to
// -0.0 and every other result is unchanged by the start value.
// Error bound: an element passes through at most ceil(chunk/256) in-lane
// additions, 8 tree levels, 4 in-lane additions of pass 2 and 8 more tree
// levels, so |sum - exact| <= (ceil(chunk/256) + 20) * 2^-24 * sum|x|
// (one block: ceil(n/256) + 8).
template <bool CONTIG>
__global__ void __launch_bounds__(256) sum_pass1(const float *x, PwGeom g, int64_t chunk, float *partial) {
    __shared__ float red[256];
    const int64_t begin = (int64_t)blockIdx.x * chunk;
    const int64_t end = begin + chunk < g.numel ? begin + chunk : g.numel;
    auto offset_of = [&](int64_t e) -> int64_t {
        if constexpr (CONTIG) {
            return g.ioff[0] + e;
        } else {
            int64_t oo, io[1];
            decode_outer<1>(g, g.rank, e, oo, io);
            return io[0];
        }
    };
    // The lane's elements are added one by one in index order; only the
    // loads run ahead: U of them are issued before their U additions, so a
    // lane waits for memory once per U elements instead of once per element
    // (the additions, and so the bits, are those of the plain loop).
    constexpr int U = 8;
    float acc = -0.0f;
    int64_t e = begin + threadIdx.x;
    for (; e + (U - 1) * 256 < end; e += U * 256) {
        float v[U];
#pragma unroll
        for (int k = 0; k < U; k++) v[k] = x[offset_of(e + k * 256)];
#pragma unroll
        for (int k = 0; k < U; k++) acc += v[k];
    }
    for (; e < end; e += 256) acc += x[offset_of(e)];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

__global__ void __launch_bounds__(256) sum_pass2(const float *partial, int n, float *out) {
    __shared__ float red[256];
    float acc = -0.0f;
    for (int e = threadIdx.x; e < n; e += 256) acc += partial[e];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = red[0];
}

// Scratch of trs_sum_f32_noalloc: pass 1's block partials, kSumBlocks floats
// (4 KiB) in a file-scope device array that each GPU holds until the process
// ends.  In host code `scratch` names a host-side stand-in, not device
// memory: kernels receive only the address setup_sum_scratch looks up.
static __device__ __align__(256) float scratch[kSumBlocks];

__global__ void __launch_bounds__(kHelperLanes) fill_kernel(float *out, size_t n, float value, const float *src) {
    const float v = src ? src[0] : value;
    const size_t stride = (size_t)gridDim.x * kHelperLanes;
    for (size_t i = (size_t)blockIdx.x * kHelperLanes + threadIdx.x; i < n; i += stride) out[i] = v;
}

// Broadcast-reduction: grad[j] = sum over the reduced dims (row-major order)
// of up[o] * (other ? other[o] : 1), accumulated from +0.0, one thread per
// operand element j.  `kept` dims are the operand's non-broadcast dims of the
// output; `red` dims are the dims it was broadcast along.
struct ReduceGeom {
    int32_t nkept;
    int32_t nred;
    int64_t kept_size[TRS_MAX_RANK];
    int64_t kept_up[TRS_MAX_RANK];     // strides of up (output-contiguous) per kept dim
    int64_t kept_other[TRS_MAX_RANK];  // strides of other per kept dim
    int64_t red_size[TRS_MAX_RANK];
    int64_t red_up[TRS_MAX_RANK];
    int64_t red_other[TRS_MAX_RANK];
    int64_t nself;
    int64_t nred_total;
    int64_t other_off;
};

// One lane per operand element j: its reduced dims walked with an odometer,
// kUnroll loads issued ahead of their ordered adds (the adds are the
// reference's sequence; only the loads run ahead).  Used for short chains
// and for layouts whose reduced or kept dims do not merge.
constexpr int kRedUnroll = 8;

template <bool HAS_OTHER>
__global__ void __launch_bounds__(kHelperLanes) reduce_bcast_kernel(const float *up, const float *other, ReduceGeom rg,
                                                           float *grad) {
    const int64_t stride = (int64_t)gridDim.x * kHelperLanes;
    for (int64_t j = (int64_t)blockIdx.x * kHelperLanes + threadIdx.x; j < rg.nself; j += stride) {
        int64_t ub = 0, ob = rg.other_off, rem = j;
        for (int d = rg.nkept - 1; d >= 0; d--) {
            const int64_t c = rem % rg.kept_size[d];
            rem /= rg.kept_size[d];
            ub += c * rg.kept_up[d];
            ob += c * rg.kept_other[d];
        }
        float acc = 0.0f;
        // The reduced positions in row-major order: the innermost reduced dim
        // is stepped by its strides, and where it wraps the next position is
        // decoded afresh (no per-dim counters, so no local array at any rank).
        const int last = rg.nred - 1;
        const int64_t isz = rg.nred ? rg.red_size[last] : 1;
        const int64_t iup = rg.nred ? rg.red_up[last] : 0, iot = rg.nred ? rg.red_other[last] : 0;
        auto position = [&](int64_t r, int64_t &u, int64_t &o) {
            u = ub;
            o = ob;
            for (int d = last; d >= 0; d--) {
                const int64_t q = r / rg.red_size[d];
                const int64_t cd = r - q * rg.red_size[d];
                r = q;
                u += cd * rg.red_up[d];
                o += cd * rg.red_other[d];
            }
        };
        int64_t uo = ub, oo = ob, ci = 0;
        for (int64_t r0 = 0; r0 < rg.nred_total; r0 += kRedUnroll) {
            float c[kRedUnroll];
#pragma unroll
            for (int i = 0; i < kRedUnroll; i++) {
                if (r0 + i < rg.nred_total) {
                    c[i] = up[uo];
                    if constexpr (HAS_OTHER) c[i] = c[i] * other[oo];
                    if (++ci < isz) {
                        uo += iup;
                        oo += iot;
                    } else {
                        ci = 0;
                        position(r0 + i + 1, uo, oo);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kRedUnroll; i++)
                if (r0 + i < rg.nred_total) acc += c[i];
        }
        grad[j] = acc;
    }
}

// Staged broadcast reduction for `up` viewed as [KO, R, KI]: the reduced dims
// merged into R rows, the operand's kept dims into KO outer and KI inner, KI
// unit-stride in up.  grad[ko, ki] = sum over r in order of up[ko, r, ki]
// (times other[ko, r, ki]) from +0.0.  Each of the KO*KI sums is a chain of R
// dependent adds that the reference's order forbids splitting, so the chains
// are few and long (a bias gradient over [8192, 4096] has 4096 chains of
// 8192): one lane per chain could keep far too few loads in flight, and a
// chain costs R dependent adds whatever the layout (about 6 cycles each for a
// wave fed from LDS).
//
// A block owns 32 chains.  Eight producer waves load stages of SR rows of
// those 32 columns AHEAD stages in advance into registers: each lane SR/256
// blocks of 4x4 (4 rows of 4 chains), multiplied by `other` (one rounding, as
// the reference's up * other), transposed in registers and stored
// chain-major into a double-buffered LDS stage.  A ninth wave adds: lane c
// reads chain c's rows 4 at a time (ds_read_b128) and adds them in row order,
// one stage behind the producers, so its adds overlap the next stage's loads
// and stores.  The producer and adder roles are wave-uniform and each runs
// the same number of barriers.  The launcher uses SR = 256 (66.5 KB of LDS,
// two blocks per CU); 512-row stages measured no faster.
constexpr int kStRows = 256;
constexpr int kStChains = 32;                    // chains per block (adder lanes 0..31)
constexpr int kStProducers = 8;                  // producer waves; wave 8 adds
constexpr int kStLanes = (kStProducers + 1) * 64;

struct RedColsGeom {
    int64_t KO, R, KI;
    int64_t up_ko, up_r;          // up strides (the ki stride is 1)
    int64_t ot_ko, ot_r, ot_ki;   // other strides
    int64_t other_off;
};

// How the producers read `other`: not at all, as 16-byte vectors along ki
// (4 chains of a row), as vectors along r (4 rows of a chain, a transposed
// view such as c.mT), or one float at a time.
enum RedOther { kOtNone = 0, kOtVecKi = 1, kOtVecR = 2, kOtScalar = 3 };

// Raw buffer descriptor word 3 (32-bit data format: untyped loads, no
// swizzle).
constexpr int kRawBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t stage_rsrc(const float *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, bytes, kRawBufferWord3);
}

// Bytes a stage's descriptor covers: from the stage's first row through
// `tail` floats past the start of the last of `rem` remaining rows (rows
// `row_stride` floats apart); none when no rows remain.
__device__ __forceinline__ int stage_span(int64_t rem, int64_t row_stride, int64_t tail) {
    if (rem <= 0) return 0;
    const int64_t b = ((rem - 1) * row_stride + tail) * 4;
    return (int)(uint32_t)(b < 0xFFFFFFFFll ? b : 0xFFFFFFFFll);
}

__device__ __forceinline__ vf4 buffer_vf4(__amdgpu_buffer_rsrc_t rs, int off) {
    return __builtin_bit_cast(vf4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
}

// A register copy the compiler cannot move or merge: without a product the
// transpose is plain copies, which the register allocator would otherwise
// gather at the loop's back edge, where they wait for every load in flight.
__device__ __forceinline__ float stage_copy(float x) {
    float y;
    asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
    return y;
}

// CH = 32 or 16 chains per block.  A producer wave covers CH/4 chain quads
// by RQ = 256/CH row quads.  With 16, a block reads 64 B of each row, and
// blocks b and b + 8 (one XCD) take the two halves of each 128 B line, so
// the line is fetched once into that XCD's L2; the launcher uses it when
// 32-chain blocks would leave CUs idle.
template <int OT, int AHEAD, int SR, int CH = kStChains>
__global__ void __launch_bounds__(kStLanes) reduce_stage_kernel(const float *up, const float *other, RedColsGeom g,
                                                                 float *grad) {
    static_assert(CH == 32 || CH == 16, "chains per block");
    constexpr int RQ = 256 / CH;                // row quads per producer wave
    constexpr int QUADS = kStProducers * RQ;    // row quads per producer pass
    constexpr int NQ = SR / (4 * QUADS);        // 4x4 blocks per producer lane per stage
    // Floats per chain in a stage: (SR + 4) / 4 is 1 mod 16, so the b128
    // accesses of 8 consecutive lanes (chain-strided for the adder,
    // row-strided for the producers) fall on distinct 4-bank groups.
    constexpr int PITCH = SR + 4;
    static_assert(NQ >= 1 && NQ * 4 * QUADS == SR && (PITCH / 4) % 16 == 1, "stage shape");
    __shared__ __attribute__((aligned(16))) float stage[2][CH][PITCH];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t groups = g.KI / CH;
    const int64_t ko = blockIdx.x / groups;
    int64_t gi = blockIdx.x % groups;
    if (CH == 16 && groups % 16 == 0)  // blocks b, b + 8: the two halves of one 128 B line
        gi = (gi / 16) * 16 + 2 * (gi % 8) + (gi / 8) % 2;
    const int64_t ki0 = gi * CH;
    const int64_t nst = (g.R + SR - 1) / SR;
    const int64_t nit = (nst + AHEAD - 1) / AHEAD * AHEAD;  // stages run, padded to whole rings
    if (wave < kStProducers) {
        const int cq = lane / RQ;  // chains cq*4 .. cq*4+3
        // row quads j*QUADS + wave*RQ + lane%RQ of a stage, j < NQ
        const int quad0 = wave * RQ + lane % RQ;
        // Loads go through a buffer descriptor per stage, built in scalar
        // registers from the block's base and the stage index: a lane's byte
        // offsets within a stage never change, and the descriptor's extent
        // ends after the last row below R, so the hardware returns 0 for the
        // rows past R (never added) without any per-row address arithmetic.
        const float *ub = up + ko * g.up_ko + ki0;
        const float *ob = OT != kOtNone ? other + g.other_off + ko * g.ot_ko + ki0 * g.ot_ki : nullptr;
        int vu[NQ][4], vo[NQ][4];
#pragma unroll
        for (int j = 0; j < NQ; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t row = (j * QUADS + quad0) * 4 + i;
                vu[j][i] = (int)((row * g.up_r + cq * 4) * 4);
                if constexpr (OT == kOtVecKi) vo[j][i] = (int)((row * g.ot_r + cq * 4) * 4);
                else if constexpr (OT == kOtVecR)
                    vo[j][i] = (int)(((int64_t)(cq * 4 + i) * g.ot_ki + (j * QUADS + quad0) * 4) * 4);
                else vo[j][i] = 0;
            }
        // ru[s][j][i]: row i's 4 chains; ro[s][j][i]: the same for kOtVecKi
        // and kOtScalar, chain i's 4 rows for kOtVecR.
        vf4 ru[AHEAD][NQ][4], ro[AHEAD][NQ][4];
        auto issue = [&](int slot, int64_t st) {
            const int64_t sc = st < nst ? st : nst - 1;  // past the end: no rows, base kept in range
            const int64_t rem = g.R - st * SR;            // rows from this stage's first on
            const auto rs = stage_rsrc(ub + sc * SR * g.up_r, stage_span(rem, g.up_r, CH));
#pragma unroll
            for (int j = 0; j < NQ; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) ru[slot][j][i] = buffer_vf4(rs, vu[j][i]);
            if constexpr (OT == kOtVecKi) {
                const auto os = stage_rsrc(ob + sc * SR * g.ot_r, stage_span(rem, g.ot_r, CH));
#pragma unroll
                for (int j = 0; j < NQ; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) ro[slot][j][i] = buffer_vf4(os, vo[j][i]);
            } else if constexpr (OT == kOtVecR) {
                // the last chain's remaining rows end the extent
                const auto os = stage_rsrc(ob + sc * SR, stage_span(rem, 1, (CH - 1) * g.ot_ki + 1));
#pragma unroll
                for (int j = 0; j < NQ; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) ro[slot][j][i] = buffer_vf4(os, vo[j][i]);
            } else if constexpr (OT == kOtScalar) {
                const float *oc = ob + cq * 4 * g.ot_ki;
#pragma unroll
                for (int j = 0; j < NQ; j++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int64_t r = st * SR + (j * QUADS + quad0) * 4 + i;
                        const float *op = oc + (r < g.R ? r : g.R - 1) * g.ot_r;
                        ro[slot][j][i] = vf4{op[0], op[g.ot_ki], op[2 * g.ot_ki], op[3 * g.ot_ki]};
                    }
            }
        };
        // The ring starts at zero and the loop starts AHEAD stages early (the
        // stores of stages below 0 are never read): the first loads are then
        // issued by the loop's own code, into the registers every later load
        // of their slot uses, and the wait before each stage's transpose
        // covers that stage's loads only.
#pragma unroll
        for (int k = 0; k < AHEAD; k++)
#pragma unroll
            for (int j = 0; j < NQ; j++)
#pragma unroll
                for (int i = 0; i < 4; i++) ru[k][j][i] = ro[k][j][i] = vf4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int64_t s0 = -AHEAD; s0 < nit; s0 += AHEAD) {
#pragma unroll
            for (int k = 0; k < AHEAD; k++) {
                const int64_t st = s0 + k;
                // keeps this stage's register transpose (which waits for this
                // stage's loads only) from being hoisted with the others
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < NQ; j++) {
                    vf4 w[4];  // w[c]: chain c's 4 rows
#pragma unroll
                    for (int c = 0; c < 4; c++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            float v;
                            if constexpr (OT == kOtVecR) v = ru[k][j][i][c] * ro[k][j][c][i];
                            else if constexpr (OT != kOtNone) v = ru[k][j][i][c] * ro[k][j][i][c];
                            else v = stage_copy(ru[k][j][i][c]);
                            w[c][i] = v;
                        }
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        *(vf4 *)&stage[st & 1][cq * 4 + c][(j * QUADS + quad0) * 4] = w[c];
                }
                issue(k, st + AHEAD);
                __syncthreads();
            }
        }
    } else {
        float acc = 0.0f;
        const bool active = lane < CH;
        auto add_stage = [&](int64_t st) {
            const float *row = &stage[st & 1][lane & (CH - 1)][0];
            const int64_t left = g.R - st * SR;
            if (left >= SR) {
                // SR/4 quads in groups of 8, the next group read before the
                // current one is added
                vf4 a[8], b[8];
#pragma unroll
                for (int q = 0; q < 8; q++) a[q] = *(const vf4 *)&row[q * 4];
#pragma unroll
                for (int grp = 0; grp < SR / 32; grp++) {
                    if (grp + 1 < SR / 32) {
#pragma unroll
                        for (int q = 0; q < 8; q++) b[q] = *(const vf4 *)&row[(grp + 1) * 32 + q * 4];
                    }
                    __builtin_amdgcn_sched_barrier(0);  // keep those reads ahead of these adds
#pragma unroll
                    for (int q = 0; q < 8; q++) {
                        acc += a[q][0];
                        acc += a[q][1];
                        acc += a[q][2];
                        acc += a[q][3];
                    }
#pragma unroll
                    for (int q = 0; q < 8; q++) a[q] = b[q];
                }
            } else {
                for (int64_t r = 0; r < left; r++) acc += row[r];
            }
        };
        for (int64_t it = -AHEAD; it < nit; it++) {
            if (it >= 1 && it - 1 < nst && active) add_stage(it - 1);
            __syncthreads();
        }
        if (nit == nst && active) add_stage(nst - 1);  // written before the last barrier
        if (active) grad[ko * g.KI + ki0 + lane] = acc;
    }
}

// Merges a reduction's dims into [KO, R, KI] for the staged kernel: the
// reduced dims (in order) into one of R rows, the trailing kept dims into KI
// (unit stride in up), the other kept dims into KO.  Adjacent dims merge when
// the outer one's stride is the inner one's stride times its size, for up and
// (when present) for other.  False when the layout does not reduce to that.
bool reduce_cols_plan(const ReduceGeom &rg, bool has_other, RedColsGeom *cg) {
    auto merge = [&](int n, const int64_t *size, const int64_t *su, const int64_t *so, int first, int last,
                     int64_t *msize, int64_t *mu, int64_t *mo) -> bool {
        // dims [first, last] merge into one (row-major)
        int64_t sz = 1, u = 0, o = 0;
        for (int d = last; d >= first; d--) {
            if (d == last) {
                sz = size[d];
                u = su[d];
                o = so[d];
                continue;
            }
            if (su[d] != su[d + 1] * size[d + 1]) return false;
            if (has_other && so[d] != so[d + 1] * size[d + 1]) return false;
            sz *= size[d];
        }
        (void)n;
        *msize = sz;
        *mu = u;
        *mo = o;
        return true;
    };
    if (rg.nred < 1 || rg.nkept < 1) return false;
    int64_t R, ur, orr;
    if (!merge(rg.nred, rg.red_size, rg.red_up, rg.red_other, 0, rg.nred - 1, &R, &ur, &orr)) return false;
    // KI: the longest run of trailing kept dims that merges and ends with up
    // stride 1; KO: the rest (one merged dim, or none).
    if (rg.kept_up[rg.nkept - 1] != 1) return false;
    int first = rg.nkept - 1;
    while (first > 0) {
        const int d = first - 1;
        if (rg.kept_up[d] != rg.kept_up[d + 1] * rg.kept_size[d + 1]) break;
        if (has_other && rg.kept_other[d] != rg.kept_other[d + 1] * rg.kept_size[d + 1]) break;
        first = d;
    }
    int64_t KI, uki, oki;
    if (!merge(rg.nkept, rg.kept_size, rg.kept_up, rg.kept_other, first, rg.nkept - 1, &KI, &uki, &oki)) return false;
    int64_t KO = 1, uko = 0, oko = 0;
    if (first > 0 && !merge(rg.nkept, rg.kept_size, rg.kept_up, rg.kept_other, 0, first - 1, &KO, &uko, &oko))
        return false;
    cg->KO = KO;
    cg->R = R;
    cg->KI = KI;
    cg->up_ko = uko;
    cg->up_r = ur;
    cg->ot_ko = oko;
    cg->ot_r = orr;
    cg->ot_ki = oki;
    cg->other_off = rg.other_off;
    return true;
}

int reduce_to_operand(const float *up, const trs_layout *lout, const float *other,
                      const trs_layout *lother, const trs_layout *lself, float *grad) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    int rc = check_layout(lout, "output");
    if (!rc) rc = check_layout(lself, "operand");
    if (!rc && other) rc = check_layout(lother, "other");
    if (rc) return rc;
    if (lself->rank > lout->rank) return set_error(TRS_E_SHAPE_MISMATCH, "operand rank above output rank");
    ReduceGeom rg{};
    const int lead = lout->rank - lself->rank;
    const int olead = other ? lout->rank - lother->rank : 0;
    int64_t ustride[TRS_MAX_RANK];
    {
        int64_t s = 1;
        for (int d = lout->rank - 1; d >= 0; d--) {
            ustride[d] = s;
            s *= lout->shape[d];
        }
    }
    // Kept dims (the operand's own) and reduced dims (broadcast along), each
    // in output order.  Size-1 dims index nothing and are dropped; a dim that
    // continues the previous one of its kind in both up and other (stride =
    // next stride * next size) is merged into it.  Either way the operand's
    // row-major index and the row-major order of each chain are unchanged.
    struct DimList {
        int n = 0;
        int64_t size[TRS_MAX_RANK], up[TRS_MAX_RANK], ot[TRS_MAX_RANK];
        void add(int64_t sz, int64_t u, int64_t o) {
            if (n > 0 && up[n - 1] == u * sz && ot[n - 1] == o * sz) {
                size[n - 1] *= sz;
                up[n - 1] = u;
                ot[n - 1] = o;
                return;
            }
            size[n] = sz;
            up[n] = u;
            ot[n] = o;
            n++;
        }
    } kept, red;
    for (int d = 0; d < lout->rank; d++) {
        const int64_t osz = lout->shape[d];
        const bool self_bcast = d < lead || (lself->shape[d - lead] == 1 && osz != 1);
        if (d >= lead && lself->shape[d - lead] != osz && lself->shape[d - lead] != 1)
            return set_error(TRS_E_SHAPE_MISMATCH, "operand does not broadcast to the output");
        int64_t ost = 0;
        if (other && d >= olead) {
            const int64_t s = lother->shape[d - olead];
            if (s != osz && s != 1) return set_error(TRS_E_SHAPE_MISMATCH, "other does not broadcast");
            ost = (s == 1) ? 0 : lother->stride[d - olead];
        }
        if (osz == 1) continue;
        if (self_bcast) red.add(osz, ustride[d], ost);
        else kept.add(osz, ustride[d], ost);
    }
    rg.nkept = kept.n;
    rg.nred = red.n;
    for (int d = 0; d < kept.n; d++) {
        rg.kept_size[d] = kept.size[d];
        rg.kept_up[d] = kept.up[d];
        rg.kept_other[d] = kept.ot[d];
    }
    for (int d = 0; d < red.n; d++) {
        rg.red_size[d] = red.size[d];
        rg.red_up[d] = red.up[d];
        rg.red_other[d] = red.ot[d];
    }
    rg.nself = layout_numel(lself);
    rg.nred_total = 1;
    for (int d = 0; d < rg.nred; d++) rg.nred_total *= rg.red_size[d];
    rg.other_off = other ? lother->offset : 0;
    if (rg.nself == 0) return TRS_OK;
    if (layout_numel(lout) == 0) {  // nothing reaches the operand: +0.0
        const int64_t grid = std::min<int64_t>((rg.nself + 255) / 256, (int64_t)dev->cu_count * 8);
        hipLaunchKernelGGL(fill_kernel, dim3((unsigned)grid), dim3(kHelperLanes), 0, dev->stream, grad,
                           (size_t)rg.nself, 0.0f, (const float *)nullptr);
        TRS_LAUNCH_CHECK("fill kernel");
        return TRS_OK;
    }
    // The staged kernel: reduced dims merging into at least one full stage
    // of rows, kept dims merging into an outer and an inner part whose up
    // stride is 1 and whose size is a multiple of 32, 16-byte aligned.
    // Byte offsets within a stage are 32-bit: (256 * stride + 32) * 4 must
    // stay below 2^31 for each operand read through a descriptor.
    auto fits = [](int64_t extent) { return extent >= 0 && extent * 4 < (int64_t)INT32_MAX; };
    RedColsGeom cg{};
    if (reduce_cols_plan(rg, other != nullptr, &cg) && cg.R >= kStRows && cg.KI % kStChains == 0 &&
        cg.KO * (cg.KI / kStChains) <= INT32_MAX && (uintptr_t)up % 16 == 0 && cg.up_ko % 4 == 0 &&
        cg.up_r % 4 == 0 && fits(kStRows * cg.up_r + kStChains) &&
        (!other || (cg.ot_ko >= 0 && cg.ot_r >= 0 && cg.ot_ki >= 0))) {
        auto launch = [&]<int CH, int SR>() {
            const int64_t grid = cg.KO * (cg.KI / CH);
            const dim3 gd((unsigned)grid), bd(kStLanes);
            if (!other) {
                hipLaunchKernelGGL((reduce_stage_kernel<kOtNone, 2, SR, CH>), gd, bd, 0, dev->stream, up, other, cg,
                                   grad);
            } else {
                const bool base16 = (uintptr_t)(other + cg.other_off) % 16 == 0 && cg.ot_ko % 4 == 0;
                if (base16 && cg.ot_ki == 1 && cg.ot_r % 4 == 0 && fits(SR * cg.ot_r + CH))
                    hipLaunchKernelGGL((reduce_stage_kernel<kOtVecKi, 2, SR, CH>), gd, bd, 0, dev->stream, up, other,
                                       cg, grad);
                else if (base16 && cg.ot_r == 1 && cg.ot_ki % 4 == 0 && cg.R % 4 == 0 && fits(CH * cg.ot_ki + SR))
                    hipLaunchKernelGGL((reduce_stage_kernel<kOtVecR, 2, SR, CH>), gd, bd, 0, dev->stream, up, other,
                                       cg, grad);
                else
                    hipLaunchKernelGGL((reduce_stage_kernel<kOtScalar, 2, SR, CH>), gd, bd, 0, dev->stream, up, other,
                                       cg, grad);
            }
        };
        // 16-chain blocks with 512-row stages when 32-chain blocks would
        // leave CUs idle (a bias gradient over [8192, 4096]: 128 blocks).
        if (cg.KO * (cg.KI / kStChains) < dev->cu_count && cg.R >= 2 * kStRows && fits(2 * kStRows * cg.up_r + 16))
            launch.template operator()<16, 2 * kStRows>();
        else
            launch.template operator()<kStChains, kStRows>();
        TRS_LAUNCH_CHECK("staged broadcast reduction kernel");
        return TRS_OK;
    }
    const int64_t grid = std::min<int64_t>((rg.nself + 255) / 256, (int64_t)dev->cu_count * 8);
    if (other)
        hipLaunchKernelGGL(reduce_bcast_kernel<true>, dim3((unsigned)grid), dim3(kHelperLanes), 0, dev->stream, up,
                           other, rg, grad);
    else
        hipLaunchKernelGGL(reduce_bcast_kernel<false>, dim3((unsigned)grid), dim3(kHelperLanes), 0, dev->stream, up,
                           (const float *)nullptr, rg, grad);
    TRS_LAUNCH_CHECK("broadcast reduction kernel");
    return TRS_OK;
}

// Called by device_state() at a device's set-up, with that device current.
void setup_sum_scratch(DeviceState *dev) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        dev->sum_scratch = nullptr;
        std::snprintf(dev->sum_scratch_error, sizeof dev->sum_scratch_error, "hipGetSymbolAddress(scratch): %s (%d)",
                      hipGetErrorString(e), (int)e);
        return;
    }
    dev->sum_scratch = (float *)p;
}

// Sum of x into out[0]; pass 1's partials go to `partial` (kSumBlocks floats)
// or, when it is null, to a buffer from the block cache.
int sum_launch(DeviceState *dev, const float *x, const trs_layout *lx, float *out, float *partial) {
    int rc = check_layout(lx, "input");
    if (rc) return rc;
    if (!out) return set_error(TRS_E_INVALID_ARGUMENT, "null output");
    const int64_t n = layout_numel(lx);
    if (n == 0) return trs_fill_f32(out, 1, -0.0f);
    if (!x) return set_error(TRS_E_INVALID_ARGUMENT, "null input");
    // The tree adds elements by their position in row-major logical order.
    // Dropping size-1 dims and merging contiguous ones keeps every position,
    // so the merged view gives the same bits.
    trs_layout lm;
    merge_layout_dims(lx, &lm);
    if (lm.rank > kMaxRank) {
        // More dims than the kernel decodes: copy the view to a contiguous
        // buffer of this call's own (the same elements in the same order)
        // and sum that.
        if (partial)
            return set_error(TRS_E_INVALID_ARGUMENT,
                             "the no-allocation sum takes views that merge to at most %d dims; this one keeps %d",
                             kMaxRank, lm.rank);
        void *tmp = nullptr;
        rc = trs_alloc((size_t)n * sizeof(float), &tmp);
        if (rc) return rc;
        trs_layout lc{};
        lc.rank = lx->rank;
        int64_t s = 1;
        for (int d = lx->rank - 1; d >= 0; d--) {
            lc.shape[d] = lx->shape[d];
            lc.stride[d] = s;
            s *= lx->shape[d];
        }
        rc = trs_unary_f32(TRS_COPY, x, lx, (float *)tmp, &lc);
        trs_layout l1{};
        l1.rank = 1;
        l1.shape[0] = n;
        l1.stride[0] = 1;
        if (!rc) rc = sum_launch(dev, (const float *)tmp, &l1, out, nullptr);
        const int frc = trs_free(tmp);
        return rc ? rc : frc;
    }
    // Geometry for logical-order decode of a strided input.
    PwGeom g;
    std::memset(&g, 0, sizeof g);
    g.numel = n;
    g.rank = lm.rank;
    g.ioff[0] = lm.offset;
    for (int d = 0; d < lm.rank; d++) {
        g.size[d] = lm.shape[d];
        g.istride[0][d] = lm.stride[d];
        if (lm.shape[d] > (int64_t)UINT32_MAX) g.wide = 1;
        g.fd[d] = make_fast_div(lm.shape[d] > (int64_t)UINT32_MAX ? 1u : (uint32_t)lm.shape[d]);
    }
    const bool contig = layout_is_contiguous(&lm);
    // Up to kSumOneBlock elements: pass 1 alone, one block writing the result
    // (one launch and no partials; the order is still fixed by n).
    if (n <= kSumOneBlock) {
        if (contig)
            hipLaunchKernelGGL(sum_pass1<true>, dim3(1), dim3(256), 0, dev->stream, x, g, n, out);
        else
            hipLaunchKernelGGL(sum_pass1<false>, dim3(1), dim3(256), 0, dev->stream, x, g, n, out);
        TRS_LAUNCH_CHECK("sum one pass");
        return TRS_OK;
    }
    const int64_t chunk = (n + kSumBlocks - 1) / kSumBlocks;
    const int blocks = (int)((n + chunk - 1) / chunk);  // <= kSumBlocks partials for every n
    if (blocks > kSumBlocks)  // cannot happen; the scratch holds kSumBlocks partials
        return set_error(TRS_E_INVALID_ARGUMENT, "sum of %lld elements needs %d partials, above the %d the scratch holds",
                         (long long)n, blocks, kSumBlocks);
    // Without a caller buffer, the partials take a buffer of this call's own:
    // the block cache returns it in stream order, so concurrent callers on
    // one device never share it.
    void *owned = nullptr;
    if (!partial) {
        rc = trs_alloc(kSumBlocks * sizeof(float), &owned);
        if (rc) return rc;
        partial = (float *)owned;
    }
    if (contig)
        hipLaunchKernelGGL(sum_pass1<true>, dim3(blocks), dim3(256), 0, dev->stream, x, g, chunk, partial);
    else
        hipLaunchKernelGGL(sum_pass1<false>, dim3(blocks), dim3(256), 0, dev->stream, x, g, chunk, partial);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) {
        hipLaunchKernelGGL(sum_pass2, dim3(1), dim3(256), 0, dev->stream, partial, blocks, out);
        e = hipGetLastError();
    }
    rc = e == hipSuccess ? TRS_OK : hip_fail(e, "sum launch");
    if (owned) {
        const int frc = trs_free(owned);
        if (!rc) rc = frc;
    }
    return rc;
}

}  // namespace trs

using namespace trs;

extern "C" {

int trs_accumulate_f32(float *dst, const float *src, size_t n) {
    trs_layout l{};
    l.rank = 1;
    l.shape[0] = (int64_t)n;
    l.stride[0] = 1;
    return trs_binary_f32(TRS_ADD, dst, &l, src, &l, dst, &l);  // in place: the same view
}

int trs_fill_f32(float *out, size_t n, float value) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    if (n == 0) return TRS_OK;
    if (!out) return set_error(TRS_E_INVALID_ARGUMENT, "null output");
    const int64_t grid = std::min<int64_t>(((int64_t)n + 255) / 256, (int64_t)dev->cu_count * 8);
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)grid), dim3(kHelperLanes), 0, dev->stream, out, n, value,
                       (const float *)nullptr);
    TRS_LAUNCH_CHECK("fill kernel");
    return TRS_OK;
}

int trs_fill_from_device_f32(float *out, size_t n, const float *value) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    if (n == 0) return TRS_OK;
    if (!out || !value) return set_error(TRS_E_INVALID_ARGUMENT, "null pointer");
    const int64_t grid = std::min<int64_t>(((int64_t)n + 255) / 256, (int64_t)dev->cu_count * 8);
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)grid), dim3(kHelperLanes), 0, dev->stream, out, n, 0.0f, value);
    TRS_LAUNCH_CHECK("fill kernel");
    return TRS_OK;
}

int trs_mul_backward_f32(const float *up, const trs_layout *lout, const float *other, const trs_layout *lother,
                         const trs_layout *lself, float *grad) {
    int rc = check_layout(lout, "output");
    if (!rc) rc = check_layout(lself, "operand");
    if (rc) return rc;
    // An empty output reads nothing (an empty operand's storage may be null).
    if (!other && layout_numel(lout) != 0) return set_error(TRS_E_INVALID_ARGUMENT, "null other operand");
    if (layout_numel(lself) == layout_numel(lout)) {
        // No broadcast: one contribution per element, stored as is.
        const trs_layout lc = contiguous_like(lout);
        return trs_binary_f32(TRS_MUL, up, &lc, other, lother, grad, &lc);
    }
    return reduce_to_operand(up, lout, other, lother, lself, grad);
}

int trs_reduce_to_shape_f32(const float *up, const trs_layout *lout, const trs_layout *lself, float *grad) {
    int rc = check_layout(lout, "output");
    if (!rc) rc = check_layout(lself, "operand");
    if (rc) return rc;
    if (layout_numel(lself) == layout_numel(lout)) {
        const size_t n = (size_t)layout_numel(lout);
        return trs_memcpy_d2d(grad, up, n * sizeof(float));
    }
    return reduce_to_operand(up, lout, nullptr, nullptr, lself, grad);
}

int trs_pointwise_plan(int n_inputs, const void *const *inputs, const trs_layout *const *layouts,
                       const int *elem_bytes, const float *out, const trs_layout *lo, int cu_count, int roles,
                       trs_pw_plan_info *info) {
    if (!info) return set_error(TRS_E_INVALID_ARGUMENT, "null plan info");
    if (n_inputs < 1 || n_inputs > kMaxIn)
        return set_error(TRS_E_INVALID_ARGUMENT, "pointwise plans take 1 to %d inputs, got %d", kMaxIn, n_inputs);
    if (!inputs || !layouts) return set_error(TRS_E_INVALID_ARGUMENT, "null input arrays");
    if (cu_count < 1) return set_error(TRS_E_INVALID_ARGUMENT, "cu_count must be positive, got %d", cu_count);
    int eb[kMaxIn];
    for (int i = 0; i < n_inputs; i++) eb[i] = elem_bytes ? elem_bytes[i] : 4;
    PwPlan pl;
    const int rc = plan_pointwise(lo, const_cast<float *>(out), n_inputs, inputs, layouts, eb, cu_count, &pl, 1,
                                  nullptr, roles != 0);
    if (rc) return rc;
    *info = trs_pw_plan_info{};
    info->variant = (int32_t)pl.variant;
    if (pl.variant == PwVariant::Empty) return TRS_OK;
    info->rank = pl.g.rank;
    info->vec = pl.vec;
    info->fixed_rank = pl.rk;
    info->skew = pl.g.skew;
    info->walk = pl.walk;
    info->trans = pl.trans;
    info->held = pl.held;
    info->once = pl.once;
    info->block = pl.block;
    info->grid = pl.grid;
    info->split = pl.nsplit;
    int64_t launches = pl.variant == PwVariant::Empty ? 0 : 1;
    for (int d = 0; d < pl.nsplit; d++) launches = std::min<int64_t>(launches * pl.ssize[d], INT32_MAX);
    info->launches = (int32_t)launches;
    return TRS_OK;
}

int trs_sum_f32(const float *x, const trs_layout *lx, float *out) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    return sum_launch(dev, x, lx, out, nullptr);
}

int trs_sum_f32_noalloc(const float *x, const trs_layout *lx, float *out) {
    DeviceState *dev = device_state();
    if (!dev) return TRS_E_NO_DEVICE;
    if (!dev->sum_scratch)
        return set_error(TRS_E_HIP, "the no-allocation sum's scratch is unavailable on device %d: %s", dev->index,
                         dev->sum_scratch_error);
    return sum_launch(dev, x, lx, out, dev->sum_scratch);
}

}  // extern "C"
