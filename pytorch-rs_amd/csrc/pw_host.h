// pw_host.h -- host-side launch planning for the pointwise engine (pw_core.h).
//
// plan_pointwise() turns (output layout, input layouts) into a normalised
// PwGeom and picks the kernel variant:
//   1. align inputs to the output rank (right-aligned broadcasting,
//      BroadcastPlan in src/tensor.rs:3601-3693): stride 0 on broadcast dims;
//   2. drop size-1 dims, order dims by decreasing output stride so the kernel
//      walks the output in physical order, and merge adjacent dims that are
//      contiguous for every operand;
//   3. choose flat / rows / xpose / generic and whether 16-byte vector
//      accesses are legal (alignment of every unit-stride operand).
#pragma once

#include <cstdint>
#include <cstring>

#include "pw_core.h"
#include "trs_internal.h"

namespace trs {

enum class PwVariant { Empty, Flat, Rows, Xpose, Generic };

// Dims a plan can walk on the host beyond the kernel geometry's kMaxRank.
constexpr int kMaxSplit = TRS_MAX_RANK - kMaxRank;

// pw_xpose tile: 4 x 2 waves = 128 (t) x 64 (x).  On (a + b) * c.mT over
// [64, 512, 1024] this shape's access pattern measured fastest of 64-256 x
// 32-256 (its reads of c are 512 B runs); walking 8 outer tuples per block
// with the invariant operand held in registers measured faster than one
// tuple per block, which reloads it from L2 for every tuple.
constexpr int kXposeWT = 4, kXposeWX = 2;
constexpr int kXposeBT = 32 * kXposeWT, kXposeBX = 32 * kXposeWX;
constexpr int kXposeWalk = 8;  // largest walk: 8, 4 or 2 tuples, dividing the tuple count
constexpr int kXposeResident = 4;  // about the pw_xpose blocks (512 lanes) resident per CU

struct PwPlan {
    PwVariant variant = PwVariant::Empty;
    bool vec = false;
    bool contig = false;  // Flat + vec with every input unit-stride and read once
    int ntransposed = 0;
    // Xpose: operand role masks (transposed, held over the outer tuples,
    // loaded once per tuple, stride 0 along x) and the tuples each block
    // walks (g.rows = g.groups * walk).
    uint32_t trans = 0, held = 0, once = 0, xbc = 0;
    int walk = 1;
    // The compile-time fast case, 0 if none: the rank (Rows: 2, 3 or 4;
    // Xpose: 3) of a launch with fewer than 2^32 tiles and every element
    // offset below 2^32.
    int rk = 0;
    // Xpose with rk = 3 and vector access: every tile interior and taken in
    // plain order (no diagonal skew), so the kernel tests neither per block.
    bool plain = false;
    int nin = 0;
    int block = 256;  // lanes per block (kFlatBlock for the flat variants)
    int64_t grid = 0;
    PwGeom g;
    PwPtrs p;
    // Views that keep more than kMaxRank dims after merging: nsplit dims
    // (those with the fewest indices) are walked on the host, one launch of
    // the other kMaxRank dims per index tuple, each with the base offsets
    // moved by that tuple (for_each_part).
    int nsplit = 0;
    int64_t ssize[kMaxSplit];
    int64_t sos[kMaxSplit];
    int64_t sis[kMaxIn][kMaxSplit];
};

// Calls launch(g) once per part of the plan: with no split, on the plan's
// geometry; otherwise on a copy whose output and input offsets are moved to
// each index tuple of the split dims, in row-major order.  The parts write
// disjoint output elements, so their order does not change any result.
template <class L>
int for_each_part(const PwPlan &pl, L &&launch) {
    // pw_rows and pw_xpose take a block's first tile unchecked: never more
    // blocks than tiles.
    const int64_t tiles = pl.variant == PwVariant::Rows    ? pl.g.rows * pl.g.chunks
                          : pl.variant == PwVariant::Xpose ? pl.g.groups * pl.g.chunks
                                                           : INT64_MAX;
    if (pl.grid < 1 || pl.grid > tiles)
        return set_error(TRS_E_INVALID_ARGUMENT, "pointwise launch of %lld blocks over %lld tiles", (long long)pl.grid,
                         (long long)tiles);
    if (pl.nsplit == 0) return launch(pl.g);
    PwGeom g = pl.g;
    int64_t idx[kMaxSplit] = {};
    for (;;) {
        g.ooff = pl.g.ooff;
        for (int i = 0; i < kMaxIn; i++) g.ioff[i] = pl.g.ioff[i];
        for (int d = 0; d < pl.nsplit; d++) {
            g.ooff += idx[d] * pl.sos[d];
            for (int i = 0; i < kMaxIn; i++) g.ioff[i] += idx[d] * pl.sis[i][d];
        }
        const int rc = launch(g);
        if (rc) return rc;
        int d = pl.nsplit - 1;
        while (d >= 0 && ++idx[d] == pl.ssize[d]) idx[d--] = 0;
        if (d < 0) return TRS_OK;
    }
}

inline FastDiv make_fast_div(uint32_t d) {
    FastDiv f{};
    f.div = d;
    uint32_t shift = 0;
    while (shift < 32 && (1ull << shift) < d) shift++;
    const uint64_t two32 = 1ull << 32;
    const uint64_t m = (two32 * ((1ull << shift) - d)) / d + 1;
    f.mul = (uint32_t)m;
    f.shift = shift;
    return f;
}

// Lanes per vector pw_rows block (one float4 per lane): the fewest that give
// a block at least 2 KiB of HBM traffic, counting the outputs and the inputs
// read once (`streamed`; broadcast operands come from cache).  The GPU starts
// about 4.4 blocks per nanosecond, so a kernel whose blocks each move 1 KiB
// is bound by block dispatch, not HBM: a write-only pass over 128 MiB took
// 29.9 us on one-wave blocks and 20.4 us on 256-lane blocks, and a [64, 512,
// 1024] broadcast add (a and b from cache, the output written) 30.1 us on
// one wave against 20.6 on two.  Where inputs stream as well, one wave is
// fastest: relu(x + b) over [4096, 4096] measured 21.2 us per launch on
// one-wave blocks, 22.7 on 256 lanes and 22.8 on 2,048-column tiles of 256
// lanes with two float4 each.
inline int rows_lanes(uint32_t streamed, int nin, const int *elem_bytes, int nout) {
    int per_element = 4 * nout;
    for (int i = 0; i < nin; i++)
        if ((streamed >> i) & 1u) per_element += elem_bytes[i];
    for (int lanes = 64; lanes < kRowLanesMax; lanes *= 2)
        if (lanes * 4 * per_element >= 2048) return lanes;
    return kRowLanesMax;
}

// `elem_bytes[i]` is 4 for f32 inputs and 1 for u8 inputs.  A program with
// several outputs passes outputs 1.. in `more` (nout - 1 of them); they share
// the output layout `lo`.  `roles`: the launcher can run pw_xpose specialised
// on held / once-per-tuple operands (the fusion compiler); otherwise an
// Xpose plan takes one outer tuple per block and no roles.
inline int plan_pointwise(const trs_layout *lo, float *out, int nin, const void *const *bases,
                          const trs_layout *const *lins, const int *elem_bytes, int cu_count,
                          PwPlan *plan, int nout = 1, float *const *more = nullptr, bool roles = false) {
    int rc = check_layout(lo, "output");
    if (rc) return rc;
    if (nin > kMaxIn) return set_error(TRS_E_INVALID_ARGUMENT, "too many pointwise inputs (%d)", nin);
    if (nout < 1 || nout > kMaxOut || (nout > 1 && more == nullptr))
        return set_error(TRS_E_INVALID_ARGUMENT, "bad pointwise output count (%d)", nout);
    for (int i = 0; i < nin; i++) {
        rc = check_layout(lins[i], "input");
        if (rc) return rc;
        if (lins[i]->rank > lo->rank)
            return set_error(TRS_E_SHAPE_MISMATCH, "input %d has rank %d above the output rank %d", i,
                             lins[i]->rank, lo->rank);
        const int lead = lo->rank - lins[i]->rank;
        for (int d = 0; d < lins[i]->rank; d++) {
            const int64_t s = lins[i]->shape[d], o = lo->shape[lead + d];
            if (s != o && s != 1)
                return set_error(TRS_E_SHAPE_MISMATCH,
                                 "The size of tensor a (%lld) must match the size of tensor b "
                                 "(%lld) at non-singleton dimension %d",
                                 (long long)s, (long long)o, lead + d);
        }
    }
    *plan = PwPlan{};
    plan->nin = nin;
    PwGeom &g = plan->g;
    std::memset(&g, 0, sizeof(g));
    plan->p.out = out;
    for (int i = 0; i < nin; i++) plan->p.in[i] = bases[i];
    for (int o = 1; o < nout; o++) plan->p.more[o - 1] = more[o - 1];

    int64_t numel = layout_numel(lo);
    if (numel == 0) {
        plan->variant = PwVariant::Empty;
        return TRS_OK;
    }
    if (out == nullptr) return set_error(TRS_E_INVALID_ARGUMENT, "null output pointer");
    for (int o = 1; o < nout; o++)
        if (more[o - 1] == nullptr) return set_error(TRS_E_INVALID_ARGUMENT, "null output pointer %d", o);
    for (int i = 0; i < nin; i++)
        if (bases[i] == nullptr) return set_error(TRS_E_INVALID_ARGUMENT, "null input pointer %d", i);
    // An input may share memory with an output only as the very same view
    // (element-wise in place: every lane reads and writes its own elements);
    // any other overlap would race across lanes.  Outputs never share memory.
    for (int o = 0; o < nout; o++) {
        float *const base = o == 0 ? out : more[o - 1];
        const ByteRange ro = byte_range(base, lo, 4);
        for (int i = 0; i < nin; i++) {
            if (layout_numel(lins[i]) == 0) continue;
            const ByteRange ri = byte_range(bases[i], lins[i], elem_bytes[i]);
            if (!ranges_overlap(ro, ri)) continue;
            if (elem_bytes[i] == 4 && ri.begin == ro.begin && same_view_shape(lins[i], lo)) continue;
            return set_error(TRS_E_INVALID_ARGUMENT, "output %d overlaps input %d other than as the same view", o,
                             i);
        }
        for (int q = 0; q < o; q++) {
            if (ranges_overlap(ro, byte_range(q == 0 ? out : more[q - 1], lo, 4)))
                return set_error(TRS_E_INVALID_ARGUMENT, "outputs %d and %d overlap", q, o);
        }
    }

    // 1-2. align, drop singleton dims.
    int rank = 0;
    int64_t size[TRS_MAX_RANK], os[TRS_MAX_RANK], is[kMaxIn][TRS_MAX_RANK];
    for (int d = 0; d < lo->rank; d++) {
        if (lo->shape[d] == 1) continue;
        size[rank] = lo->shape[d];
        os[rank] = lo->stride[d];
        for (int i = 0; i < nin; i++) {
            const int lead = lo->rank - lins[i]->rank;
            is[i][rank] = (d < lead || lins[i]->shape[d - lead] == 1) ? 0 : lins[i]->stride[d - lead];
        }
        rank++;
    }
    // Order by decreasing output stride (stable insertion sort).
    for (int a = 1; a < rank; a++) {
        for (int b = a; b > 0 && os[b - 1] < os[b]; b--) {
            std::swap(size[b - 1], size[b]);
            std::swap(os[b - 1], os[b]);
            for (int i = 0; i < nin; i++) std::swap(is[i][b - 1], is[i][b]);
        }
    }
    // The output must not overlap itself (each element written once).
    for (int d = 0; d + 1 < rank; d++) {
        if (os[d] < os[d + 1] * size[d + 1])
            return set_error(TRS_E_INVALID_ARGUMENT, "output layout overlaps itself");
    }
    if (rank > 0 && os[rank - 1] == 0)
        return set_error(TRS_E_INVALID_ARGUMENT, "output layout overlaps itself");
    // Merge dims that are contiguous for every operand.
    {
        int64_t nsize[TRS_MAX_RANK], nos[TRS_MAX_RANK], nis[kMaxIn][TRS_MAX_RANK];
        int nr = 0;
        // Walk from innermost to outermost, building reversed list.
        for (int d = rank - 1; d >= 0; d--) {
            if (nr > 0) {
                const int q = nr - 1;
                bool ok = os[d] == nos[q] * nsize[q];
                for (int i = 0; ok && i < nin; i++) ok = is[i][d] == nis[i][q] * nsize[q];
                if (ok) {
                    nsize[q] *= size[d];
                    continue;
                }
            }
            nsize[nr] = size[d];
            nos[nr] = os[d];
            for (int i = 0; i < nin; i++) nis[i][nr] = is[i][d];
            nr++;
        }
        rank = nr;
        for (int d = 0; d < rank; d++) {
            size[d] = nsize[rank - 1 - d];
            os[d] = nos[rank - 1 - d];
            for (int i = 0; i < nin; i++) is[i][d] = nis[i][rank - 1 - d];
        }
    }
    if (rank == 0) {  // a single element
        rank = 1;
        size[0] = 1;
        os[0] = 1;
        for (int i = 0; i < nin; i++) is[i][0] = 0;
    }
    // More dims than a kernel's geometry holds: split off, onto the host, the
    // dims with the fewest indices (never the innermost; the outermost of
    // equal sizes), so the launches number the product of the smallest
    // sizes: [100000, 2, 2, ...] runs as 2 launches, not 100,000.  Both the
    // split and the kept dims stay in stride order.
    if (rank > kMaxRank) {
        const int ns = rank - kMaxRank;
        bool split[TRS_MAX_RANK] = {};
        for (int n = 0; n < ns; n++) {
            int best = -1;
            for (int d = 0; d < rank - 1; d++)
                if (!split[d] && (best < 0 || size[d] < size[best])) best = d;
            split[best] = true;
        }
        plan->nsplit = ns;
        int w = 0, k = 0;
        for (int d = 0; d < rank; d++) {
            if (split[d]) {
                plan->ssize[w] = size[d];
                plan->sos[w] = os[d];
                for (int i = 0; i < nin; i++) plan->sis[i][w] = is[i][d];
                numel /= size[d];
                w++;
            } else {
                size[k] = size[d];
                os[k] = os[d];
                for (int i = 0; i < nin; i++) is[i][k] = is[i][d];
                k++;
            }
        }
        rank = kMaxRank;
    }

    g.rank = rank;
    g.numel = numel;
    g.ooff = lo->offset;
    for (int d = 0; d < rank; d++) {
        g.size[d] = size[d];
        g.ostride[d] = os[d];
        if (size[d] > (int64_t)UINT32_MAX) g.wide = 1;
        g.fd[d] = make_fast_div(size[d] > (int64_t)UINT32_MAX ? 1u : (uint32_t)size[d]);
    }
    for (int i = 0; i < nin; i++) {
        g.ioff[i] = lins[i]->offset;
        bool bcast = false;
        for (int d = 0; d < rank; d++) {
            g.istride[i][d] = is[i][d];
            bcast |= is[i][d] == 0;
        }
        for (int d = 0; d < plan->nsplit; d++) bcast |= plan->sis[i][d] == 0;
        if (!bcast) g.streamed |= 1u << i;
    }

    // Alignment of a unit-stride access along dim `ud` for operand bytes, in
    // every part of a split launch (`sst`: the operand's split-dim strides).
    auto aligned = [&](const void *base, int64_t off, const int64_t *strides, const int64_t *sst, int ud, int eb) {
        const uint64_t addr = (uint64_t)(uintptr_t)base + (uint64_t)off * (uint64_t)eb;
        if (addr % (uint64_t)(4 * eb) != 0) return false;
        for (int d = 0; d < rank; d++)
            if (d != ud && strides[d] % 4 != 0) return false;
        for (int d = 0; d < plan->nsplit; d++)
            if (sst[d] % 4 != 0) return false;
        return true;
    };

    const int inner = rank - 1;
    auto outputs_aligned = [&]() {
        bool ok = aligned(out, lo->offset, os, plan->sos, inner, 4);
        for (int o = 1; o < nout; o++) ok = ok && aligned(more[o - 1], lo->offset, os, plan->sos, inner, 4);
        return ok;
    };
    // Every element offset the launch forms (in any part) is below 2^32:
    // strides are non-negative, so the largest is offset + sum (size - 1) *
    // stride over the inner and the split dims.
    auto offsets_fit32 = [&]() {
        auto last = [&](int64_t off, const int64_t *st, const int64_t *sst) {
            for (int d = 0; d < rank; d++) off += (size[d] - 1) * st[d];
            for (int d = 0; d < plan->nsplit; d++) off += (plan->ssize[d] - 1) * sst[d];
            return off;
        };
        if (last(g.ooff, os, plan->sos) > (int64_t)UINT32_MAX) return false;
        for (int i = 0; i < nin; i++)
            if (last(g.ioff[i], is[i], plan->sis[i]) > (int64_t)UINT32_MAX) return false;
        return true;
    };
    bool unit_or_bcast = os[inner] == 1;
    for (int i = 0; i < nin; i++) unit_or_bcast &= is[i][inner] == 0 || is[i][inner] == 1;
    const int64_t cap = g_pw_grid_cap.load(std::memory_order_relaxed);
    const int64_t want = cap > 0 ? cap : kMaxGrid;

    if (unit_or_bcast) {
        bool vec = outputs_aligned();
        for (int i = 0; i < nin; i++)
            if (is[i][inner] == 1) vec &= aligned(bases[i], g.ioff[i], is[i], plan->sis[i], inner, elem_bytes[i]);
        if (rank == 1) {
            plan->variant = PwVariant::Flat;
            plan->vec = vec;
            bool all_unit = true;
            for (int i = 0; i < nin; i++) all_unit &= is[i][0] == 1;
            plan->contig = vec && all_unit;
            const int64_t work = vec ? numel / 4 : numel;
            plan->block = kFlatBlock;
            plan->grid = std::min<int64_t>(std::max<int64_t>(1, (work + kFlatBlock - 1) / kFlatBlock), want);
        } else {
            plan->variant = PwVariant::Rows;
            plan->vec = vec && size[inner] % 4 == 0;
            plan->block = plan->vec ? rows_lanes(g.streamed, nin, elem_bytes, nout) : 256;
            g.chunkcols = plan->vec ? 4 * plan->block : 0;
            g.rows = numel / size[inner];
            const int64_t chunk = plan->vec ? g.chunkcols : kRowChunk;
            g.chunks = (size[inner] + chunk - 1) / chunk;
            g.fdchunks = make_fast_div(g.chunks > (int64_t)UINT32_MAX ? 1u : (uint32_t)g.chunks);
            const bool fast = g.rows * g.chunks <= (int64_t)UINT32_MAX && offsets_fit32();
            plan->rk = fast && rank <= 4 ? rank : 0;
            plan->grid = std::min<int64_t>(g.rows * g.chunks, want);
        }
        return TRS_OK;
    }

    // Transposed operands: unit stride along one common dim t < inner.
    if (os[inner] == 1 && rank >= 2) {
        int tdim = -1;
        bool ok = true;
        uint32_t tmask = 0;
        for (int i = 0; i < nin && ok; i++) {
            if (is[i][inner] == 0 || is[i][inner] == 1) continue;
            int t = -1;
            for (int d = 0; d < inner; d++)
                if (is[i][d] == 1) t = d;
            if (t < 0 || (tdim >= 0 && t != tdim)) ok = false;
            tdim = t;
            tmask |= 1u << i;
        }
        int nt = __builtin_popcount(tmask);
        if (ok && tdim >= 0) {
            g.tdim = tdim;
            g.transposed = tmask;
            bool vec = outputs_aligned();
            for (int i = 0; i < nin; i++) {
                if ((tmask >> i) & 1u) {
                    vec &= aligned(bases[i], g.ioff[i], is[i], plan->sis[i], tdim, elem_bytes[i]);
                } else if (is[i][inner] == 1) {
                    vec &= aligned(bases[i], g.ioff[i], is[i], plan->sis[i], inner, elem_bytes[i]);
                }
            }
            plan->vec = vec;
            plan->ntransposed = nt;
            g.rows = numel / (size[tdim] * size[inner]);
            plan->variant = PwVariant::Xpose;
            plan->trans = tmask;
            plan->block = 64 * kXposeWT * kXposeWX;
            if (roles) {
                for (int i = 0; i < nin; i++) {
                    if ((tmask >> i) & 1u) continue;
                    if (is[i][inner] == 0) plan->xbc |= 1u << i;
                    bool outer_zero = true;
                    for (int d = 0; d < inner; d++)
                        if (d != tdim && is[i][d] != 0) outer_zero = false;
                    if (outer_zero) plan->held |= 1u << i;
                    else if (is[i][tdim] == 0) plan->once |= 1u << i;
                }
            }
            // When an operand is held, each block walks the largest of 8, 4
            // or 2 tuples that divides the tuple count (the held operand is
            // then loaded once for all of them); else one tuple per block.
            plan->walk = 1;
            if (plan->held)
                for (int w = kXposeWalk; w >= 2; w /= 2)
                    if (g.rows % w == 0) {
                        plan->walk = w;
                        break;
                    }
            g.groups = g.rows / plan->walk;
            g.ttiles = (size[tdim] + kXposeBT - 1) / kXposeBT;
            const int64_t xtiles = (size[inner] + kXposeBX - 1) / kXposeBX;
            g.chunks = g.ttiles * xtiles;
            const bool small = g.groups * g.chunks <= (int64_t)UINT32_MAX;
            g.fdchunks = make_fast_div(small ? (uint32_t)g.chunks : 1u);
            g.fdttiles = make_fast_div(small ? (uint32_t)g.ttiles : 1u);
            // Diagonal tile order when one tuple has more tiles than the GPU
            // holds at once (about kXposeResident blocks per CU).
            g.skew = xtiles > 1 && g.chunks > (int64_t)kXposeResident * cu_count;
            g.fdxtiles = make_fast_div(small ? (uint32_t)xtiles : 1u);
            plan->rk = rank == 3 && small && offsets_fit32() ? 3 : 0;
            plan->plain = plan->rk == 3 && vec && !g.skew && size[tdim] % kXposeBT == 0 &&
                          size[inner] % kXposeBX == 0;
            plan->grid = std::min<int64_t>(g.groups * g.chunks, want);
            return TRS_OK;
        }
    }
    plan->variant = PwVariant::Generic;
    plan->block = kGenericBlock;
    const int64_t per_block = kGenericBlock * kGenericUnroll;
    plan->grid = std::min<int64_t>(std::max<int64_t>(1, (numel + per_block - 1) / per_block), want);
    return TRS_OK;
}

}  // namespace trs
