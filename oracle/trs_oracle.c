/*
 * trs_oracle.c -- CPU restatement of the pytorch-rs tensor hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library under pytorch-rs_amd/.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only to check or to time the
 * reference algorithm -- never as the code path that is measured or shipped.
 *
 * Every function restates one piece of /root/reference/src/tensor.rs (Rust,
 * single-threaded, f32) and cites the lines it follows.  Conventions:
 *   - shapes, strides and offsets are element counts (usize in the reference,
 *     uint64_t here; the reference never has negative strides, tensor.rs:212-221);
 *   - every binary op is exactly one IEEE-754 binary32 operation with
 *     round-to-nearest-even and no contraction (build with -ffp-contract=off);
 *   - exp is the platform libm expf, exactly what Rust's f32::exp calls on
 *     linux-gnu (tensor.rs:2398-2400).
 *
 * Pinning (which check fixes what) is listed per function; functions with no
 * independent check say "parity unpinned".
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <gnu/libc-version.h>
#include <pthread.h>

#define ORC_MAX_RANK 25

/* Error codes; the same numbering as the product ABI (include/trs_hip.h). */
enum {
    ORC_OK = 0,
    ORC_E_ALLOCATION = -1,
    ORC_E_INDEX_OVERFLOW = -2,
    ORC_E_STRIDE_OVERFLOW = -3,
    ORC_E_SHAPE_MISMATCH = -4,
    ORC_E_MATMUL_INNER = -5,
    ORC_E_MATMUL_RANK = -6,
    ORC_E_INVALID = -7,
    ORC_E_ELEMENT_OVERFLOW = -11,
};

/* Same binary layout as trs_layout in include/trs_hip.h. */
typedef struct {
    int32_t rank;
    int32_t reserved;
    int64_t shape[ORC_MAX_RANK];
    int64_t stride[ORC_MAX_RANK];
    int64_t offset;
} orc_layout;

const char *orc_libc_version(void) { return gnu_get_libc_version(); }

/* ------------------------------------------------------------------------ */
/* Layout predicates and stride builders                                     */
/* ------------------------------------------------------------------------ */

static const uint64_t ISIZE_MAX_U = (uint64_t)INT64_MAX;

/* element_count (tensor.rs:4174-4180) */
int orc_element_count(int rank, const uint64_t *shape, uint64_t *out) {
    uint64_t n = 1;
    for (int i = 0; i < rank; i++) {
        if (__builtin_mul_overflow(n, shape[i], &n)) return ORC_E_ELEMENT_OVERFLOW;
    }
    *out = n;
    return ORC_OK;
}

/* checked_stride_product (tensor.rs:4434-4439): stride * max(dim,1) <= isize::MAX */
static int checked_stride_product(uint64_t stride, uint64_t dim, uint64_t *out) {
    uint64_t d = dim > 1 ? dim : 1, p;
    if (__builtin_mul_overflow(stride, d, &p) || p > ISIZE_MAX_U) return ORC_E_STRIDE_OVERFLOW;
    *out = p;
    return ORC_OK;
}

/* contiguous_strides (tensor.rs:4198-4209) */
int orc_contiguous_strides(int rank, const uint64_t *shape, uint64_t *strides) {
    uint64_t stride = 1;
    for (int axis = rank - 1; axis >= 0; axis--) {
        strides[axis] = stride;
        if (axis > 0) {
            int rc = checked_stride_product(stride, shape[axis], &stride);
            if (rc) return rc;
        }
    }
    return ORC_OK;
}

/* layout_is_contiguous (tensor.rs:3695-3715): singleton dims ignored */
int orc_layout_is_contiguous(int rank, const uint64_t *shape, const uint64_t *strides,
                             uint64_t elements) {
    if (elements == 0) return 1;
    uint64_t expected = 1;
    for (int axis = rank - 1; axis >= 0; axis--) {
        uint64_t dim = shape[axis];
        if (dim == 1) continue;
        if (strides[axis] != expected) return 0;
        if (__builtin_mul_overflow(expected, dim, &expected)) return 0;
    }
    return 1;
}

/* layout_is_contiguous_in_order (tensor.rs:3765-3791) */
static int contiguous_in_order(int rank, const uint64_t *shape, const uint64_t *strides,
                               const int *order, int order_len) {
    if (rank != order_len) return 0;
    int is_empty = 0;
    for (int i = 0; i < rank; i++) is_empty |= shape[i] == 0;
    uint64_t expected = 1;
    for (int i = 0; i < order_len; i++) {
        int axis = order[i];
        uint64_t dim = shape[axis];
        if (dim == 1) continue;
        if (strides[axis] != expected) return 0;
        uint64_t next;
        if (__builtin_mul_overflow(expected, dim, &next)) {
            if (!is_empty) return 0;
            next = expected * dim; /* wrapping, as the reference allows for empty tensors */
        }
        expected = next;
    }
    return 1;
}

/* layout_is_channels_last_contiguous (tensor.rs:3717-3719), order [1,3,2,0] */
int orc_is_channels_last_contiguous(int rank, const uint64_t *shape, const uint64_t *strides) {
    static const int order[4] = {1, 3, 2, 0};
    return contiguous_in_order(rank, shape, strides, order, 4);
}

/* Tensor::is_non_overlapping_and_dense (tensor.rs:1019-1053) */
int orc_is_non_overlapping_and_dense(int rank, const uint64_t *shape, const uint64_t *strides,
                                     uint64_t elements) {
    if (elements == 0) return 1;
    int dims = 0;
    for (int i = 0; i < rank; i++) dims += shape[i] > 1;
    uint64_t expected = 1;
    for (int matched = 0; matched < dims; matched++) {
        int found = -1;
        for (int axis = 0; axis < rank; axis++) {
            if (shape[axis] > 1 && strides[axis] == expected) {
                if (found >= 0) return 0;
                found = axis;
            }
        }
        if (found < 0) return 0;
        if (__builtin_mul_overflow(expected, shape[found], &expected)) return 0;
    }
    return 1;
}

/* checked_physical_stride_product (tensor.rs:4441-4446) */
static int checked_physical_stride_product(uint64_t stride, uint64_t dim, uint64_t *out) {
    uint64_t p;
    if (__builtin_mul_overflow(stride, dim, &p) || p > ISIZE_MAX_U) return ORC_E_STRIDE_OVERFLOW;
    *out = p;
    return ORC_OK;
}

/* channels_last_strides via strides_in_physical_order (tensor.rs:4211-4247) */
int orc_channels_last_strides(int rank, const uint64_t *shape, uint64_t *strides) {
    static const int order[4] = {1, 3, 2, 0};
    if (rank != 4) return ORC_E_STRIDE_OVERFLOW;
    uint64_t tmp[ORC_MAX_RANK];
    int rc = orc_contiguous_strides(rank, shape, tmp);
    if (rc) return rc;
    uint64_t stride = 1;
    for (int pos = 0; pos < 4; pos++) {
        int axis = order[pos];
        strides[axis] = stride;
        if (pos + 1 < 4) {
            rc = checked_physical_stride_product(stride, shape[axis], &stride);
            if (rc) return rc;
        }
    }
    return ORC_OK;
}

/* ElementwiseLayout::aligned_broadcast_stride (tensor.rs:4114-4131) */
static uint64_t aligned_broadcast_stride(int op_rank, const uint64_t *op_shape,
                                         const uint64_t *op_strides, int out_rank, int out_axis,
                                         uint64_t out_dim) {
    int leading = out_rank - op_rank;
    if (out_axis < leading) return 0;
    int in_axis = out_axis - leading;
    if (op_shape[in_axis] == 1 && out_dim != 1) return 0;
    return op_strides[in_axis];
}

/* aligned_broadcast_stride_bytes (tensor.rs:4133-4151): wrapping i64 byte stride */
static int64_t aligned_broadcast_stride_bytes(int op_rank, const uint64_t *op_shape,
                                              const uint64_t *op_strides, int out_rank,
                                              int out_axis, uint64_t out_dim) {
    uint64_t s = aligned_broadcast_stride(op_rank, op_shape, op_strides, out_rank, out_axis,
                                          out_dim);
    return (int64_t)(s * 4u); /* wrapping multiply of the signed stride by 4 */
}

typedef struct {
    int rank;
    const uint64_t *shape;
    const uint64_t *strides;
} ew_operand;

/* compare_elementwise_dimensions (tensor.rs:4315-4336) */
static int compare_dims(int rank, const uint64_t *shape, const ew_operand *ops, int nops, int d0,
                        int d1) {
    for (int i = 0; i < nops; i++) {
        int64_t s0 = aligned_broadcast_stride_bytes(ops[i].rank, ops[i].shape, ops[i].strides,
                                                    rank, d0, shape[d0]);
        int64_t s1 = aligned_broadcast_stride_bytes(ops[i].rank, ops[i].shape, ops[i].strides,
                                                    rank, d1, shape[d1]);
        if (s0 == 0 || s1 == 0) continue;
        if (s0 < s1) return -1;
        if (s0 > s1 || shape[d0] > shape[d1]) return 1;
    }
    return 0;
}

/* elementwise_output_strides (tensor.rs:4249-4312): TensorIterator-style
 * insertion sort of dimensions, then byte strides with i64 wrap-around. */
static int elementwise_output_strides(int rank, const uint64_t *shape, const ew_operand *ops,
                                      int nops, uint64_t *out) {
    int perm[ORC_MAX_RANK];
    for (int i = 0; i < rank; i++) perm[i] = rank - 1 - i;
    for (int index = 1; index < rank; index++) {
        int d1 = index;
        for (int d0 = index - 1; d0 >= 0; d0--) {
            int c = compare_dims(rank, shape, ops, nops, perm[d0], perm[d1]);
            if (c > 0) {
                int t = perm[d0];
                perm[d0] = perm[d1];
                perm[d1] = t;
                d1 = d0;
            } else if (c < 0) {
                break;
            }
        }
    }
    int identity = 1;
    for (int i = 0; i < rank; i++) identity &= perm[i] == rank - i - 1;
    if (identity) return orc_contiguous_strides(rank, shape, out);

    int64_t byte_strides[ORC_MAX_RANK];
    int64_t next = 4;
    for (int pos = 0; pos < rank; pos++) {
        int axis = perm[pos];
        byte_strides[axis] = next;
        if (pos + 1 < rank) {
            if (shape[axis] > (uint64_t)INT64_MAX) return ORC_E_STRIDE_OVERFLOW;
            next = (int64_t)((uint64_t)next * shape[axis]); /* wrapping_mul */
        }
    }
    for (int axis = rank - 1; axis >= 0; axis--) {
        int64_t s = byte_strides[axis] / 4;
        if (s >= 0) {
            out[axis] = (uint64_t)s;
        } else if (axis + 1 == rank) {
            out[axis] = 1;
        } else {
            int rc = checked_stride_product(out[axis + 1], shape[axis + 1], &out[axis]);
            if (rc) return rc;
        }
    }
    return ORC_OK;
}

/* Public entry: nops operands given as orc_layout (only rank/shape/stride used). */
int orc_elementwise_output_strides(int rank, const int64_t *shape, int nops,
                                   const orc_layout *ops, int64_t *out) {
    ew_operand eo[4];
    uint64_t sh[4][ORC_MAX_RANK], st[4][ORC_MAX_RANK];
    if (nops > 4 || rank > ORC_MAX_RANK) return ORC_E_INVALID;
    for (int i = 0; i < nops; i++) {
        for (int d = 0; d < ops[i].rank; d++) {
            sh[i][d] = (uint64_t)ops[i].shape[d];
            st[i][d] = (uint64_t)ops[i].stride[d];
        }
        eo[i].rank = ops[i].rank;
        eo[i].shape = sh[i];
        eo[i].strides = st[i];
    }
    return elementwise_output_strides(rank, (const uint64_t *)shape, eo, nops, (uint64_t *)out);
}

static void layout_u64(const orc_layout *l, uint64_t *shape, uint64_t *strides) {
    for (int d = 0; d < l->rank; d++) {
        shape[d] = (uint64_t)l->shape[d];
        strides[d] = (uint64_t)l->stride[d];
    }
}

static uint64_t layout_elements(const orc_layout *l) {
    uint64_t n = 1;
    for (int d = 0; d < l->rank; d++) n *= (uint64_t)l->shape[d];
    return n;
}

/* Tensor::unary_output_strides (tensor.rs:2751-2766): contiguous, then
 * channels-last, then dense-preserve, then the elementwise permutation. */
int orc_unary_output_strides(const orc_layout *in, int64_t *out_strides) {
    uint64_t shape[ORC_MAX_RANK], strides[ORC_MAX_RANK];
    layout_u64(in, shape, strides);
    int rank = in->rank;
    uint64_t elements = layout_elements(in);
    uint64_t *out = (uint64_t *)out_strides;
    if (orc_layout_is_contiguous(rank, shape, strides, elements))
        return orc_contiguous_strides(rank, shape, out);
    if (orc_is_channels_last_contiguous(rank, shape, strides))
        return orc_channels_last_strides(rank, shape, out);
    if (orc_is_non_overlapping_and_dense(rank, shape, strides, elements)) {
        memcpy(out, strides, sizeof(uint64_t) * rank);
        return ORC_OK;
    }
    ew_operand op = {rank, shape, strides};
    return elementwise_output_strides(rank, shape, &op, 1, out);
}

/* Tensor::map_scalar output layout (tensor.rs:2718-2735): the elementwise
 * permutation of the single operand (no contiguous/dense shortcuts). */
int orc_scalar_output_strides(const orc_layout *in, int64_t *out_strides) {
    uint64_t shape[ORC_MAX_RANK], strides[ORC_MAX_RANK];
    layout_u64(in, shape, strides);
    ew_operand op = {in->rank, shape, strides};
    return elementwise_output_strides(in->rank, shape, &op, 1, (uint64_t *)out_strides);
}

/* broadcast_dimension (tensor.rs:4067-4077) */
static int broadcast_dimension(uint64_t l, uint64_t r, uint64_t *out) {
    if (l == r) *out = l;
    else if (l == 1) *out = r;
    else if (r == 1) *out = l;
    else return 0;
    return 1;
}

/* aligned_dimension (tensor.rs:4058-4065) */
static uint64_t aligned_dimension(int rank_in, const uint64_t *shape, int rank_out, int axis) {
    int leading = rank_out - rank_in;
    return axis < leading ? 1 : shape[axis - leading];
}

/* Output layout of a tensor-tensor binary op: zip_map (tensor.rs:2535-2557)
 * chooses zip_map_same_shape's layout rule (:2629-2656) for equal shapes and
 * BroadcastPlan::new (:3601-3693) otherwise (the trailing fast paths
 * :3376-3543 only run when that plan is contiguous, so they agree with it). */
int orc_binary_output_layout(const orc_layout *l, const orc_layout *r, orc_layout *out) {
    uint64_t ls[ORC_MAX_RANK], lt[ORC_MAX_RANK], rs[ORC_MAX_RANK], rt[ORC_MAX_RANK];
    layout_u64(l, ls, lt);
    layout_u64(r, rs, rt);
    memset(out, 0, sizeof(*out));
    int same = l->rank == r->rank;
    for (int d = 0; same && d < l->rank; d++) same = ls[d] == rs[d];
    if (same) {
        int rank = l->rank;
        uint64_t elements = layout_elements(l);
        uint64_t *os = (uint64_t *)out->stride;
        out->rank = rank;
        memcpy(out->shape, l->shape, sizeof(int64_t) * rank);
        int rc;
        if (orc_layout_is_contiguous(rank, ls, lt, elements) &&
            orc_layout_is_contiguous(rank, rs, rt, elements)) {
            rc = orc_contiguous_strides(rank, ls, os);
        } else if (orc_is_channels_last_contiguous(rank, ls, lt) &&
                   orc_is_channels_last_contiguous(rank, rs, rt)) {
            rc = orc_channels_last_strides(rank, ls, os);
        } else if (orc_is_non_overlapping_and_dense(rank, ls, lt, elements) &&
                   orc_is_non_overlapping_and_dense(rank, rs, rt, elements) &&
                   memcmp(lt, rt, sizeof(uint64_t) * rank) == 0) {
            memcpy(os, lt, sizeof(uint64_t) * rank);
            rc = ORC_OK;
        } else {
            ew_operand ops[2] = {{rank, ls, lt}, {rank, rs, rt}};
            rc = elementwise_output_strides(rank, ls, ops, 2, os);
        }
        return rc;
    }
    /* BroadcastPlan::new */
    int rank = l->rank > r->rank ? l->rank : r->rank;
    uint64_t shape[ORC_MAX_RANK];
    for (int axis = 0; axis < rank; axis++) {
        if (!broadcast_dimension(aligned_dimension(l->rank, ls, rank, axis),
                                 aligned_dimension(r->rank, rs, rank, axis), &shape[axis]))
            return ORC_E_SHAPE_MISMATCH;
    }
    uint64_t elements;
    int rc = orc_element_count(rank, shape, &elements);
    if (rc) return rc;
    if (elements > ISIZE_MAX_U / 4) return ORC_E_ALLOCATION;
    out->rank = rank;
    for (int d = 0; d < rank; d++) out->shape[d] = (int64_t)shape[d];
    ew_operand ops[2] = {{l->rank, ls, lt}, {r->rank, rs, rt}};
    return elementwise_output_strides(rank, shape, ops, 2, (uint64_t *)out->stride);
}

/* ------------------------------------------------------------------------ */
/* Scalar semantics                                                          */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* relu_value (tensor.rs:4392-4400): exact zeros pass through (keeps -0.0);
 * otherwise f32::max(v, 0.0), which returns 0.0 for NaN. */
static inline float relu_value(float v) {
    if ((f2u(v) & 0x7fffffffu) == 0) return v;
    return v > 0.0f ? v : 0.0f;
}

/* relu_backward_value (tensor.rs:4422-4432) */
static inline float relu_backward_value(float input, float up) {
    uint32_t bits = f2u(input), mag = bits & 0x7fffffffu;
    int is_nan = mag > 0x7f800000u;
    int pos_nonzero = (bits & 0x80000000u) == 0 && mag != 0;
    return (is_nan || pos_nonzero) ? up : 0.0f;
}

/* negate_value (tensor.rs:4388-4390) */
static inline float negate_value(float v) { return u2f(f2u(v) ^ 0x80000000u); }

enum { ORC_ADD = 0, ORC_SUB = 1, ORC_MUL = 2, ORC_DIV = 3 };
/* tensor.rs:2197-2247 */
static inline float binary_op(int op, float l, float r) {
    switch (op) {
    case ORC_ADD: return l + r;
    case ORC_SUB: return l - r;
    case ORC_MUL: return l * r;
    default: return l / r;
    }
}

enum { ORC_S_ADD = 0, ORC_S_SUB, ORC_S_MUL, ORC_S_DIV, ORC_S_RSUB, ORC_S_RDIV };
/* add_scalar/sub_scalar/mul_scalar/div_scalar/scalar_sub (tensor.rs:2254-2317),
 * scalar_div = scalar * recip(value) (tensor.rs:2319-2372) */
static inline float scalar_op(int op, float v, float s) {
    switch (op) {
    case ORC_S_ADD: return v + s;
    case ORC_S_SUB: return v - s;
    case ORC_S_MUL: return v * s;
    case ORC_S_DIV: return v / s;
    case ORC_S_RSUB: return s - v;
    default: return s * (1.0f / v);
    }
}

enum { ORC_EXP = 0, ORC_RELU = 1, ORC_NEG = 2, ORC_COPY = 3 };
static inline float unary_op(int op, float v) {
    switch (op) {
    case ORC_EXP: return expf(v); /* tensor.rs:2398-2400 -> libm expf */
    case ORC_RELU: return relu_value(v);
    case ORC_NEG: return negate_value(v);
    default: return v;
    }
}

/* ------------------------------------------------------------------------ */
/* Logical iteration                                                         */
/* ------------------------------------------------------------------------ */

/* logical_offset_for_linear_index (tensor.rs:3815-3841) */
static inline uint64_t logical_offset(const orc_layout *l, uint64_t index) {
    uint64_t off = (uint64_t)l->offset;
    for (int axis = l->rank - 1; axis >= 0; axis--) {
        uint64_t dim = (uint64_t)l->shape[axis];
        off += (index % dim) * (uint64_t)l->stride[axis];
        index /= dim;
    }
    return off;
}

/* Storage offset of the operand element that output coordinate `coord`
 * reads under right-aligned broadcasting (SavedTensor::broadcast_position,
 * tensor.rs:2850-2874, and aligned_broadcast_stride, :4079-4096). Also
 * returns the operand's logical (row-major) index. */
static inline uint64_t broadcast_offset(const orc_layout *op, int out_rank, const uint64_t *coord,
                                        uint64_t *logical) {
    int leading = out_rank - op->rank;
    uint64_t off = (uint64_t)op->offset, li = 0;
    for (int a = 0; a < op->rank; a++) {
        uint64_t dim = (uint64_t)op->shape[a];
        uint64_t c = dim == 1 ? 0 : coord[leading + a];
        li = li * dim + c;
        off += c * (uint64_t)op->stride[a];
    }
    if (logical) *logical = li;
    return off;
}

static inline void decode(const orc_layout *l, uint64_t index, uint64_t *coord) {
    for (int axis = l->rank - 1; axis >= 0; axis--) {
        uint64_t dim = (uint64_t)l->shape[axis];
        coord[axis] = index % dim;
        index /= dim;
    }
}

/* ------------------------------------------------------------------------ */
/* Pointwise                                                                 */
/* ------------------------------------------------------------------------ */

/* Tensor-tensor binary op: every path of zip_map (tensor.rs:2535-2716,
 * 3376-3599) computes out[logical i] = op(left at broadcast position,
 * right at broadcast position), each a single rounding; this loop visits the
 * output in logical row-major order and writes at the output layout. */
int orc_binary_f32(int op, const float *lbuf, const orc_layout *l, const float *rbuf,
                   const orc_layout *r, float *out, const orc_layout *lo) {
    uint64_t n = layout_elements(lo), coord[ORC_MAX_RANK];
    for (uint64_t i = 0; i < n; i++) {
        decode(lo, i, coord);
        float a = lbuf[broadcast_offset(l, lo->rank, coord, NULL)];
        float b = rbuf[broadcast_offset(r, lo->rank, coord, NULL)];
        out[logical_offset(lo, i)] = binary_op(op, a, b);
    }
    return ORC_OK;
}

/* map_scalar (tensor.rs:2718-2735) */
int orc_scalar_f32(int op, const float *buf, const orc_layout *l, float s, float *out,
                   const orc_layout *lo) {
    uint64_t n = layout_elements(l);
    for (uint64_t i = 0; i < n; i++)
        out[logical_offset(lo, i)] = scalar_op(op, buf[logical_offset(l, i)], s);
    return ORC_OK;
}

/* unary_map + materialize_with_strides (tensor.rs:2737-2749, 1805-1838) */
int orc_unary_f32(int op, const float *buf, const orc_layout *l, float *out,
                  const orc_layout *lo) {
    uint64_t n = layout_elements(l);
    for (uint64_t i = 0; i < n; i++)
        out[logical_offset(lo, i)] = unary_op(op, buf[logical_offset(l, i)]);
    return ORC_OK;
}

/* Contiguous fast path of unary_map for large buffers (the same loop the
 * reference runs at tensor.rs:1812-1813 when input and output are dense). */
void orc_unary_contig_f32(int op, const float *in, float *out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = unary_op(op, in[i]);
}

void orc_binary_contig_f32(int op, const float *a, const float *b, float *out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = binary_op(op, a[i], b[i]);
}

void orc_scalar_contig_f32(int op, const float *a, float s, float *out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = scalar_op(op, a[i], s);
}

/* Trailing-vector fast path, materialize_contiguous_trailing_broadcast
 * (tensor.rs:3454-3543), vector on the right: out[r, j] = op(x[r, j], v[j]). */
void orc_row_broadcast_f32(int op, const float *x, const float *v, float *out, uint64_t rows,
                           uint64_t cols) {
    for (uint64_t r = 0; r < rows; r++)
        for (uint64_t j = 0; j < cols; j++) out[r * cols + j] = binary_op(op, x[r * cols + j], v[j]);
}

/* Dropout-apply as the reference composes it (python_nn_functional.rs:117-200
 * has no sampling; the config applies a precomputed mask): mul (tensor.rs:2217)
 * by the mask converted u8 -> f32 0/1 at ingest (python.rs:10396-10444), then
 * mul_scalar (tensor.rs:2274). Two roundings: (h * m) * s. */
void orc_mask_apply_f32(const float *h, const uint8_t *mask, float s, float *out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        float t = h[i] * (float)mask[i];
        out[i] = t * s;
    }
}

/* ------------------------------------------------------------------------ */
/* Reductions                                                                */
/* ------------------------------------------------------------------------ */

/* Tensor::sum (tensor.rs:2413-2431): logical_values().sum(), a sequential
 * left fold in row-major order.  Rust 1.92's f32 Sum starts from -0.0; that
 * start value only shows for empty or all-(-0.0) inputs (parity unpinned:
 * tests/tensor_baseline.rs:1201-1210 checks only the magnitude). */
float orc_sum_f32(const float *buf, const orc_layout *l) {
    uint64_t n = layout_elements(l);
    float acc = -0.0f;
    for (uint64_t i = 0; i < n; i++) acc += buf[logical_offset(l, i)];
    return acc;
}

/* Sum of |x| in double: the error budget for a reordered float sum. */
double orc_sum_abs_f64(const float *buf, uint64_t n) {
    double acc = 0.0;
    for (uint64_t i = 0; i < n; i++) acc += fabs((double)buf[i]);
    return acc;
}

/* ------------------------------------------------------------------------ */
/* Matmul                                                                    */
/* ------------------------------------------------------------------------ */

/* Tensor::matmul (tensor.rs:2453-2533): every path (contiguous row-blocked
 * :3919-3966, owned strided :2478-2506, checked fallback :2507-2525) starts
 * each output at +0.0 and adds left[i,k]*right[k,j] for k ascending, one
 * multiply and one add rounding per step.  Rank 2 only; `batch` > 1 applies
 * it to `batch` independent matrices (the reference has no bmm: its harness
 * calls rank-2 matmul per batch index).  The output is contiguous. */
int orc_matmul_f32(const float *a, const orc_layout *la, const float *b, const orc_layout *lb,
                   float *c, int64_t batch, int64_t bsa, int64_t bsb) {
    if (la->rank != 2 || lb->rank != 2) return ORC_E_MATMUL_RANK;
    uint64_t M = la->shape[0], K = la->shape[1], K2 = lb->shape[0], N = lb->shape[1];
    if (K != K2) return ORC_E_MATMUL_INNER;
    uint64_t sam = la->stride[0], sak = la->stride[1], sbk = lb->stride[0], sbn = lb->stride[1];
    for (int64_t t = 0; t < batch; t++) {
        const float *A = a + la->offset + t * bsa, *B = b + lb->offset + t * bsb;
        float *C = c + (uint64_t)t * M * N;
        for (uint64_t i = 0; i < M * N; i++) C[i] = 0.0f;
        for (uint64_t i = 0; i < M; i++) {
            float *crow = C + i * N;
            for (uint64_t k = 0; k < K; k++) {
                float av = A[i * sam + k * sak];
                const float *brow = B + k * sbk;
                if (sbn == 1) {
                    for (uint64_t j = 0; j < N; j++) crow[j] += av * brow[j];
                } else {
                    for (uint64_t j = 0; j < N; j++) crow[j] += av * brow[j * sbn];
                }
            }
        }
    }
    return ORC_OK;
}

/* Selected rows of a contiguous-output matmul (same order as above): the
 * full-size parity check evaluates a sample of rows. */
/* contiguous_matmul_row_blocked (tensor.rs:3919-3966): contiguous operands,
 * rows taken four at a time with depth outermost, so each right-hand row is
 * streamed once per 4-row block; leftover rows one at a time.  Per output
 * element the additions run in the same order as orc_matmul_f32 (k
 * ascending from +0.0), so the two are bit-identical; this one exists for
 * timing the reference's CPU path at its own speed (CONTIGUOUS_MATMUL_ROW_BLOCK
 * = 4, tensor.rs:17-19). */
void orc_matmul_row_blocked_f32(const float *left, const float *right, float *out, uint64_t rows,
                                uint64_t inner, uint64_t cols) {
    for (uint64_t i = 0; i < rows * cols; i++) out[i] = 0.0f;
    const uint64_t blocked = rows / 4 * 4;
    for (uint64_t r = 0; r < blocked; r += 4) {
        const float *l0 = left + r * inner, *l1 = l0 + inner, *l2 = l1 + inner, *l3 = l2 + inner;
        float *o0 = out + r * cols, *o1 = o0 + cols, *o2 = o1 + cols, *o3 = o2 + cols;
        for (uint64_t d = 0; d < inner; d++) {
            const float a0 = l0[d], a1 = l1[d], a2 = l2[d], a3 = l3[d];
            const float *rr = right + d * cols;
            for (uint64_t c = 0; c < cols; c++) {
                const float b = rr[c];
                o0[c] += a0 * b;
                o1[c] += a1 * b;
                o2[c] += a2 * b;
                o3[c] += a3 * b;
            }
        }
    }
    for (uint64_t r = blocked; r < rows; r++) {
        const float *l = left + r * inner;
        float *o = out + r * cols;
        for (uint64_t d = 0; d < inner; d++) {
            const float a = l[d];
            const float *rr = right + d * cols;
            for (uint64_t c = 0; c < cols; c++) o[c] += a * rr[c];
        }
    }
}

/* The row-blocked loop above split over `threads` POSIX threads by ranges of
 * output rows (multiples of 4, so every thread's rows are blocked exactly as
 * the single-threaded loop blocks them).  Each output element still starts at
 * +0.0 and adds left[i,k]*right[k,j] for k ascending, so the result is
 * bit-identical to orc_matmul_row_blocked_f32 and orc_matmul_f32 (pinned by
 * tests/test_oracle_properties.py).  Checker only: it lets the full-size
 * parity tests compare every element of a large product. */
typedef struct {
    const float *left, *right;
    float *out;
    uint64_t rows, inner, cols;
} mm_chunk;

static void *mm_chunk_worker(void *arg) {
    mm_chunk *c = (mm_chunk *)arg;
    orc_matmul_row_blocked_f32(c->left, c->right, c->out, c->rows, c->inner, c->cols);
    return NULL;
}

void orc_matmul_row_blocked_threads_f32(const float *left, const float *right, float *out, uint64_t rows,
                                        uint64_t inner, uint64_t cols, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    uint64_t per = (rows + (uint64_t)threads - 1) / (uint64_t)threads;
    per = (per + 3) / 4 * 4;
    pthread_t tid[64];
    mm_chunk ch[64];
    int started[64] = {0};
    int nt = 0;
    for (uint64_t r0 = 0; r0 < rows && nt < 64; r0 += per, nt++) {
        const uint64_t n = r0 + per < rows ? per : rows - r0;
        ch[nt].left = left + r0 * inner;
        ch[nt].right = right;
        ch[nt].out = out + r0 * cols;
        ch[nt].rows = n;
        ch[nt].inner = inner;
        ch[nt].cols = cols;
        started[nt] = pthread_create(&tid[nt], NULL, mm_chunk_worker, &ch[nt]) == 0;
        if (!started[nt]) mm_chunk_worker(&ch[nt]);
    }
    for (int t = 0; t < nt; t++)
        if (started[t]) pthread_join(tid[t], NULL);
}

int orc_matmul_rows_f32(const float *a, const orc_layout *la, const float *b, const orc_layout *lb,
                        const int64_t *rows, int64_t nrows, float *out_rows) {
    uint64_t K = la->shape[1], N = lb->shape[1];
    uint64_t sam = la->stride[0], sak = la->stride[1], sbk = lb->stride[0], sbn = lb->stride[1];
    const float *A = a + la->offset, *B = b + lb->offset;
    for (int64_t r = 0; r < nrows; r++) {
        float *crow = out_rows + (uint64_t)r * N;
        for (uint64_t j = 0; j < N; j++) crow[j] = 0.0f;
        uint64_t i = (uint64_t)rows[r];
        for (uint64_t k = 0; k < K; k++) {
            float av = A[i * sam + k * sak];
            const float *brow = B + k * sbk;
            for (uint64_t j = 0; j < N; j++) crow[j] += av * brow[j * sbn];
        }
    }
    return ORC_OK;
}

/* Elementwise error budget for a reordered fp32 product: (|A| |B|)[i, :] for
 * the same sampled rows, accumulated in double. */
int orc_matmul_abs_rows_f64(const float *a, const orc_layout *la, const float *b,
                            const orc_layout *lb, const int64_t *rows, int64_t nrows,
                            double *out_rows) {
    uint64_t K = la->shape[1], N = lb->shape[1];
    uint64_t sam = la->stride[0], sak = la->stride[1], sbk = lb->stride[0], sbn = lb->stride[1];
    const float *A = a + la->offset, *B = b + lb->offset;
    for (int64_t r = 0; r < nrows; r++) {
        double *crow = out_rows + (uint64_t)r * N;
        for (uint64_t j = 0; j < N; j++) crow[j] = 0.0;
        uint64_t i = (uint64_t)rows[r];
        for (uint64_t k = 0; k < K; k++) {
            double av = fabs((double)A[i * sam + k * sak]);
            const float *brow = B + k * sbk;
            for (uint64_t j = 0; j < N; j++) crow[j] += av * fabs((double)brow[j * sbn]);
        }
    }
    return ORC_OK;
}

/* ------------------------------------------------------------------------ */
/* Autograd VJPs                                                             */
/* ------------------------------------------------------------------------ */

/* apply_relu_vjp (tensor.rs:3161-3176): gradient in the input's logical
 * order, relu'(x) * up via relu_backward_value. `up` is logical-contiguous. */
void orc_relu_backward_f32(const float *input, const orc_layout *li, const float *up,
                           float *grad) {
    uint64_t n = layout_elements(li);
    for (uint64_t i = 0; i < n; i++)
        grad[i] = relu_backward_value(input[logical_offset(li, i)], up[i]);
}

/* GradFn::Multiply VJP for one operand (tensor.rs:3031-3097) with the
 * GradientAccumulator rule (:3204-3228): `up` has the output shape (logical
 * order); grad[j] for the operand `self_l` accumulates up[o] * other[o] over
 * output indices o in row-major order.  With no broadcast (operand elements
 * == output elements) the first contribution is stored as is; otherwise the
 * accumulation starts from +0.0. `grad` is in the operand's logical order. */
void orc_mul_backward_f32(const float *up, const orc_layout *lout, const float *other,
                          const orc_layout *lother, const orc_layout *lself, float *grad) {
    uint64_t nout = layout_elements(lout), nself = layout_elements(lself);
    int preserve_first = nself == nout;
    uint8_t *init = (uint8_t *)calloc(nself ? nself : 1, 1);
    for (uint64_t j = 0; j < nself; j++) {
        grad[j] = 0.0f;
        init[j] = (uint8_t)!preserve_first;
    }
    uint64_t coord[ORC_MAX_RANK];
    for (uint64_t o = 0; o < nout; o++) {
        decode(lout, o, coord);
        uint64_t self_index;
        broadcast_offset(lself, lout->rank, coord, &self_index);
        float contribution = up[o] * other[broadcast_offset(lother, lout->rank, coord, NULL)];
        if (init[self_index]) {
            grad[self_index] += contribution;
        } else {
            grad[self_index] = contribution;
            init[self_index] = 1;
        }
    }
    free(init);
}

/* Sum of `up` (output shape, logical order) over the dimensions an operand of
 * shape `lself` was broadcast along, accumulated from +0.0 in output-major
 * order -- the GradientAccumulator order of tensor.rs:3204-3228 applied to a
 * unit multiplier.  This is the VJP of a broadcasting tensor-tensor add, which
 * the reference does not record (tensor.rs:2197-2209); it is pinned by
 * composition: add's VJP equals mul's VJP against an all-ones operand. */
void orc_reduce_to_shape_f32(const float *up, const orc_layout *lout, const orc_layout *lself,
                             float *grad) {
    uint64_t nout = layout_elements(lout), nself = layout_elements(lself);
    if (nself == nout) {
        memcpy(grad, up, sizeof(float) * nout);
        return;
    }
    for (uint64_t j = 0; j < nself; j++) grad[j] = 0.0f;
    uint64_t coord[ORC_MAX_RANK];
    for (uint64_t o = 0; o < nout; o++) {
        decode(lout, o, coord);
        uint64_t self_index;
        broadcast_offset(lself, lout->rank, coord, &self_index);
        grad[self_index] += up[o];
    }
}

/* transform_backward, Permute (tensor.rs:3230-3300): the gradient of a
 * permuted view, returned in the input's logical order. */
void orc_permute_backward_f32(const float *up, int rank, const int64_t *out_shape,
                              const int64_t *dims, const int64_t *in_shape, float *grad) {
    uint64_t in_strides[ORC_MAX_RANK], stride = 1, n = 1;
    for (int a = rank - 1; a >= 0; a--) {
        in_strides[a] = stride;
        stride *= (uint64_t)in_shape[a];
    }
    for (int a = 0; a < rank; a++) n *= (uint64_t)out_shape[a];
    uint64_t coord[ORC_MAX_RANK];
    for (uint64_t o = 0; o < n; o++) {
        uint64_t rem = o;
        for (int a = rank - 1; a >= 0; a--) {
            coord[a] = rem % (uint64_t)out_shape[a];
            rem /= (uint64_t)out_shape[a];
        }
        uint64_t idx = 0;
        for (int a = 0; a < rank; a++) idx += coord[a] * in_strides[dims[a]];
        grad[idx] = up[o];
    }
}

/* add_gradient / accumulate_leaf_gradient (tensor.rs:3302-3341,
 * storage.rs:85-100): dst[i] += src[i]. */
void orc_accumulate_f32(float *dst, const float *src, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) dst[i] += src[i];
}

/* ------------------------------------------------------------------------ */
/* Exhaustive exp checker                                                    */
/* ------------------------------------------------------------------------ */

/* Largest distance, in representable floats, between got[i] and glibc
 * expf(x) for the n consecutive bit patterns x = first_bits + i (both NaN
 * counts as 0).  Split over `threads` POSIX threads; each computes the same
 * expf the reference calls (tensor.rs:2398-2400).  Checker only. */
typedef struct {
    const float *got;
    uint32_t first;
    uint64_t begin, end;
    uint64_t worst;
    uint64_t worst_index;
} exp_chunk;

static int64_t ordered_bits(float f) {
    int32_t i;
    memcpy(&i, &f, 4);
    return i < 0 ? -(int64_t)(i & 0x7fffffff) : (int64_t)i;
}

static void *exp_check_worker(void *arg) {
    exp_chunk *c = (exp_chunk *)arg;
    for (uint64_t i = c->begin; i < c->end; i++) {
        const float x = u2f((uint32_t)(c->first + i));
        const float want = expf(x), got = c->got[i];
        uint64_t d;
        if (want != want || got != got) d = (want != want && got != got) ? 0 : UINT64_MAX;
        else {
            int64_t a = ordered_bits(got), b = ordered_bits(want);
            d = (uint64_t)(a > b ? a - b : b - a);
        }
        if (d > c->worst) {
            c->worst = d;
            c->worst_index = i;
        }
    }
    return NULL;
}

uint64_t orc_exp_max_ulp(const float *got, uint32_t first_bits, uint64_t n, int threads,
                         uint64_t *worst_index) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t tid[64];
    exp_chunk ch[64];
    int started[64] = {0};
    const uint64_t per = (n + (uint64_t)threads - 1) / (uint64_t)threads;
    for (int t = 0; t < threads; t++) {
        ch[t].got = got;
        ch[t].first = first_bits;
        ch[t].begin = (uint64_t)t * per < n ? (uint64_t)t * per : n;
        ch[t].end = ch[t].begin + per < n ? ch[t].begin + per : n;
        ch[t].worst = 0;
        ch[t].worst_index = 0;
        started[t] = pthread_create(&tid[t], NULL, exp_check_worker, &ch[t]) == 0;
        if (!started[t]) exp_check_worker(&ch[t]);
    }
    uint64_t worst = 0, wi = 0;
    for (int t = 0; t < threads; t++) {
        if (started[t]) pthread_join(tid[t], NULL);
        if (ch[t].worst > worst) {
            worst = ch[t].worst;
            wi = ch[t].worst_index;
        }
    }
    if (worst_index) *worst_index = wi;
    return worst;
}
