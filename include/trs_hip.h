/*
 * trs_hip.h -- C ABI of libtrs_hip.so, the MI355X (gfx950) device backend for
 * the pytorch-rs tensor hot path: strided/broadcast pointwise ops, the
 * pointwise fusion compiler, fp32 matmul and the backward helpers autograd
 * needs.
 *
 * The reference (bobrenjc93/pytorch-rs) has no FFI or plugin boundary for
 * this path: arithmetic is called directly from Tensor methods in
 * src/tensor.rs, and the storage seam is the (device, dtype) match in
 * Storage::from_owned (src/storage.rs:116-124).  Each entry point below names
 * the reference function whose per-element work it replaces.
 *
 * Conventions
 *   - Every function returns int: 0 on success, a negative TRS_E_* code on
 *     failure; trs_last_error() then holds a thread-local message.  The codes
 *     mirror TensorError (src/tensor_error.rs:7-108).  No C++ exception
 *     crosses this boundary: a failed host allocation inside the library
 *     returns TRS_E_ALLOCATION_FAILED, and the message buffer itself is a
 *     fixed thread-local array.
 *   - Tensor operands are (base pointer, trs_layout): `base` is element 0 of
 *     the storage and layout.offset the element offset of the view, as in the
 *     reference Tensor struct (src/tensor.rs:212-221).  Strides are in
 *     elements and never negative.
 *   - The caller allocates every output (trs_alloc) and computes its layout;
 *     the output layout of the reference's planner (elementwise_output_strides,
 *     src/tensor.rs:4249-4312) is a host-side property.
 *   - An output must not overlap itself, and may share memory with an input
 *     only as the very same view (same address, shape and strides: in place,
 *     element for element).  A matmul output shares no memory with A or B.
 *     Other overlaps are rejected with TRS_E_INVALID_ARGUMENT before any
 *     launch.
 *   - A non-empty view whose element count, last element offset or last byte
 *     offset leaves 64 bits is rejected with TRS_E_INDEX_OVERFLOW.
 *   - All work is queued in order on one HIP stream per device (trs_stream);
 *     only trs_memcpy_d2h and trs_synchronize block the host.
 *   - Callable from any thread; the allocator and the fusion cache are
 *     internally locked.
 */
#ifndef TRS_HIP_H
#define TRS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Views of up to TRS_MAX_RANK dims (the reference's shapes are vectors of
 * any length).  Kernels index at most 8 dims after size-1 dims are dropped
 * and contiguous dims merged; a pointwise view with more than that is run as
 * one launch per index tuple of its outermost dims. */
#define TRS_MAX_RANK 25

/* Status codes (TensorError variants, src/tensor_error.rs:7-108). */
#define TRS_OK 0
#define TRS_E_ALLOCATION_FAILED (-1)      /* AllocationFailed */
#define TRS_E_INDEX_OVERFLOW (-2)         /* IndexCalculationOverflow */
#define TRS_E_STRIDE_OVERFLOW (-3)        /* StrideCalculationOverflow */
#define TRS_E_SHAPE_MISMATCH (-4)         /* ShapeMismatch */
#define TRS_E_MATMUL_INNER_MISMATCH (-5)  /* MatmulInnerDimensionMismatch */
#define TRS_E_MATMUL_REQUIRES_MATRICES (-6) /* MatmulRequiresMatrices */
#define TRS_E_INVALID_ARGUMENT (-7)       /* bad op code, rank > TRS_MAX_RANK, null pointer */
#define TRS_E_HIP (-8)                    /* HIP runtime failure */
#define TRS_E_FUSION (-9)                 /* fusion IR parse or hipRTC failure */
#define TRS_E_NO_DEVICE (-10)             /* no usable gfx950 device */

/* A strided view: rank <= TRS_MAX_RANK, shape/stride/offset in elements (the Tensor
 * metadata of src/tensor.rs:212-221). */
typedef struct trs_layout {
    int32_t rank;
    int32_t reserved;
    int64_t shape[TRS_MAX_RANK];
    int64_t stride[TRS_MAX_RANK];
    int64_t offset;
} trs_layout;

/* ---- device and memory (Storage / Device: src/storage.rs:7-18, src/device.rs:5-9) */

/* Initialise HIP, select device 0 and create its stream.  Idempotent. */
int trs_init(void);
int trs_device_count(int *count);
int trs_set_device(int device);
int trs_get_device(int *device);
/* Device name, CU count and max engine clock (kHz) of the current device. */
int trs_device_info(char *name, size_t name_len, int *cu_count, int *clock_khz);
/* Storage allocation (filled_storage, src/tensor.rs:4434-4442, without the
 * fill).  Blocks come from a per-device cache (512 B granules below 1 MiB,
 * 2 MiB above) and trs_free returns them to it without synchronising: the
 * release is stream-ordered, so a block must not be used outside this
 * library's stream after it is freed.  Pointers not from trs_alloc are
 * released with a stream sync and hipFree. */
int trs_alloc(size_t bytes, void **ptr);
/* Test hook (no counterpart in the reference; for the tests of this
 * library's fallbacks, which nothing else can reach): after `n` more
 * successful trs_alloc calls in this process, every trs_alloc fails with
 * TRS_E_ALLOCATION_FAILED until the hook is called again; n < 0 removes the
 * limit.  The fallbacks it reaches: a matmul whose gather buffers for
 * operands with no unit stride cannot be had runs the one-lane-per-output
 * kernel; a split K whose workspace cannot be had runs unsplit. */
int trs_debug_fail_allocs_after(int64_t n);
/* Test hook (no counterpart in the reference; for the tests of the
 * pointwise kernels' grid-stride loops, which only launches of more than
 * 2^22 blocks reach otherwise): every pointwise launch planned after it uses
 * at most `blocks` blocks, its blocks looping over the remaining tiles;
 * blocks = 0 restores the default cap.  Process-wide; negative is
 * TRS_E_INVALID_ARGUMENT. */
int trs_debug_pointwise_grid_cap(int64_t blocks);
int trs_free(void *ptr);
/* Return every cached block to HIP (after draining the device stream). */
int trs_empty_cache(void);
/* Bytes in live (allocated) and cached (freed, kept) blocks on the device. */
int trs_memory_stats(size_t *live_bytes, size_t *cached_bytes);
/* Page-locked host memory (hipHostMalloc).  Copies to and from it run as one
 * DMA.  Ingest and egress of whole buffers replace the reference's per-element
 * buffer conversion (src/python.rs:10329-10403) and Python-list egress
 * (src/python.rs:3744-3756, 4031-4052).  trs_host_free waits for the device
 * stream before releasing the buffer. */
int trs_host_alloc(size_t bytes, void **ptr);
int trs_host_free(void *ptr);
/* Host <-> device copies, ordered on the device stream.  h2d and d2h return
 * once the copy is complete, so the host buffer may be reused at once.
 * Pageable host memory of 16 MiB or more (h2d) or 4 MiB or more (d2h) is
 * pipelined through two page-locked chunks per device with a host copy pool;
 * smaller or page-locked buffers go as one DMA.  d2d does not block. */
int trs_memcpy_h2d(void *dst, const void *src, size_t bytes);
int trs_memcpy_d2h(void *dst, const void *src, size_t bytes);
int trs_memcpy_d2d(void *dst, const void *src, size_t bytes);
/* Zero `bytes` with a fill kernel (no hipMemset node, so it is graph-safe). */
int trs_memset_zero(void *dst, size_t bytes);
int trs_synchronize(void);
/* The hipStream_t all entry points enqueue on (for event timing). */
int trs_stream(void **stream);
/* Thread-local message for the last failing call on this thread. */
const char *trs_last_error(void);

/* ---- pointwise (zip_map / map_scalar / unary_map, src/tensor.rs:2535-2794) */

/* Tensor-tensor ops: add/sub/mul/div (src/tensor.rs:2197-2247). */
#define TRS_ADD 0
#define TRS_SUB 1
#define TRS_MUL 2
#define TRS_DIV 3
/* Tensor-scalar ops (src/tensor.rs:2254-2372): v+s, v-s, v*s, v/s, s-v,
 * and s*(1/v) (scalar_div's reciprocal multiplication). */
#define TRS_S_ADD 0
#define TRS_S_SUB 1
#define TRS_S_MUL 2
#define TRS_S_DIV 3
#define TRS_S_RSUB 4
#define TRS_S_RDIV 5
/* Unary ops: exp (src/tensor.rs:2398), relu (:2378, relu_value :4392-4400),
 * neg (negate_value :4388-4390), copy (materialize_with_strides :1805-1838,
 * used by contiguous()/clone). */
#define TRS_EXP 0
#define TRS_RELU 1
#define TRS_NEG 2
#define TRS_COPY 3

/* out = op(a, b) elementwise.  `lo` is the output layout; a and b broadcast
 * to lo's shape by right alignment (BroadcastPlan, src/tensor.rs:3601-3693).
 * Replaces zip_map (src/tensor.rs:2535-2716) and its trailing fast paths
 * (:3376-3543) and odometer (:3546-3599).  Bit-exact: one IEEE op each. */
int trs_binary_f32(int op, const float *a, const trs_layout *la, const float *b,
                   const trs_layout *lb, float *out, const trs_layout *lo);
/* out = op(a, s) elementwise; replaces map_scalar (src/tensor.rs:2718-2735). */
int trs_binary_scalar_f32(int op, const float *a, const trs_layout *la, float s, float *out,
                          const trs_layout *lo);
/* out = op(a) elementwise; replaces unary_map + materialize_with_strides
 * (src/tensor.rs:2737-2749, 1805-1838). */
int trs_unary_f32(int op, const float *a, const trs_layout *la, float *out,
                  const trs_layout *lo);
/* Dropout-apply with a precomputed keep-mask: out = (h * f32(mask)) * scale,
 * two roundings.  Replaces the reference composition mul (src/tensor.rs:2217)
 * then mul_scalar (:2274) of a mask ingested as f32 0/1
 * (src/python.rs:10396-10444); the mask stays uint8 in HBM. */
int trs_mask_apply_f32(const float *h, const trs_layout *lh, const uint8_t *mask,
                       const trs_layout *lm, float scale, float *out, const trs_layout *lo);

/* ---- reductions and backward helpers (src/tensor.rs:2413-2431, 2881-3341) */

/* *out (one device float) = sum of x.  Replaces Tensor::sum
 * (src/tensor.rs:2413-2431); a fixed-order two-level tree rather than the
 * reference's sequential fold, so it matches within the float summation
 * bound, not bit for bit: |sum - exact| <= (d u / (1 - d u)) * sum|x| with
 * u = 2^-24 and d = ceil(n/256) + 8 up to 32,768 elements, else
 * ceil(ceil(n/1024)/256) + 20.  Every partial sum starts from -0.0, as
 * Rust's f32 Sum does, so an all-(-0.0) input gives -0.0; an empty one gives
 * -0.0 too.  Elements are added by their row-major logical position: a view
 * that keeps more than 8 dims after size-1 dims are dropped and contiguous
 * dims merged is first copied to a contiguous buffer of the call's own, which
 * gives the same bits. */
int trs_sum_f32(const float *x, const trs_layout *lx, float *out);
/* trs_sum_f32 that allocates nothing: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same kernels and
 * the same result bits as trs_sum_f32.  Above 32,768 elements the block
 * partials (at most 1,024 floats for any input size, so no size is refused)
 * go to a static 4 KiB device array that each GPU holds until the process
 * ends, shared by every call on that GPU: the calls are ordered on the
 * device's library stream, and calls that ran on different streams of one
 * GPU at once would race on it.  Nothing needs clearing between calls (pass
 * 1 writes every partial pass 2 reads).  Its device address is looked up
 * once per device when the library sets the device up (trs_init).  It cannot
 * copy, so a view that keeps more than 8 dims after merging is refused
 * (TRS_E_INVALID_ARGUMENT). */
int trs_sum_f32_noalloc(const float *x, const trs_layout *lx, float *out);
/* out[0..n) = *value (a device float): the Sum VJP fill (src/tensor.rs:3008-3013). */
int trs_fill_from_device_f32(float *out, size_t n, const float *value);
/* out[0..n) = value. */
int trs_fill_f32(float *out, size_t n, float value);
/* grad = (up * scale) * f32(mask): the gradient of dropout-apply, as the
 * reference's graph computes it for mul then mul_scalar -- the MultiplyScalar
 * VJP (src/tensor.rs:3014-3021) followed by the Multiply VJP (:3031-3097) --
 * in one pass, two roundings. */
int trs_mask_backward_f32(const float *up, const trs_layout *lu, const uint8_t *mask,
                          const trs_layout *lm, float scale, float *grad, const trs_layout *lg);
/* grad (input-logical order) = relu'(input) * up; apply_relu_vjp
 * (src/tensor.rs:3161-3176) with relu_backward_value (:4422-4432).  `up` is
 * contiguous in the input's logical order. */
int trs_relu_backward_f32(const float *input, const trs_layout *li, const float *up,
                          float *grad);
/* One operand's Multiply VJP (src/tensor.rs:3031-3097) with the
 * GradientAccumulator rule (:3204-3228): grad[j] = sum over output indices o
 * that read operand element j, in row-major order, of up[o] * other[o];
 * no-broadcast operands store the single contribution as is, broadcast ones
 * accumulate from +0.0.  `up` is contiguous with shape lout; `grad` is
 * contiguous with the operand shape lself (only rank/shape read). */
int trs_mul_backward_f32(const float *up, const trs_layout *lout, const float *other,
                         const trs_layout *lother, const trs_layout *lself, float *grad);
/* grad = up summed over the dims lself was broadcast along, from +0.0 in
 * row-major output order (the add VJP; the reference records none for
 * tensor-tensor add, src/tensor.rs:2197-2209). */
int trs_reduce_to_shape_f32(const float *up, const trs_layout *lout, const trs_layout *lself,
                            float *grad);
/* dst[i] += src[i]; add_gradient and accumulate_leaf_gradient
 * (src/tensor.rs:3302-3341, src/storage.rs:85-100). */
int trs_accumulate_f32(float *dst, const float *src, size_t n);

/* ---- matmul (Tensor::matmul, src/tensor.rs:2453-2533, 3872-3994) */

/* C = A @ B in fp32 on CDNA4 FP32 MFMA.  Rank 2 ([M,K] @ [K,N]) or rank 3
 * ([b,M,K] @ [b,K,N], the batch the reference spells as rank-2 calls).
 * Operands may be transposed views (unit stride in either matrix dim,
 * e.g. `.mT`).  An operand with no unit stride is first copied into a
 * contiguous buffer from the library's block cache (as large as the operand,
 * returned at the end of the call); if that memory cannot be allocated, a
 * one-thread-per-output kernel runs in the reference's own k order.  `lc`
 * must be contiguous.
 * Tolerance versus the reference's sequential order: |dC| <= 1e-5*sqrt(K) *
 * (|A||B|) elementwise.  A single matrix whose tiles would leave CUs idle
 * may split K into S slices summed in slice order: a 16-byte-aligned one
 * with M and N multiples of 256, fewer 256x256 tiles than CUs and a long K
 * (S <= 8, when S slices fill at least half the CUs or give at least as
 * many blocks as the unsplit tile), else one whose 128x128 or 64x128 tile
 * gives at most one block per CU (S <= 16, slices of at least 128 k).  The
 * partial products then take S*M*N floats of device memory from the
 * library's block cache for the duration of the call (at most 65,536
 * floats per CU: 64 MiB on a 256-CU device).  If that memory cannot be
 * allocated the call runs the unsplit tile instead.  A product whose
 * 256x256 tiles would leave CUs idle in their last round, or number fewer
 * than the CUs with no power-of-two split filling them (6144^3: 576 tiles;
 * 3072^3: 144), may instead run stream-K: one block per CU takes an equal
 * share of all (tile, k-slice) steps, and a tile split between blocks has
 * its pieces added in k order by a second pass; its workspace is two 256x256
 * tiles per CU (128 MiB on a 256-CU device) from the block cache, and
 * without it the call runs the plan stream-K replaced.  An output with at
 * most 32 rows or columns (a matrix-vector
 * product, a small-batch linear layer) runs a kernel that streams the long
 * operand once; it splits K to fill the device when the partial products
 * (splits * M * N * batch floats, from the block cache) move at most 1/8 of
 * the long operand's bytes, and runs unsplit when that memory cannot be had.
 * The order of summation, and so the low bits of a result,
 * depends on the shape, the layout and the device's CU count (not on the
 * operands' alignment); for fixed values of these the result is
 * deterministic.
 * Empty outputs launch nothing; K = 0 writes +0.0 and then the operands may
 * be null (src/tensor.rs:4817-4839). */
int trs_matmul_f32(const float *a, const trs_layout *la, const float *b, const trs_layout *lb,
                   float *c, const trs_layout *lc);
/* Diagnostic (no counterpart in the reference): the kernel trs_matmul_f32
 * would run for these operands on the current device, without launching or
 * allocating.  Pointers are used only for their alignment and may be null.
 * *tile_m x *tile_n x *tile_k is one block's C tile and k depth (all 0
 * when nothing is launched; operands with no unit stride report the tile
 * their contiguous copies run on; a short output side reports its padded
 * rows, 16 or 32, by 64 and the k per slice),
 * *splits the number of K slices (1 = unsplit, 0 = stream-K), *blocks the
 * blocks of the main launch.  Any out pointer may be null. */
int trs_matmul_plan_f32(const float *a, const trs_layout *la, const float *b, const trs_layout *lb,
                        const float *c, const trs_layout *lc, int *tile_m, int *tile_n, int *tile_k,
                        int64_t *splits, int64_t *blocks);

/* Diagnostic (no counterpart in the reference): the launch plan the
 * pointwise entry points would use for these layouts (or, with roles = 1, a
 * fused program, which also specialises on held and once-per-tuple operands),
 * without launching anything or touching a device.  `inputs` and `out` are
 * used only for their alignment and the overlap checks and may be any
 * addresses; `elem_bytes` gives each input's element size (4 for f32, 1 for
 * a u8 mask; null means all 4); `cu_count` is the compute-unit count the plan
 * assumes.  Errors are those of the pointwise entry points. */
typedef struct trs_pw_plan_info {
    int32_t variant;    /* 0 nothing to do, 1 flat, 2 rows, 3 transposing, 4 generic */
    int32_t rank;       /* rank after dropping size-1 dims and merging contiguous ones */
    int32_t vec;        /* 16-byte vector accesses */
    int32_t fixed_rank; /* rank the kernel is compiled for (32-bit offsets), 0 = decoded at run time */
    int32_t skew;       /* transposing: a tuple's tiles taken in diagonal order */
    int32_t walk;       /* transposing: outer tuples per block */
    uint32_t trans;     /* transposing: inputs read transposed (bit i = input i) */
    uint32_t held;      /* transposing with roles: inputs loaded once per block */
    uint32_t once;      /* transposing with roles: inputs loaded once per outer tuple */
    int32_t block;      /* lanes per block */
    int64_t grid;       /* blocks per launch */
    int32_t split;      /* dims walked on the host, one launch per index tuple,
                         * when more than 8 dims remain after merging (those
                         * with the fewest indices, never the innermost) */
    int32_t launches;   /* kernel launches per call (saturates at INT32_MAX) */
} trs_pw_plan_info;
int trs_pointwise_plan(int n_inputs, const void *const *inputs, const trs_layout *const *layouts,
                       const int *elem_bytes, const float *out, const trs_layout *lo, int cu_count, int roles,
                       trs_pw_plan_info *info);

/* ---- pointwise fusion compiler (new; no counterpart in the reference) */

/* Compile a pointwise IR program to a gfx950 kernel with hipRTC (-O3,
 * -ffp-contract=off), cached by IR text in the process and on disk: the code
 * object is kept under TRS_FUSION_CACHE_DIR (empty disables), else
 * $XDG_CACHE_HOME/trs_hip/fusion or $HOME/.cache/trs_hip/fusion, keyed by the
 * hipRTC version, options and full source.  IR grammar, one instruction per
 * line, values numbered from 0 in order of definition:
 *     in f32 | in u8           -- next kernel input
 *     const <hex f32 bits>     -- scalar constant
 *     add|sub|mul|div %a %b    -- binary32 op, one rounding
 *     exp|relu|neg %a          -- unary op with the reference semantics
 *     relub %x %g              -- relu's VJP: g where x is NaN or > 0, else +0
 *                                 (relu_backward_value, src/tensor.rs:4422-4432)
 *     out %a                   -- an output; the `out` lines end the program,
 *                                 at most 8 of them, in output order
 * Each instruction rounds exactly as the eager op it mirrors, so a fused
 * chain is bit-identical to the eager chain except through exp. */
int trs_fusion_compile(const char *ir, size_t ir_len, uint64_t *kernel_id);
/* Launch a compiled one-output program: inputs broadcast to lo's shape. */
int trs_fusion_launch(uint64_t kernel_id, int n_inputs, const void *const *inputs,
                      const trs_layout *in_layouts, float *out, const trs_layout *lo);
/* Launch a program with n_outputs outputs in one kernel; every output has the
 * layout lo.  Outputs share no memory with each other; an output may share
 * memory with an input only as the very same view. */
int trs_fusion_launch_multi(uint64_t kernel_id, int n_inputs, const void *const *inputs,
                            const trs_layout *in_layouts, int n_outputs, float *const *outputs,
                            const trs_layout *lo);
/* Number of outputs of a compiled program. */
int trs_fusion_outputs(uint64_t kernel_id, int *n_outputs);
/* Generated HIP C++ source of a compiled program (for inspection). */
int trs_fusion_source(uint64_t kernel_id, char *buf, size_t buf_len, size_t *needed);
/* Milliseconds spent producing this program's code object: the hipRTC
 * compile, or the load from the disk cache (reported apart from timings). */
int trs_fusion_compile_ms(uint64_t kernel_id, double *ms);
/* *hit = 1 when the code object came from the disk cache, else 0. */
int trs_fusion_from_disk_cache(uint64_t kernel_id, int *hit);

#ifdef __cplusplus
}
#endif

#endif /* TRS_HIP_H */
