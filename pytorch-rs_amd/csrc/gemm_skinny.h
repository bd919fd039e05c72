// gemm_skinny.h -- products with a short output side (at most 32 rows or
// columns), shared by gemm.hip (which chooses them) and gemm_skinny.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace trs {

// out(i, j) = sum_k X(i, k) * Y(k, j) for i < R, j < L, k < K, per batch.
// X is the short operand, Y the long one.  Y has a unit stride along k
// (`dot`, element (k, j) at y + j*yl + k) or along j (element at
// y + k*yl + j).  Output element (i, j) of batch b is at
// out + b*bo + i*oi + j*oj, with bo = R*L when left 0; a whole contiguous
// product has (oi, oj) = (L, 1) or (1, R), a block of columns or rows of a
// larger output (a GEMM's rim) its row stride in oi or oj.
struct SkinnyProblem {
    const float *x = nullptr;
    const float *y = nullptr;
    float *out = nullptr;
    int64_t xi = 0, xk = 0;
    int64_t yl = 0;
    bool dot = false;
    int64_t oi = 0, oj = 0, bo = 0;
    int64_t bx = 0, by = 0;
    int64_t R = 0, L = 0, K = 0, batch = 1;
};

struct SkinnyPlan {
    // The VALU matrix-vector kernel (dot form, R <= 4): row_groups is then
    // the short rows it is compiled for (1, 2 or 4) and kc the k per wave.
    bool gemv = false;
    // The VALU kernel for the other form (Y unit-stride along j, R <= 8):
    // row_groups is then the rows it is compiled for (1, 2, 4 or 8, at
    // least R) and kc the rows of Y per slice.
    bool axpy = false;
    // The MFMA kernel that streams Y through LDS (dot form, 5..32 short
    // rows): kLdsSkinnyCols columns per block, kc a multiple of 32.
    bool lds = false;
    int row_groups = 1;   // 16-row MFMA groups covering R
    bool yvec = false;    // Y read as float4 (else four scalar loads)
    bool xvec = false;    // X rows read as float4 along k
    int64_t kc = 0;       // k per split (a multiple of 16)
    int64_t splits = 1;   // K split into this many slices, summed in slice order
    int64_t blocks = 0;
};

constexpr int64_t kSkinnyMaxRows = 32;
constexpr int kSkinnyCols = 64;  // output columns per block
constexpr int kAxpyCols = 256;   // output columns per block of the VALU axpy kernel
constexpr int kLdsSkinnyCols = 64;  // output columns per block of the LDS-streaming kernel

// Fills `plan` and returns true when the kernel takes the problem (R at
// most kSkinnyMaxRows).  Y is read as float4 wherever a whole float4 lies in
// its row (dword alignment suffices); X likewise when xk is 1.
bool plan_skinny(const SkinnyProblem &p, int cu_count, SkinnyPlan *plan);

// ((p0 + p1) + p2) + ... over S partial products in slice order, slice s of
// batch b at ws[(b*S + s)*mn + e]; one float per lane, so any mn and
// alignment.  The sum of element e goes to c[b*mn + e], or with `scatter`
// (e = i*L + j) to c[b*bo + i*oi + j*oj].
struct SliceOut {
    bool scatter = false;
    int64_t L = 0, oi = 0, oj = 0, bo = 0;
};
int launch_slice_sum(const float *ws, float *c, int64_t mn, int64_t batch, int64_t S, hipStream_t s,
                     const SliceOut &out = SliceOut{});

// Runs the plan on stream `s`.  A split plan takes a workspace of
// splits * R * L * batch floats from the block cache; without one it runs
// unsplit.
int run_skinny(const SkinnyProblem &p, const SkinnyPlan &plan, hipStream_t s);

}  // namespace trs
