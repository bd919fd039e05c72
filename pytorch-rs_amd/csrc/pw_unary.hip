// pw_unary.hip -- unary pointwise entry point (exp, relu, neg, copy) and relu's
// backward.
// The ops, their kernels and the launcher are in pw_ops.h.
#include "pw_ops.h"

using namespace trs;

extern "C" {

int trs_unary_f32(int op, const float *a, const trs_layout *la, float *out, const trs_layout *lo) {
    const void *bases[1] = {a};
    const trs_layout *ls[1] = {la};
    const int eb[1] = {4};
    if (la && lo && la->rank != lo->rank)
        return set_error(TRS_E_SHAPE_MISMATCH, "unary op output rank differs from input rank");
    switch (op) {
    case TRS_EXP: return run_pointwise(UnaryF<TRS_EXP>{}, lo, out, 1, bases, ls, eb);
    case TRS_RELU: return run_pointwise(UnaryF<TRS_RELU>{}, lo, out, 1, bases, ls, eb);
    case TRS_NEG: return run_pointwise(UnaryF<TRS_NEG>{}, lo, out, 1, bases, ls, eb);
    case TRS_COPY: return run_pointwise(UnaryF<TRS_COPY>{}, lo, out, 1, bases, ls, eb);
    default: return set_error(TRS_E_INVALID_ARGUMENT, "unknown unary op %d", op);
    }
}

int trs_relu_backward_f32(const float *input, const trs_layout *li, const float *up, float *grad) {
    int rc = check_layout(li, "input");
    if (rc) return rc;
    const trs_layout lc = contiguous_like(li);
    const void *bases[2] = {input, up};
    const trs_layout *ls[2] = {li, &lc};
    const int eb[2] = {4, 4};
    return run_pointwise(ReluBackwardF{}, &lc, grad, 2, bases, ls, eb);
}

}  // extern "C"
