// pw_scalar.hip -- tensor-scalar pointwise entry point.
// The ops, their kernels and the launcher are in pw_ops.h.
#include "pw_ops.h"

using namespace trs;

extern "C" {

int trs_binary_scalar_f32(int op, const float *a, const trs_layout *la, float s, float *out,
                          const trs_layout *lo) {
    const void *bases[1] = {a};
    const trs_layout *ls[1] = {la};
    const int eb[1] = {4};
    if (la && lo && la->rank != lo->rank)
        return set_error(TRS_E_SHAPE_MISMATCH, "scalar op output rank differs from input rank");
    switch (op) {
    case TRS_S_ADD: return run_pointwise(ScalarF<TRS_S_ADD>{s}, lo, out, 1, bases, ls, eb);
    case TRS_S_SUB: return run_pointwise(ScalarF<TRS_S_SUB>{s}, lo, out, 1, bases, ls, eb);
    case TRS_S_MUL: return run_pointwise(ScalarF<TRS_S_MUL>{s}, lo, out, 1, bases, ls, eb);
    case TRS_S_DIV: return run_pointwise(ScalarF<TRS_S_DIV>{s}, lo, out, 1, bases, ls, eb);
    case TRS_S_RSUB: return run_pointwise(ScalarF<TRS_S_RSUB>{s}, lo, out, 1, bases, ls, eb);
    case TRS_S_RDIV: return run_pointwise(ScalarF<TRS_S_RDIV>{s}, lo, out, 1, bases, ls, eb);
    default: return set_error(TRS_E_INVALID_ARGUMENT, "unknown scalar op %d", op);
    }
}

}  // extern "C"
