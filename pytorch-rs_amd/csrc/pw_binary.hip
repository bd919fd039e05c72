// pw_binary.hip -- binary pointwise entry point (add, sub, mul, div over broadcast
// and strided operands).
// The ops, their kernels and the launcher are in pw_ops.h.  mul and div are
// instantiated in pw_binary_muldiv.hip, so the two halves compile in parallel.
#include "pw_ops.h"

namespace trs {
extern template int run_pointwise<BinaryF<TRS_MUL>, 0u>(const BinaryF<TRS_MUL> &, const trs_layout *, float *, int,
                                                        const void *const *, const trs_layout *const *, const int *);
extern template int run_pointwise<BinaryF<TRS_DIV>, 0u>(const BinaryF<TRS_DIV> &, const trs_layout *, float *, int,
                                                        const void *const *, const trs_layout *const *, const int *);
}  // namespace trs

using namespace trs;

extern "C" {

int trs_binary_f32(int op, const float *a, const trs_layout *la, const float *b, const trs_layout *lb,
                   float *out, const trs_layout *lo) {
    const void *bases[2] = {a, b};
    const trs_layout *ls[2] = {la, lb};
    const int eb[2] = {4, 4};
    switch (op) {
    case TRS_ADD: return run_pointwise(BinaryF<TRS_ADD>{}, lo, out, 2, bases, ls, eb);
    case TRS_SUB: return run_pointwise(BinaryF<TRS_SUB>{}, lo, out, 2, bases, ls, eb);
    case TRS_MUL: return run_pointwise(BinaryF<TRS_MUL>{}, lo, out, 2, bases, ls, eb);
    case TRS_DIV: return run_pointwise(BinaryF<TRS_DIV>{}, lo, out, 2, bases, ls, eb);
    default: return set_error(TRS_E_INVALID_ARGUMENT, "unknown binary op %d", op);
    }
}

}  // extern "C"
