// pw_binary_muldiv.hip -- the mul and div instances of the binary pointwise
// launcher (their kernels), called from trs_binary_f32 in pw_binary.hip.
#include "pw_ops.h"

namespace trs {
template int run_pointwise<BinaryF<TRS_MUL>, 0u>(const BinaryF<TRS_MUL> &, const trs_layout *, float *, int,
                                                 const void *const *, const trs_layout *const *, const int *);
template int run_pointwise<BinaryF<TRS_DIV>, 0u>(const BinaryF<TRS_DIV> &, const trs_layout *, float *, int,
                                                 const void *const *, const trs_layout *const *, const int *);
}  // namespace trs
