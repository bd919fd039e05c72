// pw_mask.hip -- dropout mask-apply and its backward (u8 keep-mask operand).
// The ops, their kernels and the launcher are in pw_ops.h.
#include "pw_ops.h"

using namespace trs;

extern "C" {

int trs_mask_apply_f32(const float *h, const trs_layout *lh, const uint8_t *mask, const trs_layout *lm,
                       float scale, float *out, const trs_layout *lo) {
    const void *bases[2] = {h, mask};
    const trs_layout *ls[2] = {lh, lm};
    const int eb[2] = {4, 1};
    return run_pointwise<MaskApplyF, 2u>(MaskApplyF{scale}, lo, out, 2, bases, ls, eb);
}

int trs_mask_backward_f32(const float *up, const trs_layout *lu, const uint8_t *mask, const trs_layout *lm,
                          float scale, float *grad, const trs_layout *lg) {
    const void *bases[2] = {up, mask};
    const trs_layout *ls[2] = {lu, lm};
    const int eb[2] = {4, 1};
    return run_pointwise<MaskBackwardF, 2u>(MaskBackwardF{scale}, lg, grad, 2, bases, ls, eb);
}

}  // extern "C"
