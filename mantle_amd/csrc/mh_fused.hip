// mh_fused.hip -- graph-level entry points that cover several forward_op / backward_op
// calls of one graph pattern: bias ADD followed by RELU (a Linear layer's bias + activation,
// or an NCHW per-channel bias).
#include "mh_internal.h"

using namespace mh;

extern "C" {

int mh_bias_relu_fwd(float* y, float* r, const float* x, const mh_shape* psx, const float* bias,
                     const mh_shape* psbias) {
    MH_SHAPE_ARG(sx);
    MH_SHAPE_ARG(sbias);
    MH_TRY(check_shape(sx, "x"));
    MH_TRY(check_shape(sbias, "bias"));
    mh_shape bs;
    MH_TRY(broadcast_shapes(sx, sbias, &bs));
    if (!shape_eq(bs, sx)) return fail(MH_ERR_SHAPE, "mh_bias_relu_fwd: bias must broadcast to x");
    const int64_t n = numel(sx);
    if (n == 0) return MH_OK;
    if (!y || !r || !x || !bias) return fail(MH_ERR_NULL, "mh_bias_relu_fwd: null tensor");
    MH_TRY(mh_binary_fwd(MH_ADD, y, &sx, x, &sx, bias, &sbias));  // ADD.forward
    return mh_unary_fwd(MH_RELU, r, y, n);                     // RELU.forward
}

int mh_bias_relu_bwd_accum(float* g_y, float* grad_x, float* grad_bias, const float* y, const float* ug,
                           const mh_shape* psx, const mh_shape* psbias) {
    MH_SHAPE_ARG(sx);
    MH_SHAPE_ARG(sbias);
    MH_TRY(check_shape(sx, "x"));
    MH_TRY(check_shape(sbias, "bias"));
    mh_shape bs;
    MH_TRY(broadcast_shapes(sx, sbias, &bs));
    if (!shape_eq(bs, sx)) return fail(MH_ERR_SHAPE, "mh_bias_relu_bwd_accum: bias must broadcast to x");
    const int64_t n = numel(sx);
    if (n == 0) return MH_OK;
    if (!y || !ug) return fail(MH_ERR_NULL, "mh_bias_relu_bwd_accum: null tensor");
    MH_TRY(require_init());
    float* gy = g_y;
    if (!gy) {  // the grad of y starts at zero: stage it
        MH_TRY(stage((size_t)n * sizeof(float), reinterpret_cast<void**>(&gy)));
        MH_TRY(mh_zero(gy, n));
    }
    MH_TRY(mh_unary_bwd_accum(MH_RELU, gy, y, ug, n));  // RELU backward_op
    if (grad_x) MH_TRY(mh_binary_bwd_accum(MH_ADD, 0, grad_x, &sx, gy, &sx, y, &sx, y, &sbias));
    if (grad_bias) MH_TRY(mh_binary_bwd_accum(MH_ADD, 1, grad_bias, &sbias, gy, &sx, y, &sx, y, &sbias));
    return MH_OK;
}

}  // extern "C"
