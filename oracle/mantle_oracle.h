/*
 * mantle_oracle.h -- CPU restatement of Mantle's elementwise / broadcast / reduction path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP path in
 * mantle_amd/: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only to check or to time the reference semantics. The product path never
 * links, loads or calls it.
 *
 * Every function restates one piece of the reference (paths relative to the Mantle
 * checkout): mantle/core/tensorutils.mojo, mantle/core/math_util.mojo,
 * mantle/autograd/ops/{basics,mlops,ops}.mojo. The fp32 expression order of each op is
 * kept exactly (built with -ffp-contract=off; fmaf only where the restated algorithm uses
 * a fused multiply-add).
 *
 * Pinning status (what checks each function; see tests/test_oracle.py):
 *   - closed-form single-IEEE-op functions (add/sub/mul/div, relu, max, broadcast index
 *     math, accumulate, tie routing): reference fixtures from the tests/mojo test files plus
 *     brute-force checks against numpy on small inputs;
 *   - or_exp / or_log: reference special points plus fp64 bounds over the config domains
 *     (exp <= 2 ulp on [-30, 30], <= 6 ulp on [-88, 88]; log <= 2 ulp; the sigmoid built on
 *     exp <= 3 ulp). Bit-level agreement with Mojo's stdlib exp/log (mojo
 *     1.0.0b3.dev2026061606, not installable here) is PARITY UNPINNED;
 *   - or_powf restates the stdlib's `_powf_scalar` (std/builtin/simd.mojo, the float
 *     `SIMD ** SIMD` of basics.mojo:353,373). Its formula is pinned: wherever or_log and
 *     or_exp are correctly rounded, or_powf has exactly the bits of RN(exp(fl32(y * RN(log x)))),
 *     which a correctly rounded powf misses in 37-56 % of samples at config 2's exponents
 *     (test_powf_is_exp_of_y_times_log). Its fp64 bound is <= 8 ulp (the product's rounding,
 *     |y log x| * 2^-24 relative). What stays unpinned is only the exp/log bits it inherits;
 *   - or_tanh: the cancellation formula is pinned the same way (test_tanh_is_the_exp_...);
 *   - lane-ordered sums (or_reduce_*): exact-integer fixtures plus an fp64 bound; the
 *     reduce_add lane-combine shape is PARITY UNPINNED at the bit level (rtol class).
 */
#ifndef MANTLE_ORACLE_H
#define MANTLE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_MAX_RANK 8 /* mantle/core/tensor.mojo:20 MAX_RANK */

/* Same layout as mh_shape in include/mantle_hip.h: rank, then row-major dims. */
typedef struct {
    int32_t rank;
    int64_t dims[OR_MAX_RANK];
} or_shape;

/* Mantle OP ids (mantle/autograd/ops/ops.mojo:57-83). */
enum {
    OR_ADD = 0, OR_SUB = 1, OR_MUL = 2, OR_DIV = 3, OR_EXP = 4, OR_LOG = 5, OR_POW = 6,
    OR_SUM = 8, OR_MEAN = 9, OR_MAX = 10, OR_SIGMOID = 13, OR_RELU = 14, OR_TANH = 15
};

/* Return codes. */
enum { OR_OK = 0, OR_ERR_SHAPE = -2, OR_ERR_RANK = -3, OR_ERR_OP = -4 };

/* nelts = 2 * simd_width_of[f32]() (mantle/__init__.mojo:21): the lane count that fixes
 * the CPU summation order. 32 on an AVX-512 host (the default here). */
void or_set_nelts(int nelts);
int or_get_nelts(void);

/* ---- scalar math (mantle/core/math_util.mojo:149-196, mlops.mojo:27-235) ---- */
float or_exp(float x);
float or_log(float x);
float or_powi(float x, int64_t n);
float or_powf(float x, float y);
float or_sigmoid(float x);
float or_tanh(float x);
float or_relu(float x);

/* ---- tensorutils primitives ---- */
void or_fill(float* t, int64_t n, float v);
int or_broadcast_shapes(const or_shape* s1, const or_shape* s2, or_shape* out);
void or_broadcast_calculate_strides(int size, const or_shape* shape, int64_t* strides);
int64_t or_get_real_index(int size, const int64_t* strides, const or_shape* bshape, int64_t i);
int or_elwise_transform(int op, float* res, const float* t, int64_t n);
void or_elwise_pow(float* res, const float* t, int64_t n, int64_t x);
int or_elwise_op(int op, float* res, const float* t1, const or_shape* s1,
                 const float* t2, const or_shape* s2);
int or_accumulate_grad(float* grad, const or_shape* sg, const float* rg, const or_shape* srg);
float or_reduce_all(int op, const float* t, int64_t n);
int or_reduce_axis(int op, float* res, const float* t, const or_shape* s, int axis);
/* or_reduce_axis with its outputs split over nthreads threads (the reference's parallelize
 * over outputs, tensorutils.mojo:682); identical results. For the CPU baseline. */
int or_reduce_axis_mt(int op, float* res, const float* t, const or_shape* s, int axis, int nthreads);

/* ---- op-level dispatch (mantle/autograd/ops/ops.mojo:243-311, 355-463) ----
 * axis < 0 means "no axis attribute" (reduce over all elements). */
int or_forward_op(int op, float* res, const float* t1, const or_shape* s1,
                  const float* t2, const or_shape* s2, int axis);
int or_backward_op(int tensor_id, int op, const float* ug, const or_shape* sug,
                   const float* t1, const or_shape* s1, const float* t2, const or_shape* s2,
                   int axis, float* grad);

/* ---- optimizer (mantle/nn/optim.mojo:94-140) ----
 * One Adam.step for one parameter tensor of n elements at iteration `iter` (already
 * incremented, as step() does before the update). Updates param, m (momentum) and v (rms)
 * in place. Pinned by: fp64 Adam within a small bound, the exact g = 0 invariant, and the
 * first-step closed form lr * g / (|g| + eps) (tests/test_oracle.py). */
void or_adam_step(float* param, const float* grad, float* m, float* v, int64_t n, float lr,
                  float beta1, float beta2, float eps, int64_t iter);

/* ---- adjacent elementwise ops (basics.mojo:759-817, mlops.mojo:128-186, 238-299) ----
 * FMA uses fmaf (one rounding). CLIP's min / max follow LLVM minnum / maxnum, so a NaN input
 * clips to hi; the NaN behaviour of Mojo's SIMD min / max is PARITY UNPINNED (finite and
 * infinite inputs are pinned by brute-force comparisons in tests/test_oracle.py). */
void or_fma_fwd(float* res, const float* t1, const float* t2, const float* t3, int64_t n);
int or_fma_bwd_accum(int tensor_id, float* grad, const float* ug, const float* t1, const float* t2, int64_t n);
void or_leakyrelu_fwd(float* res, const float* x, int64_t n, float slope);
void or_leakyrelu_bwd_accum(float* grad, const float* x, const float* ug, int64_t n, float slope);
void or_clip_fwd(float* res, const float* x, int64_t n, float lo, float hi);
void or_clip_bwd_accum(float* grad, const float* x, const float* ug, int64_t n, float lo, float hi);

/* ---- tstd (tensorutils.mojo:724-741, 776-840) ----
 * Standard deviation over all elements or one axis (population: divide by the count).
 * The axis form reads each output line correctly, where the reference's index arithmetic
 * does not for most shapes (see the C source); pinned by the reference's own expected
 * values and by fp64 standard deviations. */
float or_tstd_all(const float* t, int64_t n);
int or_tstd_axis(float* res, const float* t, const or_shape* s, int axis);

#ifdef __cplusplus
}
#endif
#endif
