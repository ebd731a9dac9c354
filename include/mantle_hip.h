/*
 * mantle_hip.h -- C ABI of libmantle_hip.so: Mantle's elementwise / broadcast / reduction
 * op layer as hand-written HIP kernels for gfx950 (MI355X).
 *
 * This is the drop-in boundary for Mantle's op structs. Each entry point replaces the body
 * of one reference function (paths relative to the Mantle checkout, cited per entry):
 * mantle/core/tensorutils.mojo primitives and the op structs of
 * mantle/autograd/ops/basics.mojo and mantle/autograd/ops/mlops.mojo, reached through
 * forward_op / backward_op in mantle/autograd/ops/ops.mojo.
 *
 * Conventions
 *   - Plain C types only; no exceptions cross the ABI. Every int-returning call returns
 *     MH_OK (0) or a negative mh_status; mh_last_error() gives a thread-local message.
 *   - Tensors are fp32, row-major contiguous, rank 1..8 (mantle/core/tensor.mojo:20-155),
 *     described by an mh_shape passed by pointer (const mh_shape*, read during the call
 *     only), so that any FFI can pass it without struct-by-value rules. Tensor pointers
 *     are device pointers from mh_malloc (or any device allocation on the initialised
 *     device). The library never frees caller memory.
 *   - Shapes are validated before any device work: a pair that does not broadcast (which
 *     the reference only prints about, tensorutils.mojo:116-122), rank outside 1..8, a
 *     negative dim or a null tensor pointer returns an error and launches nothing.
 *   - One context per process, one HIP stream (default priority). Calls are complete when
 *     they return unless mh_init was given MH_INIT_ASYNC; then mh_sync() waits.
 *   - Backward entry points ACCUMULATE into grad (grad = grad + op gradient), fusing the
 *     op struct's backward with accumulate_grad exactly as backward_op does
 *     (ops.mojo:355-463). Pass a zeroed grad to get the plain gradient.
 *   - Not re-entrant across host threads (the reference calls ops from one thread).
 */
#ifndef MANTLE_HIP_H
#define MANTLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MH_MAX_RANK 8 /* mantle/core/tensor.mojo:20 MAX_RANK */

/* TensorShape (mantle/core/tensor.mojo:28-229): rank and row-major dims. */
typedef struct {
    int32_t rank;
    int64_t dims[MH_MAX_RANK];
} mh_shape;

/* Op ids: the same numbers as Mantle's OP registry (mantle/autograd/ops/ops.mojo:57-83). */
enum mh_op {
    MH_ADD = 0, MH_SUB = 1, MH_MUL = 2, MH_DIV = 3, MH_EXP = 4, MH_LOG = 5, MH_POW = 6,
    MH_SUM = 8, MH_MEAN = 9, MH_MAX = 10, MH_SIGMOID = 13, MH_RELU = 14, MH_TANH = 15,
    MH_FMA = 19, MH_CLIP = 20, MH_LEAKYRELU = 28
};

enum mh_status {
    MH_OK = 0,
    MH_ERR_INVALID = -1,   /* bad argument (tensor_id, axis, flag ...) */
    MH_ERR_SHAPE = -2,     /* shapes do not broadcast / do not match the op */
    MH_ERR_RANK = -3,      /* rank outside 1..8 or a negative dim */
    MH_ERR_NULL = -4,      /* null pointer for a non-empty tensor */
    MH_ERR_OP = -5,        /* op id not supported by this entry point */
    MH_ERR_NOT_INIT = -6,  /* mh_init has not succeeded */
    MH_ERR_HIP = -7,       /* a HIP runtime call failed (message in mh_last_error) */
    MH_ERR_NO_DEVICE = -8, /* no usable gfx950 device */
    MH_ERR_OVERFLOW = -9   /* element count or byte size overflow */
};

#define MH_INIT_ASYNC 1u /* do not synchronise at the end of each call */

/* ---- context and memory (the device-resident side of Tensor / Collection) ---- */
/* mh_init also reads two environment variables (again at every call):
 *   MANTLE_HIP_TRACE=1   every entry point that queues GPU work opens a roctx range named after
 *                        itself and its op (roctx found with dlopen; absent, tracing stays off);
 *   MANTLE_HIP_FAIL_AT=k the k-th HIP runtime call after this mh_init fails with MH_ERR_HIP
 *                        without being made (failure-path tests). */
int mh_init(int device, uint64_t flags);
int mh_shutdown(void);
int mh_sync(void);
const char* mh_last_error(void);
const char* mh_status_string(int status);
int mh_device_count(int* count);

/* Tensor storage: Tensor[f32] allocation and zero-init (tensor.mojo:250-302). */
int mh_malloc(void** dptr, size_t bytes);
int mh_free(void* dptr);
int mh_memcpy_h2d(void* dst, const void* src, size_t bytes);
int mh_memcpy_d2h(void* dst, const void* src, size_t bytes);
/* Tensor.copy (tensor.mojo:345-361): device-to-device deep copy. */
int mh_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Tensor.zero / Collection.set_zero (collection.mojo:221-224); a fill kernel, not a memset. */
int mh_zero(float* t, int64_t n);

/* fill, tensorutils.mojo:29-44: t[i] = v. */
int mh_fill(float* t, float v, int64_t n);

/* ---- forward ---- */

/* ADD/SUB/MUL/DIV forward: the elwise_op dispatcher, tensorutils.mojo:242-357
 * (same shape :277-290, tensor-scalar :293-304, scalar-tensor :307-318,
 * broadcast_elwise_op :321-357) as called by ADD/SUB/MUL/DIV.forward
 * (basics.mojo:36-43, 66-73, 102-109, 140-147). sres must equal broadcast(sa, sb). */
int mh_binary_fwd(int op, float* res, const mh_shape* sres, const float* a, const mh_shape* sa,
                  const float* b, const mh_shape* sb);

/* EXP/LOG/SIGMOID/RELU/TANH forward: elwise_transform, tensorutils.mojo:181-200, with the
 * functions of EXP.forward (basics.mojo:266-270), LOG.forward (:294-298),
 * SIGMOID.sigmoid (mlops.mojo:35-42), RELU.relu (:85-90), TANH.tanh (:195-201). */
int mh_unary_fwd(int op, float* res, const float* x, int64_t n);

/* POW.forward, basics.mojo:320-327 -> elwise_pow, tensorutils.mojo:226-239:
 * res = powi(x, Int(exponent[0])), the exponent truncated toward zero. `exponent` is the
 * device pointer of the shape-(1) graph scalar t2. */
int mh_pow_fwd(float* res, const float* x, int64_t n, const float* exponent);

/* elwise_pow, tensorutils.mojo:226-239: res = powi(x, n_int) with the integer exponent
 * given by the caller (Mojo's `SIMD ** Int`: square-and-multiply from 1, 1 / result for a
 * negative exponent). */
int mh_powi_fwd(float* res, const float* x, int32_t n_int, int64_t n);

/* SUM/MEAN/MAX forward: SUM.forward (basics.mojo:393-406), MEAN.forward (:440-452),
 * MAX.forward (:521-534) -> reduce all (tensorutils.mojo:564-598, tsum/tmean/tmax
 * :694-720, :850-862) or reduce axis (:622-684, :746-772, :865-876). axis = -1 reduces all
 * elements into res[0]; otherwise res has get_reduce_shape(sx, axis) (:601-619). */
int mh_reduce_fwd(int op, float* res, const float* x, const mh_shape* sx, int32_t axis);

/* mh_reduce_fwd without any device allocation. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP-graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Same kernels and results as mh_reduce_fwd, but the
 * split partials live in a fixed 16 MiB device array per GPU (held from library load until
 * the process ends) instead of library scratch; shapes whose partials would need more return
 * MH_ERR_OVERFLOW before any device work (every reduction over a non-last axis fits, and
 * last-axis or all-element reductions of up to 2^32 elements). All calls in a process share
 * its GPU's array: calls that overlap on one GPU (issued from several host threads) race, and
 * must not be made. */
int mh_reduce_fwd_noalloc(int op, float* res, const float* x, const mh_shape* sx, int32_t axis);

/* ---- backward (accumulating) ---- */

/* backward_op for ADD/SUB/MUL/DIV (ops.mojo:408-463): the struct backward of operand
 * tensor_id (ADD :46-55, SUB :82-91, MUL :118-129, DIV :155-219 of basics.mojo) followed
 * by accumulate_grad[grad_shape = s_k, res_grad_shape = broadcast(s1, s2)]
 * (tensorutils.mojo:454-487), i.e. un-broadcast by summation when the operand was
 * broadcast. sug must equal broadcast(s1, s2); sgrad must equal s1 (id 0) or s2 (id 1). */
int mh_binary_bwd_accum(int op, int tensor_id, float* grad, const mh_shape* sgrad,
                        const float* ug, const mh_shape* sug, const float* t1, const mh_shape* s1,
                        const float* t2, const mh_shape* s2);

/* Both operand gradients of a same-shape ADD/SUB/MUL/DIV in one pass (the two
 * backward_op calls that Model.backward makes when both operands are trainable,
 * model.mojo:233-270). Requires s1 == s2 == sug; either grad pointer may be NULL to skip
 * that operand. grad1 == grad2 (one symbol as both operands, x * x) accumulates both
 * gradients into it, operand 0's first: grad = (grad + rg0) + rg1, as the two calls do.
 * Gradient ranges that overlap without being equal run as the two calls, id 0 then id 1. */
int mh_binary_bwd_accum2(int op, float* grad1, float* grad2, const float* ug,
                         const float* t1, const float* t2, const mh_shape* s);

/* backward_op for EXP/LOG/SIGMOID/RELU/TANH (ops.mojo:355-405): EXP.backward
 * (basics.mojo:272-285), LOG.backward (:300-309), SIGMOID.backward (mlops.mojo:50-76),
 * RELU.backward (:99-125), TANH.backward (:209-235), then the same-shape
 * accumulate_grad (tensorutils.mojo:442-451): grad = grad + f'(x) * ug. */
int mh_unary_bwd_accum(int op, float* grad, const float* x, const float* ug, int64_t n);

/* backward_op for POW (ops.mojo:408-463 with POW.backward, basics.mojo:329-378).
 * tensor_id 0: grad = grad + (a * powf(x + 1e-12, a - 1)) * ug, a = exponent[0].
 * tensor_id 1: grad[0] = grad[0] + sum(powf(x, a) * (isinf(log x) ? 0 : log x) * ug), a sum
 * whose order differs from the reference's (rtol 1e-5); where x + 1e-12 rounds to x and
 * powf(x + 1e-12, a - 1) and x times it are normal and below 2e38, a term takes powf(x, a) as
 * that product (a few ulp from it), the power tensor_id 0 evaluates.
 * n is the element count of x and ug. */
int mh_pow_bwd_accum(int tensor_id, float* grad, const float* x, const float* exponent,
                     const float* ug, int64_t n);

/* The two POW backward_op calls Model.backward makes when both x and the exponent are
 * trainable (model.mojo:233-270 with POW.backward, basics.mojo:329-378), in one pass that reads
 * x and ug once: grad_x as tensor_id 0, grad_exp[0] as tensor_id 1. The results have the bits
 * of mh_pow_bwd_accum(0, ...) then mh_pow_bwd_accum(1, ...). A null gradient skips its part;
 * a grad_x that overlaps x, ug, the exponent or grad_exp runs as those two calls in order. */
int mh_pow_bwd_accum2(float* grad_x, float* grad_exp, const float* x, const float* exponent,
                      const float* ug, int64_t n);

/* backward_op for SUM/MEAN/MAX (ops.mojo:355-405): SUM.backward (basics.mojo:408-425),
 * MEAN.backward (:454-506), MAX.backward (:536-615, ties split as fl(1/count) * ug),
 * then the same-shape accumulate_grad. ug has the reduced shape (axis >= 0) or (1). */
int mh_reduce_bwd_accum(int op, float* grad, const float* x, const mh_shape* sx, const float* ug,
                        int32_t axis);

/* accumulate_grad, tensorutils.mojo:442-487: grad += rg for equal shapes, grad += rg[0]
 * for rg of shape (1), otherwise grad += un-broadcast(rg) (sum over the broadcast axes).
 * Pairs that are not numpy-broadcastable (which the reference indexes out of bounds with,
 * tensorutils.mojo:149-175 and :482-484) return MH_ERR_SHAPE. */
int mh_accumulate_grad(float* grad, const mh_shape* sgrad, const float* rg, const mh_shape* srg);

/* ---- adjacent ops (same-shape, flat element count) ---- */

/* FMA.forward (mantle/autograd/ops/basics.mojo:768-788): res = fma(t1, t2, t3), one rounding.
 * FMA.result_shape (:759-766) assumes all three shapes equal; so does this entry point. */
int mh_fma_fwd(float* res, const float* t1, const float* t2, const float* t3, int64_t n);

/* FMA.backward (basics.mojo:790-817) accumulated as the ternary backward_op does
 * (ops.mojo:466-497): tensor_id 0 grad += ug * t2; 1 grad += ug * t1; 2 grad += ug. */
int mh_fma_bwd_accum(int tensor_id, float* grad, const float* ug, const float* t1, const float* t2, int64_t n);

/* LEAKYRELU (mantle/autograd/ops/mlops.mojo:128-186), attribute negative_slope:
 * fwd res = x > 0 ? x : x * slope; bwd grad += (x > 0 ? 1 : slope) * ug. */
int mh_leakyrelu_fwd(float* res, const float* x, int64_t n, float negative_slope);
int mh_leakyrelu_bwd_accum(float* grad, const float* x, const float* ug, int64_t n, float negative_slope);

/* CLIP (mlops.mojo:238-299), attributes min / max (absent: pass -FLT_MAX / FLT_MAX, the
 * reference's min_finite / max_finite): fwd res = max(min(x, max_val), min_val) with
 * minnum / maxnum semantics (a NaN input gives max_val); bwd grad += (x >= min_val &&
 * x <= max_val) ? ug : 0. */
int mh_clip_fwd(float* res, const float* x, int64_t n, float min_val, float max_val);
int mh_clip_bwd_accum(float* grad, const float* x, const float* ug, int64_t n, float min_val, float max_val);

/* tstd (mantle/core/tensorutils.mojo:724-741 all elements, :776-840 one axis): population
 * standard deviation, sqrt(sum((x - mean)^2) / count), with the mean of tmean. axis -1 = all
 * elements (res has one element), else res has get_reduce_shape(sx, axis). Each output line
 * is the line tmean reads; the reference's axis form reads other lines for most shapes (its
 * index arithmetic takes i % shape[k] without dividing), which is not reproduced. */
int mh_tstd(float* res, const float* x, const mh_shape* sx, int32_t axis);

/* ---- fused graph-level entry points (no single reference counterpart) ---- */

/* Linear-layer / NCHW bias + RELU forward: y = ADD(x, bias) (broadcast) and
 * r = RELU(y) in one pass, the two forward_op calls of a graph ADD -> RELU
 * (ADD.forward basics.mojo:36-43, RELU.forward mlops.mojo:92-97). Writes both y (needed
 * by RELU's backward) and r. sbias must broadcast to sx. */
int mh_bias_relu_fwd(float* y, float* r, const float* x, const mh_shape* sx, const float* bias,
                     const mh_shape* sbias);

/* Backward of the same graph: g_y = g_y + relu'(y) * ug (RELU backward_op), then both
 * ADD backward_op calls: grad_x += g_y and grad_bias += un-broadcast(g_y). g_y may be NULL
 * when the graph's grad of y starts at zero and is not needed afterwards; then the sum
 * uses relu'(y) * ug directly. grad_x or grad_bias may be NULL to skip that operand. */
int mh_bias_relu_bwd_accum(float* g_y, float* grad_x, float* grad_bias, const float* y,
                           const float* ug, const mh_shape* sx, const mh_shape* sbias);

/* Row-fused forward of the classifier-head graph over x [rows, classes] (classes <= 2047):
 *   MAX(x, axis 1) -> SUB -> EXP -> SUM(axis 1) -> DIV -> LOG -> MUL(target) -> MEAN
 * i.e. Softmax (mantle/nn/activations.mojo:74-87) followed by LOG, MUL and MEAN
 * (basics.mojo:288-309, 94-129, 428-506): loss[0] = mean(log(softmax(x)) * target), with no
 * sign change. Per element the same values as the eight forward_op calls; the final mean
 * sums in another order (rtol class). Reads x and target once. */
int mh_softmax_log_mul_mean_fwd(float* loss, const float* x, const float* target, int64_t rows,
                                int64_t classes);

/* Backward of the same graph from ug = the grad of the loss (a device scalar), accumulated:
 * grad_x = grad_x + d(loss)/dx, bit-identical to the ten backward_op calls Model.backward
 * makes for the graph (model.mojo:194-330) from zeroed intermediate grads. Reads x and
 * target, updates grad_x, in one pass. */
int mh_softmax_log_mul_mean_bwd_accum(float* grad_x, const float* x, const float* target,
                                      const float* ug, int64_t rows, int64_t classes);

/* Row-fused graphs over the last axis of x [rows, classes], classes <= 2047 (longer rows
 * return MH_ERR_INVALID: use the op-by-op entry points). Outputs and gradients are
 * bit-identical to the op-by-op forward_op / backward_op calls for finite inputs (each row
 * sum runs in the order the library's row reductions use for that length); only a loss's
 * all-element sum runs in another order (rtol class).
 *
 * Softmax (mantle/nn/activations.mojo:74-87): MAX(axis) -> SUB -> EXP -> SUM(axis) -> DIV.
 * The backward takes grad_out, the gradient of the Softmax output, and accumulates into
 * grad_x what the graph's five backward nodes give from zeroed intermediate gradients. */
int mh_softmax_fwd(float* out, const float* x, int64_t rows, int64_t classes);
int mh_softmax_bwd_accum(float* grad_x, const float* x, const float* grad_out, int64_t rows, int64_t classes);

/* LogSoftmax (activations.mojo:94-108): MAX(axis) -> SUB -> EXP -> SUM(axis) -> LOG ->
 * SUB(x - max, log sum). Backward as for Softmax. */
int mh_logsoftmax_fwd(float* out, const float* x, int64_t rows, int64_t classes);
int mh_logsoftmax_bwd_accum(float* grad_x, const float* x, const float* grad_out, int64_t rows, int64_t classes);

/* CrossEntropyLoss (mantle/nn/loss.mojo:45-61) of predictions x [rows, classes] against
 * target: LogSoftmax(x, axis 1) -> MUL(target, .) -> SUM -> MUL(., f32(-1 / rows)); loss is a
 * device scalar. The backward takes ug, the gradient of the loss (a device scalar). */
int mh_cross_entropy_fwd(float* loss, const float* x, const float* target, int64_t rows, int64_t classes);
int mh_cross_entropy_bwd_accum(float* grad_x, const float* x, const float* target, const float* ug, int64_t rows,
                               int64_t classes);

/* ---- graph and model: Graph (mantle/autograd/graph.mojo:33-217), Model
 * (mantle/nn/model.mojo:55-340) and its Collections (mantle/autograd/collection.mojo:24-224)
 * in device memory ---- */

/* AttributeVector entries of the ops on this path (mantle/autograd/attributes.mojo): the
 * reduce "axis", LEAKYRELU "negative_slope", CLIP "min" / "max"; flags say which are set. */
#define MH_ATTR_AXIS 1
#define MH_ATTR_NEGATIVE_SLOPE 2
#define MH_ATTR_MIN 4
#define MH_ATTR_MAX 8
typedef struct {
    int32_t flags;
    int32_t axis;
    float negative_slope;
    float min_val;
    float max_val;
} mh_attrs;

enum mh_symbol_kind { MH_SYM_INPUT = 0, MH_SYM_PARAM = 1, MH_SYM_NODE = 2 };
enum mh_copy_from { MH_FROM_HOST = 0, MH_FROM_DEVICE = 1 };
/* mh_model_create flag: run an ADD whose output only feeds the RELU node right after it as
 * the fused bias + RELU kernels (every tensor and grad slot still holds the op-by-op value). */
#define MH_MODEL_FUSE_BIAS_RELU 1u
/* mh_model_create flag: run the node groups nn.Softmax, nn.LogSoftmax, nn.CrossEntropyLoss
 * (activations.mojo:74-108, loss.mojo:45-61) and Softmax -> LOG -> MUL(target) -> MEAN over
 * the last axis (at most 2047 classes) as one row-fused kernel each way, when the group's
 * nodes are consecutive and its intermediates are read by the group alone. The group's
 * output (or loss) and grad_x get the op-by-op values; the intermediate tensor and gradient
 * slots are not written, and the backward assumes their gradients start at zero (as after
 * mh_model_zero_grad). */
#define MH_MODEL_FUSE_ROWS 2u

typedef struct mh_graph mh_graph;
typedef struct mh_model mh_model;

/* Graph() and its builders: input (graph.mojo:85-86), param with optional data (:88-94;
 * without data the parameter is zero, model.mojo:371-373), scalar (:96-97: a shape-(1)
 * non-trainable parameter), op (:110-129: result shape from static_result_shape, trainable
 * if any operand is, :212-217), out (:104-105) and loss (:107-108). Symbols are numbered in
 * creation order. Host-only calls: no device is needed. */
int mh_graph_create(mh_graph** out);
int mh_graph_destroy(mh_graph* g);
int mh_graph_input(mh_graph* g, const mh_shape* shape, int trainable, int32_t* sym);
int mh_graph_param(mh_graph* g, const mh_shape* shape, int trainable, const float* data, int64_t ndata,
                   int32_t* sym);
int mh_graph_scalar(mh_graph* g, float value, int32_t* sym);
int mh_graph_op(mh_graph* g, int op, int32_t noperands, const int32_t* operands, const mh_attrs* attrs,
                int32_t* sym);
int mh_graph_out(mh_graph* g, int32_t sym);
int mh_graph_loss(mh_graph* g, int32_t sym);
int mh_graph_symbol(const mh_graph* g, int32_t sym, mh_shape* shape, int* trainable, int* kind);
int mh_graph_counts(const mh_graph* g, int32_t* nsymbols, int32_t* nnodes, int32_t* ninputs, int32_t* nparams,
                    int32_t* noutputs);

/* Model(g) (model.mojo:58-78 with allocate_tensor_memory / allocate_grad_memory, :332-395):
 * one device arena for every symbol's tensor and one for every trainable symbol's gradient,
 * zeroed, parameters with data copied in. The graph is copied: it may be destroyed after. */
int mh_model_create(const mh_graph* g, uint64_t flags, mh_model** out);
int mh_model_destroy(mh_model* m);

/* Model.forward (model.mojo:80-96, execute :113-171): copies the inputs (in graph input
 * order, from host or device memory) into their slots and runs every node. Read the loss
 * through mh_model_tensor. */
int mh_model_forward(mh_model* m, int32_t ninputs, const float* const* inputs, int from);
/* Model.inference (model.mojo:98-111): runs the nodes up to the last one that writes a
 * graph output (n_inference_nodes, model.mojo:39-48). */
int mh_model_inference(mh_model* m, int32_t ninputs, const float* const* inputs, int from);
/* Model.backward (model.mojo:173-330): with nupper == 0 the loss gradient is filled with
 * 1.0, else the last node's output gradient is set to upper_grads[0]; then every node in
 * reverse order accumulates into the gradient of each trainable operand. Gradients
 * accumulate across calls until mh_model_zero_grad, as in the reference. */
int mh_model_backward(mh_model* m, int32_t nupper, const float* const* upper_grads, int from);
/* Collection.__getitem__ (collection.mojo:194-200) of parameters.tensors / .grads: the
 * device address of a symbol's slot (aliasing, like share()). */
int mh_model_tensor(mh_model* m, int32_t sym, float** dptr);
int mh_model_grad(mh_model* m, int32_t sym, float** dptr);
/* parameters.grads.set_zero (collection.mojo:221-224): one fill over the gradient arena. */
int mh_model_zero_grad(mh_model* m);
/* HIP-graph form of the passes: mh_model_capture runs the pass once (library buffers reach
 * their sizes), then records its launches on the library stream into a graph; mh_model_replay
 * launches the graph. MH_PASS_FORWARD is every node (inputs are not part of it: write them into
 * their slots first, through mh_model_tensor); MH_PASS_BACKWARD seeds the loss gradient with 1.0
 * and runs every node in reverse; MH_PASS_STEP is a training step's device work in one graph:
 * the gradient arena zeroed (mh_model_zero_grad), then the forward and backward passes. A graph
 * launch costs the host about as much as launching a handful of kernels, so a step replays
 * fastest as one MH_PASS_STEP graph: for a deep chain of small tensors (24 MUL/ADD/RELU layers
 * over [32, 32]) 1.5-2 times as fast as the eager step, whose host launches bound it; a short
 * step or one over large tensors runs as fast eagerly. The graph holds kernel launches only
 * (no memset or host-copy nodes). Capturing again replaces the graph. A captured graph keeps
 * the library buffers it was recorded with (a library buffer that grows while any graph exists
 * is kept, at least doubling, and freed once no captured graph is left); after mh_shutdown and
 * mh_init, replay returns MH_ERR_INVALID until the pass is captured again. */
#define MH_PASS_FORWARD 0
#define MH_PASS_BACKWARD 1
#define MH_PASS_STEP 2
int mh_model_capture(mh_model* m, int pass);
int mh_model_replay(mh_model* m, int pass);

/* The trainable parameters (graph params with trainable set, get_trainable_parameters,
 * optim.mojo:27-44) occupy the start of the tensor arena, and their gradients the start of
 * the gradient arena, in the same order and slot sizes: two parallel spans of n floats
 * (padding between slots is zero in both). mh_adam_step over the two spans updates every
 * parameter in one launch; padding stays zero. NULL spans and n = 0 without trainable
 * parameters. */
int mh_model_param_span(mh_model* m, float** params, float** grads, int64_t* n);
/* fused_groups: bias + RELU pairs plus row groups the model runs fused. */
int mh_model_info(const mh_model* m, int32_t* n_inference_nodes, int64_t* tensor_bytes, int64_t* grad_bytes,
                  int32_t* fused_groups);

/* ---- optimizer ---- */

/* Adam.step for one parameter tensor (mantle/nn/optim.mojo:94-140, per-element body :101-132):
 * m = b1*m + (1-b1)*g; v = b2*v + ((1-b2)*g)*g; p = p - lr*((m/(1-b1**iter)) /
 * (sqrt(v/(1-b2**iter)) + eps)), in that order, with iter >= 1 the already-incremented step
 * count. Updates param, m and v in place (28 bytes per element). */
int mh_adam_step(float* param, const float* grad, float* m, float* v, int64_t n, float lr, float beta1,
                 float beta2, float eps, int64_t iter);

/* Adam.step over every trainable parameter of a model (the parallelize over parameters,
 * optim.mojo:140): arrays of ntensors device pointers and sizes, one launch per 80 tensors.
 * Same arithmetic as mh_adam_step. */
int mh_adam_step_multi(int64_t ntensors, float* const* params, const float* const* grads, float* const* m,
                       float* const* v, const int64_t* sizes, float lr, float beta1, float beta2, float eps,
                       int64_t iter);

/* Seeded synthetic fill (the device counterpart of rand_uniform / rand_normal,
 * mantle/core/rand_utils.mojo:23-63): element i of stream `seed` comes from a counter-based
 * SplitMix64, so the result does not depend on the launch shape. U(lo, hi) and N(mean, std). */
int mh_rand_uniform(float* t, int64_t n, uint64_t seed, float lo, float hi);
int mh_rand_normal(float* t, int64_t n, uint64_t seed, float mean, float std);

/* ---- timing (events on the library's stream) ---- */
int mh_event_create(void** ev);
int mh_event_destroy(void* ev);
int mh_event_record(void* ev);
int mh_event_elapsed_ms(float* ms, void* start, void* stop);

/* ---- diagnostics ---- */

/* How mh_binary_fwd would execute (sres, sa, sb): after dropping size-1 dims and merging
 * dims that are contiguous for every operand. kind: 0 same-shape, 1 b is one element,
 * 2 a is one element, 3 strided broadcast. Host-only, needs no device. */
typedef struct {
    int32_t kind;
    int32_t rank;
    int64_t dims[MH_MAX_RANK];
    int64_t stride_a[MH_MAX_RANK];
    int64_t stride_b[MH_MAX_RANK];
} mh_plan_info;
int mh_plan_binary(const mh_shape* sres, const mh_shape* sa, const mh_shape* sb, mh_plan_info* out);

/* The chain of single-axis reductions that un-broadcasting rg into grad runs: the number
 * of steps and, per step, the [A, B, C] view reduced over B. Host-only. */
typedef struct {
    int32_t nsteps; /* 0: same shape (no reduction) */
    int64_t a[MH_MAX_RANK];
    int64_t b[MH_MAX_RANK];
    int64_t c[MH_MAX_RANK];
} mh_reduce_plan_info;
int mh_plan_unbroadcast(const mh_shape* sgrad, const mh_shape* srg, mh_reduce_plan_info* out);

/* The 1-D launches an element-streaming entry point makes over n elements (host-only): `what`
 * names it, and *out gets the kernel form (Adam: 0 the one-quad-per-thread k_adam_al, 1 the
 * grid-stride k_adam; 0 elsewhere), the workgroup size, the number of workgroups of a launch
 * and the number of launches. Every grid stays below the 2^32 work-items of one dispatch: the
 * one-quad-per-thread kernels (fill, copy, same-shape ops) cover at most 2^31 quads per launch
 * and longer tensors take several launches; the unaligned fill and k_adam loop over their grid
 * (k_adam_al, which does not, only takes tensors its grid covers). MH_LAUNCH_ROWS16 counts rows,
 * not elements: the row-fused losses' forward and every row-fused backward over rows of at most
 * 32 classes run 64-row workgroups, several launches past one dispatch (none for zero rows). */
enum {
    MH_LAUNCH_FILL = 0,            /* mh_fill / mh_zero, 16-byte-aligned tensor */
    MH_LAUNCH_FILL_UNALIGNED = 1,  /* mh_fill / mh_zero, other tensors */
    MH_LAUNCH_COPY = 2,            /* mh_memcpy_d2d of n floats, 16-byte aligned */
    MH_LAUNCH_SAME_SHAPE = 3,      /* same-shape elementwise forward / backward, aligned */
    MH_LAUNCH_ADAM = 4,            /* mh_adam_step, all four tensors 16-byte aligned */
    MH_LAUNCH_ADAM_UNALIGNED = 5,  /* mh_adam_step, other tensors */
    MH_LAUNCH_ROWS16 = 6           /* row-fused one-shot kernels over n rows of <= 32 classes, aligned */
};
typedef struct {
    int32_t kernel;
    int32_t threads;
    int64_t blocks;
    int64_t launches;
} mh_launch_info;
int mh_plan_launch(int32_t what, int64_t n, mh_launch_info* out);

#ifdef __cplusplus
}
#endif
#endif
