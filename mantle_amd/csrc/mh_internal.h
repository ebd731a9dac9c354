// mh_internal.h -- host-side internals of libmantle_hip.so: context, error reporting,
// shape validation and the collapsed launch plans shared by the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstring>
#include <type_traits>
#include <vector>

#include "../../include/mantle_hip.h"

namespace mh {

// A float4 as a clang vector type: arrays and struct members of it stay in registers, where
// HIP's union float4 can be put in scratch memory.
typedef float vf4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------------------
struct Context {
    bool initialized = false;
    int device = -1;
    uint64_t flags = 0;
    hipStream_t stream = nullptr;
    void* scratch = nullptr;  // library-owned, grown on demand (two-pass reductions)
    size_t scratch_bytes = 0;
    void* stage = nullptr;  // library-owned staging for materialised intermediates
    size_t stage_bytes = 0;
    uint32_t* tickets = nullptr;  // zeroed arrival counters of single-launch reductions
    int64_t ntickets = 0;
    int num_cus = 256;
    // Captured HIP graphs hold the addresses of scratch, stage and tickets. While any exists,
    // a buffer that grows is retired (kept allocated) instead of freed, so that every graph
    // still points at live memory; retired buffers are freed when the last graph is
    // released, or at mh_shutdown.
    int64_t graphs_live = 0;
    std::vector<void*> retired;
    uint64_t epoch = 0;  // bumped by every mh_init: a graph replays only in its own epoch
};
Context& ctx();
// A captured graph that holds library buffer addresses comes into / goes out of existence;
// graph_release takes the epoch the graph was captured in (graphs of an earlier epoch no
// longer count: mh_shutdown freed what they pointed at).
void graph_retain();
int graph_release(uint64_t epoch);

// Error reporting: records a thread-local message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Checks the result of a HIP runtime call.
int hip_check(hipError_t e, const char* what);
// Failure injection for failure-path tests without a GPU fault: with MANTLE_HIP_FAIL_AT=<n>
// in the environment at mh_init, the n-th HIP call wrapped by MH_HIP after that init is not
// made and fails with MH_ERR_HIP instead, as if the runtime had refused it.
int hip_inject(const char* what);
#define MH_HIP(call)                                        \
    do {                                                    \
        int rc__ = ::mh::hip_inject(#call);                 \
        if (rc__ == MH_OK) rc__ = ::mh::hip_check((call), #call); \
        if (rc__ != MH_OK) return rc__;                     \
    } while (0)
#define MH_TRY(expr)                    \
    do {                                \
        int rc__ = (expr);              \
        if (rc__ != MH_OK) return rc__; \
    } while (0)

// Opt-in tracing: with MANTLE_HIP_TRACE=1 in the environment at mh_init, every entry point that
// queues GPU work opens a roctx range named after itself (and its op) for the duration of the
// call, so a `rocprofv3 --marker-trace` run shows each call around the kernels it launched.
// roctx is resolved with dlopen at mh_init; without the variable (or the library) the scopes
// test one null pointer and do nothing.
using RoctxPushFn = int (*)(const char*);
using RoctxPopFn = int (*)();
extern RoctxPushFn g_roctx_push;
extern RoctxPopFn g_roctx_pop;
void trace_init();
void trace_push_op(const char* fn, int op);  // pushes "fn(OPNAME)"
struct TraceScope {
    bool on;
    explicit TraceScope(const char* fn) : on(g_roctx_push != nullptr) {
        if (on) g_roctx_push(fn);
    }
    TraceScope(const char* fn, int op) : on(g_roctx_push != nullptr) {
        if (on) trace_push_op(fn, op);
    }
    ~TraceScope() {
        if (on) g_roctx_pop();
    }
    TraceScope(const TraceScope&) = delete;
    TraceScope& operator=(const TraceScope&) = delete;
};
#define MH_TRACE(fn) ::mh::TraceScope mh_trace_scope__(fn)
#define MH_TRACE_OP(fn, op) ::mh::TraceScope mh_trace_scope__(fn, op)

// Copies the shape argument `p<name>` (a const mh_shape* of the C ABI) into a local
// `name`, rejecting a null pointer.
#define MH_SHAPE_ARG(name)                                                                  \
    if (!p##name) return ::mh::fail(MH_ERR_NULL, "%s: null shape argument " #name, __func__); \
    const mh_shape name = *p##name

int require_init();
// End of an entry point: checks the launch and synchronises unless MH_INIT_ASYNC.
int finish(const char* what);
// Library scratch of at least `bytes` (synchronises before growing).
// A dispatch holds fewer than 2^32 work-items per grid dimension (the AQL packet's grid size
// is 32-bit), so a 1-D launch of `per_block`-thread workgroups has at most this many.
constexpr int64_t kMaxDispatchItems = ((int64_t)1 << 32) - 1;
constexpr int64_t max_grid_blocks(int per_block) { return kMaxDispatchItems / per_block; }
// Workgroups to give each of `items` a thread, clamped to what one dispatch holds; the
// kernels launched this way loop over the grid for what lies beyond.
inline int64_t grid_blocks(int64_t items, int per_block) {
    int64_t b = (items + per_block - 1) / per_block;
    if (b < 1) b = 1;
    return b > max_grid_blocks(per_block) ? max_grid_blocks(per_block) : b;
}

// The one-quad-per-thread kernels (no grid loop: at config-5 sizes a loop that runs once
// still cost 6 % of a row-broadcast op) cover at most this many quads per launch; a longer
// tensor runs as several launches over offset pointers.
constexpr int64_t kMaxLaunchQuads = (int64_t)1 << 31;
inline int64_t launch_count(int64_t nq) { return nq <= kMaxLaunchQuads ? 1 : (nq + kMaxLaunchQuads - 1) / kMaxLaunchQuads; }

// Launch shapes of the element-streaming entry points (what mh_plan_launch reports).
struct LaunchShape {
    int32_t kernel;    // entry-point specific form (Adam: 0 k_adam_al, 1 k_adam)
    int32_t threads;   // per workgroup
    int64_t blocks;    // workgroups of the (first) launch
    int64_t launches;  // launches over the tensor
};
LaunchShape fill_launch(int64_t n, bool aligned);
LaunchShape copy_launch(int64_t nquads);
LaunchShape elw_same_launch(int64_t n);
LaunchShape adam_launch(int64_t n, bool aligned);
LaunchShape row16_launch(int64_t rows);

int scratch(size_t bytes, void** out);
// A second library buffer for intermediates that live across calls using scratch().
int stage(size_t bytes, void** out);
// At least n zeroed arrival counters. A kernel that takes tickets leaves every one it
// touched at zero again when it ends (the last arrival resets it).
int tickets(int64_t n, uint32_t** out);
// The no-allocation scratch: a fixed device array of kNoAllocScratchBytes per GPU, shared by
// every call on that GPU (contents are whatever the last call left). `bytes` beyond the size
// fail with MH_ERR_OVERFLOW; the address is the current device's, resolved at mh_init.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
int noalloc_scratch(size_t bytes, float** out);

// ---------------------------------------------------------------------------------------
// shapes
// ---------------------------------------------------------------------------------------
int check_shape(const mh_shape& s, const char* name);
int64_t numel(const mh_shape& s);
bool shape_eq(const mh_shape& a, const mh_shape& b);
bool is_scalar_shape(const mh_shape& s);  // TensorShape(1)
int broadcast_shapes(const mh_shape& s1, const mh_shape& s2, mh_shape* out);
bool broadcasts_to(const mh_shape& small, const mh_shape& big);
void broadcast_strides(int size, const mh_shape& shape, int64_t* strides);
mh_shape reduced_shape(const mh_shape& s, int axis);  // get_reduce_shape; axis<0 -> (1)
mh_shape flat_shape(int64_t n);

// ---------------------------------------------------------------------------------------
// fast unsigned division by an invariant (Granlund & Montgomery, "Division by invariant
// integers using multiplication", PLDI 1994): q = (umulhi(n, mul) + n) >> shr, exact for
// all 32-bit n and 1 <= d < 2^31.
// ---------------------------------------------------------------------------------------
struct FastDiv {
    uint32_t d, mul, shr;
};
inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    f.shr = s;
    f.mul = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
    return f;
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    uint32_t t = __umulhi(n, f.mul);
    return (uint32_t)(((uint64_t)t + n) >> f.shr);
}

// ---------------------------------------------------------------------------------------
// elementwise launch plan: output shape collapsed (size-1 dims dropped, dims merged where
// every input is contiguous across the pair), one stride row per input.
// ---------------------------------------------------------------------------------------
constexpr int kMaxIn = 4;
enum InKind : int32_t { IN_FULL = 0, IN_SCALAR = 1, IN_BCAST = 2 };

struct ElwPlan {
    int64_t n = 0;   // output element count
    int32_t rank = 0;
    int32_t nin = 0;
    int32_t kind[kMaxIn] = {0, 0, 0, 0};
    int64_t dims[MH_MAX_RANK] = {};
    int64_t st[kMaxIn][MH_MAX_RANK] = {};
    FastDiv fd[MH_MAX_RANK] = {};
    int32_t vec_ok = 0;  // inner dim % 4 == 0 and each strided input has inner stride 0/1
    int32_t any_bcast = 0;
};
// Builds the plan for an output of shape `out` and inputs of the given shapes (each must
// broadcast to `out`).
int build_elw_plan(const mh_shape& out, int nin, const mh_shape* in, ElwPlan* plan);

// Streamed accesses. A full-size operand that a kernel reads once, or a result it writes once,
// goes through the non-temporal path (the nt bit of the vector load / store). On gfx950 a plain
// load of data that is not in the Infinity Cache allocates there and first writes back the
// dirty line it replaces, so reads behind other kernels' writes ran at 2.6 TB/s against 4.2 TB/s
// non-temporal (42 MB), and copies at 0.73 against 0.82 of peak (1 GiB); a non-temporal read of
// data still in the cache costs about 6 % more than a plain one. Small operands that many
// threads read again (a bias, a row's max, a column operand, split partials) stay plain.
__device__ __forceinline__ float4 ld_nt4(const float* p, int64_t q) {
    const vf4 v = __builtin_nontemporal_load(reinterpret_cast<const vf4*>(p) + q);
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ vf4 ld_ntv(const float* p, int64_t q) {
    return __builtin_nontemporal_load(reinterpret_cast<const vf4*>(p) + q);
}
__device__ __forceinline__ void st_nt4(float* p, int64_t q, float4 v) {
    const vf4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<vf4*>(p) + q);
}
__device__ __forceinline__ void st_ntv(float* p, int64_t q, vf4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<vf4*>(p) + q);
}
__device__ __forceinline__ float ld_nt(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_nt(float* p, float v) { __builtin_nontemporal_store(v, p); }

// Component j of a float4.
__device__ __forceinline__ float comp(const float4& q, int j) {
    return j == 0 ? q.x : (j == 1 ? q.y : (j == 2 ? q.z : q.w));
}

// True when some element of quad b differs in its bits from the same element of quad a, so
// that storing b over a changes memory. Sparse accumulations store only such quads: MAX
// backward adds +0 away from the line maxima, and x + 0 has the bits of x unless x is -0 (then
// +0) or a signalling NaN (then quieted), both of which this test catches.
__device__ __forceinline__ bool bits_differ4(float a0, float a1, float a2, float a3, float b0, float b1, float b2,
                                             float b3) {
    return ((__float_as_uint(a0) ^ __float_as_uint(b0)) | (__float_as_uint(a1) ^ __float_as_uint(b1)) |
            (__float_as_uint(a2) ^ __float_as_uint(b2)) | (__float_as_uint(a3) ^ __float_as_uint(b3))) != 0u;
}

// Offset type of the broadcast engine: 32-bit below 2^31 output elements (every operand is
// no larger than the output, so its offsets fit too).
template <bool BIG>
using off_type = typename std::conditional<BIG, int64_t, int32_t>::type;

// Offsets of the broadcast (IN_BCAST) operands at output element idx, the element's
// coordinate along the innermost collapsed dim (cin) and along the next outer dim (cprev, -1
// for a rank-1 plan). MAXR bounds the collapsed rank the loop covers (the caller guarantees
// pl.rank <= MAXR). BIG: 64-bit division (n >= 2^31).
template <int NIN, bool BIG, int MAXR>
__device__ __forceinline__ void bcast_decode(const ElwPlan& pl, int64_t idx, off_type<BIG>* off, int64_t* cin,
                                             int64_t* cprev) {
    using OT = off_type<BIG>;
    const int inner = pl.rank - 1;
#pragma unroll
    for (int k = 0; k < NIN; ++k) off[k] = 0;
    *cprev = -1;
    int64_t rem = idx;
    uint32_t rem32 = (uint32_t)idx;
#pragma unroll
    for (int d = MAXR - 1; d >= 0; --d) {
        if (d > inner) continue;
        int64_t c;
        if (BIG) {
            const int64_t q = rem / pl.dims[d];
            c = rem - q * pl.dims[d];
            rem = q;
        } else {
            const uint32_t q32 = fdiv(rem32, pl.fd[d]);
            c = (int64_t)(rem32 - q32 * pl.fd[d].d);
            rem32 = q32;
        }
        if (d == inner) *cin = c;
        if (d == inner - 1) *cprev = c;
#pragma unroll
        for (int k = 0; k < NIN; ++k)
            if (pl.kind[k] == IN_BCAST) off[k] += (OT)c * (OT)pl.st[k][d];
    }
}

// ---------------------------------------------------------------------------------------
// kernels (defined in mh_elementwise.hip / mh_reduce.hip)
// ---------------------------------------------------------------------------------------
// Reduction operator and epilogue ids shared by the reduce launchers.
// RED_MAXCNT_ARG: RED_MAXCNT whose split partials also hold the element index of each split's
// maximum (x of fewer than 2^32 elements).
enum RedOp : int { RED_SUM = 0, RED_MAX = 1, RED_MAXCNT = 2, RED_MAXCNT_ARG = 3 };
enum Epi : int {
    EPI_STORE = 0,     // out = v
    EPI_MEAN = 1,      // out = v / (float)len
    EPI_ACCUM = 2,     // out = out + v
    EPI_ACCUM_NEG = 3,  // out = out + (-v)
    EPI_SCALE = 5,      // out = v * div
    // out = ((out + x0) + x1) + ... (x negated for _NEG): a shape-aware gradient accumulation
    // walks the full-shape gradient serially, so each row's values add into the gradient one
    // at a time. Kernels with one thread per row do exactly that; the others add the finished
    // sum (EPI_ACCUM / EPI_ACCUM_NEG).
    EPI_SEQ_ACCUM = 6,
    EPI_SEQ_ACCUM_NEG = 7
};
// Reduce x viewed as [A, B, C] over B into out[A*C] (out2: fl(1/count) for RED_MAXCNT).
// `div` is the float divisor of EPI_MEAN; `tmp` holds split partials
// (reduce_abc_tmp_floats(op, A, B, C) floats, may be null when that is 0).
// `split`, when given, says where the first pass left its split partials in tmp (RED_MAXCNT:
// the maxima, then the counts; RED_MAXCNT_ARG: then the indices): S == 1 when there are none; C == 1 (rows): chunk s of line r
// (kRowChunk elements from r * B + s * span) at tmp[r * S + s]; columns: split s (rows
// [s * span, (s + 1) * span) of every line) at tmp[s * A * C + line].
struct RedSplit {
    int64_t S = 1, span = 0;
};
size_t reduce_abc_tmp_floats(int op, int64_t A, int64_t B, int64_t C);
int reduce_abc(int op, int epi, const float* x, int64_t A, int64_t B, int64_t C, float* out,
               float* out2, float div, float* tmp, RedSplit* split = nullptr);
// Sum over all n elements of the POW exponent-gradient term, accumulated into grad[0]; with
// grad_x, the x gradient of every element is accumulated into grad_x in the same pass.
int pow_exponent_grad(float* grad, const float* x, const float* exponent, const float* ug,
                      int64_t n, float* grad_x = nullptr);
// grad += un-broadcast(rg) (or += -un-broadcast(rg)): the chain of single-axis reductions.
size_t unbroadcast_scratch_floats(const mh_shape& sgrad, const mh_shape& srg);
int unbroadcast_accum_scratch(float* grad, const mh_shape& sgrad, const float* rg,
                              const mh_shape& srg, bool negate, float* tmp);
int plan_unbroadcast(const mh_shape& sgrad, const mh_shape& srg, mh_reduce_plan_info* info);
// The cross-entropy graph (loss.mojo:45-61) with its final scale given (the value of the
// graph scalar it multiplies by); mh_cross_entropy_* use f32(-1 / rows).
int cross_entropy_fwd_c(float* loss, const float* x, const float* tg, int64_t rows, int64_t K, float scale);
int cross_entropy_bwd_c(float* gx, const float* x, const float* tg, const float* ug, int64_t rows, int64_t K,
                        float scale);

// grad += un-broadcast(rg) of a broadcast MUL / DIV backward with rg computed inside the
// reduction (single-step plans whose per-element operand has the full shape); *done says
// whether it ran.
int unbroadcast_binrg(int op, int id, bool divs, float* grad, const mh_shape& sgrad, const float* ug,
                      const mh_shape& sug, const float* t1, const mh_shape& s1, const float* t2,
                      const mh_shape& s2, bool* done);

// Elementwise helpers used by the reduction and fused entry points.
int map_max_route(float* grad, const mh_shape& sx, const float* x, const mh_shape& sline,
                  const float* m, const float* f, const float* ug);
int map_scale_bcast(float* grad, const mh_shape& sx, const float* ug, const mh_shape& sug,
                    float c, bool twice);
int map_mean_all(float* grad, int64_t n, const float* ug, float c);
int map_accum_same(float* grad, const float* rg, int64_t n, bool scalar_rg);

}  // namespace mh
