// mh_softmax.hip -- row-fused forward and backward of the classifier-head graph
//
//   MAX(x, axis 1) -> SUB -> EXP -> SUM(axis 1) -> DIV -> LOG -> MUL(target) -> MEAN
//
// over x [rows, classes]: Mantle's Softmax (mantle/nn/activations.mojo:74-87) followed by LOG,
// MUL and MEAN (mantle/autograd/ops/basics.mojo:288-309, 94-129, 428-506). Op by op that is 8
// forward and 10 backward kernels and about 14 passes over [rows, classes]; here the forward
// reads x and target once and the backward reads x and target and updates grad_x once.
//
// Every per-element value is computed with the same expression, in the same order, as the
// op-by-op chain, and every gradient accumulation happens in Model.backward's node order
// (model.mojo:194-330), so grad_x is bit-identical to the ten backward_op calls starting from
// zeroed intermediate grads. Row sums run in element order (as both the reference's scalar
// tail loop and the op-by-op GPU path do for rows this short). Only the final MEAN over all
// elements sums in another order (the rtol class).
//
// One thread owns one row, held in registers (loops unrolled to 8, 16 or 32 classes); a block
// of 256 threads stages RB rows (256, fewer when wide rows would exceed 64 KB of LDS) of each
// operand in LDS with coalesced loads (rows of up to 32 classes).
#include <cfloat>

#include "mh_internal.h"
#include "mh_math.h"

namespace mh {

constexpr int kSThreads = 256;
constexpr int kSMaxClasses = 32;
constexpr int64_t kSLdsFloats = 16384;  // 64 KB of tiles per block

// Rows per block: 256, halved until `tiles` tiles of rb * K floats fit the LDS budget.
static inline int rows_per_block(int tiles, int64_t K) {
    int rb = kSThreads;
    while (rb > 64 && (int64_t)tiles * rb * K > kSLdsFloats) rb >>= 1;
    return rb;
}

// Copies rows [r0, r0 + rows) of a [*, K] array into LDS (16-byte aligned source: float4).
__device__ __forceinline__ void stage_tile(float* dst, const float* __restrict__ src, int64_t base, int cnt,
                                           bool al) {
    const int t = threadIdx.x;
    int done = 0;
    if (al) {
        const int nq = cnt >> 2;
        const float4* s4 = reinterpret_cast<const float4*>(src + base);
        for (int i = t; i < nq; i += kSThreads) reinterpret_cast<float4*>(dst)[i] = s4[i];
        done = nq << 2;
    }
    for (int i = done + t; i < cnt; i += kSThreads) dst[i] = src[base + i];
}

__device__ __forceinline__ float block_sum_rows(float v, float* ws) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

// Forward: part[block] = sum over the block's rows of sum_j log(softmax(x)_j) * target_j.
// The row lives in registers (KM >= K: loops unrolled, elements j >= K skipped); LDS only
// stages the coalesced loads.
template <int KM>
__global__ void __launch_bounds__(kSThreads)
    k_smlm_fwd(const float* __restrict__ x, const float* __restrict__ tg, int64_t rows, int K, int rb, bool al,
               float* __restrict__ part) {
    extern __shared__ float4 smem4[];
    __shared__ float ws[4];
    float* xs = reinterpret_cast<float*>(smem4);
    float* ts = xs + rb * K;
    const int64_t r0 = (int64_t)blockIdx.x * rb;
    const int nr = (int)((rows - r0) < rb ? (rows - r0) : rb);
    const int64_t base = r0 * K;
    stage_tile(xs, x, base, nr * K, al);
    stage_tile(ts, tg, base, nr * K, al);
    __syncthreads();
    float rowsum = 0.0f;
    const int t = threadIdx.x;
    if (t < nr) {
        float xr[KM], e[KM];
#pragma unroll
        for (int j = 0; j < KM; ++j) xr[j] = j < K ? xs[t * K + j] : 0.0f;
        float m = -FLT_MAX;  // MAX.forward: reduce with max_simd from min_finite
#pragma unroll
        for (int j = 0; j < KM; ++j)
            if (j < K) m = m > xr[j] ? m : xr[j];
        float s = 0.0f;  // SUM.forward over the row, in element order
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                e[j] = mexp(xr[j] - m);  // SUB.forward, EXP.forward
                s = s + e[j];
            }
        }
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float sm = e[j] / s;                 // DIV.forward
                const float lp = mlog(sm);                 // LOG.forward
                rowsum = rowsum + lp * ts[t * K + j];      // MUL.forward, then the MEAN's sum
            }
        }
    }
    const float tot = block_sum_rows(rowsum, ws);
    if (t == 0) part[blockIdx.x] = tot;
}

// Backward from ug = d loss (shape (1)), accumulated into grad_x:
//   MEAN  : g_t   = 0 + f32(1/f64(N)) * ug
//   MUL   : g_lp  = 0 + g_t * target                      (target not trainable)
//   LOG   : g_sm  = 0 + g_lp / sm
//   DIV 0 : g_e   = 0 + g_sm / s
//   DIV 1 : g_s   = 0 + sum_j ((-e_j) / (s * s)) * g_sm_j
//   SUM   : g_e   = g_e + 1 * g_s   ((1 * g_s) * g_s for one class: see below)
//   EXP   : g_xm  = 0 + exp(xm) * g_e
//   SUB 0 : grad_x = grad_x + g_xm
//   SUB 1 : g_max = 0 + (-sum_j g_xm_j)
//   MAX   : grad_x = grad_x + (x == m ? fl(1/count) * g_max : 0)
// Registers hold the row (KM >= K); LDS stages x, target and grad_x (written back in place).
template <int KM>
__global__ void __launch_bounds__(kSThreads)
    k_smlm_bwd(float* __restrict__ g, const float* __restrict__ x, const float* __restrict__ tg,
               const float* __restrict__ ug, int64_t rows, int K, int rb, bool al, float cmean) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    float* ts = xs + rb * K;
    float* gs = ts + rb * K;
    const int64_t r0 = (int64_t)blockIdx.x * rb;
    const int nr = (int)((rows - r0) < rb ? (rows - r0) : rb);
    const int64_t base = r0 * K;
    const int cnt = nr * K;
    stage_tile(xs, x, base, cnt, al);
    stage_tile(ts, tg, base, cnt, al);
    stage_tile(gs, g, base, cnt, al);
    __syncthreads();
    const int t = threadIdx.x;
    if (t < nr) {
        float xr[KM], e[KM], w[KM];
#pragma unroll
        for (int j = 0; j < KM; ++j) xr[j] = j < K ? xs[t * K + j] : 0.0f;
        // forward values: the row max as MAX.forward takes it (max_simd from min_finite),
        // e = exp(x - m), s = sum e; and, as MAX.backward recomputes it, the max with its
        // count (an element that is neither above nor below the running max -- equal, or
        // NaN -- adds to the count)
        float m = -FLT_MAX, mb = -FLT_MAX;
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float v = xr[j];
                m = m > v ? m : v;
                if (mb > v) {
                } else if (v > mb) {
                    mb = v;
                    c = 1;
                } else {
                    c += 1;
                }
            }
        }
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                e[j] = mexp(xr[j] - m);
                s = s + e[j];
            }
        }
        const float gt = 0.0f + cmean * ug[0];  // MEAN backward (all elements)
        const float s2 = s * s;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float sm = e[j] / s;
                const float glp = 0.0f + gt * ts[t * K + j];  // MUL backward, operand 0
                const float gsm = 0.0f + glp / sm;            // LOG backward
                w[j] = 0.0f + gsm / s;                        // DIV backward, operand 0: g_e
                acc = acc + ((-e[j]) / s2) * gsm;             // DIV backward, operand 1
            }
        }
        const float gS = 0.0f + acc;
        // SUM backward: rg = 1 * g_s, except over a size-1 axis (K == 1), where the reduced
        // shape equals the input shape and accumulate_op applies the multiply twice
        // (tensorutils.mojo:380-393): rg = (1 * g_s) * g_s
        const float rgs = K == 1 ? (1.0f * gS) * gS : 1.0f * gS;
        float acc2 = 0.0f;
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float ge = w[j] + rgs;  // SUM backward
                w[j] = 0.0f + e[j] * ge;      // EXP backward: g_xm
                acc2 = acc2 + w[j];
            }
        }
        const float gmax = 0.0f + (-acc2);          // SUB backward, operand 1
        const float sg = (1.0f / (float)c) * gmax;  // MAX backward factor
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float a = gs[t * K + j] + w[j];           // SUB backward, operand 0
                gs[t * K + j] = a + (xr[j] == mb ? sg : 0.0f);  // MAX backward
            }
        }
    }
    __syncthreads();
    // write the grad tile back
    if (al) {
        const int nq = cnt >> 2;
        float4* g4 = reinterpret_cast<float4*>(g + base);
        for (int i = t; i < nq; i += kSThreads) g4[i] = reinterpret_cast<const float4*>(gs)[i];
        for (int i = (nq << 2) + t; i < cnt; i += kSThreads) g[base + i] = gs[i];
    } else {
        for (int i = t; i < cnt; i += kSThreads) g[base + i] = gs[i];
    }
}

static int check_smlm(const char* what, const float* x, const float* tg, int64_t rows, int64_t classes) {
    if (rows < 0 || classes < 0) return fail(MH_ERR_INVALID, "%s: negative size", what);
    if (classes > kSMaxClasses)
        return fail(MH_ERR_INVALID, "%s: %lld classes; the fused kernels take rows of at most %d (use the op-by-op path)",
                    what, (long long)classes, kSMaxClasses);
    if (rows > 0 && classes > 0 && (!x || !tg)) return fail(MH_ERR_NULL, "%s: null tensor", what);
    if ((double)rows * (double)classes > 9.0e15) return fail(MH_ERR_OVERFLOW, "%s: size overflow", what);
    return MH_OK;
}

static inline bool al16s(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace mh

using namespace mh;

extern "C" {

int mh_softmax_log_mul_mean_fwd(float* loss, const float* x, const float* target, int64_t rows, int64_t classes) {
    MH_TRY(check_smlm("mh_softmax_log_mul_mean_fwd", x, target, rows, classes));
    if (!loss) return fail(MH_ERR_NULL, "mh_softmax_log_mul_mean_fwd: null loss");
    MH_TRY(require_init());
    const int64_t n = rows * classes;
    if (n == 0) return mh_fill(loss, __builtin_nanf(""), 1);  // the mean of no elements: 0 / 0
    const int rb = rows_per_block(2, classes);
    const int64_t nblocks = (rows + rb - 1) / rb;
    if (nblocks > 0x7fffffff) return fail(MH_ERR_OVERFLOW, "mh_softmax_log_mul_mean_fwd: too many rows");
    const size_t np = ((size_t)nblocks + 63) & ~(size_t)63;
    const size_t t = reduce_abc_tmp_floats(RED_SUM, 1, nblocks, 1);
    float* part = nullptr;
    MH_TRY(scratch((np + t + 64) * sizeof(float), reinterpret_cast<void**>(&part)));
    const bool al = al16s(x) && al16s(target);
    const size_t lds = 2 * (size_t)rb * (size_t)classes * sizeof(float);
    dim3 g((unsigned)nblocks), b(kSThreads);
    hipStream_t st = ctx().stream;
    if (classes <= 8) hipLaunchKernelGGL(k_smlm_fwd<8>, g, b, lds, st, x, target, rows, (int)classes, rb, al, part);
    else if (classes <= 16) hipLaunchKernelGGL(k_smlm_fwd<16>, g, b, lds, st, x, target, rows, (int)classes, rb, al, part);
    else hipLaunchKernelGGL(k_smlm_fwd<32>, g, b, lds, st, x, target, rows, (int)classes, rb, al, part);
    // MEAN.forward: the sum of every element divided by f32(N)
    MH_TRY(reduce_abc(RED_SUM, EPI_MEAN, part, 1, nblocks, 1, loss, nullptr, (float)n, part + np));
    return finish("mh_softmax_log_mul_mean_fwd");
}

int mh_softmax_log_mul_mean_bwd_accum(float* grad_x, const float* x, const float* target, const float* ug,
                                      int64_t rows, int64_t classes) {
    MH_TRY(check_smlm("mh_softmax_log_mul_mean_bwd_accum", x, target, rows, classes));
    const int64_t n = rows * classes;
    if (n == 0) return MH_OK;
    if (!grad_x || !ug) return fail(MH_ERR_NULL, "mh_softmax_log_mul_mean_bwd_accum: null tensor");
    MH_TRY(require_init());
    const int rb = rows_per_block(3, classes);
    const int64_t nblocks = (rows + rb - 1) / rb;
    if (nblocks > 0x7fffffff) return fail(MH_ERR_OVERFLOW, "mh_softmax_log_mul_mean_bwd_accum: too many rows");
    const bool al = al16s(x) && al16s(target) && al16s(grad_x);
    const size_t lds = 3 * (size_t)rb * (size_t)classes * sizeof(float);
    const float cmean = (float)(1.0 / (double)n);  // MEAN.backward, basics.mojo:470-487
    dim3 g((unsigned)nblocks), b(kSThreads);
    hipStream_t st = ctx().stream;
    if (classes <= 8)
        hipLaunchKernelGGL(k_smlm_bwd<8>, g, b, lds, st, grad_x, x, target, ug, rows, (int)classes, rb, al, cmean);
    else if (classes <= 16)
        hipLaunchKernelGGL(k_smlm_bwd<16>, g, b, lds, st, grad_x, x, target, ug, rows, (int)classes, rb, al, cmean);
    else
        hipLaunchKernelGGL(k_smlm_bwd<32>, g, b, lds, st, grad_x, x, target, ug, rows, (int)classes, rb, al, cmean);
    return finish("mh_softmax_log_mul_mean_bwd_accum");
}

}  // extern "C"
