// mh_softmax.hip -- row-fused forward and backward of Mantle's row graphs over the last axis
// of x [rows, classes]:
//
//   Softmax      (mantle/nn/activations.mojo:74-87)
//                MAX(axis) -> SUB -> EXP -> SUM(axis) -> DIV                    -> out
//   LogSoftmax   (activations.mojo:94-108)
//                MAX(axis) -> SUB -> EXP -> SUM(axis) -> LOG -> SUB(xm, ls)     -> out
//   CrossEntropyLoss (mantle/nn/loss.mojo:45-61)
//                LogSoftmax -> MUL(target, .) -> SUM -> MUL(., f32(-1 / rows))  -> loss
//   the config-5 head
//                Softmax -> LOG -> MUL(., target) -> MEAN                       -> loss
//
// Op by op each graph is 5-9 forward and 7-10 backward kernels and 8-14 passes over
// [rows, classes]; fused, the forward reads x (and the target) once and the backward reads
// x, the target or upstream gradient, and updates grad_x once.
//
// Every per-element value uses the same expression, in the same order, as the op-by-op
// chain, every gradient accumulates in Model.backward's node order (model.mojo:194-330), and
// every row sum runs in the order the library's own row reductions use for that row length,
// so grad_x (and the Softmax / LogSoftmax outputs) are bit-identical to the op-by-op
// backward_op calls starting from zeroed intermediate gradients, for finite inputs. The row
// reductions' orders:
//   classes <= 64    element order from +0 (k_rows_lds / k_rows_thread): one thread per row,
//                    the row in registers, LDS staging of coalesced loads; or (17-64
//                    classes) P lanes per row carrying each running value across in order;
//   64 < classes < 2048
//                    k_rows_wave's order (per lane, quads lane + 64 q accumulated in groups
//                    of four, the tail into the first group, the sixteen partials summed in
//                    order, then an xor butterfly; lane-strided elements when classes is not
//                    a multiple of 4): one wavefront per row, the row across its lanes.
// Only the all-element sum of a loss graph (MEAN or SUM) runs in another order (the rtol
// class).
//
// Backward, per element, in node order (0 + v is an accumulation into a zeroed gradient):
//   Softmax    g_sm given                       | head graph: g_t = 0 + c * ug; g_lp = 0 + g_t * t;
//                                               |             g_sm = 0 + g_lp / sm
//              DIV 0: g_e = 0 + g_sm / s;  DIV 1: g_s = 0 + sum((-e) / (s * s) * g_sm)
//   LogSoftmax g_lsm given                      | cross entropy: g_ret = 0 + ug * c;
//                                               |   g_tl = 0 + 1 * g_ret; g_lsm = 0 + g_tl * t
//              SUB 0: g_xm = 0 + g_lsm;  SUB 1: g_ls = 0 + (-sum(g_lsm));  LOG: g_s = 0 + g_ls / s
//   then       SUM: rg = 1 * g_s ((1 * g_s) * g_s over one class, tensorutils.mojo:380-393)
//              EXP: g_xm = g_xm + e * (g_e + rg)
//              SUB(x, max): grad_x += g_xm;  g_max = 0 + (-sum(g_xm))
//              MAX: grad_x += (x == max ? fl(1 / count) * g_max : 0)
#include <cfloat>
#include <unordered_map>

#include "mh_internal.h"
#include "mh_math.h"

namespace mh {

enum RowGraph : int { G_SMLM = 0, G_CE = 1, G_SOFTMAX = 2, G_LOGSOFTMAX = 3 };

constexpr int kSThreads = 256;
constexpr int kSThreadMax = 64;         // rows up to this length: one thread per row
constexpr int kSWaveMax = 2047;         // longer rows (up to this): one wavefront per row
constexpr int kSLaneElems = 32;         // per-lane slots of the wavefront engine (64 * 32 > 2047)
constexpr int64_t kSLdsFloats = 16384;  // 64 KB of tiles per block

// Graphs whose backward starts from g_sm (DIV) rather than g_lsm (SUB).
template <int V>
constexpr bool from_softmax() {
    return V == G_SMLM || V == G_SOFTMAX;
}

__device__ __forceinline__ float max_simd(float a, float b) { return a > b ? a : b; }

// One element v into a row's running (maximum, count) from (-FLT_MAX, 0): a larger v starts
// a new count, an equal one adds to it, a smaller one or a NaN changes nothing. Selects over
// the comparisons: the if / else-if chain this replaces compiled to a branch per element.
__device__ __forceinline__ void max_count_add(float& mb, uint32_t& cnt, float v) {
    const bool gt = v > mb, eq = v == mb;
    cnt = gt ? 1u : (eq ? cnt + 1u : cnt);
    mb = gt ? v : mb;
}

// Two (maximum, count) pairs whose maxima are not NaN: the larger maximum with its count,
// equal maxima with both counts.
__device__ __forceinline__ void max_count_merge(float& mb, uint32_t& cnt, float om, uint32_t oc) {
    const bool gt = om > mb, eq = om == mb;
    cnt = gt ? oc : (eq ? cnt + oc : cnt);
    mb = gt ? om : mb;
}


// Rows per block of the thread engine: 256, halved until `tiles` tiles of rb * K floats fit.
static inline int rows_per_block(int tiles, int64_t K) {
    int rb = kSThreads;
    while (rb > 32 && (int64_t)tiles * rb * K > kSLdsFloats) rb >>= 1;
    return rb;
}

// Copies `cnt` floats from src + base into LDS (16-byte aligned source: float4), and back.
// Loads go out four per thread before their LDS stores, so a thread waits for memory once per
// four quads rather than once per quad.
__device__ __forceinline__ void stage_tile(float* dst, const float* __restrict__ src, int64_t base, int cnt,
                                           bool al) {
    const int t = threadIdx.x;
    int done = 0;
    if (al) {
        const int nq = cnt >> 2;
        float4* d4 = reinterpret_cast<float4*>(dst);
        int i = t;
        for (; i + 3 * kSThreads < nq; i += 4 * kSThreads) {
            float4 q[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) q[u] = ld_nt4(src + base, i + u * kSThreads);
#pragma unroll
            for (int u = 0; u < 4; ++u) d4[i + u * kSThreads] = q[u];
        }
        for (; i < nq; i += kSThreads) d4[i] = ld_nt4(src + base, i);
        done = nq << 2;
    }
    int i = done + t;
    for (; i + 3 * kSThreads < cnt; i += 4 * kSThreads) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = ld_nt(src + base + i + u * kSThreads);
#pragma unroll
        for (int u = 0; u < 4; ++u) dst[i + u * kSThreads] = v[u];
    }
    for (; i < cnt; i += kSThreads) dst[i] = ld_nt(src + base + i);
}

__device__ __forceinline__ void unstage_tile(float* __restrict__ dst, const float* src, int64_t base, int cnt,
                                             bool al) {
    const int t = threadIdx.x;
    int done = 0;
    if (al) {
        const int nq = cnt >> 2;
        for (int i = t; i < nq; i += kSThreads) st_nt4(dst + base, i, reinterpret_cast<const float4*>(src)[i]);
        done = nq << 2;
    }
    for (int i = done + t; i < cnt; i += kSThreads) st_nt(dst + base + i, src[i]);
}

// The same with each row of K floats at a stride of K + 1 in LDS (K a multiple of 4, so no quad
// straddles two rows; fk divides by K): the thread engine reads row t at t * (K + 1), and with K
// a multiple of 8 the rows at stride K put a wavefront's reads on a few LDS banks (at 32
// classes all on one).
__device__ __forceinline__ void stage_tile_pad(float* dst, const float* __restrict__ src, int64_t base, int cnt,
                                               FastDiv fk) {
    const int t = threadIdx.x;
    const int nq = cnt >> 2;
    int i = t;
    for (; i + 3 * kSThreads < nq; i += 4 * kSThreads) {
        float4 q[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) q[u] = ld_nt4(src + base, i + u * kSThreads);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t e = 4u * (uint32_t)(i + u * kSThreads);
            float* d = dst + e + fdiv(e, fk);
            d[0] = q[u].x; d[1] = q[u].y; d[2] = q[u].z; d[3] = q[u].w;
        }
    }
    for (; i < nq; i += kSThreads) {
        const float4 q = ld_nt4(src + base, i);
        const uint32_t e = 4u * (uint32_t)i;
        float* d = dst + e + fdiv(e, fk);
        d[0] = q.x; d[1] = q.y; d[2] = q.z; d[3] = q.w;
    }
}

__device__ __forceinline__ void unstage_tile_pad(float* __restrict__ dst, const float* src, int64_t base, int cnt,
                                                 FastDiv fk) {
    const int t = threadIdx.x;
    const int nq = cnt >> 2;
    for (int i = t; i < nq; i += kSThreads) {
        const uint32_t e = 4u * (uint32_t)i;
        const float* s4 = src + e + fdiv(e, fk);
        st_nt4(dst + base, i, make_float4(s4[0], s4[1], s4[2], s4[3]));
    }
}

__device__ __forceinline__ float block_sum(float v, float* ws) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

// The upstream gradient of the row part, per element: g_sm (from_softmax) or g_lsm.
template <int V>
__device__ __forceinline__ float upstream(float u, float e, float s, float gconst) {
    if constexpr (V == G_SMLM) {
        const float glp = 0.0f + gconst * u;  // MUL backward, operand 0 (gconst = g_t)
        return 0.0f + glp / (e / s);          // LOG backward
    } else if constexpr (V == G_CE) {
        return 0.0f + gconst * u;  // MUL(target, .) backward, operand 1 (gconst = g_tl)
    } else {
        return u;
    }
}

// The head graph's zero-target shortcut. An element whose target is +-0 adds
// log(e / s) * 0 = +-0 to the loss sum, and in the backward gets g_sm = 0 + (0 + g_t * 0) / (e / s)
// = +0, so g_e = 0 + g_sm / s = +0 and its DIV-1 term ((-e) / (s * s)) * g_sm = -0, whenever g_t is
// finite and e / s is a positive finite number: e >= 2^-100 guarantees that, as s lies in
// [1, classes]. A sum that starts at +0 never becomes -0 and is unchanged by adding a zero, so
// skipping such an element's divisions and log changes no bit of any result; every other
// element (a nonzero target, e below the bound, NaN) takes the full expression.
constexpr float kSkipMinE = 0x1p-100f;

__device__ __forceinline__ bool smlm_skip(float t, float e) { return t == 0.0f && e >= kSkipMinE; }

// Thread engines, head-graph forward of one row (x and target slots xr / tr in LDS): adds
// log(e_j / s) * t_j to acc in element order over the elements the shortcut keeps. They are
// listed first, so that a wavefront evaluates the log once per kept element of its busiest
// lane rather than once per class; e_j is recomputed from x (the same bits as e[j]).
template <int KM>
__device__ __forceinline__ float smlm_fwd_row(float acc, const float* xr, const float* tr, const float (&e)[KM],
                                              float m, float s, int K) {
    uint64_t need = 0;
#pragma unroll
    for (int j = 0; j < KM; ++j)
        if (j < K && !smlm_skip(tr[j], e[j])) need |= 1ull << j;
    while (need != 0) {
        const int j = __builtin_ctzll(need);
        need &= need - 1;
        acc = acc + mlog(mexp(xr[j] - m) / s) * tr[j];  // DIV, LOG, MUL, the MEAN's sum
    }
    return acc;
}

// Thread engines, head-graph backward of one row up to the DIV-1 row sum, which it returns:
// pre[j] = g_e of every element (+0 where the shortcut skips). The target slots ur are
// overwritten with g_e of the kept elements. skip_ok: g_t is finite.
template <int KM>
__device__ __forceinline__ float smlm_bwd_row(float (&pre)[KM], const float* xr, float* ur, const float (&e)[KM],
                                              float m, float s, float gconst, bool skip_ok, int K) {
    const float s2 = s * s;
    uint64_t need = 0;
#pragma unroll
    for (int j = 0; j < KM; ++j)
        if (j < K && !(skip_ok && smlm_skip(ur[j], e[j]))) need |= 1ull << j;
    float acc = 0.0f;
    for (uint64_t nd = need; nd != 0; nd &= nd - 1) {
        const int j = __builtin_ctzll(nd);
        const float ej = mexp(xr[j] - m);
        const float gsm = upstream<G_SMLM>(ur[j], ej, s, gconst);
        ur[j] = 0.0f + gsm / s;
        acc = acc + ((-ej) / s2) * gsm;
    }
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        float p = 0.0f;
        if (j < K && ((need >> j) & 1)) p = ur[j];
        pre[j] = p;
    }
    return acc;
}

// One row of a row graph's forward from LDS (x row xrow, target row trow, K elements, K <= KM):
// MAX, SUB, EXP, SUM over the row, then the loss graphs add the row's terms to rowsum (and
// return it) and Softmax / LogSoftmax overwrite the x row with the output row.
template <int V, int KM>
__device__ __forceinline__ float row_fwd(float* xrow, const float* trow, float rowsum, int K) {
    float xr[KM], e[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) xr[j] = j < K ? xrow[j] : 0.0f;
    float m = -FLT_MAX;  // MAX.forward: max_simd from min_finite, element order
#pragma unroll
    for (int j = 0; j < KM; ++j)
        if (j < K) m = max_simd(m, xr[j]);
    float s = 0.0f;  // SUB, EXP, SUM.forward
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        if (j < K) {
            e[j] = mexp(xr[j] - m);
            s = s + e[j];
        }
    }
    const float ls = (V == G_CE || V == G_LOGSOFTMAX) ? mlog(s) : 0.0f;  // LOG.forward of the sum
    if constexpr (V == G_SMLM) rowsum = smlm_fwd_row<KM>(rowsum, xrow, trow, e, m, s, K);
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        if (V != G_SMLM && j < K) {
            if constexpr (V == G_CE) {
                rowsum = rowsum + trow[j] * ((xr[j] - m) - ls);  // SUB(xm, ls), MUL(target, .)
            } else if constexpr (V == G_SOFTMAX) {
                xrow[j] = e[j] / s;  // DIV.forward
            } else {
                xrow[j] = (xr[j] - m) - ls;  // SUB(xm, ls).forward
            }
        }
    }
    return rowsum;
}

// ---------------------------------------------------------------------------------------
// thread engine: rows of at most KM (<= 64) elements, element-order row sums
// ---------------------------------------------------------------------------------------
// Forward. Loss graphs write a block partial of the all-element sum; Softmax / LogSoftmax
// write the output tile (through LDS, coalesced).
template <int V, int KM>
__global__ void __launch_bounds__(kSThreads)
    k_rowt_fwd(const float* __restrict__ x, const float* __restrict__ tg, float* __restrict__ out, int64_t rows,
               int K, int rb, bool al, float* __restrict__ part, int Kp, FastDiv fk) {
    // Kp: the LDS row stride, K or (padded, aligned operands, K a multiple of 8) K + 1
    extern __shared__ float4 smem4[];
    __shared__ float ws[4];
    constexpr bool LOSS = V == G_SMLM || V == G_CE;
    const bool pad = Kp != K;
    float* xs = reinterpret_cast<float*>(smem4);
    float* ts = xs + rb * Kp;
    const int64_t r0 = (int64_t)blockIdx.x * rb;
    const int nr = (int)((rows - r0) < rb ? (rows - r0) : rb);
    const int64_t base = r0 * K;
    if (pad) {
        stage_tile_pad(xs, x, base, nr * K, fk);
        if (LOSS) stage_tile_pad(ts, tg, base, nr * K, fk);
    } else {
        stage_tile(xs, x, base, nr * K, al);
        if (LOSS) stage_tile(ts, tg, base, nr * K, al);
    }
    __syncthreads();
    float rowsum = 0.0f;
    const int t = threadIdx.x;
    if (t < nr) rowsum = row_fwd<V, KM>(xs + t * Kp, ts + t * Kp, rowsum, K);
    if constexpr (LOSS) {
        const float tot = block_sum(rowsum, ws);
        if (t == 0) part[blockIdx.x] = tot;
    } else {
        __syncthreads();
        if (pad) unstage_tile_pad(out, xs, base, nr * K, fk);
        else unstage_tile(out, xs, base, nr * K, al);
    }
}

// Backward, accumulated into grad_x. `up` is the target (loss graphs) or the upstream
// gradient of the output (Softmax / LogSoftmax); `ug` the loss gradient (shape (1)); `c` the
// graph constant: f32(1 / f64(rows * classes)) for the MEAN, f32(-1 / f64(rows)) for the
// cross-entropy scale.
template <int V, int KM>
__global__ void __launch_bounds__(kSThreads)
    k_rowt_bwd(float* __restrict__ g, const float* __restrict__ x, const float* __restrict__ up,
               const float* __restrict__ ug, int64_t rows, int K, int rb, bool al, float c) {
    extern __shared__ float4 smem4[];
    float* xs = reinterpret_cast<float*>(smem4);
    float* us = xs + rb * K;
    float* gs = us + rb * K;
    const int64_t r0 = (int64_t)blockIdx.x * rb;
    const int nr = (int)((rows - r0) < rb ? (rows - r0) : rb);
    const int64_t base = r0 * K;
    const int cnt = nr * K;
    stage_tile(xs, x, base, cnt, al);
    stage_tile(us, up, base, cnt, al);
    stage_tile(gs, g, base, cnt, al);
    __syncthreads();
    const int t = threadIdx.x;
    if (t < nr) {
        float xr[KM], e[KM], pre[KM];
#pragma unroll
        for (int j = 0; j < KM; ++j) xr[j] = j < K ? xs[t * K + j] : 0.0f;
        // the forward row max (MAX.forward) and, as MAX.backward recomputes it, the max with
        // its count (an element neither above nor below the running max adds to the count)
        float m = -FLT_MAX, mb = -FLT_MAX;
        uint32_t cntm = 0;
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float v = xr[j];
                m = max_simd(m, v);
                max_count_add(mb, cntm, v);  // a NaN element is not counted
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
        const float gconst = V == G_SMLM ? 0.0f + c * ug[0]                       // MEAN backward
                             : V == G_CE ? 0.0f + 1.0f * (0.0f + ug[0] * c)       // MUL(., c), SUM backward
                                         : 0.0f;
        // pre: g_e after DIV (from_softmax), or g_xm after SUB(xm, ls)
        float acc = 0.0f, gS;
        if constexpr (V == G_SMLM) {
            const bool skip_ok = gconst - gconst == 0.0f;
            gS = 0.0f + smlm_bwd_row<KM>(pre, xs + t * K, us + t * K, e, m, s, gconst, skip_ok, K);
        } else if constexpr (from_softmax<V>()) {
            const float s2 = s * s;
#pragma unroll
            for (int j = 0; j < KM; ++j) {
                if (j < K) {
                    const float gsm = upstream<V>(us[t * K + j], e[j], s, gconst);
                    pre[j] = 0.0f + gsm / s;
                    acc = acc + ((-e[j]) / s2) * gsm;
                }
            }
            gS = 0.0f + acc;
        } else {
#pragma unroll
            for (int j = 0; j < KM; ++j) {
                if (j < K) {
                    const float glsm = upstream<V>(us[t * K + j], e[j], s, gconst);
                    pre[j] = 0.0f + glsm;
                    acc = acc + glsm;
                }
            }
            gS = 0.0f + (0.0f + (-acc)) / s;
        }
        const float rgs = K == 1 ? (1.0f * gS) * gS : 1.0f * gS;
        float acc2 = 0.0f;
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                if constexpr (from_softmax<V>()) pre[j] = 0.0f + e[j] * (pre[j] + rgs);
                else pre[j] = pre[j] + e[j] * (0.0f + rgs);
                acc2 = acc2 + pre[j];
            }
        }
        const float sg = (1.0f / (float)cntm) * (0.0f + (-acc2));  // SUB 1, then the MAX factor
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float a = gs[t * K + j] + pre[j];
                gs[t * K + j] = a + (xr[j] == mb ? sg : 0.0f);
            }
        }
    }
    __syncthreads();
    unstage_tile(g, gs, base, cnt, al);
}

// ---------------------------------------------------------------------------------------
// pipelined thread engine: Softmax / LogSoftmax forward over rows of at most 16 classes,
// 16-byte aligned operands
// ---------------------------------------------------------------------------------------
// A persistent grid walks 256-row tiles; while a block computes tile i from LDS, the loads of
// its next tile are already in flight into registers, so the chip never alternates between
// a whole-grid load phase and a whole-grid compute phase. A tile is at most 4096 floats (four
// float4 per thread per operand); rows are computed exactly as in k_rowt_fwd / k_rowt_bwd.
// Each class count 1..16 has its own kernel (KM = K at compile time: every loop over a row
// unrolled without per-class guards), 5-6 % faster at 10 classes than one kernel for all
// counts up to 16. Only the Softmax and LogSoftmax forward run here: at [2^20, 10] it took
// 16.0-18.8 us against 16.2-20.3 us for the one-shot engine (which writes each 64-row block's
// output as its last step), box to box; the loss graphs and every backward run one-shot.
constexpr int kPQ = 4;  // float4 per thread per operand tile (q0..q3 below)

// Four float4 of one operand tile per thread, as named registers (an array here ends up in
// scratch memory).
struct TileRegs {
    vf4 q0, q1, q2, q3;
    float tail;
};

// Loads tile floats [0, cnt) at src + base into registers: quad i of the tile goes to thread
// i % 256, slot i / 256; the cnt % 4 tail floats to threads 0..2.
__device__ __forceinline__ void tile_load(TileRegs& r, const float* __restrict__ src, int64_t base, int cnt) {
    const int t = threadIdx.x;
    const int nq = cnt >> 2;
    const float* sb = src + base;
    if (t < nq) r.q0 = ld_ntv(sb, t);
    if (t + kSThreads < nq) r.q1 = ld_ntv(sb, t + kSThreads);
    if (t + 2 * kSThreads < nq) r.q2 = ld_ntv(sb, t + 2 * kSThreads);
    if (t + 3 * kSThreads < nq) r.q3 = ld_ntv(sb, t + 3 * kSThreads);
    const int tl = (nq << 2) + t;
    if (t < 4 && tl < cnt) r.tail = ld_nt(sb + tl);
}

__device__ __forceinline__ void tile_to_lds(float* dst, const TileRegs& r, int cnt) {
    const int t = threadIdx.x;
    const int nq = cnt >> 2;
    vf4* d4 = reinterpret_cast<vf4*>(dst);
    if (t < nq) d4[t] = r.q0;
    if (t + kSThreads < nq) d4[t + kSThreads] = r.q1;
    if (t + 2 * kSThreads < nq) d4[t + 2 * kSThreads] = r.q2;
    if (t + 3 * kSThreads < nq) d4[t + 3 * kSThreads] = r.q3;
    const int tl = (nq << 2) + t;
    if (t < 4 && tl < cnt) dst[tl] = r.tail;
}

template <int V, int KM>
__global__ void __launch_bounds__(kSThreads)
    k_rowp_fwd(const float* __restrict__ x, float* __restrict__ out, int64_t rows) {
    static_assert(V == G_SOFTMAX || V == G_LOGSOFTMAX, "the pipelined engine runs the output-writing graphs");
    constexpr int K = KM;  // compiled for the exact class count
    __shared__ float4 xs4[kPQ * kSThreads];
    float* xs = reinterpret_cast<float*>(xs4);
    const int64_t ntiles = (rows + kSThreads - 1) / kSThreads;
    const int t = threadIdx.x;
    TileRegs rx{};
    int64_t tile = blockIdx.x;
    if (tile < ntiles) {
        const int64_t r0 = tile * kSThreads;
        const int cnt = (int)(((rows - r0) < kSThreads ? (rows - r0) : kSThreads) * K);
        tile_load(rx, x, r0 * K, cnt);
    }
    for (; tile < ntiles; tile += gridDim.x) {
        const int64_t r0 = tile * kSThreads;
        const int nr = (int)((rows - r0) < kSThreads ? (rows - r0) : kSThreads);
        const int cnt = nr * K;
        tile_to_lds(xs, rx, cnt);
        __syncthreads();
        const int64_t nxt = tile + gridDim.x;  // the next tile's loads overlap this tile's work
        if (nxt < ntiles) {
            const int64_t n0 = nxt * kSThreads;
            const int ncnt = (int)(((rows - n0) < kSThreads ? (rows - n0) : kSThreads) * K);
            tile_load(rx, x, n0 * K, ncnt);
        }
        if (t < nr) row_fwd<V, KM>(xs + t * K, xs + t * K, 0.0f, K);  // no target: unread
        __syncthreads();
        unstage_tile(out, xs, r0 * K, cnt, true);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------
// one-shot engine: rows of at most 16 classes, aligned operands
// ---------------------------------------------------------------------------------------
// A one-wavefront block takes 64 rows and issues every load of its tiles (ceil(K / 4) float4
// per thread per operand, the 64 * K % 4 tail floats on threads 0..2) before it uses any; the
// tiles go through LDS and thread t computes row t (row_fwd, the op-by-op chain's expressions
// and element-order sums). The forward runs the loss graphs: a block's partial is the
// wavefront's butterfly sum of its row sums, which k_loss_comb then sums. The backward runs
// every graph. Each class count 1..16 has its own kernel (every loop over a row unrolled
// without per-class guards). Many small blocks (5 KB of LDS each at 10 classes) keep the CU
// full of waves, so the loads of some overlap the exp work of others: at config 5 the pass
// reads its 84 MB in 15.3 us, against 16.7 us for a persistent grid of 256-thread blocks that
// prefetched each next 256-row tile into registers while computing the current one.
constexpr int kORows = 64;

// A tile quad's index for the one-shot kernels' loads. With K >= 4 every block holds at least
// one whole quad (nq >= 1), so a quad past the tile reloads the tile's last one and the loads
// need no branch (under a branch the compiler zeroed every tile register first: about three
// VALU instructions per element); smaller K keeps the guarded load.
template <int K>
__device__ __forceinline__ int tile_quad(int q, int nq) {
    if constexpr (K >= 4) return q < nq ? q : nq - 1;
    return q;
}

// The one-shot tiles' LDS row stride: K, or K + 1 for 24 and 32 classes (at stride K the
// wavefront's row reads t * K + j fall on a few banks, at 32 classes on one). Quads go in and
// out as float4 at stride K; at stride K + 1 (K a multiple of 4, so a quad never straddles two
// rows) element e sits at e + e / K. At 8 and 16 classes the padded tiles measured no faster
// (the CrossEntropy forward 0.3-0.7 us slower over 8M elements).
template <int K>
constexpr int tile_stride() {
    return K % 8 == 0 && K > 16 ? K + 1 : K;
}
template <int K>
__device__ __forceinline__ int tile_el(int e) {
    return tile_stride<K>() == K ? e : e + e / K;
}
template <int K>
__device__ __forceinline__ void tile_put(float* s, int qi, const vf4& q) {
    if constexpr (tile_stride<K>() == K) {
        reinterpret_cast<vf4*>(s)[qi] = q;
    } else {
        float* d = s + tile_el<K>(4 * qi);
        d[0] = q[0]; d[1] = q[1]; d[2] = q[2]; d[3] = q[3];
    }
}
template <int K>
__device__ __forceinline__ vf4 tile_get(const float* s, int qi) {
    if constexpr (tile_stride<K>() == K) {
        return reinterpret_cast<const vf4*>(s)[qi];
    } else {
        const float* d = s + tile_el<K>(4 * qi);
        return vf4{d[0], d[1], d[2], d[3]};
    }
}
constexpr int64_t kOMaxBlocks = max_grid_blocks(kORows);  // blocks of one launch

template <int V, int K>
__global__ void __launch_bounds__(kORows)
    k_rowo_fwd(const float* __restrict__ x, const float* __restrict__ tg, int64_t rows, float* __restrict__ part) {
    static_assert(V == G_SMLM || V == G_CE, "the one-shot forward runs the loss graphs");
    constexpr int QPT = (K + 3) / 4;  // 16 K quads per tile over 64 threads
    constexpr int KP = tile_stride<K>();
    __shared__ vf4 xs4[(kORows * KP + 3) / 4 + 1], ts4[(kORows * KP + 3) / 4 + 1];
    float* xs = reinterpret_cast<float*>(xs4);
    float* ts = reinterpret_cast<float*>(ts4);
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * kORows;
    const int nr = (int)((rows - r0) < kORows ? (rows - r0) : kORows);
    const int cnt = nr * K, nq = cnt >> 2;
    const int64_t base = r0 * K;  // a multiple of 64: 16-byte aligned
    vf4 qx[QPT], qt[QPT];
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int qi = tile_quad<K>(t + kORows * u, nq);
        if (K >= 4 || t + kORows * u < nq) {
            qx[u] = ld_ntv(x + base, qi);
            qt[u] = ld_ntv(tg + base, qi);
        }
    }
    const int tl = (nq << 2) + t;
    float tx = 0.0f, tt = 0.0f;
    if (tl < cnt) {
        tx = ld_nt(x + base + tl);
        tt = ld_nt(tg + base + tl);
    }
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        if (t + kORows * u < nq) {
            tile_put<K>(xs, t + kORows * u, qx[u]);
            tile_put<K>(ts, t + kORows * u, qt[u]);
        }
    }
    if (tl < cnt) {
        xs[tile_el<K>(tl)] = tx;
        ts[tile_el<K>(tl)] = tt;
    }
    __syncthreads();
    float rowsum = 0.0f;
    if (t < nr) rowsum = row_fwd<V, K>(xs + t * KP, ts + t * KP, rowsum, K);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) rowsum = rowsum + __shfl_xor(rowsum, m);
    if (t == 0) part[blockIdx.x] = rowsum;
}

// A loss's all-element sum over np block partials (16-byte aligned) in one 1024-thread block:
// thread t adds the partials' float4 quads t, t + 1024, ... in order, four loads in flight per
// round, each quad summed left to right, then the np % 4 tail (threads 0..2); an xor butterfly
// per wavefront and the sixteen wavefront sums in order finish it. The loss is the sum / lscale
// (MEAN, lscale = f32(N)) or the sum * lscale (cross entropy, lscale = its scale). One launch
// with every load of a round in flight: at config 5 (16384 partials) 2.4 us after the pass,
// against 2.8-3.3 us for two rounds of scalar loads (256 threads of sixteen loads each measured
// the same). It takes up to kLossCombMax partials (four rounds); more go through the library's
// multi-block all-element reduction.
constexpr int kLCThreads = 1024;
constexpr int64_t kLossCombMax = 4 * 4 * kLCThreads;

template <int V>
__global__ void __launch_bounds__(kLCThreads)
    k_loss_comb(const float* __restrict__ part, int64_t np, float* __restrict__ loss, float lscale) {
    __shared__ float ws[kLCThreads / 64];
    const int t = threadIdx.x;
    const int64_t nq = np >> 2;
    const vf4* p4 = reinterpret_cast<const vf4*>(part);
    float a = 0.0f;
    for (int64_t b = 0; b < nq; b += 4 * kLCThreads) {
        vf4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t i = b + t + (int64_t)u * kLCThreads;
            v[u] = i < nq ? p4[i] : vf4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) a = a + (((v[u][0] + v[u][1]) + v[u][2]) + v[u][3]);
    }
    if (t < (int)(np & 3)) a = a + part[(nq << 2) + t];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) a = a + __shfl_xor(a, m);
    if ((t & 63) == 0) ws[t >> 6] = a;
    __syncthreads();
    if (t == 0) {
        float w = ws[0];
        for (int k = 1; k < kLCThreads / 64; ++k) w = w + ws[k];
        loss[0] = V == G_SMLM ? w / lscale : w * lscale;
    }
}

// One row of a row graph's backward from LDS (x row xrow, upstream row urow: the target of a
// loss graph, the output's gradient otherwise; K elements, K <= KM). Returns the row in xr,
// pre[j] = every node's gradient term of element j up to SUB(x, max) in node order, and the MAX
// node's route: sg goes to the elements equal to the row max mb (NaN elements never). The
// caller adds (grad + pre[j]) + (xr[j] == mb ? sg : 0). The head graph overwrites urow.
template <int V, int KM>
__device__ __forceinline__ void row_bwd(float (&xr)[KM], float (&pre)[KM], float& mb, float& sg, const float* xrow,
                                        float* urow, float gconst, bool skip_ok, int K) {
    float e[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) xr[j] = j < K ? xrow[j] : 0.0f;
    float m = -FLT_MAX;
    mb = -FLT_MAX;
    uint32_t cntm = 0;
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        if (j < K) {
            const float v = xr[j];
            m = max_simd(m, v);
            max_count_add(mb, cntm, v);  // a NaN element is not counted
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
    float acc = 0.0f, gS;
    if constexpr (V == G_SMLM) {
        gS = 0.0f + smlm_bwd_row<KM>(pre, xrow, urow, e, m, s, gconst, skip_ok, K);
    } else if constexpr (from_softmax<V>()) {
        const float s2 = s * s;
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float gsm = upstream<V>(urow[j], e[j], s, gconst);
                pre[j] = 0.0f + gsm / s;
                acc = acc + ((-e[j]) / s2) * gsm;
            }
        }
        gS = 0.0f + acc;
    } else {
#pragma unroll
        for (int j = 0; j < KM; ++j) {
            if (j < K) {
                const float glsm = upstream<V>(urow[j], e[j], s, gconst);
                pre[j] = 0.0f + glsm;
                acc = acc + glsm;
            }
        }
        gS = 0.0f + (0.0f + (-acc)) / s;
    }
    const float rgs = K == 1 ? (1.0f * gS) * gS : 1.0f * gS;
    float acc2 = 0.0f;
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        if (j < K) {
            if constexpr (from_softmax<V>()) pre[j] = 0.0f + e[j] * (pre[j] + rgs);
            else pre[j] = pre[j] + e[j] * (0.0f + rgs);
            acc2 = acc2 + pre[j];
        }
    }
    sg = (1.0f / (float)cntm) * (0.0f + (-acc2));
}

// One-shot backward over rows of at most 16 classes, aligned operands: a one-wavefront block
// takes 64 rows and issues every load of its x, upstream (a loss graph's target, else the
// output's gradient) and grad_x tiles first. The grad_x quads stay in registers; x and the
// upstream tile go through LDS, where thread t computes row t (row_bwd) and writes pre over its
// x row and the MAX route over its upstream row. Each thread then stores its grad_x quads as
// (g + pre) + route, the op-by-op chain's sums in its order. Two tiles in LDS (5 KB per
// wavefront at 10 classes): 29.9 us at config 5 against 31.3 us for the persistent grid, which
// staged grad_x as a third tile and so fitted three 256-thread blocks per CU.
template <int V, int K>
__global__ void __launch_bounds__(kORows)
    k_rowo_bwd(float* __restrict__ g, const float* __restrict__ x, const float* __restrict__ up,
               const float* __restrict__ ug, int64_t rows, float c) {
    constexpr int QPT = (K + 3) / 4;
    constexpr int KP = tile_stride<K>();
    __shared__ vf4 xs4[(kORows * KP + 3) / 4 + 1], us4[(kORows * KP + 3) / 4 + 1];
    float* xs = reinterpret_cast<float*>(xs4);
    float* us = reinterpret_cast<float*>(us4);
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * kORows;
    const int nr = (int)((rows - r0) < kORows ? (rows - r0) : kORows);
    const int cnt = nr * K, nq = cnt >> 2;
    const int64_t base = r0 * K;  // a multiple of 64: 16-byte aligned
    vf4 qx[QPT], qu[QPT], qg[QPT];
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int qi = tile_quad<K>(t + kORows * u, nq);
        if (K >= 4 || t + kORows * u < nq) {
            qx[u] = ld_ntv(x + base, qi);
            qu[u] = ld_ntv(up + base, qi);
            qg[u] = ld_ntv(g + base, qi);
        }
    }
    const int tl = (nq << 2) + t;
    float tx = 0.0f, tu = 0.0f, tg = 0.0f;
    if (tl < cnt) {
        tx = ld_nt(x + base + tl);
        tu = ld_nt(up + base + tl);
        tg = ld_nt(g + base + tl);
    }
    // the loss's upstream gradient as a vector load behind the tiles' loads: as a scalar load
    // at its first use it cost every block a memory round trip after its barrier
    float u0 = 0.0f;
    if constexpr (V == G_SMLM || V == G_CE) u0 = __hip_atomic_load(ug, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float gconst = V == G_SMLM ? 0.0f + c * u0 : V == G_CE ? 0.0f + 1.0f * (0.0f + u0 * c) : 0.0f;
    const bool skip_ok = gconst - gconst == 0.0f;  // g_t finite (the head graph's zero-target shortcut)
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        if (t + kORows * u < nq) {
            tile_put<K>(xs, t + kORows * u, qx[u]);
            tile_put<K>(us, t + kORows * u, qu[u]);
        }
    }
    if (tl < cnt) {
        xs[tile_el<K>(tl)] = tx;
        us[tile_el<K>(tl)] = tu;
    }
    __syncthreads();
    if (t < nr) {
        float xr[K], pre[K], mb, sg;
        row_bwd<V, K>(xr, pre, mb, sg, xs + t * KP, us + t * KP, gconst, skip_ok, K);
#pragma unroll
        for (int j = 0; j < K; ++j) {
            xs[t * KP + j] = pre[j];
            us[t * KP + j] = xr[j] == mb ? sg : 0.0f;
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        if (t + kORows * u < nq) {
            const vf4 p = tile_get<K>(xs, t + kORows * u), r = tile_get<K>(us, t + kORows * u);
            vf4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = (qg[u][j] + p[j]) + r[j];
            st_ntv(g + base, t + kORows * u, o);
        }
    }
    if (tl < cnt) st_nt(g + base + tl, (tg + xs[tile_el<K>(tl)]) + us[tile_el<K>(tl)]);
}


// ---------------------------------------------------------------------------------------
// wavefront engine: 64 < classes <= 2047, one wavefront per row, k_rows_wave's order
// ---------------------------------------------------------------------------------------
// Lane slot i holds element 4 (lane + 64 (i / 4)) + i % 4 (VEC: classes % 4 == 0, quads
// lane + 64 q) or lane + 64 i (otherwise).
template <bool VEC>
__device__ __forceinline__ int slot_elem(int lane, int i) {
    return VEC ? 4 * (lane + 64 * (i >> 2)) + (i & 3) : lane + 64 * i;
}

struct OpAdd {
    __device__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
    __device__ float operator()(float a, float b) const { return a > b ? a : b; }
};

// One row's reduction in the order of k_rows_wave<R, LD, VEC> with a single chunk.
template <bool VEC, int NE, class OP>
__device__ __forceinline__ float wave_row_reduce(const float* v, int lane, int K, float init, OP op) {
    float acc = init;
    if constexpr (VEC) {
        constexpr int NQ = NE / 4;
        const int nq = K >> 2;
        float a4[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) a4[u][j] = init;
        int done = 0;  // quads taken by the four-quad main loop (a prefix of the groups)
#pragma unroll
        for (int q0 = 0; q0 + 3 < NQ; q0 += 4) {
            if (lane + 64 * (q0 + 3) < nq) {
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int j = 0; j < 4; ++j) a4[u][j] = op(a4[u][j], v[(q0 + u) * 4 + j]);
                done = q0 + 4;
            }
        }
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            if (q >= done && lane + 64 * q < nq) {
#pragma unroll
                for (int j = 0; j < 4; ++j) a4[0][j] = op(a4[0][j], v[q * 4 + j]);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = op(acc, a4[u][j]);
    } else {
#pragma unroll
        for (int i = 0; i < NE; ++i)
            if (lane + 64 * i < K) acc = op(acc, v[i]);
    }
#pragma unroll
    for (int mm = 32; mm >= 1; mm >>= 1) acc = op(acc, __shfl_xor(acc, mm));
    return acc;
}

template <bool VEC, int NE>
__device__ __forceinline__ void load_row(float* v, const float* __restrict__ src, int lane, int K, bool al) {
    if (VEC && al) {
#pragma unroll
        for (int q = 0; q < NE / 4; ++q) {
            const int qi = lane + 64 * q;
            if (4 * qi < K) {
                const float4 f = ld_nt4(src, qi);
                v[4 * q] = f.x;
                v[4 * q + 1] = f.y;
                v[4 * q + 2] = f.z;
                v[4 * q + 3] = f.w;
            } else {
                v[4 * q] = v[4 * q + 1] = v[4 * q + 2] = v[4 * q + 3] = 0.0f;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const int k = slot_elem<VEC>(lane, i);
            v[i] = k < K ? ld_nt(src + k) : 0.0f;
        }
    }
}

template <bool VEC, int NE>
__device__ __forceinline__ void store_row(float* __restrict__ dst, const float* v, int lane, int K, bool al) {
    if (VEC && al) {
#pragma unroll
        for (int q = 0; q < NE / 4; ++q) {
            const int qi = lane + 64 * q;
            if (4 * qi < K)
                st_nt4(dst, qi, make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]));
        }
    } else {
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const int k = slot_elem<VEC>(lane, i);
            if (k < K) st_nt(dst + k, v[i]);
        }
    }
}

// Row max (MAX.forward's order), e = exp(x - m) and s = sum e (SUM.forward's order).
template <bool VEC, int NE>
__device__ __forceinline__ void wave_row_softmax(const float* xv, float* e, int lane, int K, float* m_out,
                                                 float* s_out) {
    const float m = wave_row_reduce<VEC, NE>(xv, lane, K, -FLT_MAX, OpMax{});
#pragma unroll
    for (int i = 0; i < NE; ++i) e[i] = slot_elem<VEC>(lane, i) < K ? mexp(xv[i] - m) : 0.0f;
    *m_out = m;
    *s_out = wave_row_reduce<VEC, NE>(e, lane, K, 0.0f, OpAdd{});
}

template <int V, bool VEC, int NE>
__global__ void __launch_bounds__(kSThreads)
    k_roww_fwd(const float* __restrict__ x, const float* __restrict__ tg, float* __restrict__ out, int64_t rows,
               int K, bool al, float* __restrict__ part) {
    __shared__ float ws[4];
    constexpr bool LOSS = V == G_SMLM || V == G_CE;
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    float rowsum = 0.0f;
    if (row < rows) {  // uniform per wavefront
        const int64_t base = row * (int64_t)K;
        float xv[NE], e[NE];
        load_row<VEC, NE>(xv, x + base, lane, K, al);
        float m, s;
        wave_row_softmax<VEC, NE>(xv, e, lane, K, &m, &s);
        const float ls = (V == G_CE || V == G_LOGSOFTMAX) ? mlog(s) : 0.0f;
        if constexpr (LOSS) {
            float tv[NE];
            load_row<VEC, NE>(tv, tg + base, lane, K, al);
#pragma unroll
            for (int i = 0; i < NE; ++i) {
                if (slot_elem<VEC>(lane, i) < K) {
                    if constexpr (V == G_SMLM) {
                        if (!smlm_skip(tv[i], e[i])) rowsum = rowsum + mlog(e[i] / s) * tv[i];
                    }
                    else rowsum = rowsum + tv[i] * ((xv[i] - m) - ls);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NE; ++i) xv[i] = V == G_SOFTMAX ? e[i] / s : (xv[i] - m) - ls;
            store_row<VEC, NE>(out + base, xv, lane, K, al);
        }
    }
    if constexpr (LOSS) {  // every wavefront reaches the barrier
        const float tot = block_sum(rowsum, ws);
        if (threadIdx.x == 0) part[blockIdx.x] = tot;
    }
}

template <int V, bool VEC, int NE>
__global__ void __launch_bounds__(kSThreads)
    k_roww_bwd(float* __restrict__ g, const float* __restrict__ x, const float* __restrict__ up,
               const float* __restrict__ ug, int64_t rows, int K, bool al, float c) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // uniform per wavefront; no block barrier below
    const int64_t base = row * (int64_t)K;
    float xv[NE], e[NE], pre[NE], tmp[NE];
    load_row<VEC, NE>(xv, x + base, lane, K, al);
    float m, s;
    wave_row_softmax<VEC, NE>(xv, e, lane, K, &m, &s);
    // the max with its count, as MAX.backward recomputes it (lane order, then a butterfly)
    float mb = -FLT_MAX;
    uint32_t cntm = 0;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        if (slot_elem<VEC>(lane, i) < K) {
            const float v = xv[i];
            max_count_add(mb, cntm, v);  // a NaN element is not counted
        }
    }
#pragma unroll
    for (int mm = 32; mm >= 1; mm >>= 1) {
        const float om = __shfl_xor(mb, mm);
        const uint32_t oc = (uint32_t)__shfl_xor((int)cntm, mm);
        max_count_merge(mb, cntm, om, oc);
    }
    load_row<VEC, NE>(tmp, up + base, lane, K, al);
    const float gconst = V == G_SMLM ? 0.0f + c * ug[0] : V == G_CE ? 0.0f + 1.0f * (0.0f + ug[0] * c) : 0.0f;
    float gS;
    if constexpr (from_softmax<V>()) {
        const float s2 = s * s;
        const bool skip_ok = V == G_SMLM && gconst - gconst == 0.0f;
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            if (skip_ok && (slot_elem<VEC>(lane, i) >= K || smlm_skip(tmp[i], e[i]))) {
                pre[i] = 0.0f;  // the values of the full expression (slots past the row are unused)
                tmp[i] = -0.0f;
            } else {
                const float gsm = upstream<V>(tmp[i], e[i], s, gconst);
                pre[i] = 0.0f + gsm / s;
                tmp[i] = ((-e[i]) / s2) * gsm;
            }
        }
        gS = 0.0f + wave_row_reduce<VEC, NE>(tmp, lane, K, 0.0f, OpAdd{});
    } else {
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            const float glsm = upstream<V>(tmp[i], e[i], s, gconst);
            pre[i] = 0.0f + glsm;
            tmp[i] = glsm;
        }
        gS = 0.0f + (0.0f + (-wave_row_reduce<VEC, NE>(tmp, lane, K, 0.0f, OpAdd{}))) / s;
    }
    const float rgs = 1.0f * gS;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        if constexpr (from_softmax<V>()) pre[i] = 0.0f + e[i] * (pre[i] + rgs);
        else pre[i] = pre[i] + e[i] * (0.0f + rgs);
    }
    const float sg = (1.0f / (float)cntm) * (0.0f + (-wave_row_reduce<VEC, NE>(pre, lane, K, 0.0f, OpAdd{})));
    load_row<VEC, NE>(tmp, g + base, lane, K, al);
#pragma unroll
    for (int i = 0; i < NE; ++i) tmp[i] = (tmp[i] + pre[i]) + (xv[i] == mb ? sg : 0.0f);
    store_row<VEC, NE>(g + base, tmp, lane, K, al);
}

// ---------------------------------------------------------------------------------------
// multi-lane engine: rows of 17-64 classes, P = ceil(classes / 16) lanes per row
// ---------------------------------------------------------------------------------------
// Lane c of a row's P lanes holds elements [16 c, min(16 c + 16, classes)) in registers, loaded
// straight from HBM (no LDS tiles, whose size per row held the thread engine to a few waves
// per CU). Every order-dependent row quantity (the max, the max with its count, every row sum)
// is carried across the P lanes in element order: lane c starts from the value lane c - 1
// ended with, so each row sees the same sequence of operations as one thread walking the row
// (the thread engine's and the library's row reductions' order), and results keep their bits.
// A wavefront holds 64 / P rows (lanes past 64 / P * P idle), a 256-thread block four times
// that; a loss graph's all-element sum adds per lane, then per block (the rtol class).
constexpr int kMNE = 16;  // elements per lane

template <int P>
struct RowLanes {
    static constexpr int R = 64 / P;  // rows per wavefront
    int lane, r, c, cnt;              // lane in the wavefront, row in the wavefront, chunk, elements
    bool live;                        // this lane holds a chunk of a row that exists
};

// Shuffles of the values a row chain carries (the running max, max with count, or sum).
__device__ __forceinline__ float row_chain_shfl(float v, int src) { return __shfl(v, src & 63); }
struct MaxCount {
    float m;
    uint32_t c;
};
__device__ __forceinline__ MaxCount row_chain_shfl(MaxCount v, int src) {
    return MaxCount{__shfl(v.m, src & 63), (uint32_t)__shfl((int)v.c, src & 63)};
}

// The row's lanes in chunk order run `fold` (which walks the lane's elements in order from the
// value it is given): lane c starts from lane c - 1's result (init for c == 0). Every lane of
// the row returns the row's final value (that of its last lane). All lanes of the wavefront
// take part (the shuffles); `fold` runs only on the lane whose turn it is.
template <int P, class T, class F>
__device__ __forceinline__ T row_chain(const RowLanes<P>& L, T init, F fold) {
    T v = init;
#pragma unroll
    for (int k = 0; k < P; ++k) {
        const T in = row_chain_shfl(v, L.lane - 1);
        if (L.c == k && L.live) v = fold(k == 0 ? init : in);
    }
    return row_chain_shfl(v, L.lane - L.c + (P - 1));
}

// A lane's chunk [off, off + cnt) straight from HBM with plain (cacheable) loads: a lane's
// quads are 64 bytes from its neighbours', so each load instruction touches pieces of many
// lines, and the next instructions find those lines in the caches (non-temporal loads fetched
// them again: the 40-class Softmax forward took 70 us instead of 35). Staging the wavefront's
// contiguous rows through LDS with coalesced loads was no faster forward and slower backward
// (its three tiles held the grid to three blocks per CU). Rows of whole quads (VEC) load the
// chunk's quads; other rows load the aligned quads that cover the chunk (the tensor's last,
// partial quad element by element) and shift them into place: loading each element on its own
// made such rows' forward twice as slow. `base` is 16-byte aligned, n the tensor's elements.
__device__ __forceinline__ float shifted(const float* w, int j, int s) {
    return s == 0 ? w[j] : s == 1 ? w[j + 1] : s == 2 ? w[j + 2] : w[j + 3];
}

// A chunk's loads in two steps, so that a kernel issues every tensor's quad loads before it
// waits for any: chunk_issue loads every quad unconditionally (a quad the chunk does not need
// loads one that is sure to exist: the chunk's first, or the tensor's last whole quad; n >= 17
// here), chunk_finish keeps the needed ones by selects and, for a chunk that reaches the
// tensor's last, partial quad, loads its elements one by one. Loads under per-quad branches
// made the compiler copy the registers at each join, and each copy waited for the loads
// before it: one memory round trip per quad.
struct ChunkQuads {
    vf4 t[kMNE / 4 + 1];
};

template <bool VEC>
__device__ __forceinline__ void chunk_issue(ChunkQuads& c, const float* __restrict__ base, int64_t off, int cnt,
                                            int64_t n) {
    if constexpr (VEC) {  // off and cnt multiples of 4; a lane with no chunk has off = 0
        const vf4* p = reinterpret_cast<const vf4*>(base + off);
#pragma unroll
        for (int q = 0; q < kMNE / 4; ++q) c.t[q] = p[4 * q < cnt ? q : 0];
    } else {
        const int64_t a0 = off & ~(int64_t)3;
        const int64_t last = off + cnt;       // one past the chunk
        const int64_t nq4 = n & ~(int64_t)3;  // the tensor's elements in whole quads
#pragma unroll
        for (int q = 0; q < kMNE / 4 + 1; ++q) {
            const int64_t e = a0 + 4 * q;
            c.t[q] = *reinterpret_cast<const vf4*>(base + (e < last && e < nq4 ? e : nq4 - 4));
        }
    }
}

template <bool VEC>
__device__ __forceinline__ void chunk_finish(float (&v)[kMNE], const ChunkQuads& c, const float* __restrict__ base,
                                             int64_t off, int cnt, int64_t n) {
    if constexpr (VEC) {
#pragma unroll
        for (int q = 0; q < kMNE / 4; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[4 * q + i] = 4 * q < cnt ? c.t[q][i] : 0.0f;
    } else {
        const int64_t a0 = off & ~(int64_t)3;
        const int s = (int)(off - a0);
        const int64_t last = off + cnt;
        const int64_t nq4 = n & ~(int64_t)3;
        float w[kMNE + 4];
#pragma unroll
        for (int q = 0; q < kMNE / 4 + 1; ++q) {
            const int64_t e = a0 + 4 * q;
            const bool in = e < last && e < nq4;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[4 * q + i] = in ? c.t[q][i] : 0.0f;
        }
        if (last > nq4) {  // the tensor's last, partial quad
#pragma unroll
            for (int q = 0; q < kMNE / 4 + 1; ++q) {
                const int64_t e = a0 + 4 * q;
                if (e == nq4)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (e + i < n) w[4 * q + i] = base[e + i];
            }
        }
#pragma unroll
        for (int j = 0; j < kMNE; ++j) v[j] = j < cnt ? shifted(w, j, s) : 0.0f;
    }
}

// The chunk back: VEC rows as quads; other rows write the whole quads inside the chunk (this
// lane's alone) as float4 and the elements before the first and after the last 16-byte
// boundary one by one (their quads are shared with the neighbouring chunks).
template <bool VEC>
__device__ __forceinline__ void store_chunk(float* __restrict__ base, const float (&v)[kMNE], int64_t off, int cnt) {
    if constexpr (VEC) {
        float* p = base + off;
#pragma unroll
        for (int q = 0; q < kMNE / 4; ++q)
            if (4 * q < cnt) reinterpret_cast<vf4*>(p)[q] = vf4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
    } else {
        const int64_t end = off + cnt;
        const int64_t q0 = (off + 3) & ~(int64_t)3;  // first 16-byte boundary at or after off
        const int64_t q1 = end & ~(int64_t)3;        // last boundary at or before end
        const int d = (int)(q0 - off);                // v index of element q0
        float w[kMNE + 4];                             // v, padded for the shifted reads
#pragma unroll
        for (int j = 0; j < kMNE + 4; ++j) w[j] = j < kMNE ? v[j] : 0.0f;
#pragma unroll
        for (int j = 0; j < kMNE; ++j) {
            const int64_t e = off + j;
            if (j < cnt && (e < q0 || e >= q1)) base[e] = v[j];
        }
#pragma unroll
        for (int k = 0; k < kMNE / 4; ++k) {
            const int64_t e = q0 + 4 * k;
            if (e + 4 <= q1)
                *reinterpret_cast<vf4*>(base + e) = vf4{shifted(w, 4 * k, d), shifted(w, 4 * k + 1, d),
                                                        shifted(w, 4 * k + 2, d), shifted(w, 4 * k + 3, d)};
        }
    }
}

template <int P>
__device__ __forceinline__ RowLanes<P> row_lanes(int64_t rows, int K, int64_t* row_out) {
    RowLanes<P> L;
    L.lane = threadIdx.x & 63;
    L.r = L.lane / P;
    L.c = L.lane - L.r * P;
    const int64_t row = ((int64_t)blockIdx.x * (kSThreads / 64) + (threadIdx.x >> 6)) * RowLanes<P>::R + L.r;
    const int rem = K - kMNE * L.c;
    L.cnt = rem < 0 ? 0 : (rem < kMNE ? rem : kMNE);
    L.live = L.r < RowLanes<P>::R && row < rows;
    *row_out = row;
    return L;
}

template <int V, int P, bool VEC>
__global__ void __launch_bounds__(kSThreads)
    k_rowm_fwd(const float* __restrict__ x, const float* __restrict__ tg, float* __restrict__ out, int64_t rows,
               int K, float* __restrict__ part) {
    __shared__ float ws[4];
    constexpr bool LOSS = V == G_SMLM || V == G_CE;
    int64_t row;
    const RowLanes<P> L = row_lanes<P>(rows, K, &row);
    const int64_t off = row * (int64_t)K + kMNE * L.c;
    float xv[kMNE], tv[kMNE], e[kMNE];
    const int cnt = L.live ? L.cnt : 0;
    const int64_t n = rows * (int64_t)K;
    const int64_t o = L.live ? off : 0;
    ChunkQuads cx, ct;
    chunk_issue<VEC>(cx, x, o, cnt, n);
    if constexpr (LOSS) chunk_issue<VEC>(ct, tg, o, cnt, n);
    chunk_finish<VEC>(xv, cx, x, o, cnt, n);
    if constexpr (LOSS) chunk_finish<VEC>(tv, ct, tg, o, cnt, n);
    // MAX.forward: max_simd from min_finite, element order
    const float m = row_chain<P>(L, -FLT_MAX, [&](float a) {
#pragma unroll
        for (int j = 0; j < kMNE; ++j)
            if (j < cnt) a = max_simd(a, xv[j]);
        return a;
    });
#pragma unroll
    for (int j = 0; j < kMNE; ++j) e[j] = j < cnt ? mexp(xv[j] - m) : 0.0f;  // SUB, EXP
    const float s = row_chain<P>(L, 0.0f, [&](float a) {  // SUM.forward
#pragma unroll
        for (int j = 0; j < kMNE; ++j)
            if (j < cnt) a = a + e[j];
        return a;
    });
    const float ls = (V == G_CE || V == G_LOGSOFTMAX) ? mlog(s) : 0.0f;  // LOG.forward of the sum
    if constexpr (LOSS) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kMNE; ++j) {
            if (j < cnt) {
                if constexpr (V == G_SMLM) {
                    if (!smlm_skip(tv[j], e[j])) acc = acc + mlog(e[j] / s) * tv[j];  // DIV, LOG, MUL
                } else {
                    acc = acc + tv[j] * ((xv[j] - m) - ls);  // SUB(xm, ls), MUL(target, .)
                }
            }
        }
        const float tot = block_sum(acc, ws);
        if (threadIdx.x == 0) part[blockIdx.x] = tot;
    } else {
#pragma unroll
        for (int j = 0; j < kMNE; ++j) xv[j] = V == G_SOFTMAX ? e[j] / s : (xv[j] - m) - ls;  // DIV / SUB
        if (L.live) store_chunk<VEC>(out, xv, off, cnt);
    }
}

template <int V, int P, bool VEC>
__global__ void __launch_bounds__(kSThreads)
    k_rowm_bwd(float* __restrict__ g, const float* __restrict__ x, const float* __restrict__ up,
               const float* __restrict__ ug, int64_t rows, int K, float c) {
    int64_t row;
    const RowLanes<P> L = row_lanes<P>(rows, K, &row);
    const int64_t off = row * (int64_t)K + kMNE * L.c;
    const int cnt = L.live ? L.cnt : 0;
    float xv[kMNE], uv[kMNE], gv[kMNE], e[kMNE];
    const int64_t n = rows * (int64_t)K;
    const int64_t o = L.live ? off : 0;
    ChunkQuads cx, cu, cg;
    chunk_issue<VEC>(cx, x, o, cnt, n);
    chunk_issue<VEC>(cu, up, o, cnt, n);
    chunk_issue<VEC>(cg, g, o, cnt, n);
    chunk_finish<VEC>(xv, cx, x, o, cnt, n);
    chunk_finish<VEC>(uv, cu, up, o, cnt, n);
    chunk_finish<VEC>(gv, cg, g, o, cnt, n);
    // the forward row max (MAX.forward) and, as MAX.backward recomputes it, the max with its
    // count (an element neither above nor below the running max adds to the count)
    const float m = row_chain<P>(L, -FLT_MAX, [&](float a) {
#pragma unroll
        for (int j = 0; j < kMNE; ++j)
            if (j < cnt) a = max_simd(a, xv[j]);
        return a;
    });
    const MaxCount mc = row_chain<P>(L, MaxCount{-FLT_MAX, 0u}, [&](MaxCount a) {
#pragma unroll
        for (int j = 0; j < kMNE; ++j) {
            if (j < cnt) {
                max_count_add(a.m, a.c, xv[j]);  // a NaN element is not counted
            }
        }
        return a;
    });
#pragma unroll
    for (int j = 0; j < kMNE; ++j) e[j] = j < cnt ? mexp(xv[j] - m) : 0.0f;
    const float s = row_chain<P>(L, 0.0f, [&](float a) {
#pragma unroll
        for (int j = 0; j < kMNE; ++j)
            if (j < cnt) a = a + e[j];
        return a;
    });
    const float gconst = V == G_SMLM ? 0.0f + c * ug[0]                       // MEAN backward
                         : V == G_CE ? 0.0f + 1.0f * (0.0f + ug[0] * c)       // MUL(., c), SUM backward
                                     : 0.0f;
    // pre: g_e after DIV (from_softmax), or g_xm after SUB(xm, ls); uv becomes the row-sum terms
    float pre[kMNE];
    bool keep[kMNE];
    float gS;
    if constexpr (from_softmax<V>()) {
        const float s2 = s * s;
        const bool skip_ok = V == G_SMLM && gconst - gconst == 0.0f;
#pragma unroll
        for (int j = 0; j < kMNE; ++j) {
            keep[j] = j < cnt && !(skip_ok && smlm_skip(uv[j], e[j]));
            if (keep[j]) {
                const float gsm = upstream<V>(uv[j], e[j], s, gconst);
                pre[j] = 0.0f + gsm / s;
                uv[j] = ((-e[j]) / s2) * gsm;
            } else {
                pre[j] = 0.0f;
            }
        }
        gS = 0.0f + row_chain<P>(L, 0.0f, [&](float a) {
#pragma unroll
            for (int j = 0; j < kMNE; ++j)
                if (keep[j]) a = a + uv[j];
            return a;
        });
    } else {
#pragma unroll
        for (int j = 0; j < kMNE; ++j) {
            const float glsm = upstream<V>(uv[j], e[j], s, gconst);
            pre[j] = 0.0f + glsm;
            uv[j] = glsm;
        }
        gS = 0.0f + (0.0f + (-row_chain<P>(L, 0.0f, [&](float a) {
                               #pragma unroll
                               for (int j = 0; j < kMNE; ++j)
                                   if (j < cnt) a = a + uv[j];
                               return a;
                           }))) / s;
    }
    const float rgs = 1.0f * gS;  // SUM backward (classes > 1)
#pragma unroll
    for (int j = 0; j < kMNE; ++j) {
        if constexpr (from_softmax<V>()) pre[j] = 0.0f + e[j] * (pre[j] + rgs);
        else pre[j] = pre[j] + e[j] * (0.0f + rgs);
    }
    const float acc2 = row_chain<P>(L, 0.0f, [&](float a) {
#pragma unroll
        for (int j = 0; j < kMNE; ++j)
            if (j < cnt) a = a + pre[j];
        return a;
    });
    const float sg = (1.0f / (float)mc.c) * (0.0f + (-acc2));  // SUB 1, then the MAX factor
#pragma unroll
    for (int j = 0; j < kMNE; ++j) gv[j] = (gv[j] + pre[j]) + (xv[j] == mc.m ? sg : 0.0f);
    if (L.live) store_chunk<VEC>(g, gv, off, cnt);
}

// ---------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------
static inline bool al16s(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The class counts with row kernels of their own (one-shot and pipelined).
#define MH_ROW16_CLASSES(X) \
    X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13) X(14) X(15) X(16)
// the one-shot kernels' class counts: up to 32
#define MH_ONESHOT_CLASSES(X) \
    MH_ROW16_CLASSES(X)       \
    X(17) X(18) X(19) X(20) X(21) X(22) X(23) X(24) X(25) X(26) X(27) X(28) X(29) X(30) X(31) X(32)
static inline bool oneshot_classes(int K) { return K <= 32; }

// Blocks of a persistent kernel: as many as can be resident at once (queried once per
// kernel), so no block waits for another to finish.
static int64_t pipe_grid(const void* kernel) {
    static std::unordered_map<const void*, int> resident;
    auto it = resident.find(kernel);
    if (it == resident.end()) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, kSThreads, 0) != hipSuccess || n < 1) n = 1;
        it = resident.emplace(kernel, n).first;
    }
    return (int64_t)it->second * ctx().num_cus;
}

// The one-shot engine's launches over `rows` rows (what mh_plan_launch reports): blocks of 64
// rows, at most kOMaxBlocks per launch, each launch over the next run of rows.
LaunchShape row16_launch(int64_t rows) {
    const int64_t nb = (rows + kORows - 1) / kORows;
    return LaunchShape{0, kORows, nb < kOMaxBlocks ? nb : kOMaxBlocks, (nb + kOMaxBlocks - 1) / kOMaxBlocks};
}

static int check_rows(const char* what, int64_t rows, int64_t classes) {
    if (rows < 0 || classes < 0) return fail(MH_ERR_INVALID, "%s: negative size", what);
    if (classes > kSWaveMax)
        return fail(MH_ERR_INVALID, "%s: %lld classes; the fused row kernels take rows of at most %d (use the op-by-op path)",
                    what, (long long)classes, kSWaveMax);
    if ((double)rows * (double)classes > 9.0e15) return fail(MH_ERR_OVERFLOW, "%s: size overflow", what);
    return MH_OK;
}

// Loss graphs leave one partial per block in `part` (the caller sums them); Softmax and
// LogSoftmax write `out`. With aligned operands, Softmax and LogSoftmax over rows of up to 16
// classes run the pipelined engine, and the loss graphs over rows of up to 32 classes the
// one-shot engine, in several launches (each over its own rows and partials) past one
// dispatch.
template <int V>
static int launch_fwd(const float* x, const float* tg, float* out, int64_t rows, int K, float* part,
                      int64_t* nblocks_out) {
    hipStream_t st = ctx().stream;
    constexpr bool LOSS = V == G_SMLM || V == G_CE;
    const bool al = al16s(x) && (!LOSS || al16s(tg)) && (LOSS || al16s(out));
    if constexpr (!LOSS) {
        if (K <= 16 && al) {  // persistent, pipelined
            const void* kern = nullptr;
            switch (K) {
#define MH_K(KK) \
    case KK: kern = reinterpret_cast<const void*>(&k_rowp_fwd<V, KK>); break;
                MH_ROW16_CLASSES(MH_K)
#undef MH_K
                default: return fail(MH_ERR_INVALID, "row kernel: %d classes", K);
            }
            const int64_t ntiles = (rows + kSThreads - 1) / kSThreads;
            const int64_t pg = pipe_grid(kern);
            const int64_t nb = ntiles < pg ? ntiles : pg;
            *nblocks_out = nb;
            dim3 g((unsigned)nb), b(kSThreads);
            switch (K) {
#define MH_K(KK) \
    case KK: hipLaunchKernelGGL((k_rowp_fwd<V, KK>), g, b, 0, st, x, out, rows); break;
                MH_ROW16_CLASSES(MH_K)
#undef MH_K
            }
            return MH_OK;
        }
    } else {
        // one-shot blocks of 64 rows, up to 32 classes (streamed over 8M elements, the
        // CrossEntropy forward of 17-32 classes 15.1-16.8 us against 16.3-27.6 us in the
        // multi-lane and thread engines)
        if (oneshot_classes(K) && al) {
            const int64_t nb = (rows + kORows - 1) / kORows;
            *nblocks_out = nb;
            for (int64_t b0 = 0; b0 < nb; b0 += kOMaxBlocks) {
                const int64_t cnt = nb - b0 < kOMaxBlocks ? nb - b0 : kOMaxBlocks;
                const int64_t r0 = b0 * kORows, off = r0 * K;  // 16-byte aligned: r0 is a multiple of 64
                const int64_t nr = rows - r0 < cnt * kORows ? rows - r0 : cnt * kORows;
                dim3 g((unsigned)cnt), b(kORows);
                switch (K) {
#define MH_K(KK) \
    case KK: hipLaunchKernelGGL((k_rowo_fwd<V, KK>), g, b, 0, st, x + off, tg + off, nr, part + b0); break;
                    MH_ONESHOT_CLASSES(MH_K)
#undef MH_K
                    default: return fail(MH_ERR_INVALID, "row kernel: %d classes", K);
                }
            }
            return MH_OK;
        }
    }
    // multi-lane engine, aligned operands: loss rows of 33-64 classes (up to 32 the one-shot
    // kernels take them), and Softmax / LogSoftmax rows of whole quads of 40, 48 or more than
    // 52 classes.
    // Streamed over 8M elements, Softmax quad rows run 14.1-19 us in the thread engine at 20-36,
    // 44 and 52 classes (32 with its rows padded in LDS: 14.5 against 36 us unpadded) against
    // 19.6-20.7 us here; at 40-64 classes the thread engine's LDS tiles (and, above 32, its
    // 64-element registers) hold a CU to two or three blocks, and how its blocks fall into
    // rounds decides (18-31 us against 20.6-21.0 us here). Rows that are not whole quads run
    // 15-19 us there (32 us at 63 classes) against 30-31 us here.
    const bool rowm_map = K % 4 == 0 && K > 32 && (K % 8 == 0 || K > 52);
    if (K > 16 && K <= 4 * kMNE && al && (LOSS || rowm_map)) {
        const int P = (K + kMNE - 1) / kMNE;
        const int64_t rpb = (int64_t)(kSThreads / 64) * (64 / P);
        const int64_t nb = (rows + rpb - 1) / rpb;
        if (nb > 0x7fffffff) return fail(MH_ERR_OVERFLOW, "too many rows");
        *nblocks_out = nb;
        const bool vec = K % 4 == 0;
        dim3 g((unsigned)nb), b(kSThreads);
#define MH_RM(PP, VV) hipLaunchKernelGGL((k_rowm_fwd<V, PP, VV>), g, b, 0, st, x, tg, out, rows, K, part)
        if (vec) {
            if (P == 2) MH_RM(2, true);
            else if (P == 3) MH_RM(3, true);
            else MH_RM(4, true);
        } else {
            if (P == 2) MH_RM(2, false);
            else if (P == 3) MH_RM(3, false);
            else MH_RM(4, false);
        }
#undef MH_RM
        return MH_OK;
    }
    if (K <= kSThreadMax) {
        // rows of a multiple of 8 floats at a stride of K + 1 in LDS (aligned operands)
        const int Kp = al && K % 8 == 0 ? K + 1 : K;
        const int rb = rows_per_block(LOSS ? 2 : 1, Kp);
        const int64_t nb = (rows + rb - 1) / rb;
        if (nb > 0x7fffffff) return fail(MH_ERR_OVERFLOW, "too many rows");
        *nblocks_out = nb;
        const size_t lds = (LOSS ? 2 : 1) * (size_t)rb * (size_t)Kp * sizeof(float);
        const FastDiv fk = make_fastdiv((uint32_t)K);
        dim3 g((unsigned)nb), b(kSThreads);
#define MH_RT(KM) \
    hipLaunchKernelGGL((k_rowt_fwd<V, KM>), g, b, lds, st, x, tg, out, rows, K, rb, al, part, Kp, fk)
        if (K <= 8) MH_RT(8);
        else if (K <= 16) MH_RT(16);
        else if (K <= 32) MH_RT(32);
        else MH_RT(64);
#undef MH_RT
        return MH_OK;
    }
    const int64_t nb = (rows + 3) / 4;
    if (nb > 0x7fffffff) return fail(MH_ERR_OVERFLOW, "too many rows");
    *nblocks_out = nb;
    dim3 g((unsigned)nb), b(kSThreads);
#define MH_RW(VEC, NE) hipLaunchKernelGGL((k_roww_fwd<V, VEC, NE>), g, b, 0, st, x, tg, out, rows, K, al, part)
    if (K % 4 == 0) {
        if (K <= 1024) MH_RW(true, 16);
        else MH_RW(true, kSLaneElems);
    } else {
        if (K <= 1024) MH_RW(false, 16);
        else MH_RW(false, kSLaneElems);
    }
#undef MH_RW
    return MH_OK;
}

template <int V>
static int launch_bwd(float* gx, const float* x, const float* up, const float* ug, int64_t rows, int K, float c) {
    hipStream_t st = ctx().stream;
    const bool al = al16s(x) && al16s(up) && al16s(gx);
    if (oneshot_classes(K) && al) {  // one-shot blocks of 64 rows, several launches past one dispatch
        const int64_t nb = (rows + kORows - 1) / kORows;
        for (int64_t b0 = 0; b0 < nb; b0 += kOMaxBlocks) {
            const int64_t cnt = nb - b0 < kOMaxBlocks ? nb - b0 : kOMaxBlocks;
            const int64_t r0 = b0 * kORows, off = r0 * K;
            const int64_t nr = rows - r0 < cnt * kORows ? rows - r0 : cnt * kORows;
            dim3 g((unsigned)cnt), b(kORows);
            switch (K) {
#define MH_K(KK) \
    case KK: hipLaunchKernelGGL((k_rowo_bwd<V, KK>), g, b, 0, st, gx + off, x + off, up + off, ug, nr, c); break;
                MH_ONESHOT_CLASSES(MH_K)
#undef MH_K
                default: return fail(MH_ERR_INVALID, "row kernel: %d classes", K);
            }
        }
        return MH_OK;
    }
    // multi-lane engine, aligned operands, rows of 33-64 classes (up to 32 the one-shot kernels
    // above take them: streamed over 8M elements, backwards of 17-32 classes 24-28 us there
    // against 30-56 us in this and the thread engine)
    if (K > 16 && K <= 4 * kMNE && al) {
        const int P = (K + kMNE - 1) / kMNE;
        const int64_t rpb = (int64_t)(kSThreads / 64) * (64 / P);
        const int64_t nb = (rows + rpb - 1) / rpb;
        if (nb > 0x7fffffff) return fail(MH_ERR_OVERFLOW, "too many rows");
        const bool vec = K % 4 == 0;
        dim3 g((unsigned)nb), b(kSThreads);
#define MH_RM(PP, VV) hipLaunchKernelGGL((k_rowm_bwd<V, PP, VV>), g, b, 0, st, gx, x, up, ug, rows, K, c)
        if (vec) {
            if (P == 2) MH_RM(2, true);
            else if (P == 3) MH_RM(3, true);
            else MH_RM(4, true);
        } else {
            if (P == 2) MH_RM(2, false);
            else if (P == 3) MH_RM(3, false);
            else MH_RM(4, false);
        }
#undef MH_RM
        return MH_OK;
    }
    if (K <= kSThreadMax) {
        const int rb = rows_per_block(3, K);
        const int64_t nb = (rows + rb - 1) / rb;
        if (nb > 0x7fffffff) return fail(MH_ERR_OVERFLOW, "too many rows");
        const size_t lds = 3 * (size_t)rb * (size_t)K * sizeof(float);
        dim3 g((unsigned)nb), b(kSThreads);
#define MH_RT(KM) hipLaunchKernelGGL((k_rowt_bwd<V, KM>), g, b, lds, st, gx, x, up, ug, rows, K, rb, al, c)
        if (K <= 8) MH_RT(8);
        else if (K <= 16) MH_RT(16);
        else if (K <= 32) MH_RT(32);
        else MH_RT(64);
#undef MH_RT
        return MH_OK;
    }
    const int64_t nb = (rows + 3) / 4;
    if (nb > 0x7fffffff) return fail(MH_ERR_OVERFLOW, "too many rows");
    dim3 g((unsigned)nb), b(kSThreads);
#define MH_RW(VEC, NE) hipLaunchKernelGGL((k_roww_bwd<V, VEC, NE>), g, b, 0, st, gx, x, up, ug, rows, K, al, c)
    if (K % 4 == 0) {
        if (K <= 1024) MH_RW(true, 16);
        else MH_RW(true, kSLaneElems);
    } else {
        if (K <= 1024) MH_RW(false, 16);
        else MH_RW(false, kSLaneElems);
    }
#undef MH_RW
    return MH_OK;
}

// Loss graphs: block partials, then the all-element sum with the graph's epilogue.
// `cscale` of the cross entropy: the graph scalar it multiplies by (NaN: f32(-1 / rows)).
template <int V>
static int loss_fwd(const char* what, float* loss, const float* x, const float* tg, int64_t rows, int64_t K,
                    float cscale = __builtin_nanf("")) {
    MH_TRY(check_rows(what, rows, K));
    if (!loss) return fail(MH_ERR_NULL, "%s: null loss", what);
    if (rows * K > 0 && (!x || !tg)) return fail(MH_ERR_NULL, "%s: null tensor", what);
    MH_TRY(require_init());
    const int64_t n = rows * K;
    const float ce = cscale == cscale ? cscale : (float)(-1.0 / (double)rows);
    if (n == 0) {  // MEAN of nothing: 0 / 0; the cross-entropy sum of nothing: 0 * the scale
        const float v = V == G_SMLM ? __builtin_nanf("") : 0.0f * ce;
        MH_TRY(mh_fill(loss, v, 1));
        return finish(what);
    }
    const int64_t nb_max = K <= kSThreadMax ? (rows + 31) / 32 : (rows + 3) / 4;  // >= any grid used
    const size_t np = ((size_t)nb_max + 63) & ~(size_t)63;
    const size_t t = reduce_abc_tmp_floats(RED_SUM, 1, nb_max, 1);
    float* part = nullptr;
    MH_TRY(scratch((np + t + 64) * sizeof(float), reinterpret_cast<void**>(&part)));
    int64_t nb = 0;
    const float lscale = V == G_SMLM ? (float)n : ce;
    MH_TRY(launch_fwd<V>(x, tg, nullptr, rows, (int)K, part, &nb));
    if (nb <= kLossCombMax) {  // MEAN.forward: / f32(N); cross entropy: SUM, then MUL(., f32(-1 / f64(rows)))
        hipLaunchKernelGGL((k_loss_comb<V>), dim3(1), dim3(kLCThreads), 0, ctx().stream, part, nb, loss, lscale);
        return finish(what);
    }
    if (V == G_SMLM)  // MEAN.forward: the sum of every element / f32(N)
        MH_TRY(reduce_abc(RED_SUM, EPI_MEAN, part, 1, nb, 1, loss, nullptr, (float)n, part + np));
    else  // SUM.forward, then MUL(., f32(-1 / f64(rows))) (loss.mojo:58-59)
        MH_TRY(reduce_abc(RED_SUM, EPI_SCALE, part, 1, nb, 1, loss, nullptr, ce, part + np));
    return finish(what);
}

template <int V>
static int loss_bwd(const char* what, float* gx, const float* x, const float* tg, const float* ug, int64_t rows,
                    int64_t K, float cscale = __builtin_nanf("")) {
    MH_TRY(check_rows(what, rows, K));
    const int64_t n = rows * K;
    if (n == 0) return MH_OK;
    if (!gx || !x || !tg || !ug) return fail(MH_ERR_NULL, "%s: null tensor", what);
    MH_TRY(require_init());
    const float c = V == G_SMLM ? (float)(1.0 / (double)n)  // MEAN.backward, basics.mojo:470-487
                                : (cscale == cscale ? cscale : (float)(-1.0 / (double)rows));  // loss.mojo:59
    MH_TRY(launch_bwd<V>(gx, x, tg, ug, rows, (int)K, c));
    return finish(what);
}

template <int V>
static int map_fwd(const char* what, float* out, const float* x, int64_t rows, int64_t K) {
    MH_TRY(check_rows(what, rows, K));
    if (rows * K == 0) return MH_OK;
    if (!out || !x) return fail(MH_ERR_NULL, "%s: null tensor", what);
    MH_TRY(require_init());
    int64_t nb = 0;
    MH_TRY(launch_fwd<V>(x, nullptr, out, rows, (int)K, nullptr, &nb));
    return finish(what);
}

template <int V>
static int map_bwd(const char* what, float* gx, const float* x, const float* gout, int64_t rows, int64_t K) {
    MH_TRY(check_rows(what, rows, K));
    if (rows * K == 0) return MH_OK;
    if (!gx || !x || !gout) return fail(MH_ERR_NULL, "%s: null tensor", what);
    MH_TRY(require_init());
    MH_TRY(launch_bwd<V>(gx, x, gout, nullptr, rows, (int)K, 0.0f));
    return finish(what);
}

int cross_entropy_fwd_c(float* loss, const float* x, const float* tg, int64_t rows, int64_t K, float scale) {
    return loss_fwd<G_CE>("cross entropy (graph)", loss, x, tg, rows, K, scale);
}

int cross_entropy_bwd_c(float* gx, const float* x, const float* tg, const float* ug, int64_t rows, int64_t K,
                        float scale) {
    return loss_bwd<G_CE>("cross entropy backward (graph)", gx, x, tg, ug, rows, K, scale);
}

}  // namespace mh

using namespace mh;

extern "C" {

int mh_softmax_log_mul_mean_fwd(float* loss, const float* x, const float* target, int64_t rows, int64_t classes) {
    MH_TRACE("mh_softmax_log_mul_mean_fwd");
    return loss_fwd<G_SMLM>("mh_softmax_log_mul_mean_fwd", loss, x, target, rows, classes);
}

int mh_softmax_log_mul_mean_bwd_accum(float* grad_x, const float* x, const float* target, const float* ug,
                                      int64_t rows, int64_t classes) {
    MH_TRACE("mh_softmax_log_mul_mean_bwd_accum");
    return loss_bwd<G_SMLM>("mh_softmax_log_mul_mean_bwd_accum", grad_x, x, target, ug, rows, classes);
}

int mh_cross_entropy_fwd(float* loss, const float* x, const float* target, int64_t rows, int64_t classes) {
    MH_TRACE("mh_cross_entropy_fwd");
    return loss_fwd<G_CE>("mh_cross_entropy_fwd", loss, x, target, rows, classes);
}

int mh_cross_entropy_bwd_accum(float* grad_x, const float* x, const float* target, const float* ug, int64_t rows,
                               int64_t classes) {
    MH_TRACE("mh_cross_entropy_bwd_accum");
    return loss_bwd<G_CE>("mh_cross_entropy_bwd_accum", grad_x, x, target, ug, rows, classes);
}

int mh_softmax_fwd(float* out, const float* x, int64_t rows, int64_t classes) {
    MH_TRACE("mh_softmax_fwd");
    return map_fwd<G_SOFTMAX>("mh_softmax_fwd", out, x, rows, classes);
}

int mh_softmax_bwd_accum(float* grad_x, const float* x, const float* grad_out, int64_t rows, int64_t classes) {
    MH_TRACE("mh_softmax_bwd_accum");
    return map_bwd<G_SOFTMAX>("mh_softmax_bwd_accum", grad_x, x, grad_out, rows, classes);
}

int mh_logsoftmax_fwd(float* out, const float* x, int64_t rows, int64_t classes) {
    MH_TRACE("mh_logsoftmax_fwd");
    return map_fwd<G_LOGSOFTMAX>("mh_logsoftmax_fwd", out, x, rows, classes);
}

int mh_logsoftmax_bwd_accum(float* grad_x, const float* x, const float* grad_out, int64_t rows, int64_t classes) {
    MH_TRACE("mh_logsoftmax_bwd_accum");
    return map_bwd<G_LOGSOFTMAX>("mh_logsoftmax_bwd_accum", grad_x, x, grad_out, rows, classes);
}

}  // extern "C"
