// mh_elementwise.hip -- forward and accumulating-backward elementwise kernels.
//
// One engine serves every elementwise entry point: an output stream (written, or
// read-modify-written for "grad = grad + rg") and up to four input streams, each FULL (same
// shape as the output), SCALAR (one element, loaded once per thread) or BCAST (strided in the
// collapsed output space). Same-shape work takes the float4 path: one-wavefront workgroups,
// one 128-bit access per stream per thread, all loads issued before any arithmetic. Two common
// broadcast forms of a [rows, K] output have engines of their own: per-row operands ([rows, 1],
// K >= 4: one fast division per quad) and per-column operands ([1, K], K % 4 == 0: one fast
// modulo per quad). Other broadcasts decode the output coordinate of each quad with
// precomputed fast divisors; an inner dimension divisible by 4 keeps 128-bit accesses for
// every operand whose inner stride is 0 or 1.
#include "mh_internal.h"
#include "mh_math.h"

namespace mh {

// One wavefront per workgroup: with non-temporal streams, 64-thread workgroups of one quad per
// thread streamed fastest on gfx950 for every operand count measured (a binary forward at 0.84
// of peak against 0.80 with 256 threads, the two-gradient backward 0.81 against 0.76).
constexpr int kThreads = 64;

struct DevScal {
    const float* p[4];
};

template <int N>
struct InPtrs {
    const float* p[N > 0 ? N : 1];
};

// ---------------------------------------------------------------------------------------
// functors: operator()(v) with v[k] the k-th input value; setup() reads device scalars.
// ---------------------------------------------------------------------------------------
template <int OP>
struct FBin {  // add/sub/mul/div, math_util.mojo:37-126
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const {
        if constexpr (OP == MH_ADD) return v[0] + v[1];
        else if constexpr (OP == MH_SUB) return v[0] - v[1];
        else if constexpr (OP == MH_MUL) return v[0] * v[1];
        else return v[0] / v[1];
    }
};

template <int OP>
struct FUn {  // elwise_transform bodies
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const {
        if constexpr (OP == MH_EXP) return mexp(v[0]);
        else if constexpr (OP == MH_LOG) return mlog(v[0]);
        else if constexpr (OP == MH_SIGMOID) return msigmoid(v[0]);
        else if constexpr (OP == MH_RELU) return mrelu(v[0]);
        else return mtanh(v[0]);
    }
};

struct FPowi {  // POW.forward: powi(x, Int(t2[0])), basics.mojo:320-327
    int64_t n;
    __device__ void setup(const DevScal& s) {
        float e = s.p[0][0];
        n = (e != e) ? 0 : (int64_t)__builtin_truncf(e);
    }
    __device__ float operator()(const float* v) const { return mpowi(v[0], n); }
};

struct FPowiN {  // elwise_pow with its integer exponent given, tensorutils.mojo:226-239
    int64_t n;
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const { return mpowi(v[0], n); }
};

template <int OP>
struct FUnBwd {  // v[0] = x, v[1] = ug: the rg of each unary struct backward
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const {
        const float x = v[0], ug = v[1];
        if constexpr (OP == MH_EXP) return mexp(x) * ug;  // basics.mojo:281-284
        else if constexpr (OP == MH_LOG) return ug / x;   // basics.mojo:305-309
        else if constexpr (OP == MH_SIGMOID) {            // mlops.mojo:50-76
            float s = msigmoid(x);
            return (s * (1.0f - s)) * ug;
        } else if constexpr (OP == MH_RELU) {             // mlops.mojo:99-125
            return (x > 0.0f ? 1.0f : 0.0f) * ug;
        } else {                                          // mlops.mojo:209-235
            float t = mtanh(x);
            return (1.0f - t * t) * ug;
        }
    }
};

struct FPowBwdX {  // basics.mojo:345-357: (a * (x + 1e-12) ** (a - 1)) * ug
    float a, am1;
    __device__ void setup(const DevScal& s) {
        a = s.p[0][0];
        am1 = a - 1.0f;
    }
    __device__ float operator()(const float* v) const { return (a * mpowf(v[0] + 1e-12f, am1)) * v[1]; }
};

// Binary struct backward of one operand (basics.mojo:28-219). Inputs: v[0] = ug, then
//   ADD, SUB id0: -            -> ug
//   SUB id1:      -            -> ug * -1
//   MUL id0:      v[1] = t2    -> ug * t2        MUL id1: v[1] = t1 -> ug * t1
//   DIV id0:      v[1] = t2    -> ug / t2
//   DIV id1:      v[1] = t1, v[2] = t2 -> ((-t1) / (t2 * t2)) * ug
//   DIV id1 with t2 of shape (1) (DIVS): v[1] = t1, f = -1 / (s * s) -> (f * t1) * ug
template <int OP, int ID, bool DIVS>
struct FBinRg {
    float f;
    __device__ void setup(const DevScal& s) {
        if constexpr (DIVS) {
            const float t = s.p[0][0];
            f = -1.0f / (t * t);
        }
    }
    __device__ float operator()(const float* v) const {
        const float ug = v[0];
        if constexpr (OP == MH_ADD) return ug;
        else if constexpr (OP == MH_SUB) return ID == 0 ? ug : ug * -1.0f;
        else if constexpr (OP == MH_MUL) return ug * v[1];
        else if constexpr (ID == 0) return ug / v[1];
        else if constexpr (DIVS) return (f * v[1]) * ug;
        else return ((-v[1]) / (v[2] * v[2])) * ug;
    }
};

// SUM/MEAN axis backward (basics.mojo:416-425, 489-506): fill(c) then accumulate_op[mul]
// with the broadcast ug: rg = c * ug; TWICE (rg = (c * ug) * ug) when the reduced shape
// equals the input shape (accumulate_op applies func twice then, tensorutils.mojo:380-393).
template <bool TWICE>
struct FScaleBcast {
    float c;
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const {
        if constexpr (TWICE) return (c * v[0]) * v[0];
        else return c * v[0];
    }
};

// MEAN all-element backward (basics.mojo:470-487): g = f32(1/N) * ug[0], filled.
struct FMeanAll {
    float c, g;
    __device__ void setup(const DevScal& s) { g = c * s.p[0][0]; }
    __device__ float operator()(const float*) const { return g; }
};

// MAX backward routing (basics.mojo:567-577, 597-613): v[0] = x, v[1] = line max,
// v[2] = fl(1/count) of the line, v[3] = ug of the line.
struct FMaxRoute {
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const { return v[0] == v[1] ? v[2] * v[3] : 0.0f; }
};

// Accumulating functors whose contribution is +0 almost everywhere: the engines store a quad
// only when its bits change (bits_differ4), which leaves memory exactly as storing every quad
// would, without writing back the untouched ones.
template <class F>
constexpr bool kSparseAccum = false;
template <>
constexpr bool kSparseAccum<FMaxRoute> = true;

struct FFma {  // FMA.forward, basics.mojo:782-786: t1.fma(t2, t3), a single rounding
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const { return __builtin_fmaf(v[0], v[1], v[2]); }
};

struct FLeaky {  // LEAKYRELU.forward, mlops.mojo:141-154
    float slope;
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const { return v[0] > 0.0f ? v[0] : v[0] * slope; }
};

struct FLeakyBwd {  // v[0] = x, v[1] = ug: LEAKYRELU.backward, mlops.mojo:164-184
    float slope;
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const { return (v[0] > 0.0f ? 1.0f : slope) * v[1]; }
};

// min / max as LLVM minnum / maxnum: a NaN operand yields the other one, equal operands the
// first, so a NaN input clips to hi.
__device__ __forceinline__ float minnum_f(float a, float b) { return (b < a || a != a) ? b : a; }
__device__ __forceinline__ float maxnum_f(float a, float b) { return (b > a || a != a) ? b : a; }

struct FClip {  // CLIP.forward, mlops.mojo:243-266: max(min(x, hi), lo)
    float lo, hi;
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const { return maxnum_f(minnum_f(v[0], hi), lo); }
};

struct FClipBwd {  // v[0] = x, v[1] = ug: CLIP.backward, mlops.mojo:281-297
    float lo, hi;
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const { return (v[0] >= lo && v[0] <= hi) ? v[1] : 0.0f; }
};

template <int ID>
struct FFmaRg {  // FMA.backward, basics.mojo:804-817: id 0 ug * t2, id 1 ug * t1, id 2 ug
    __device__ void setup(const DevScal&) {}
    __device__ float operator()(const float* v) const {
        if constexpr (ID == 2) return v[0];
        else return v[0] * v[1];
    }
};

// ---------------------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------------------

// Same-shape engine: all inputs FULL or SCALAR (bit k of smask). One quad (16 B per
// stream) per thread, and no loop: on gfx950 this streams faster than several quads per
// thread (fewer bytes in flight per wave, more waves resident), and at config-5 sizes a grid
// loop that ran once still cost about 6 %. A launch covers at most kMaxLaunchQuads quads
// (the launcher splits longer tensors); block 0's first thread takes the n % 4 tail.
template <class F, int NIN, bool ACCUM>
__global__ void __launch_bounds__(kThreads)
    k_same4(float* __restrict__ out, InPtrs<NIN> in, int smask, int64_t n, DevScal ds, F f) {
    const int64_t nq = n >> 2;
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    float4 iv[NIN > 0 ? NIN : 1];
    float4 ov;
    if (q < nq) {
#pragma unroll
        for (int k = 0; k < NIN; ++k)
            if (!((smask >> k) & 1)) iv[k] = ld_nt4(in.p[k], q);
        if (ACCUM) ov = ld_nt4(out, q);
    }
    // device scalars (the functor's, scalar operands) after the quads' loads: read first, the
    // wave waited for them before its quads' loads went out
    __builtin_amdgcn_sched_barrier(0);
    f.setup(ds);
    float sv[NIN > 0 ? NIN : 1];
#pragma unroll
    for (int k = 0; k < NIN; ++k) sv[k] = ((smask >> k) & 1) ? in.p[k][0] : 0.0f;
    if (q < nq) {
        float r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v[NIN > 0 ? NIN : 1];
#pragma unroll
            for (int k = 0; k < NIN; ++k) v[k] = ((smask >> k) & 1) ? sv[k] : comp(iv[k], j);
            r[j] = f(v);
            if (ACCUM) r[j] = comp(ov, j) + r[j];
        }
        if (!(ACCUM && kSparseAccum<F>) || bits_differ4(ov.x, ov.y, ov.z, ov.w, r[0], r[1], r[2], r[3]))
            st_nt4(out, q, make_float4(r[0], r[1], r[2], r[3]));
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        for (int64_t i = nq << 2; i < n; ++i) {
            float v[NIN > 0 ? NIN : 1];
#pragma unroll
            for (int k = 0; k < NIN; ++k) v[k] = ((smask >> k) & 1) ? sv[k] : in.p[k][i];
            float r = f(v);
            out[i] = ACCUM ? out[i] + r : r;
        }
    }
}

// Same-shape engine, scalar accesses (some pointer not 16-byte aligned).
template <class F, int NIN, bool ACCUM>
__global__ void __launch_bounds__(kThreads)
    k_same1(float* __restrict__ out, InPtrs<NIN> in, int smask, int64_t n, DevScal ds, F f) {
    f.setup(ds);
    float sv[NIN > 0 ? NIN : 1];
#pragma unroll
    for (int k = 0; k < NIN; ++k) sv[k] = ((smask >> k) & 1) ? in.p[k][0] : 0.0f;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        float v[NIN > 0 ? NIN : 1];
#pragma unroll
        for (int k = 0; k < NIN; ++k) v[k] = ((smask >> k) & 1) ? sv[k] : ld_nt(in.p[k] + i);
        float r = f(v);
        st_nt(out + i, ACCUM ? ld_nt(out + i) + r : r);
    }
}

// Kind of operand k in the row/column/plane engines, from two bits per operand in kinds. A
// lone operand is the broadcast one (these engines run only on plans with one), which makes
// its kind a compile-time constant: no scalar load or kind test at wave start. KS >= 0 fixes
// the kinds of two operands at compile time (a full operand and a broadcast one, in either
// order: KS_FB, KS_BF); with kinds known only at run time, each operand's loads sit in a branch
// on its kind, and the compiler waits at the branch's end for the loads issued so far, so a
// broadcast operand ahead of a full one cost a second memory round trip.
constexpr int KS_RUN = -1;
constexpr int KS_FB = IN_FULL | (IN_BCAST << 2);
constexpr int KS_BF = IN_BCAST | (IN_FULL << 2);
template <int NIN, int KS = KS_RUN>
__device__ __forceinline__ int bc_kind(int kinds, int k) {
    if constexpr (NIN == 1) return (int)IN_BCAST;
    return ((KS >= 0 ? KS : kinds) >> (2 * k)) & 3;
}

// KS for a launch: the compile-time form for two operands of those kinds
static inline int bc_static_kinds(int nin, int kinds) {
    return nin == 2 && (kinds == KS_FB || kinds == KS_BF) ? kinds : KS_RUN;
}

// The general engine's kind of operand k: from the plan, or fixed by KS
template <int NIN, int KS>
__device__ __forceinline__ int bc_kind_pl(const ElwPlan& pl, int k) {
    if constexpr (KS >= 0) return (KS >> (2 * k)) & 3;
    return pl.kind[k];
}

// Row-broadcast engine: output [rows, K] with K >= 4 and fewer than 2^31 elements, every
// IN_BCAST operand a contiguous per-row vector ([rows, 1], as a row max or row sum is), the
// output and FULL operands 16-byte aligned. One quad per thread: the quad's first row comes
// from one fast division, and as K >= 4 at most one row boundary falls inside it, so a row
// operand contributes its values at rows r0 and r0 + 1. Both are loaded unconditionally (the
// second from an index clamped to the last row, used only where the quad reaches that row),
// so the two loads are in flight together: loading the second under a branch made every
// quad wait for the first before issuing it. kinds holds two bits of InKind per operand.
// Element values are the same single operations as every engine.
template <class F, int NIN, bool ACCUM, int KS = KS_RUN>
__global__ void __launch_bounds__(kThreads)
    k_rowbc4(float* __restrict__ out, InPtrs<NIN> in, int kinds, int64_t n, uint32_t K, uint32_t last_row,
             FastDiv fk, DevScal ds, F f) {
    constexpr int NA = NIN > 0 ? NIN : 1;
    f.setup(ds);
    float sv[NA];
#pragma unroll
    for (int k = 0; k < NIN; ++k) sv[k] = bc_kind<NIN, KS>(kinds, k) == IN_SCALAR ? in.p[k][0] : 0.0f;
    const int64_t nq = n >> 2;
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (q < nq) {
        const uint32_t e0 = (uint32_t)(q << 2);
        const uint32_t r0 = fdiv(e0, fk);
        const uint32_t c0 = e0 - r0 * K;
        const int jc = c0 + 3 >= K ? (int)(K - c0) : 4;  // first element of the quad in row r0 + 1
        const uint32_t r1 = r0 < last_row ? r0 + 1 : last_row;
        float v[4][NA];
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
            const int kind = bc_kind<NIN, KS>(kinds, k);
            if (kind == IN_SCALAR) {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j][k] = sv[k];
            } else if (kind == IN_FULL) {
                const vf4 t = ld_ntv(in.p[k], q);
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j][k] = t[j];
            } else {
                const float a = in.p[k][r0];
                const float b = in.p[k][r1];
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j][k] = j < jc ? a : b;
            }
        }
        vf4 o = vf4{0.f, 0.f, 0.f, 0.f};
        if (ACCUM) o = ld_ntv(out, q);
        vf4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float fv = f(v[j]);
            r[j] = ACCUM ? o[j] + fv : fv;
        }
        if (!(ACCUM && kSparseAccum<F>) || bits_differ4(o[0], o[1], o[2], o[3], r[0], r[1], r[2], r[3]))
            st_ntv(out, q, r);
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        for (int64_t i = nq << 2; i < n; ++i) {
            const int64_t row = i / (int64_t)K;
            float v[NA];
#pragma unroll
            for (int k = 0; k < NIN; ++k) {
                const int kind = bc_kind<NIN, KS>(kinds, k);
                v[k] = kind == IN_SCALAR ? sv[k] : (kind == IN_FULL ? in.p[k][i] : in.p[k][row]);
            }
            const float fv = f(v);
            out[i] = ACCUM ? out[i] + fv : fv;
        }
    }
}

// Column-broadcast engine: output [rows, C] with C % 4 == 0 and fewer than 2^31 elements,
// every IN_BCAST operand a contiguous per-column vector ([1, C], as a column max or a bias
// is), all operands and the output 16-byte aligned. One quad per thread in flat order (one
// sequential stream, as for same-shape operands); the quad's column quad is q mod C/4 (one
// fast division), whose operand quads are small enough to stay in L2.
template <class F, int NIN, bool ACCUM, int KS = KS_RUN>
__global__ void __launch_bounds__(kThreads)
    k_colbc4(float* __restrict__ out, InPtrs<NIN> in, int kinds, int64_t nq, uint32_t Cq, FastDiv fcq, DevScal ds,
             F f) {
    constexpr int NA = NIN > 0 ? NIN : 1;
    f.setup(ds);
    float sv[NA];
#pragma unroll
    for (int k = 0; k < NIN; ++k) sv[k] = bc_kind<NIN, KS>(kinds, k) == IN_SCALAR ? in.p[k][0] : 0.0f;
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (q < nq) {
        const uint32_t cq = (uint32_t)q - fdiv((uint32_t)q, fcq) * Cq;
        vf4 t[NA];
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
            const int kind = bc_kind<NIN, KS>(kinds, k);
            if (kind == IN_FULL) t[k] = ld_ntv(in.p[k], q);
            else if (kind == IN_BCAST) t[k] = reinterpret_cast<const vf4*>(in.p[k])[cq];
            else t[k] = vf4{sv[k], sv[k], sv[k], sv[k]};
        }
        vf4 o = vf4{0.f, 0.f, 0.f, 0.f};
        if (ACCUM) o = ld_ntv(out, q);
        vf4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v[NA];
#pragma unroll
            for (int k = 0; k < NIN; ++k) v[k] = t[k][j];
            const float fv = f(v);
            r[j] = ACCUM ? o[j] + fv : fv;
        }
        if (!(ACCUM && kSparseAccum<F>) || bits_differ4(o[0], o[1], o[2], o[3], r[0], r[1], r[2], r[3]))
            st_ntv(out, q, r);
    }
}

// Plane-broadcast engine: output [N, C, S] with S % 4 == 0 and fewer than 2^31 elements,
// every IN_BCAST operand a per-channel vector ([1, C, 1], as an NCHW bias is), the output and
// FULL operands 16-byte aligned. One quad per thread in flat order; a quad lies in one plane
// (S % 4 == 0), whose channel is (q / (S / 4)) mod C (two fast divisions).
template <class F, int NIN, bool ACCUM, int KS = KS_RUN>
__global__ void __launch_bounds__(kThreads)
    k_planebc4(float* __restrict__ out, InPtrs<NIN> in, int kinds, int64_t nq, uint32_t C, FastDiv fsq, FastDiv fc,
               DevScal ds, F f) {
    constexpr int NA = NIN > 0 ? NIN : 1;
    f.setup(ds);
    float sv[NA];
#pragma unroll
    for (int k = 0; k < NIN; ++k) sv[k] = bc_kind<NIN, KS>(kinds, k) == IN_SCALAR ? in.p[k][0] : 0.0f;
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (q < nq) {
        const uint32_t p = fdiv((uint32_t)q, fsq);
        const uint32_t c = p - fdiv(p, fc) * C;
        vf4 t[NA];
#pragma unroll
        for (int k = 0; k < NIN; ++k) {
            const int kind = bc_kind<NIN, KS>(kinds, k);
            if (kind == IN_FULL) {
                t[k] = ld_ntv(in.p[k], q);
            } else {
                const float b = kind == IN_BCAST ? in.p[k][c] : sv[k];
                t[k] = vf4{b, b, b, b};
            }
        }
        vf4 o = vf4{0.f, 0.f, 0.f, 0.f};
        if (ACCUM) o = ld_ntv(out, q);
        vf4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v[NA];
#pragma unroll
            for (int k = 0; k < NIN; ++k) v[k] = t[k][j];
            const float fv = f(v);
            r[j] = ACCUM ? o[j] + fv : fv;
        }
        if (!(ACCUM && kSparseAccum<F>) || bits_differ4(o[0], o[1], o[2], o[3], r[0], r[1], r[2], r[3]))
            st_ntv(out, q, r);
    }
}

// Broadcast engine, 128-bit path: the output and every FULL operand stream as flat float4
// quads whatever the shape (all must be 16-byte aligned); only the broadcast operands are
// gathered, with 32-bit offsets below 2^31 elements and a decode loop bounded by MAXR.
// The quad's first element is decoded. INNER4 (inner dim a multiple of 4, broadcast
// operands 16-byte aligned): a quad never crosses a row, and an operand contiguous along
// the inner dim is read as one float4. Otherwise elements past the end of the row are in
// the next one, whose offsets follow by addition while the next-outer coordinate does not
// wrap (a full decode per element only for rows shorter than 4 or at such a wrap); an
// operand constant along the inner dim is read once per row touched.
template <class F, int NIN, bool ACCUM, bool INNER4, bool BIG, int MAXR, int KS = KS_RUN>
__global__ void __launch_bounds__(kThreads)
    k_bcast4(float* __restrict__ out, InPtrs<NIN> in, ElwPlan pl, DevScal ds, F f) {
    constexpr int NA = NIN > 0 ? NIN : 1;
    using OT = off_type<BIG>;
    f.setup(ds);
    float sv[NA];
#pragma unroll
    for (int k = 0; k < NIN; ++k) sv[k] = bc_kind_pl<NIN, KS>(pl, k) == IN_SCALAR ? in.p[k][0] : 0.0f;
    const int inner = pl.rank - 1;
    const int64_t dinner = pl.dims[inner];
    const int64_t douter = inner > 0 ? pl.dims[inner - 1] : 1;
    const int64_t nq = pl.n >> 2;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < nq; q += stride) {
        const int64_t idx = q * 4;
        OT off0[NA];
        int64_t cin = 0, cprev = -1;
        bcast_decode<NIN, BIG, MAXR>(pl, idx, off0, &cin, &cprev);
        float v[4][NA];
        int jc = 4;         // first element of the quad in the next row (4: none)
        bool slow = false;  // per-element decode (row shorter than 4, or the next-outer coordinate wraps)
        OT offc[NA];        // offsets of element jc
        if (!INNER4 && cin + 3 >= dinner) {
            jc = (int)(dinner - cin);
            if (dinner >= 4 && inner > 0 && cprev + 1 < douter) {
#pragma unroll
                for (int k = 0; k < NIN; ++k)
                    offc[k] = off0[k] + (OT)pl.st[k][inner - 1] - (OT)cin * (OT)pl.st[k][inner];
            } else {
                slow = true;
            }
        }
        // with the kinds fixed (KS), broadcast operands go first: their loads sit under run-time
        // branches on the stride, whose joins wait for the loads issued before them, so a full
        // operand loaded ahead would be waited for there (two memory round trips per quad)
#pragma unroll
        for (int kk = 0; kk < NIN; ++kk) {
            const int k = KS == KS_FB ? NIN - 1 - kk : kk;
            if (bc_kind_pl<NIN, KS>(pl, k) == IN_SCALAR) {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j][k] = sv[k];
            } else if (bc_kind_pl<NIN, KS>(pl, k) == IN_FULL) {
                const float4 t = ld_nt4(in.p[k], q);
                v[0][k] = t.x; v[1][k] = t.y; v[2][k] = t.z; v[3][k] = t.w;
            } else if (INNER4) {
                if (pl.st[k][inner] == 1) {
                    const float4 t = *reinterpret_cast<const float4*>(in.p[k] + off0[k]);
                    v[0][k] = t.x; v[1][k] = t.y; v[2][k] = t.z; v[3][k] = t.w;
                } else {
                    const float t = in.p[k][off0[k]];
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j][k] = t;
                }
            } else if (!slow) {
                const OT si = (OT)pl.st[k][inner];
                if (si == 0) {
                    const float a = in.p[k][off0[k]];
                    const float b = jc < 4 ? in.p[k][offc[k]] : a;
#pragma unroll
                    for (int j = 0; j < 4; ++j) v[j][k] = j < jc ? a : b;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        v[j][k] = in.p[k][j < jc ? off0[k] + (OT)j * si : offc[k] + (OT)(j - jc) * si];
                }
            }
        }
        if (slow) {  // broadcast operands element by element
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                OT oj[NA];
                int64_t c1, c2;
                if (j < jc) {
#pragma unroll
                    for (int k = 0; k < NIN; ++k) oj[k] = off0[k] + (OT)j * (OT)pl.st[k][inner];
                } else {
                    bcast_decode<NIN, BIG, MAXR>(pl, idx + j, oj, &c1, &c2);
                }
#pragma unroll
                for (int k = 0; k < NIN; ++k)
                    if (bc_kind_pl<NIN, KS>(pl, k) == IN_BCAST) v[j][k] = in.p[k][oj[k]];
            }
        }
        const float4 o = ACCUM ? ld_nt4(out, q) : make_float4(0.f, 0.f, 0.f, 0.f);
        float r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r[j] = f(v[j]);
            if (ACCUM) r[j] = comp(o, j) + r[j];
        }
        if (ACCUM && kSparseAccum<F> && !bits_differ4(o.x, o.y, o.z, o.w, r[0], r[1], r[2], r[3])) continue;
        st_nt4(out, q, make_float4(r[0], r[1], r[2], r[3]));
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        for (int64_t i = nq << 2; i < pl.n; ++i) {
            OT off1[NA];
            int64_t c, c2;
            bcast_decode<NIN, BIG, MAXR>(pl, i, off1, &c, &c2);
            float v1[NA];
#pragma unroll
            for (int k = 0; k < NIN; ++k)
                v1[k] = bc_kind_pl<NIN, KS>(pl, k) == IN_SCALAR ? sv[k] : (bc_kind_pl<NIN, KS>(pl, k) == IN_FULL ? in.p[k][i] : in.p[k][off1[k]]);
            const float r1 = f(v1);
            out[i] = ACCUM ? out[i] + r1 : r1;
        }
    }
}

// Broadcast engine, scalar path (the output or a FULL operand is not 16-byte aligned).
template <class F, int NIN, bool ACCUM, bool BIG>
__global__ void __launch_bounds__(kThreads)
    k_bcast1(float* __restrict__ out, InPtrs<NIN> in, ElwPlan pl, DevScal ds, F f) {
    constexpr int NA = NIN > 0 ? NIN : 1;
    using OT = off_type<BIG>;
    f.setup(ds);
    float sv[NA];
#pragma unroll
    for (int k = 0; k < NIN; ++k) sv[k] = pl.kind[k] == IN_SCALAR ? in.p[k][0] : 0.0f;
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < pl.n; i += stride) {
        OT off[NA];
        int64_t c, c2;
        bcast_decode<NIN, BIG, MH_MAX_RANK>(pl, i, off, &c, &c2);
        float v[NA];
#pragma unroll
        for (int k = 0; k < NIN; ++k)
            v[k] = pl.kind[k] == IN_SCALAR ? sv[k] : (pl.kind[k] == IN_FULL ? in.p[k][i] : in.p[k][off[k]]);
        const float r = f(v);
        out[i] = ACCUM ? out[i] + r : r;
    }
}

// Fused two-operand backward of a same-shape binary op (both backward_op calls of
// ops.mojo:408-463 with equal shapes): g1 = g1 + rg0, g2 = g2 + rg1. One quad per thread, no
// loop, as k_same4. ALIAS: both operands are one symbol (x * x, x + x), so both calls
// accumulate into one gradient, id 0 first (model.mojo:233-270): g1 = (g1 + rg0) + rg1, and
// g2 is not used.
template <int OP, bool ALIAS = false>
__global__ void __launch_bounds__(kThreads)
    k_bwd2_same4(float* __restrict__ g1, float* __restrict__ g2, const float* __restrict__ ug,
                 const float* __restrict__ a, const float* __restrict__ b, int64_t n) {
    constexpr bool NEED_AB = (OP == MH_MUL || OP == MH_DIV);
    const int64_t nq = n >> 2;
    FBinRg<OP, 0, false> f0;
    FBinRg<OP, 1, false> f1;
    const int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (q < nq) {
        const float4 vu = ld_nt4(ug, q);
        float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
        if (NEED_AB) {
            va = ld_nt4(a, q);
            vb = ld_nt4(b, q);
        }
        const float4 v1 = ld_nt4(g1, q);
        const float4 v2 = ALIAS ? v1 : ld_nt4(g2, q);
        float r1[4], r2[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float uu = comp(vu, j);
            const float aa = comp(va, j);
            const float bb = comp(vb, j);
            float x0[3] = {uu, bb, 0.0f};  // id0 reads t2
            float x1[3] = {uu, aa, bb};    // id1 reads t1 (and t2 for DIV)
            r1[j] = comp(v1, j) + f0(x0);
            r2[j] = ALIAS ? r1[j] + f1(x1) : comp(v2, j) + f1(x1);
        }
        if (ALIAS) {
            st_nt4(g1, q, make_float4(r2[0], r2[1], r2[2], r2[3]));
        } else {
            st_nt4(g1, q, make_float4(r1[0], r1[1], r1[2], r1[3]));
            st_nt4(g2, q, make_float4(r2[0], r2[1], r2[2], r2[3]));
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        for (int64_t i = nq << 2; i < n; ++i) {
            const float aa = NEED_AB ? a[i] : 0.0f, bb = NEED_AB ? b[i] : 0.0f;
            float x0[3] = {ug[i], bb, 0.0f};
            float x1[3] = {ug[i], aa, bb};
            if (ALIAS) {
                g1[i] = (g1[i] + f0(x0)) + f1(x1);
            } else {
                g1[i] = g1[i] + f0(x0);
                g2[i] = g2[i] + f1(x1);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------
static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Workgroups of a launch of one thread per item. The one-quad-per-thread kernels get at most
// kMaxLaunchQuads items per launch (every launch site splits longer tensors); k_bcast4 and
// k_same1, which loop over their grid, take the clamped grid whatever the count.
static inline unsigned grid_for(int64_t items, int per_block) { return (unsigned)grid_blocks(items, per_block); }

// The same-shape engine's launch (k_same4, k_bwd2_same4): a thread per quad, in launches of at
// most kMaxLaunchQuads quads.
LaunchShape elw_same_launch(int64_t n) {
    const int64_t nq = n >> 2;
    return LaunchShape{0, kThreads, grid_blocks(nq < kMaxLaunchQuads ? nq : kMaxLaunchQuads, kThreads), launch_count(nq)};
}

// Runs F over the plan: out (shape = plan output) = F(inputs), or out += F(inputs).
template <class F, int NIN, bool ACCUM>
static int run_map(float* out, const ElwPlan& pl, const float* const* ptrs, const DevScal& ds, F f) {
    if (pl.n == 0) return MH_OK;
    InPtrs<NIN> in;
    for (int k = 0; k < NIN; ++k) in.p[k] = ptrs[k];
    hipStream_t st = ctx().stream;
    bool al = aligned16(out);  // the output and every FULL operand are 16-byte aligned
    for (int k = 0; k < NIN; ++k)
        if (pl.kind[k] == IN_FULL) al = al && aligned16(ptrs[k]);
    if (!pl.any_bcast) {
        int smask = 0;
        for (int k = 0; k < NIN; ++k)
            if (pl.kind[k] == IN_SCALAR) smask |= 1 << k;
        if (al) {  // a thread per quad; past kMaxLaunchQuads quads, several launches
            for (int64_t off = 0; off < pl.n; off += 4 * kMaxLaunchQuads) {
                const int64_t cnt = pl.n - off < 4 * kMaxLaunchQuads ? pl.n - off : 4 * kMaxLaunchQuads;
                InPtrs<NIN> part = in;
                for (int k = 0; k < NIN; ++k)
                    if (!((smask >> k) & 1)) part.p[k] += off;
                hipLaunchKernelGGL((k_same4<F, NIN, ACCUM>), dim3(grid_for(cnt >> 2, kThreads)), dim3(kThreads), 0,
                                   st, out + off, part, smask, cnt, ds, f);
            }
        } else {
            int64_t b = (pl.n + kThreads - 1) / kThreads;
            if (b > 65536) b = 65536;
            hipLaunchKernelGGL((k_same1<F, NIN, ACCUM>), dim3((unsigned)b), dim3(kThreads), 0, st, out,
                               in, smask, pl.n, ds, f);
        }
        return MH_OK;
    }
    const bool big = pl.n >= ((int64_t)1 << 31);
    bool al_b = true;  // broadcast operands 16-byte aligned (float4 gathers when INNER4)
    for (int k = 0; k < NIN; ++k)
        if (pl.kind[k] == IN_BCAST) al_b = al_b && aligned16(ptrs[k]);
    if (al) {
        dim3 g(grid_for(pl.n >> 2, kThreads)), b(kThreads);
        bool rowform = !big && pl.rank == 2 && pl.dims[1] >= 4;  // [rows, K] with per-row operands
        int kinds = 0;
        for (int k = 0; k < NIN; ++k) {
            if (pl.kind[k] == IN_BCAST && !(pl.st[k][0] == 1 && pl.st[k][1] == 0)) rowform = false;
            kinds |= pl.kind[k] << (2 * k);
        }
        if (rowform) {
            const uint32_t K = (uint32_t)pl.dims[1];
            const uint32_t last_row = (uint32_t)(pl.n / K) - 1;  // pl.n > 0: empty tensors return earlier
            const FastDiv fk = make_fastdiv(K);
            if constexpr (NIN == 2) {  // a full and a broadcast operand: kinds fixed at compile time
                const int ks = bc_static_kinds(NIN, kinds);
                if (ks == KS_FB) {
                    hipLaunchKernelGGL((k_rowbc4<F, NIN, ACCUM, KS_FB>), g, b, 0, st, out, in, kinds, pl.n, K,
                                       last_row, fk, ds, f);
                    return MH_OK;
                }
                if (ks == KS_BF) {
                    hipLaunchKernelGGL((k_rowbc4<F, NIN, ACCUM, KS_BF>), g, b, 0, st, out, in, kinds, pl.n, K,
                                       last_row, fk, ds, f);
                    return MH_OK;
                }
            }
            hipLaunchKernelGGL((k_rowbc4<F, NIN, ACCUM>), g, b, 0, st, out, in, kinds, pl.n, K, last_row,
                               fk, ds, f);
            return MH_OK;
        }
        // [rows, C] with per-column operands ([1, C]), C % 4 == 0
        bool colform = !big && pl.rank == 2 && pl.dims[1] % 4 == 0 && al_b;
        for (int k = 0; k < NIN; ++k)
            if (pl.kind[k] == IN_BCAST && !(pl.st[k][0] == 0 && pl.st[k][1] == 1)) colform = false;
        // [N, C, S] with per-channel operands ([1, C, 1]), S % 4 == 0
        bool planeform = !big && pl.rank == 3 && pl.dims[2] % 4 == 0;
        for (int k = 0; k < NIN; ++k)
            if (pl.kind[k] == IN_BCAST && !(pl.st[k][0] == 0 && pl.st[k][1] == 1 && pl.st[k][2] == 0)) planeform = false;
        if (planeform) {
            const uint32_t C = (uint32_t)pl.dims[1], Sq = (uint32_t)(pl.dims[2] / 4);
            const FastDiv fsq = make_fastdiv(Sq), fc = make_fastdiv(C);
            if constexpr (NIN == 2) {  // a full and a broadcast operand: kinds fixed at compile time
                const int ks = bc_static_kinds(NIN, kinds);
                if (ks == KS_FB) {
                    hipLaunchKernelGGL((k_planebc4<F, NIN, ACCUM, KS_FB>), g, b, 0, st, out, in, kinds, pl.n >> 2, C,
                                       fsq, fc, ds, f);
                    return MH_OK;
                }
                if (ks == KS_BF) {
                    hipLaunchKernelGGL((k_planebc4<F, NIN, ACCUM, KS_BF>), g, b, 0, st, out, in, kinds, pl.n >> 2, C,
                                       fsq, fc, ds, f);
                    return MH_OK;
                }
            }
            hipLaunchKernelGGL((k_planebc4<F, NIN, ACCUM>), g, b, 0, st, out, in, kinds, pl.n >> 2, C, fsq,
                               fc, ds, f);
            return MH_OK;
        }
        if (colform) {
            const uint32_t Cq = (uint32_t)(pl.dims[1] / 4);
            const FastDiv fcq = make_fastdiv(Cq);
            if constexpr (NIN == 2) {  // a full and a broadcast operand: kinds fixed at compile time
                const int ks = bc_static_kinds(NIN, kinds);
                if (ks == KS_FB) {
                    hipLaunchKernelGGL((k_colbc4<F, NIN, ACCUM, KS_FB>), g, b, 0, st, out, in, kinds, pl.n >> 2, Cq,
                                       fcq, ds, f);
                    return MH_OK;
                }
                if (ks == KS_BF) {
                    hipLaunchKernelGGL((k_colbc4<F, NIN, ACCUM, KS_BF>), g, b, 0, st, out, in, kinds, pl.n >> 2, Cq,
                                       fcq, ds, f);
                    return MH_OK;
                }
            }
            hipLaunchKernelGGL((k_colbc4<F, NIN, ACCUM>), g, b, 0, st, out, in, kinds, pl.n >> 2, Cq, fcq, ds,
                               f);
            return MH_OK;
        }
        const bool inner4 = pl.vec_ok && al_b;
        if (big) {  // 64-bit offsets, any rank
            if (inner4) hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, true, true, MH_MAX_RANK>), g, b, 0, st, out, in, pl, ds, f);
            else hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, false, true, MH_MAX_RANK>), g, b, 0, st, out, in, pl, ds, f);
        } else if (pl.rank <= 3) {
            if constexpr (NIN == 2) {  // a full and a broadcast operand: kinds fixed at compile time
                const int ks = bc_static_kinds(NIN, kinds);
                if (ks == KS_FB) {
                    if (inner4) hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, true, false, 3, KS_FB>), g, b, 0, st, out,
                                                   in, pl, ds, f);
                    else hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, false, false, 3, KS_FB>), g, b, 0, st, out, in,
                                            pl, ds, f);
                    return MH_OK;
                }
                if (ks == KS_BF) {
                    if (inner4) hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, true, false, 3, KS_BF>), g, b, 0, st, out,
                                                   in, pl, ds, f);
                    else hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, false, false, 3, KS_BF>), g, b, 0, st, out, in,
                                            pl, ds, f);
                    return MH_OK;
                }
            }
            if (inner4) hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, true, false, 3>), g, b, 0, st, out, in, pl, ds, f);
            else hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, false, false, 3>), g, b, 0, st, out, in, pl, ds, f);
        } else {
            if (inner4) hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, true, false, MH_MAX_RANK>), g, b, 0, st, out, in, pl, ds, f);
            else hipLaunchKernelGGL((k_bcast4<F, NIN, ACCUM, false, false, MH_MAX_RANK>), g, b, 0, st, out, in, pl, ds, f);
        }
        return MH_OK;
    }
    int64_t blocks = (pl.n + kThreads - 1) / kThreads;
    if (blocks > 262144) blocks = 262144;
    if (blocks < 1) blocks = 1;
    dim3 g((unsigned)blocks), b(kThreads);
    if (big) hipLaunchKernelGGL((k_bcast1<F, NIN, ACCUM, true>), g, b, 0, st, out, in, pl, ds, f);
    else hipLaunchKernelGGL((k_bcast1<F, NIN, ACCUM, false>), g, b, 0, st, out, in, pl, ds, f);
    return MH_OK;
}

static DevScal no_scal() {
    DevScal d;
    for (int i = 0; i < 4; ++i) d.p[i] = nullptr;
    return d;
}
static DevScal scal1(const float* p) {
    DevScal d = no_scal();
    d.p[0] = p;
    return d;
}

static int check_op_binary(int op) {
    if (op < MH_ADD || op > MH_DIV) return fail(MH_ERR_OP, "op %d is not ADD/SUB/MUL/DIV", op);
    return MH_OK;
}
static int check_op_unary(int op) {
    if (op != MH_EXP && op != MH_LOG && op != MH_SIGMOID && op != MH_RELU && op != MH_TANH)
        return fail(MH_ERR_OP, "op %d is not EXP/LOG/SIGMOID/RELU/TANH", op);
    return MH_OK;
}

template <int OP>
static int binary_fwd_t(float* res, const ElwPlan& pl, const float* a, const float* b) {
    const float* p[2] = {a, b};
    return run_map<FBin<OP>, 2, false>(res, pl, p, no_scal(), FBin<OP>{});
}

template <int OP>
static int unary_fwd_t(float* res, const ElwPlan& pl, const float* x) {
    const float* p[1] = {x};
    return run_map<FUn<OP>, 1, false>(res, pl, p, no_scal(), FUn<OP>{});
}

template <int OP>
static int unary_bwd_t(float* grad, const ElwPlan& pl, const float* x, const float* ug) {
    const float* p[2] = {x, ug};
    return run_map<FUnBwd<OP>, 2, true>(grad, pl, p, no_scal(), FUnBwd<OP>{});
}

// rg of one binary operand, written (ACCUM = false) or accumulated (ACCUM = true) over the
// ug-shaped plan whose inputs are ordered as FBinRg expects.
template <int OP, int ID, bool DIVS, bool ACCUM>
static int binary_rg_t(float* out, const mh_shape& sug, const float* ug, const float* t1,
                       const mh_shape& s1, const float* t2, const mh_shape& s2) {
    using F = FBinRg<OP, ID, DIVS>;
    ElwPlan pl;
    if constexpr (OP == MH_ADD || OP == MH_SUB) {
        mh_shape in[1] = {sug};
        MH_TRY(build_elw_plan(sug, 1, in, &pl));
        const float* p[1] = {ug};
        return run_map<F, 1, ACCUM>(out, pl, p, no_scal(), F{});
    } else if constexpr ((OP == MH_MUL && ID == 0) || (OP == MH_DIV && ID == 0)) {
        mh_shape in[2] = {sug, s2};
        MH_TRY(build_elw_plan(sug, 2, in, &pl));
        const float* p[2] = {ug, t2};
        return run_map<F, 2, ACCUM>(out, pl, p, no_scal(), F{});
    } else if constexpr (OP == MH_MUL || DIVS) {
        mh_shape in[2] = {sug, s1};
        MH_TRY(build_elw_plan(sug, 2, in, &pl));
        const float* p[2] = {ug, t1};
        return run_map<F, 2, ACCUM>(out, pl, p, DIVS ? scal1(t2) : no_scal(), F{});
    } else {
        mh_shape in[3] = {sug, s1, s2};
        MH_TRY(build_elw_plan(sug, 3, in, &pl));
        const float* p[3] = {ug, t1, t2};
        return run_map<F, 3, ACCUM>(out, pl, p, no_scal(), F{});
    }
}

template <bool ACCUM>
static int binary_rg(int op, int id, bool divs, float* out, const mh_shape& sug, const float* ug,
                     const float* t1, const mh_shape& s1, const float* t2, const mh_shape& s2) {
#define MH_RG(OPV, IDV, DV) return binary_rg_t<OPV, IDV, DV, ACCUM>(out, sug, ug, t1, s1, t2, s2)
    switch (op) {
        case MH_ADD: MH_RG(MH_ADD, 0, false);
        case MH_SUB: if (id == 0) MH_RG(MH_SUB, 0, false); else MH_RG(MH_SUB, 1, false);
        case MH_MUL: if (id == 0) MH_RG(MH_MUL, 0, false); else MH_RG(MH_MUL, 1, false);
        default:
            if (id == 0) MH_RG(MH_DIV, 0, false);
            if (divs) MH_RG(MH_DIV, 1, true);
            MH_RG(MH_DIV, 1, false);
    }
#undef MH_RG
}

// Exported to mh_reduce.hip / mh_fused.hip.
int map_max_route(float* grad, const mh_shape& sx, const float* x, const mh_shape& sline,
                  const float* m, const float* f, const float* ug) {
    mh_shape in[4] = {sx, sline, sline, sline};
    ElwPlan pl;
    MH_TRY(build_elw_plan(sx, 4, in, &pl));
    const float* p[4] = {x, m, f, ug};
    return run_map<FMaxRoute, 4, true>(grad, pl, p, no_scal(), FMaxRoute{});
}

int map_scale_bcast(float* grad, const mh_shape& sx, const float* ug, const mh_shape& sug, float c,
                    bool twice) {
    mh_shape in[1] = {sug};
    ElwPlan pl;
    MH_TRY(build_elw_plan(sx, 1, in, &pl));
    const float* p[1] = {ug};
    if (twice) {
        FScaleBcast<true> f;
        f.c = c;
        return run_map<FScaleBcast<true>, 1, true>(grad, pl, p, no_scal(), f);
    }
    FScaleBcast<false> f;
    f.c = c;
    return run_map<FScaleBcast<false>, 1, true>(grad, pl, p, no_scal(), f);
}

int map_mean_all(float* grad, int64_t n, const float* ug, float c) {
    mh_shape s = flat_shape(n);
    ElwPlan pl;
    MH_TRY(build_elw_plan(s, 0, nullptr, &pl));
    FMeanAll f;
    f.c = c;
    return run_map<FMeanAll, 0, true>(grad, pl, nullptr, scal1(ug), f);
}

int map_binary_rg_store(int op, int id, bool divs, float* rg, const mh_shape& sug, const float* ug,
                        const float* t1, const mh_shape& s1, const float* t2, const mh_shape& s2) {
    return binary_rg<false>(op, id, divs, rg, sug, ug, t1, s1, t2, s2);
}

int map_accum_same(float* grad, const float* rg, int64_t n, bool scalar_rg) {
    mh_shape so = flat_shape(n);
    mh_shape si = flat_shape(scalar_rg ? 1 : n);
    ElwPlan pl;
    MH_TRY(build_elw_plan(so, 1, &si, &pl));
    const float* p[1] = {rg};
    return run_map<FBinRg<MH_ADD, 0, false>, 1, true>(grad, pl, p, no_scal(), FBinRg<MH_ADD, 0, false>{});
}

int unbroadcast_accum_scratch(float* grad, const mh_shape& sgrad, const float* rg,
                              const mh_shape& srg, bool negate, float* tmp);
size_t unbroadcast_scratch_floats(const mh_shape& sgrad, const mh_shape& srg);

}  // namespace mh

using namespace mh;

extern "C" {

int mh_binary_fwd(int op, float* res, const mh_shape* psres, const float* a, const mh_shape* psa,
                  const float* b, const mh_shape* psb) {
    MH_TRACE_OP("mh_binary_fwd", op);
    MH_SHAPE_ARG(sres);
    MH_SHAPE_ARG(sa);
    MH_SHAPE_ARG(sb);
    MH_TRY(check_op_binary(op));
    MH_TRY(check_shape(sres, "res"));
    MH_TRY(check_shape(sa, "a"));
    MH_TRY(check_shape(sb, "b"));
    mh_shape bs;
    MH_TRY(broadcast_shapes(sa, sb, &bs));
    if (!shape_eq(bs, sres)) return fail(MH_ERR_SHAPE, "mh_binary_fwd: res shape is not broadcast(a, b)");
    if (numel(sres) == 0) return MH_OK;
    if (!res || !a || !b) return fail(MH_ERR_NULL, "mh_binary_fwd: null tensor");
    MH_TRY(require_init());
    mh_shape in[2] = {sa, sb};
    ElwPlan pl;
    MH_TRY(build_elw_plan(sres, 2, in, &pl));
    switch (op) {
        case MH_ADD: MH_TRY(binary_fwd_t<MH_ADD>(res, pl, a, b)); break;
        case MH_SUB: MH_TRY(binary_fwd_t<MH_SUB>(res, pl, a, b)); break;
        case MH_MUL: MH_TRY(binary_fwd_t<MH_MUL>(res, pl, a, b)); break;
        default: MH_TRY(binary_fwd_t<MH_DIV>(res, pl, a, b)); break;
    }
    return finish("mh_binary_fwd");
}

int mh_unary_fwd(int op, float* res, const float* x, int64_t n) {
    MH_TRACE_OP("mh_unary_fwd", op);
    MH_TRY(check_op_unary(op));
    if (n < 0) return fail(MH_ERR_INVALID, "mh_unary_fwd: negative count");
    if (n == 0) return MH_OK;
    if (!res || !x) return fail(MH_ERR_NULL, "mh_unary_fwd: null tensor");
    MH_TRY(require_init());
    mh_shape s = flat_shape(n);
    ElwPlan pl;
    MH_TRY(build_elw_plan(s, 1, &s, &pl));
    switch (op) {
        case MH_EXP: MH_TRY(unary_fwd_t<MH_EXP>(res, pl, x)); break;
        case MH_LOG: MH_TRY(unary_fwd_t<MH_LOG>(res, pl, x)); break;
        case MH_SIGMOID: MH_TRY(unary_fwd_t<MH_SIGMOID>(res, pl, x)); break;
        case MH_RELU: MH_TRY(unary_fwd_t<MH_RELU>(res, pl, x)); break;
        default: MH_TRY(unary_fwd_t<MH_TANH>(res, pl, x)); break;
    }
    return finish("mh_unary_fwd");
}

int mh_pow_fwd(float* res, const float* x, int64_t n, const float* exponent) {
    MH_TRACE("mh_pow_fwd");
    if (n < 0) return fail(MH_ERR_INVALID, "mh_pow_fwd: negative count");
    if (n == 0) return MH_OK;
    if (!res || !x || !exponent) return fail(MH_ERR_NULL, "mh_pow_fwd: null tensor");
    MH_TRY(require_init());
    mh_shape s = flat_shape(n);
    ElwPlan pl;
    MH_TRY(build_elw_plan(s, 1, &s, &pl));
    const float* p[1] = {x};
    MH_TRY((run_map<FPowi, 1, false>(res, pl, p, scal1(exponent), FPowi{})));
    return finish("mh_pow_fwd");
}

int mh_powi_fwd(float* res, const float* x, int32_t n_int, int64_t n) {
    MH_TRACE("mh_powi_fwd");
    if (n < 0) return fail(MH_ERR_INVALID, "mh_powi_fwd: negative count");
    if (n == 0) return MH_OK;
    if (!res || !x) return fail(MH_ERR_NULL, "mh_powi_fwd: null tensor");
    MH_TRY(require_init());
    mh_shape s = flat_shape(n);
    ElwPlan pl;
    MH_TRY(build_elw_plan(s, 1, &s, &pl));
    const float* p[1] = {x};
    MH_TRY((run_map<FPowiN, 1, false>(res, pl, p, DevScal{}, FPowiN{(int64_t)n_int})));
    return finish("mh_powi_fwd");
}

int mh_unary_bwd_accum(int op, float* grad, const float* x, const float* ug, int64_t n) {
    MH_TRACE_OP("mh_unary_bwd_accum", op);
    MH_TRY(check_op_unary(op));
    if (n < 0) return fail(MH_ERR_INVALID, "mh_unary_bwd_accum: negative count");
    if (n == 0) return MH_OK;
    if (!grad || !x || !ug) return fail(MH_ERR_NULL, "mh_unary_bwd_accum: null tensor");
    MH_TRY(require_init());
    mh_shape s = flat_shape(n);
    mh_shape in[2] = {s, s};
    ElwPlan pl;
    MH_TRY(build_elw_plan(s, 2, in, &pl));
    switch (op) {
        case MH_EXP: MH_TRY(unary_bwd_t<MH_EXP>(grad, pl, x, ug)); break;
        case MH_LOG: MH_TRY(unary_bwd_t<MH_LOG>(grad, pl, x, ug)); break;
        case MH_SIGMOID: MH_TRY(unary_bwd_t<MH_SIGMOID>(grad, pl, x, ug)); break;
        case MH_RELU: MH_TRY(unary_bwd_t<MH_RELU>(grad, pl, x, ug)); break;
        default: MH_TRY(unary_bwd_t<MH_TANH>(grad, pl, x, ug)); break;
    }
    return finish("mh_unary_bwd_accum");
}

int mh_pow_bwd_accum(int tensor_id, float* grad, const float* x, const float* exponent,
                     const float* ug, int64_t n) {
    MH_TRACE("mh_pow_bwd_accum");
    if (tensor_id != 0 && tensor_id != 1) return fail(MH_ERR_INVALID, "mh_pow_bwd_accum: tensor_id %d", tensor_id);
    if (n < 0) return fail(MH_ERR_INVALID, "mh_pow_bwd_accum: negative count");
    if (n == 0) return MH_OK;
    if (!grad || !x || !ug || !exponent) return fail(MH_ERR_NULL, "mh_pow_bwd_accum: null tensor");
    MH_TRY(require_init());
    if (tensor_id == 1) {
        MH_TRY(pow_exponent_grad(grad, x, exponent, ug, n));
        return finish("mh_pow_bwd_accum");
    }
    mh_shape s = flat_shape(n);
    mh_shape in[2] = {s, s};
    ElwPlan pl;
    MH_TRY(build_elw_plan(s, 2, in, &pl));
    const float* p[2] = {x, ug};
    MH_TRY((run_map<FPowBwdX, 2, true>(grad, pl, p, scal1(exponent), FPowBwdX{})));
    return finish("mh_pow_bwd_accum");
}

int mh_pow_bwd_accum2(float* grad_x, float* grad_exp, const float* x, const float* exponent, const float* ug,
                      int64_t n) {
    MH_TRACE("mh_pow_bwd_accum2");
    if (n < 0) return fail(MH_ERR_INVALID, "mh_pow_bwd_accum2: negative count");
    if (n == 0) return MH_OK;
    if (!x || !ug || !exponent) return fail(MH_ERR_NULL, "mh_pow_bwd_accum2: null tensor");
    MH_TRY(require_init());
    // grad_x written while x, ug, the exponent or grad_exp are read: the two calls in order
    const auto overlaps = [&](const float* p, int64_t m) {
        return grad_x && p && p < grad_x + n && grad_x < p + m;
    };
    if (!grad_x || !grad_exp || overlaps(x, n) || overlaps(ug, n) || overlaps(exponent, 1) ||
        overlaps(grad_exp, 1)) {
        if (grad_x) MH_TRY(mh_pow_bwd_accum(0, grad_x, x, exponent, ug, n));
        if (grad_exp) MH_TRY(mh_pow_bwd_accum(1, grad_exp, x, exponent, ug, n));
        return MH_OK;
    }
    MH_TRY(pow_exponent_grad(grad_exp, x, exponent, ug, n, grad_x));
    return finish("mh_pow_bwd_accum2");
}

int mh_binary_bwd_accum(int op, int tensor_id, float* grad, const mh_shape* psgrad, const float* ug,
                        const mh_shape* psug, const float* t1, const mh_shape* ps1, const float* t2,
                        const mh_shape* ps2) {
    MH_TRACE_OP("mh_binary_bwd_accum", op);
    MH_SHAPE_ARG(sgrad);
    MH_SHAPE_ARG(sug);
    MH_SHAPE_ARG(s1);
    MH_SHAPE_ARG(s2);
    MH_TRY(check_op_binary(op));
    if (tensor_id != 0 && tensor_id != 1) return fail(MH_ERR_INVALID, "mh_binary_bwd_accum: tensor_id %d", tensor_id);
    MH_TRY(check_shape(sgrad, "grad"));
    MH_TRY(check_shape(sug, "ug"));
    MH_TRY(check_shape(s1, "t1"));
    MH_TRY(check_shape(s2, "t2"));
    mh_shape bs;
    MH_TRY(broadcast_shapes(s1, s2, &bs));
    if (!shape_eq(bs, sug)) return fail(MH_ERR_SHAPE, "mh_binary_bwd_accum: ug shape is not broadcast(t1, t2)");
    if (!shape_eq(sgrad, tensor_id == 0 ? s1 : s2))
        return fail(MH_ERR_SHAPE, "mh_binary_bwd_accum: grad shape differs from operand %d", tensor_id);
    if (numel(sug) == 0) return MH_OK;
    const bool need_t1 = (op == MH_MUL && tensor_id == 1) || (op == MH_DIV && tensor_id == 1);
    const bool need_t2 = (op == MH_MUL || op == MH_DIV);
    if (!grad || !ug || (need_t1 && !t1) || (need_t2 && !t2))
        return fail(MH_ERR_NULL, "mh_binary_bwd_accum: null tensor");
    MH_TRY(require_init());
    const bool divs = op == MH_DIV && tensor_id == 1 && is_scalar_shape(s2);
    if (shape_eq(sgrad, sug)) {
        MH_TRY(binary_rg<true>(op, tensor_id, divs, grad, sug, ug, t1, s1, t2, s2));
        return finish("mh_binary_bwd_accum");
    }
    // operand was broadcast: accumulate_grad sums rg over the broadcast axes
    const size_t red_floats = unbroadcast_scratch_floats(sgrad, sug);
    if (op == MH_ADD || op == MH_SUB) {
        float* tmp = nullptr;
        MH_TRY(scratch(red_floats * sizeof(float), reinterpret_cast<void**>(&tmp)));
        MH_TRY(unbroadcast_accum_scratch(grad, sgrad, ug, sug, op == MH_SUB && tensor_id == 1, tmp));
        return finish("mh_binary_bwd_accum");
    }
    bool done = false;  // rg summed as it is computed, when the shapes allow it
    MH_TRY(unbroadcast_binrg(op, tensor_id, divs, grad, sgrad, ug, sug, t1, s1, t2, s2, &done));
    if (done) return finish("mh_binary_bwd_accum");
    const size_t n = (size_t)numel(sug);
    const size_t rg_floats = (n + 63) & ~(size_t)63;
    float* base = nullptr;
    MH_TRY(scratch((rg_floats + red_floats) * sizeof(float), reinterpret_cast<void**>(&base)));
    float* rg = base;
    MH_TRY(binary_rg<false>(op, tensor_id, divs, rg, sug, ug, t1, s1, t2, s2));
    MH_TRY(unbroadcast_accum_scratch(grad, sgrad, rg, sug, false, base + rg_floats));
    return finish("mh_binary_bwd_accum");
}

int mh_binary_bwd_accum2(int op, float* grad1, float* grad2, const float* ug, const float* t1,
                         const float* t2, const mh_shape* ps) {
    MH_TRACE_OP("mh_binary_bwd_accum2", op);
    MH_SHAPE_ARG(s);
    MH_TRY(check_op_binary(op));
    MH_TRY(check_shape(s, "shape"));
    if (!grad1 && !grad2) return MH_OK;
    const int64_t nel = numel(s);
    // the two gradient ranges: the same tensor (one fused pass, id 0's sum first), or
    // overlapping without being equal (the two backward_op calls one after the other)
    const bool alias = grad1 && grad1 == grad2;
    const bool overlap = grad1 && grad2 && !alias && grad1 < grad2 + nel && grad2 < grad1 + nel;
    if (!grad1 || !grad2 || overlap || is_scalar_shape(s) || nel == 0 ||
        !(aligned16(grad1) && aligned16(grad2) && aligned16(ug) && aligned16(t1) && aligned16(t2))) {
        // one operand, overlapping grads, a graph scalar (DIV's scalar rule), empty or
        // unaligned: per operand, id 0 then id 1 (model.mojo:233-270)
        if (grad1) MH_TRY(mh_binary_bwd_accum(op, 0, grad1, &s, ug, &s, t1, &s, t2, &s));
        if (grad2) MH_TRY(mh_binary_bwd_accum(op, 1, grad2, &s, ug, &s, t1, &s, t2, &s));
        return MH_OK;
    }
    const bool need_ab = op == MH_MUL || op == MH_DIV;
    if (!ug || (need_ab && (!t1 || !t2))) return fail(MH_ERR_NULL, "mh_binary_bwd_accum2: null tensor");
    MH_TRY(require_init());
    hipStream_t st = ctx().stream;
    // a thread per quad; past kMaxLaunchQuads quads, several launches over offset pointers
    for (int64_t off = 0; off < nel; off += 4 * kMaxLaunchQuads) {
        const int64_t n = nel - off < 4 * kMaxLaunchQuads ? nel - off : 4 * kMaxLaunchQuads;
        dim3 g(grid_for(n >> 2, kThreads)), b(kThreads);
        float* g1 = grad1 + off;
        const float* u = ug + off;
        const float* a = t1 ? t1 + off : nullptr;  // ADD and SUB do not read the operands
        const float* c = t2 ? t2 + off : nullptr;
        if (alias) {  // g2 is not read: pass a null pointer so no access can go through it
            switch (op) {
                case MH_ADD: hipLaunchKernelGGL((k_bwd2_same4<MH_ADD, true>), g, b, 0, st, g1, nullptr, u, a, c, n); break;
                case MH_SUB: hipLaunchKernelGGL((k_bwd2_same4<MH_SUB, true>), g, b, 0, st, g1, nullptr, u, a, c, n); break;
                case MH_MUL: hipLaunchKernelGGL((k_bwd2_same4<MH_MUL, true>), g, b, 0, st, g1, nullptr, u, a, c, n); break;
                default: hipLaunchKernelGGL((k_bwd2_same4<MH_DIV, true>), g, b, 0, st, g1, nullptr, u, a, c, n); break;
            }
            continue;
        }
        float* g2 = grad2 + off;
        switch (op) {
            case MH_ADD: hipLaunchKernelGGL(k_bwd2_same4<MH_ADD>, g, b, 0, st, g1, g2, u, a, c, n); break;
            case MH_SUB: hipLaunchKernelGGL(k_bwd2_same4<MH_SUB>, g, b, 0, st, g1, g2, u, a, c, n); break;
            case MH_MUL: hipLaunchKernelGGL(k_bwd2_same4<MH_MUL>, g, b, 0, st, g1, g2, u, a, c, n); break;
            default: hipLaunchKernelGGL(k_bwd2_same4<MH_DIV>, g, b, 0, st, g1, g2, u, a, c, n); break;
        }
    }
    return finish("mh_binary_bwd_accum2");
}

int mh_accumulate_grad(float* grad, const mh_shape* psgrad, const float* rg, const mh_shape* psrg) {
    MH_TRACE("mh_accumulate_grad");
    MH_SHAPE_ARG(sgrad);
    MH_SHAPE_ARG(srg);
    MH_TRY(check_shape(sgrad, "grad"));
    MH_TRY(check_shape(srg, "rg"));
    const bool same = shape_eq(sgrad, srg);
    const bool scal = !same && is_scalar_shape(srg);
    if (!same && !scal && !broadcasts_to(sgrad, srg))
        return fail(MH_ERR_SHAPE, "mh_accumulate_grad: grad shape does not broadcast to rg shape");
    if (numel(sgrad) == 0 || numel(srg) == 0) return MH_OK;
    if (!grad || !rg) return fail(MH_ERR_NULL, "mh_accumulate_grad: null tensor");
    MH_TRY(require_init());
    if (same || scal) {
        MH_TRY(map_accum_same(grad, rg, numel(sgrad), scal));
        return finish("mh_accumulate_grad");
    }
    float* tmp = nullptr;
    MH_TRY(scratch(unbroadcast_scratch_floats(sgrad, srg) * sizeof(float), reinterpret_cast<void**>(&tmp)));
    MH_TRY(unbroadcast_accum_scratch(grad, sgrad, rg, srg, false, tmp));
    return finish("mh_accumulate_grad");
}

}  // extern "C"

namespace mh {

// ---------------------------------------------------------------------------------------
// FMA (basics.mojo:759-817), LEAKYRELU (mlops.mojo:128-186), CLIP (mlops.mojo:238-299):
// same-shape maps over a flat element count
// ---------------------------------------------------------------------------------------
static int flat_check(const char* what, int64_t n, bool ptrs_ok) {
    if (n < 0) return fail(MH_ERR_INVALID, "%s: negative count", what);
    if (n > 0 && !ptrs_ok) return fail(MH_ERR_NULL, "%s: null tensor", what);
    return MH_OK;
}

template <class F, int NIN, bool ACCUM>
static int flat_map(const char* what, float* out, const float* const* ptrs, int64_t n, F f) {
    MH_TRY(require_init());
    mh_shape s = flat_shape(n);
    mh_shape in[kMaxIn] = {s, s, s, s};
    ElwPlan pl;
    MH_TRY(build_elw_plan(s, NIN, in, &pl));
    MH_TRY((run_map<F, NIN, ACCUM>(out, pl, ptrs, no_scal(), f)));
    return finish(what);
}

}  // namespace mh

extern "C" {

int mh_fma_fwd(float* res, const float* t1, const float* t2, const float* t3, int64_t n) {
    MH_TRACE("mh_fma_fwd");
    MH_TRY(flat_check("mh_fma_fwd", n, res && t1 && t2 && t3));
    if (n == 0) return MH_OK;
    const float* p[3] = {t1, t2, t3};
    return flat_map<FFma, 3, false>("mh_fma_fwd", res, p, n, FFma{});
}

int mh_fma_bwd_accum(int tensor_id, float* grad, const float* ug, const float* t1, const float* t2, int64_t n) {
    MH_TRACE("mh_fma_bwd_accum");
    if (tensor_id < 0 || tensor_id > 2) return fail(MH_ERR_INVALID, "mh_fma_bwd_accum: tensor_id %d", tensor_id);
    const float* other = tensor_id == 0 ? t2 : t1;
    MH_TRY(flat_check("mh_fma_bwd_accum", n, grad && ug && (tensor_id == 2 || other)));
    if (n == 0) return MH_OK;
    const float* p[2] = {ug, other};
    if (tensor_id == 2) return flat_map<FFmaRg<2>, 1, true>("mh_fma_bwd_accum", grad, p, n, FFmaRg<2>{});
    return flat_map<FFmaRg<0>, 2, true>("mh_fma_bwd_accum", grad, p, n, FFmaRg<0>{});
}

int mh_leakyrelu_fwd(float* res, const float* x, int64_t n, float negative_slope) {
    MH_TRACE("mh_leakyrelu_fwd");
    MH_TRY(flat_check("mh_leakyrelu_fwd", n, res && x));
    if (n == 0) return MH_OK;
    const float* p[1] = {x};
    return flat_map<FLeaky, 1, false>("mh_leakyrelu_fwd", res, p, n, FLeaky{negative_slope});
}

int mh_leakyrelu_bwd_accum(float* grad, const float* x, const float* ug, int64_t n, float negative_slope) {
    MH_TRACE("mh_leakyrelu_bwd_accum");
    MH_TRY(flat_check("mh_leakyrelu_bwd_accum", n, grad && x && ug));
    if (n == 0) return MH_OK;
    const float* p[2] = {x, ug};
    return flat_map<FLeakyBwd, 2, true>("mh_leakyrelu_bwd_accum", grad, p, n, FLeakyBwd{negative_slope});
}

int mh_clip_fwd(float* res, const float* x, int64_t n, float min_val, float max_val) {
    MH_TRACE("mh_clip_fwd");
    MH_TRY(flat_check("mh_clip_fwd", n, res && x));
    if (n == 0) return MH_OK;
    const float* p[1] = {x};
    return flat_map<FClip, 1, false>("mh_clip_fwd", res, p, n, FClip{min_val, max_val});
}

int mh_clip_bwd_accum(float* grad, const float* x, const float* ug, int64_t n, float min_val, float max_val) {
    MH_TRACE("mh_clip_bwd_accum");
    MH_TRY(flat_check("mh_clip_bwd_accum", n, grad && x && ug));
    if (n == 0) return MH_OK;
    const float* p[2] = {x, ug};
    return flat_map<FClipBwd, 2, true>("mh_clip_bwd_accum", grad, p, n, FClipBwd{min_val, max_val});
}

}  // extern "C"
