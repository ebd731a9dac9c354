// mh_reduce.hip -- axis / all-element reductions, un-broadcast gradient accumulation, MAX
// backward tie routing and the POW exponent gradient.
//
// Every reduction is expressed on a view [A, B, C] reduced over B:
//   C == 1, B <= 32 : 64 rows (a one-wavefront block) staged in LDS by coalesced float4
//                     loads, one thread per row (unaligned x: one thread per row straight
//                     from memory);
//   C == 1, B < 2048: one wavefront (64 lanes) per row, 128-bit loads, butterfly shuffle;
//   C == 1, B >= 2048: 2048-element chunks, one 4-wave block each (two quads per thread),
//                     whose partials reduce again along the row the same way;
//   C  > 1, C % 4 == 0 and >= 1024 columns: one thread per column quad over a split of the
//                     rows (about four blocks per CU; splits on grid x), the split partials
//                     combined in one short launch (k_parts_comb);
//   C  > 1, C % 4 == 0 and >= 128 columns: a block per (strip of 64 column quads, split of
//                     rows), its four waves interleaving the rows, combined through LDS;
//   C  > 1 otherwise  : one thread per output column (a quad of columns when C % 4 == 0);
//   in every column form the rows split across blocks when that is needed to fill the chip,
//   and a second pass combines the split partials in fixed split order.
// No atomics: each output's summation order is fixed by the launch shape, so a call repeated
// on the same input returns the same bits.
// MAX backward over axis 0 and all elements routes from the split partials its max-count
// reduction leaves (k_max_route_*): x is read again only where a split holds a line maximum
// it cannot place by its recorded index.
#include <cfloat>
#include <type_traits>

#include "mh_internal.h"
#include "mh_math.h"

namespace mh {

constexpr int kRThreads = 256;
// Rows per workgroup of the LDS-staged short-row kernels (one thread per row): one wavefront.
constexpr int kLdsRows = 64;
// A launch of one thread per row or output covers at most this many (a grid holds fewer than
// 2^32 work-items per dimension); larger counts take the grid-stride kernels.
constexpr int64_t kMaxGridRows = ((int64_t)1 << 32) - 256;

// ---------------------------------------------------------------------------------------
// reduction policies
// ---------------------------------------------------------------------------------------
struct RSum {
    using T = float;
    __device__ static T init() { return 0.0f; }
    __device__ static T lift(float x) { return x; }
    __device__ static T comb(T a, T b) { return a + b; }
    __device__ static T shfl(T v, int m) { return __shfl_xor(v, m); }
};
struct RMax {  // max_simd (math_util.mojo:224-244): a > b ? a : b, start -FLT_MAX
    using T = float;
    __device__ static T init() { return -FLT_MAX; }
    __device__ static T lift(float x) { return x; }
    __device__ static T comb(T a, T b) { return a > b ? a : b; }
    __device__ static T shfl(T v, int m) { return __shfl_xor(v, m); }
};
struct MC {
    float m;
    uint32_t c;
};
// (line max, number of elements equal to it), from -FLT_MAX with count 0 (basics.mojo:551-577,
// 597-613: c = #(x == m)). A NaN element is neither the maximum nor counted: the running
// value never becomes NaN, so exactly one side of a combine can be NaN, and the other side is
// kept. Every order of combining then gives the same maximum (as a float) and count.
struct RMaxCnt {
    using T = MC;
    __device__ static T init() { return MC{-FLT_MAX, 0u}; }
    __device__ static T lift(float x) { return MC{x, 1u}; }
    // the larger side wins; equal maxima add their counts; against a NaN element the other
    // side wins. Written as selects over comparisons joined without short-circuits: early
    // returns (or || and &&) compiled to a branch per comparison, with an exec-mask save and
    // restore around each element of a line.
    __device__ static T comb(T a, T b) {
        const bool eq = a.m == b.m;
        const bool take_b = (b.m > a.m) | (!(a.m > b.m) & !eq & (a.m != a.m));
        return MC{take_b ? b.m : a.m, eq ? a.c + b.c : (take_b ? b.c : a.c)};
    }
    __device__ static T shfl(T v, int m) {
        return MC{__shfl_xor(v.m, m), (uint32_t)__shfl_xor((int)v.c, m)};
    }
};

// RMaxCnt with the element index of the maximum: the first pass of a column MAX backward.
// Maxima and counts are RMaxCnt's (the same comparisons and sums); a tie keeps the lower index.
// Where a split's count is 1, its index is the one element equal to its maximum, and the
// routing pass adds there without reading x again (a count above 1 makes it read x).
struct MCI {
    float m;
    uint32_t c, i;
};
struct RMaxCntArg {
    using T = MCI;
    __device__ static T init() { return MCI{-FLT_MAX, 0u, 0xffffffffu}; }
    __device__ static T lift(float x) { return MCI{x, 1u, 0xffffffffu}; }
    __device__ static T comb(T a, T b) {  // RMaxCnt's selects, the lower index on a tie
        const bool eq = a.m == b.m;
        const bool take_b = (b.m > a.m) | (!(a.m > b.m) & !eq & (a.m != a.m));
        return MCI{take_b ? b.m : a.m, eq ? a.c + b.c : (take_b ? b.c : a.c),
                   eq ? (a.i < b.i ? a.i : b.i) : (take_b ? b.i : a.i)};
    }
    __device__ static T shfl(T v, int m) {
        return MCI{__shfl_xor(v.m, m), (uint32_t)__shfl_xor((int)v.c, m), (uint32_t)__shfl_xor((int)v.i, m)};
    }
};

// ---------------------------------------------------------------------------------------
// loaders: get(i) -> R::T at element i; get4 for 16-byte aligned quads
// ---------------------------------------------------------------------------------------
template <class R>
struct LdPlain {
    const float* x;
    __device__ void setup() {}
    __device__ typename R::T get(int64_t i) const { return R::lift(ld_nt(x + i)); }
    __device__ void get4(int64_t i, typename R::T* o) const {
        float4 q = ld_nt4(x + i, 0);
        o[0] = R::lift(q.x); o[1] = R::lift(q.y); o[2] = R::lift(q.z); o[3] = R::lift(q.w);
    }
};

struct LdArg {  // x, each element with its index (tensors of fewer than 2^32 elements)
    const float* x;
    __device__ void setup() {}
    __device__ MCI get(int64_t i) const { return MCI{ld_nt(x + i), 1u, (uint32_t)i}; }
    __device__ void get4(int64_t i, MCI* o) const {
        const float4 q = ld_nt4(x + i, 0);
        const uint32_t k = (uint32_t)i;
        o[0] = MCI{q.x, 1u, k}; o[1] = MCI{q.y, 1u, k + 1}; o[2] = MCI{q.z, 1u, k + 2}; o[3] = MCI{q.w, 1u, k + 3};
    }
};

// Split partials of RMaxCnt (LdPairs) and RMaxCntArg (LdPairsArg): the maxima at m, the counts
// at c. The combines above the first level need no indices (only the first level's feed the
// routing), so LdPairsArg leaves them at their initial value. get4 is called at quad-aligned
// offsets only (counts of partials a multiple of 4 in 64-float-aligned scratch): two quad
// loads.
struct LdPairsArg {
    const float* m;
    const uint32_t* c;
    __device__ void setup() {}
    __device__ MCI get(int64_t k) const { return MCI{m[k], c[k], 0xffffffffu}; }
    __device__ void get4(int64_t k, MCI* o) const {
        const float4 a = *reinterpret_cast<const float4*>(m + k);
        const uint4 b = *reinterpret_cast<const uint4*>(c + k);
        o[0] = MCI{a.x, b.x, 0xffffffffu}; o[1] = MCI{a.y, b.y, 0xffffffffu};
        o[2] = MCI{a.z, b.z, 0xffffffffu}; o[3] = MCI{a.w, b.w, 0xffffffffu};
    }
};

struct LdPairs {
    const float* m;
    const uint32_t* c;
    __device__ void setup() {}
    __device__ MC get(int64_t i) const { return MC{m[i], c[i]}; }
    __device__ void get4(int64_t i, MC* o) const {
        const float4 a = *reinterpret_cast<const float4*>(m + i);
        const uint4 b = *reinterpret_cast<const uint4*>(c + i);
        o[0] = MC{a.x, b.x}; o[1] = MC{a.y, b.y}; o[2] = MC{a.z, b.z}; o[3] = MC{a.w, b.w};
    }
};

// POW exponent gradient term (basics.mojo:359-376): powf(x, a) * (isinf(log x) ? 0 : log x) * ug.
// With gx set, every element the reduction visits (each exactly once: the reduction adds
// each term once) also takes the x gradient, gx[i] = gx[i] + (a * powf(x[i] + 1e-12, a - 1))
// * ug[i] (basics.mojo:345-357, FPowBwdX's expression), from the same x and ug loads and,
// where x + 1e-12 rounds to x, the same log: both POW operand gradients in one pass.
//
// The term's power comes from p = powf(x + 1e-12, a - 1), the x gradient's power (evaluated
// for the term alone when gx is null): where x + 1e-12 rounds to x and both p and x * p are
// normal and below 2e38, no exp of either power met its clamp, x * p is powf(x, a) within the
// rounding of the two exp arguments (a few ulp where |a log x| is small), and log x is finite
// or NaN, so (x * p * log x) * ug is the term. Every other element (zero, subnormal, infinite,
// NaN or negative bases, clamped or out-of-range powers) evaluates powf(x, a) as written. The
// exponent's gradient is a sum, compared in the rtol-1e-5 class; the x gradient keeps its bits.
// frac (set once per block) marks an exponent for which powf(., a) and powf(., a - 1) both take
// the exp(y * log x) route (a and a - 1 neither NaN nor integral below 2^31): their elements
// skip the per-call tests of the exponent and take p as the bare exp polynomial, whose bits are
// mexp's wherever the band test passes (there the argument lay inside mexp's clamp range).
struct LdPowGrad {
    const float* x;
    const float* ug;
    const float* ap;
    float a;
    float* gx;
    float am1;
    bool frac;
    __device__ static bool exp_route(float y) {
        return !(y != y) && !(__builtin_truncf(y) == y && __builtin_fabsf(y) < 2147483648.0f);
    }
    __device__ __forceinline__ void setup() {
        a = ap[0];
        am1 = a - 1.0f;
        frac = exp_route(a) && exp_route(am1);
    }
    // positive, normal and below 2e38: one unsigned compare of the bits (NaN, infinities,
    // zeros, subnormals and negative values all fall outside)
    __device__ static bool in_band(float v) {
        return __float_as_uint(v) - 0x00800000u < __float_as_uint(2.0e38f) - 0x00800000u;
    }
    // mpowf_lg for an exponent on the exp route: the same bits
    __device__ static float pow_exp(float xv, float y, float lg) {
        return xv < 0.0f ? __builtin_nanf("") : mexp(y * lg);
    }
    // one element: returns the term; with GX (gx set), g becomes g + the x gradient
    template <bool FRAC, bool GX>
    __device__ __forceinline__ float elem(float xv, float u, float& g) const {
        const float lx = mlog(xv);
        const float xe = xv + 1e-12f;
        const bool same = xe == xv;  // equal values have equal bits here (xe != +-0)
        if constexpr (FRAC) {
            // the exp of (a - 1) log x without mexp's clamp and NaN pass-through or pow's
            // negative-base test: where p and x * p are in band, the argument lay inside the
            // clamp range and x was positive, so p holds mpowf_lg's bits; any other lane takes
            // the powers as written
            const float p = mexp_core(am1 * lx);
            const float t = p * xv;
            if (__builtin_expect(same && in_band(p) && in_band(t), 1)) {
                if constexpr (GX) g = g + (a * p) * u;
                return (t * lx) * u;
            }
            if constexpr (GX) {
                const float lxe = same ? lx : mlog(xe);
                g = g + (a * pow_exp(xe, am1, lxe)) * u;
            }
            const float lg = __builtin_isinf(lx) ? 0.0f : lx;
            return (pow_exp(xv, a, lx) * lg) * u;
        } else {
            float p;
            if constexpr (GX) {
                const float lxe = same ? lx : mlog(xe);
                p = mpowf_lg(xe, am1, lxe);
                g = g + (a * p) * u;
            } else {
                p = mpowf_lg(xe, am1, lx);  // read below only where xe == x
            }
            const float t = p * xv;
            if (__builtin_expect(same && in_band(p) && in_band(t), 1)) return (t * lx) * u;
            const float lg = __builtin_isinf(lx) ? 0.0f : lx;
            return (mpowf_lg(xv, a, lx) * lg) * u;
        }
    }
    // elem<true, GX>'s first branch without branches: ok says whether x is a positive normal
    // value below 2e38 (mlog's straight-line case) and the powers took that branch; where it
    // holds, g and the term are elem's, and the caller recomputes any other lane with elem.
    template <bool GX>
    __device__ __forceinline__ float elem_frac_fast(float xv, float u, float& g, bool& ok) const {
        const float lx = mlog_core(xv, 0);
        const bool same = xv + 1e-12f == xv;
        const float p = mexp_core(am1 * lx);
        const float t = p * xv;
        ok = in_band(xv) && same && in_band(p) && in_band(t);
        if constexpr (GX) g = g + (a * p) * u;
        return (t * lx) * u;
    }
    template <bool FRAC, bool GX>
    __device__ float get_t(int64_t i) const {
        const float xv = ld_nt(x + i), u = ld_nt(ug + i);
        float g = GX ? ld_nt(gx + i) : 0.0f;
        const float r = elem<FRAC, GX>(xv, u, g);
        if constexpr (GX) st_nt(gx + i, g);
        return r;
    }
    template <bool FRAC, bool GX>
    __device__ void get4_t(int64_t i, float* o) const {
        const float4 q = ld_nt4(x + i, 0);
        const float4 u = ld_nt4(ug + i, 0);
        float4 g = GX ? ld_nt4(gx + i, 0) : make_float4(0.f, 0.f, 0.f, 0.f);
        o[0] = elem<FRAC, GX>(q.x, u.x, g.x);
        o[1] = elem<FRAC, GX>(q.y, u.y, g.y);
        o[2] = elem<FRAC, GX>(q.z, u.z, g.z);
        o[3] = elem<FRAC, GX>(q.w, u.w, g.w);
        if constexpr (GX) st_nt4(gx + i, 0, g);
    }
    __device__ float get(int64_t i) const {
        if (gx) return frac ? get_t<true, true>(i) : get_t<false, true>(i);
        return frac ? get_t<true, false>(i) : get_t<false, false>(i);
    }
    __device__ void get4(int64_t i, float* o) const {
        if (gx) {
            if (frac) get4_t<true, true>(i, o);
            else get4_t<false, true>(i, o);
        } else if (frac) {
            get4_t<true, false>(i, o);
        } else {
            get4_t<false, false>(i, o);
        }
    }
};

// The rg of a broadcast MUL / DIV backward, computed inside the un-broadcast reduction
// instead of being materialised (the expressions of FBinRg: MUL ug * other; DIV operand 0
// ug / t2; operand 1 ((-t1) / (t2 * t2)) * ug, or (f * t1) * ug with f = -1 / (s * s) for
// a scalar t2). `a` is the full-shape operand; `t2` of DIV's operand 1 has the grad's shape
// and is read at the element's output line (i / (B*C)) * C + i % C. get4 takes a quad in
// one row (C == 1) or over four consecutive lines (C % 4 == 0), with 16-byte loads when
// `al`, else four scalar loads, so the reduction runs in the same order either way. COL1
// (DIV's operand 1 only): C == 1, known when the kernel is compiled, so the divisor's load has
// one form (under a branch between the two, the compiler waited at the join for every load
// issued before it, and a thread's rows in flight went out one after another).
template <int OP, int ID, bool DIVS, bool BIG, bool COL1 = false>
struct LdBinRg {
    const float* ug;
    const float* a;
    const float* t2;
    int64_t BC, C;
    FastDiv fbc, fc;
    bool al;
    float f;
    __device__ void setup() {
        if constexpr (DIVS) {
            const float t = t2[0];
            f = -1.0f / (t * t);
        }
    }
    __device__ int64_t line(int64_t i) const {
        if constexpr (BIG) {
            return (i / BC) * C + i % C;
        } else {
            const uint32_t u = (uint32_t)i;
            const uint32_t c = u - fdiv(u, fc) * (uint32_t)C;
            return (int64_t)fdiv(u, fbc) * C + c;
        }
    }
    __device__ float term(float u, float av, float d) const {
        if constexpr (OP == MH_MUL) return u * av;
        else if constexpr (ID == 0) return u / av;
        else if constexpr (DIVS) return (f * av) * u;
        else return ((-av) / (d * d)) * u;
    }
    __device__ float get(int64_t i) const {
        const float d = (OP == MH_DIV && ID == 1 && !DIVS) ? t2[line(i)] : 0.0f;
        return term(ld_nt(ug + i), ld_nt(a + i), d);
    }
    __device__ void get4(int64_t i, float* o) const {
        float4 u, v;
        if (al) {
            u = ld_nt4(ug + i, 0);
            v = ld_nt4(a + i, 0);
        } else {
            u = make_float4(ld_nt(ug + i), ld_nt(ug + i + 1), ld_nt(ug + i + 2), ld_nt(ug + i + 3));
            v = make_float4(ld_nt(a + i), ld_nt(a + i + 1), ld_nt(a + i + 2), ld_nt(a + i + 3));
        }
        float4 d = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (OP == MH_DIV && ID == 1 && !DIVS) {
            const int64_t l = line(i);
            if constexpr (COL1) d = make_float4(t2[l], t2[l], t2[l], t2[l]);
            else d = make_float4(t2[l], t2[l + 1], t2[l + 2], t2[l + 3]);
        }
        o[0] = term(u.x, v.x, d.x);
        o[1] = term(u.y, v.y, d.y);
        o[2] = term(u.z, v.z, d.z);
        o[3] = term(u.w, v.w, d.w);
    }
};

// ---------------------------------------------------------------------------------------
// epilogues
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void epi_store(float* out, float*, int64_t o, float v, int epi, float div) {
    switch (epi) {
        case EPI_STORE: out[o] = v; break;
        case EPI_MEAN: out[o] = v / div; break;
        case EPI_ACCUM: out[o] = out[o] + v; break;
        case EPI_SCALE: out[o] = v * div; break;
        case EPI_SEQ_ACCUM:
        case EPI_SEQ_ACCUM_NEG: out[o] = v; break;  // v started from out[o] (row_start)
        default: out[o] = out[o] + (-v); break;
    }
}
// The start and the values of a row that one thread sums in element order: for the serial
// accumulation epilogues (sums only) out[o] and each value negated for _NEG, else R::init()
// and the values as they are.
template <class R>
__device__ __forceinline__ typename R::T row_start(int epi, const float* out, int64_t o) {
    if constexpr (std::is_same<R, RSum>::value) {
        if (epi == EPI_SEQ_ACCUM || epi == EPI_SEQ_ACCUM_NEG) return out[o];
    }
    return R::init();
}
template <class R>
__device__ __forceinline__ typename R::T row_val(int epi, typename R::T v) {
    if constexpr (std::is_same<R, RSum>::value) {
        if (epi == EPI_SEQ_ACCUM_NEG) return -v;
    }
    return v;
}
__device__ __forceinline__ void epi_store(float* out, float* out2, int64_t o, MC v, int, float) {
    out[o] = v.m;
    out2[o] = 1.0f / (float)v.c;  // MAX.backward: factor = 1 / count, basics.mojo:573, 609
}
__device__ __forceinline__ void epi_store(float* out, float* out2, int64_t o, MCI v, int, float) {
    out[o] = v.m;
    out2[o] = 1.0f / (float)v.c;
}
// MC partials keep the counts in a second array right after the maxima, MCI partials the
// indices in a third after the counts.
__device__ __forceinline__ void part_store2(float* pm, int64_t npart, int64_t o, float v) { pm[o] = v; (void)npart; }
__device__ __forceinline__ void part_store2(float* pm, int64_t npart, int64_t o, MC v) {
    pm[o] = v.m;
    reinterpret_cast<uint32_t*>(pm + npart)[o] = v.c;
}
__device__ __forceinline__ void part_store2(float* pm, int64_t npart, int64_t o, MCI v) {
    pm[o] = v.m;
    reinterpret_cast<uint32_t*>(pm + npart)[o] = v.c;
    reinterpret_cast<uint32_t*>(pm + 2 * npart)[o] = v.i;
}

// RMaxCnt over lanes whose counts are below 16 (a first-level chunk: each lane combines at most
// eight elements): the maximum by six float shuffles, the count as four ballots, one per count
// bit, over the lanes at that maximum. The same count as wave_reduce<RMaxCnt> and a maximum
// equal to its as a float (only the sign of a zero tie may differ), with half its shuffles:
// the first pass of an all-element MAX backward took 49 us over 2^26 elements with the
// pair-valued butterfly.
__device__ __forceinline__ MC wave_reduce_mc_small(MC v) {
    float m = v.m;
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) {
        const float o = __shfl_xor(m, k);
        m = o > m ? o : m;
    }
    const uint32_t c = v.m == m ? v.c : 0u;
    uint32_t tot = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) tot += (uint32_t)__popcll(__ballot((c >> b) & 1u)) << b;
    return MC{m, tot};
}

template <class R>
__device__ __forceinline__ typename R::T wave_reduce(typename R::T v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = R::comb(v, R::shfl(v, m));
    return v;
}

// ---------------------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------------------
// One thread per row of length B (B small or zero).
template <class R, class LD>
__global__ void __launch_bounds__(kRThreads)
    k_rows_thread(LD ld, int64_t nrows, int64_t B, float* out, float* out2, int epi, float div) {
    ld.setup();
    const int64_t stride = (int64_t)gridDim.x * kRThreads;
    for (int64_t r = (int64_t)blockIdx.x * kRThreads + threadIdx.x; r < nrows; r += stride) {
        typename R::T acc = row_start<R>(epi, out, r);
        const int64_t base = r * B;
        for (int64_t j = 0; j < B; ++j) acc = R::comb(acc, row_val<R>(epi, ld.get(base + j)));
        epi_store(out, out2, r, acc, epi, div);
    }
}

// Short rows (C == 1, B <= BMAX): the block stages rows [r0, r0 + 256) -- one contiguous,
// 16-byte aligned run of floats -- in LDS with float4 loads, then thread t reduces row r0 + t
// in element order (the order of the reference's scalar tail loop for rows shorter than
// its SIMD width).
// Every quad of the tile is loaded into registers before any is stored to LDS (unrolled over
// the tile's at most BMAX / 4 quads per thread), so a block waits for memory once.
template <int BMAX>
__device__ __forceinline__ int64_t stage_rows(float* tile, const float* __restrict__ x, int64_t nrows, int B,
                                              int64_t* rows_out) {
    constexpr int QPT = BMAX / 4;  // rows * B / 4 <= kLdsRows * QPT
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * kLdsRows;
    const int64_t rows = (nrows - r0) < kLdsRows ? (nrows - r0) : kLdsRows;
    const int64_t base = r0 * B;
    const int cnt = (int)(rows * B);
    const int nq = cnt >> 2;
    float4 q[QPT];
#pragma unroll
    for (int k = 0; k < QPT; ++k)
        if (t + k * kLdsRows < nq) q[k] = ld_nt4(x + base, t + k * kLdsRows);
    const int tl = (nq << 2) + t;  // the cnt % 4 tail floats: threads 0..2
    const float tv = tl < cnt ? ld_nt(x + base + tl) : 0.0f;
#pragma unroll
    for (int k = 0; k < QPT; ++k)
        if (t + k * kLdsRows < nq) reinterpret_cast<float4*>(tile)[t + k * kLdsRows] = q[k];
    if (tl < cnt) tile[tl] = tv;
    *rows_out = rows;
    return base;
}

template <class R, int BMAX>
__global__ void __launch_bounds__(kLdsRows)
    k_rows_lds(const float* __restrict__ x, int64_t nrows, int B, float* out, float* out2, int epi, float div) {
    __shared__ float4 tile4[kLdsRows * BMAX / 4];
    float* tile = reinterpret_cast<float*>(tile4);
    const int t = threadIdx.x;
    const int64_t o = (int64_t)blockIdx.x * kLdsRows + t;
    // the row's starting value (the gradient, for a sequential accumulation) is loaded with the tile
    typename R::T acc = o < nrows ? row_start<R>(epi, out, o) : R::init();
    int64_t rows;
    stage_rows<BMAX>(tile, x, nrows, B, &rows);
    __syncthreads();
    if (t < rows) {
        for (int j = 0; j < B; ++j) acc = R::comb(acc, row_val<R>(epi, R::lift(tile[t * B + j])));
        epi_store(out, out2, o, acc, epi, div);
    }
}

// Short rows (C == 1, B <= BMAX) through any loader: the block's threads compute the values
// of rows [r0, r0 + 256) at consecutive element indices (coalesced, ld.get handles any
// position), stage them in LDS, then thread t reduces row r0 + t in element order -- the
// order of k_rows_lds and k_rows_thread.
template <class R, class LD, int BMAX>
__global__ void __launch_bounds__(kLdsRows)
    k_rows_lds_ld(LD ld, int64_t nrows, int B, float* out, float* out2, int epi, float div) {
    using T = typename R::T;
    __shared__ T tile[kLdsRows * BMAX];
    ld.setup();
    const int64_t r0 = (int64_t)blockIdx.x * kLdsRows;
    const int64_t rows = (nrows - r0) < kLdsRows ? (nrows - r0) : kLdsRows;
    const int64_t base = r0 * B;
    const int cnt = (int)(rows * B);
    const int t = threadIdx.x;
    // every value of the tile and the row's starting value are loaded before any LDS store
    // (unrolled over at most BMAX values per thread), so a block waits for memory once
    T acc = t < rows ? row_start<R>(epi, out, r0 + t) : R::init();
    T v[BMAX];
#pragma unroll
    for (int k = 0; k < BMAX; ++k)
        if (t + k * kLdsRows < cnt) v[k] = ld.get(base + t + k * kLdsRows);
#pragma unroll
    for (int k = 0; k < BMAX; ++k)
        if (t + k * kLdsRows < cnt) tile[t + k * kLdsRows] = v[k];
    __syncthreads();
    if (t < rows) {
        for (int j = 0; j < B; ++j) acc = R::comb(acc, row_val<R>(epi, tile[t * B + j]));
        epi_store(out, out2, r0 + t, acc, epi, div);
    }
}

// MAX backward over short rows in one pass (basics.mojo:581-615 for a last-axis reduce):
// the row max m and count c from the LDS tile, then grad[i] = grad[i] + (x[i] == m ?
// fl(1/c) * ug[row] : 0), x read once from HBM. Every load of the block (its x quads, its
// grad quads, its rows' ug) is issued before the first barrier, so a block waits for memory
// once; the grad quads wait in registers while the rows' maxima are found. Every grad quad
// is stored, unlike the long-row kernels' sparse stores: with rows of at most 32 elements
// every 128-byte line holds a row maximum, and 16-byte stores into most lines cost more than
// writing the lines whole (config 5's rows of 10: 28.6 us sparse, 22.7 us dense).
template <int BMAX>
__global__ void __launch_bounds__(kLdsRows)
    k_max_bwd_rows(float* __restrict__ grad, const float* __restrict__ x, const float* __restrict__ ug,
                   int64_t nrows, int B, FastDiv fdB) {
    constexpr int QPT = BMAX / 4;  // quads per thread: rows * B / 4 <= kLdsRows * BMAX / 4
    __shared__ float4 tile4[kLdsRows * BMAX / 4];
    __shared__ float sm[kLdsRows], sg[kLdsRows];
    float* tile = reinterpret_cast<float*>(tile4);
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * kLdsRows;
    const int64_t rows = (nrows - r0) < kLdsRows ? (nrows - r0) : kLdsRows;
    const int64_t base = r0 * B;
    const int cnt = (int)(rows * B);
    const int nq = cnt >> 2;
    float* gb = grad + base;
    // a quad past the tile reloads the tile's last one (the loads need no per-lane guard, under
    // which the compiler zeroed the registers first); a tile of no whole quad loads none
    float4 xq[QPT], gq[QPT];
    if (nq > 0) {
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int i = t + u * kLdsRows;
            xq[u] = ld_nt4(x + base, i < nq ? i : nq - 1);
            gq[u] = ld_nt4(gb, i < nq ? i : nq - 1);
        }
    }
    const float ugt = t < rows ? ug[r0 + t] : 0.0f;
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int i = t + u * kLdsRows;
        if (i < nq) tile4[i] = xq[u];
    }
    for (int i = (nq << 2) + t; i < cnt; i += kLdsRows) tile[i] = ld_nt(x + base + i);
    __syncthreads();
    if (t < rows) {
        MC acc = RMaxCnt::init();
        for (int j = 0; j < B; ++j) acc = RMaxCnt::comb(acc, RMaxCnt::lift(tile[t * B + j]));
        const float f = 1.0f / (float)acc.c;  // basics.mojo:609
        sm[t] = acc.m;
        sg[t] = f * ugt;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < QPT; ++u) {
        const int i = t + u * kLdsRows;
        if (i >= nq) break;
        const float4 o = gq[u];
        float r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * i + j;
            const int row = (int)fdiv((uint32_t)e, fdB);
            r[j] = tile[e] == sm[row] ? sg[row] : 0.0f;
        }
        const float4 g = make_float4(o.x + r[0], o.y + r[1], o.z + r[2], o.w + r[3]);
        st_nt4(gb, i, g);
    }
    for (int e = (nq << 2) + t; e < cnt; e += kLdsRows) {
        const int row = (int)fdiv((uint32_t)e, fdB);
        grad[base + e] = grad[base + e] + (tile[e] == sm[row] ? sg[row] : 0.0f);
    }
}

// One wavefront per (row, chunk): virtual row vr = r * S + s covers elements
// [r*B + s*L, r*B + min((s+1)*L, B)). S == 1 writes the epilogue, S > 1 writes partials.
template <class R, class LD, bool VEC>
__global__ void __launch_bounds__(kRThreads)
    k_rows_wave(LD ld, int64_t nvrows, int64_t S, int64_t B, int64_t L, float* out, float* out2,
                int epi, float div, float* part) {
    ld.setup();
    using T = typename R::T;
    const int lane = threadIdx.x & 63;
    const int64_t vr = (int64_t)blockIdx.x * (kRThreads / 64) + (threadIdx.x >> 6);
    if (vr >= nvrows) return;  // uniform per wavefront; no block-level barrier follows
    const int64_t r = vr / S, s = vr - r * S;
    const int64_t start = r * B + s * L;
    const int64_t rem = B - s * L;
    const int64_t len = rem < L ? rem : L;
    T acc = R::init();
    if (VEC) {
        const int64_t nq = len >> 2;
        T a4[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) a4[u][j] = R::init();
        int64_t q = lane;
        for (; q + 192 < nq; q += 256) {
            T v[4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) ld.get4(start + (q + 64 * u) * 4, v[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) a4[u][j] = R::comb(a4[u][j], v[u][j]);
        }
        for (; q < nq; q += 64) {
            T v[4];
            ld.get4(start + q * 4, v);
#pragma unroll
            for (int j = 0; j < 4; ++j) a4[0][j] = R::comb(a4[0][j], v[j]);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = R::comb(acc, a4[u][j]);
    } else {
        for (int64_t j = lane; j < len; j += 64) acc = R::comb(acc, ld.get(start + j));
    }
    acc = wave_reduce<R>(acc);
    if (lane == 0) {
        if (S == 1) epi_store(out, out2, r, acc, epi, div);
        else part_store2(part, nvrows, vr, acc);
    }
}

// Short columns (B <= 64) of a serial accumulation (EPI_SEQ_ACCUM / _NEG): one thread per
// output element walks its B values in row order, eight loads in flight, adding each into the
// output one at a time (row_start / row_val) in one launch with no split.
template <class R, class LD>
__global__ void __launch_bounds__(kRThreads)
    k_cols_seq(LD ld, int64_t A, int64_t B, int64_t C, float* out, float* out2, int epi, float div) {
    ld.setup();
    using T = typename R::T;
    const int64_t o = (int64_t)blockIdx.x * kRThreads + threadIdx.x;
    if (o >= A * C) return;
    const int64_t a = o / C, c = o - a * C;
    const int64_t base = a * B * C + c;
    T acc = row_start<R>(epi, out, o);
    int64_t b = 0;
    for (; b + 7 < B; b += 8) {
        T v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ld.get(base + (b + u) * C);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = R::comb(acc, row_val<R>(epi, v[u]));
    }
    for (; b < B; ++b) acc = R::comb(acc, row_val<R>(epi, ld.get(base + b * C)));
    epi_store(out, out2, o, acc, epi, div);
}

// Column reduction: item = a quad (VEC) or one element of the flattened [A, C] output; the
// rows [b0, b1) of split blockIdx.y. S == 1 writes the epilogue, S > 1 writes partials at
// s * (A * C) + o.
template <class R, class LD, bool VEC, bool SPLIT_X = false>
__global__ void __launch_bounds__(kRThreads)
    k_cols(LD ld, int64_t A, int64_t B, int64_t C, int64_t rps, int64_t S, float* out, float* out2,
           int epi, float div, float* part) {
    ld.setup();
    using T = typename R::T;
    constexpr int W = VEC ? 4 : 1;
    const int64_t AC = A * C;
    const int64_t item = (int64_t)(SPLIT_X ? blockIdx.y : blockIdx.x) * kRThreads + threadIdx.x;
    const int64_t o = item * W;
    if (o >= AC) return;
    const int64_t a = o / C, c = o - a * C;
    const int64_t s = SPLIT_X ? blockIdx.x : blockIdx.y;
    const int64_t b0 = s * rps;
    const int64_t b1 = (b0 + rps < B) ? b0 + rps : B;
    const int64_t base = a * B * C + c;
    T acc[W];
#pragma unroll
    for (int j = 0; j < W; ++j) acc[j] = R::init();
    int64_t b = b0;
    constexpr int RU = VEC ? 2 : 4;  // rows in flight
    for (; b + RU - 1 < b1; b += RU) {
        T v[RU][W];
#pragma unroll
        for (int u = 0; u < RU; ++u) {
            if (VEC) ld.get4(base + (b + u) * C, v[u]);
            else v[u][0] = ld.get(base + (b + u) * C);
        }
#pragma unroll
        for (int u = 0; u < RU; ++u)
#pragma unroll
            for (int j = 0; j < W; ++j) acc[j] = R::comb(acc[j], v[u][j]);
    }
    for (; b < b1; ++b) {
        T v[W];
        if (VEC) ld.get4(base + b * C, v);
        else v[0] = ld.get(base + b * C);
#pragma unroll
        for (int j = 0; j < W; ++j) acc[j] = R::comb(acc[j], v[j]);
    }
#pragma unroll
    for (int j = 0; j < W; ++j) {
        if (S == 1) epi_store(out, out2, o + j, acc[j], epi, div);
        else part_store2(part, S * AC, s * AC + o + j, acc[j]);
    }
}

// A pass over chunk partials (a row of at most kCombineMax elements per block, one block per
// row): 1024 threads, each with all of its (up to eight) quads' loads in flight, so the row
// takes one memory round trip; the sixteen wave results combine by a fixed butterfly.
constexpr int kCombThreads = 1024;
template <class R, class LD, bool VEC>
__global__ void __launch_bounds__(kCombThreads)
    k_row_comb(LD ld, int64_t B, float* out, float* out2, int epi, float div) {
    using T = typename R::T;
    __shared__ T ws[kCombThreads / 64];
    ld.setup();
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int64_t r = blockIdx.x, start = r * B;
    T acc = R::init();
    if (VEC) {
        constexpr int U = 8;  // kCombineMax / (4 * kCombThreads)
        T v[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t e = ((int64_t)u * kCombThreads + t) * 4;
            if (e < B) ld.get4(start + e, v[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t e = ((int64_t)u * kCombThreads + t) * 4;
            if (e < B)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc = R::comb(acc, v[u][j]);
        }
    } else {
        for (int64_t e = t; e < B; e += kCombThreads) acc = R::comb(acc, ld.get(start + e));
    }
    acc = wave_reduce<R>(acc);
    if (lane == 0) ws[w] = acc;
    __syncthreads();
    if (w == 0) {  // the sixteen wave results by a butterfly within lanes 0-15 (a serial fold of
                   // max-count pairs took 2 us more)
        static_assert(kCombThreads / 64 == 16, "sixteen waves");
        T v = lane < 16 ? ws[lane] : R::init();
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1) v = R::comb(v, R::shfl(v, m));
        if (lane == 0) epi_store(out, out2, r, v, epi, div);
    }
}

// Combine of S split partials [S, n] (n % 4 == 0) in one launch with few memory round trips:
// a block is kPcQuads column quads x kPcGroups row groups; group r adds the partial rows
// [r * rpg, min((r + 1) * rpg, S)) in order, eight rows' loads in flight, and the groups' results
// fold in LDS as a fixed tree (group r with r + h for h = 16, 8, ..., 1), after which group 0
// writes the epilogue. Folding the groups one after another into group 0 cost 2-2.5 us more
// with max-count pairs ([8192, 8192] axis 0, 128 splits: 8.5 against 6.0 us in a probe).
constexpr int kPcQuads = 8, kPcGroups = kRThreads / kPcQuads;
template <class R, class LD>
__global__ void __launch_bounds__(kRThreads)
    k_parts_comb(LD ld, int64_t S, int64_t n, int64_t rpg, float* out, float* out2, int epi, float div) {
    using T = typename R::T;
    __shared__ T lds[kPcGroups][kPcQuads][4];
    ld.setup();
    const int q = threadIdx.x % kPcQuads, r = threadIdx.x / kPcQuads;
    const int64_t o = ((int64_t)blockIdx.x * kPcQuads + q) * 4;
    const bool active = o < n;
    T acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = R::init();
    if (active) {
        const int64_t s0 = r * rpg;
        const int64_t s1 = s0 + rpg < S ? s0 + rpg : S;
        for (int64_t s = s0; s < s1; s += 8) {
            T v[8][4];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s + u < s1) ld.get4((s + u) * n + o, v[u]);
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s + u < s1)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[j] = R::comb(acc[j], v[u][j]);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) lds[r][q][j] = acc[j];
    __syncthreads();
#pragma unroll
    for (int h = kPcGroups / 2; h >= 1; h >>= 1) {  // every thread reaches every barrier
        if (r < h)
#pragma unroll
            for (int j = 0; j < 4; ++j) lds[r][q][j] = R::comb(lds[r][q][j], lds[r + h][q][j]);
        __syncthreads();
    }
    if (r == 0 && active) {
#pragma unroll
        for (int j = 0; j < 4; ++j) epi_store(out, out2, o + j, lds[0][q][j], epi, div);
    }
}

// Rows of >= 2048 elements: one block (4 waves) per (row, chunk) of L = 2048 elements, two
// quads per thread in flight (small one-shot blocks stream best on gfx950). Block
// vr = r * S + s covers elements [r*B + s*L, r*B + min((s+1)*L, B)); the four wave results
// combine in wave order. S == 1 writes the row's epilogue, S > 1 the partial part[vr].
constexpr int64_t kRowChunk = 2048;
template <class R, class LD, bool VEC>
__global__ void __launch_bounds__(kRThreads)
    k_rows_block(LD ld, int64_t S, int64_t B, int64_t L, float* out, float* out2, int epi, float div,
                 float* part, int64_t npart) {
    using T = typename R::T;
    __shared__ T ws[4];
    ld.setup();
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int64_t vr = blockIdx.x;
    const int64_t r = vr / S, s = vr - r * S;
    const int64_t start = r * B + s * L;
    const int64_t rem = B - s * L;
    const int64_t len = rem < L ? rem : L;
    T acc = R::init();
    constexpr bool kMaxCntFirst = std::is_same<R, RMaxCnt>::value && std::is_same<LD, LdPlain<RMaxCnt>>::value;
    if constexpr (VEC && kMaxCntFirst) {
        // a first-level max-count chunk (L <= kRowChunk: at most two quads per thread): the
        // lane's maximum by comparisons, then its count as the elements equal to it, which is
        // RMaxCnt's count (NaN, also the filler of a missing quad, is neither) without the
        // pairwise combining (46.8 -> 39.4 us over 2^26 elements, the plain maximum's time)
        static_assert(kRowChunk <= 8 * kRThreads, "a first-level chunk is at most two quads per thread");
        const int64_t nq = len >> 2;
        const float nan = __builtin_nanf("");
        const float4 fq = make_float4(nan, nan, nan, nan);
        const float* xs = ld.x + start;
        const float4 qa = t < nq ? ld_nt4(xs, t) : fq;
        const float4 qb = t + kRThreads < nq ? ld_nt4(xs, t + kRThreads) : fq;
        const float v[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        float m = -FLT_MAX;
#pragma unroll
        for (int j = 0; j < 8; ++j) m = v[j] > m ? v[j] : m;
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) c += v[j] == m ? 1u : 0u;
        acc = MC{m, c};
    } else if (VEC) {
        const int64_t nq = len >> 2;
        T a2[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) a2[u][j] = R::init();
        int64_t q = t;
        for (; q + kRThreads < nq; q += 2 * kRThreads) {
            T v[2][4];
            ld.get4(start + q * 4, v[0]);
            ld.get4(start + (q + kRThreads) * 4, v[1]);
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) a2[u][j] = R::comb(a2[u][j], v[u][j]);
        }
        if (q < nq) {
            T v[4];
            ld.get4(start + q * 4, v);
#pragma unroll
            for (int j = 0; j < 4; ++j) a2[0][j] = R::comb(a2[0][j], v[j]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = R::comb(acc, a2[u][j]);
    } else {
        for (int64_t j = t; j < len; j += kRThreads) acc = R::comb(acc, ld.get(start + j));
    }
    if constexpr (std::is_same<R, RMaxCnt>::value && std::is_same<LD, LdPlain<RMaxCnt>>::value)
        acc = wave_reduce_mc_small(acc);  // L <= kRowChunk: at most eight elements per lane
    else
        acc = wave_reduce<R>(acc);
    if (lane == 0) ws[w] = acc;
    __syncthreads();
    if (t == 0) {
        const T tot = R::comb(R::comb(R::comb(ws[0], ws[1]), ws[2]), ws[3]);
        if (S == 1) epi_store(out, out2, r, tot, epi, div);
        else part_store2(part, npart, vr, tot);
    }
}

// Strided-axis reduction over [A, B, C] with C % 4 == 0: block (a * nstrips + strip, s) owns
// the 64 column quads [strip * 64, strip * 64 + 64) of slab a (lane = quad) and the rows
// [s * rps, min((s + 1) * rps, B)), which its four waves interleave (wave w: rows b0 + w,
// b0 + w + 4, ...). Every wave reads 1 KiB contiguous per row; the wave results combine in
// wave order through LDS. S == 1 writes the epilogue, S > 1 partials at s * (A * C) + o.
template <class R, class LD>
__global__ void __launch_bounds__(kRThreads)
    k_cols_strip(LD ld, int64_t A, int64_t B, int64_t C, int64_t nstrips, int64_t rps, int64_t S,
                 float* out, float* out2, int epi, float div, float* part) {
    using T = typename R::T;
    __shared__ T lds[3][64][4];
    ld.setup();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t bx = blockIdx.x;
    const int64_t a = bx / nstrips, strip = bx - a * nstrips;
    const int64_t cq = strip * 64 + lane;
    const bool active = cq < (C >> 2);
    const int64_t s = blockIdx.y;
    const int64_t b0 = s * rps;
    const int64_t b1 = (b0 + rps < B) ? b0 + rps : B;
    T acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = R::init();
    if (active) {
        const int64_t base = a * B * C + cq * 4;
        int64_t b = b0 + w;
        for (; b + 12 < b1; b += 16) {
            T v[4][4];
#pragma unroll
            for (int u = 0; u < 4; ++u) ld.get4(base + (b + 4 * u) * C, v[u]);
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[j] = R::comb(acc[j], v[u][j]);
        }
        for (; b < b1; b += 4) {
            T v[4];
            ld.get4(base + b * C, v);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = R::comb(acc[j], v[j]);
        }
    }
    if (w > 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) lds[w - 1][lane][j] = acc[j];
    }
    __syncthreads();
    if (w == 0 && active) {
#pragma unroll
        for (int ww = 0; ww < 3; ++ww)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = R::comb(acc[j], lds[ww][lane][j]);
        const int64_t o = a * C + cq * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (S == 1) epi_store(out, out2, o + j, acc[j], epi, div);
            else part_store2(part, S * A * C, s * A * C + o + j, acc[j]);
        }
    }
}

// MAX backward over rows of B <= 16384 elements (B % 4 == 0), one pass: the row is held in
// registers (NQ quads per thread, WPR waves per row), its max and count reduced across the
// row's threads, then grad[i] = grad[i] + (x[i] == m ? fl(1/c) * ug[row] : 0) from the same
// registers (basics.mojo:581-615 for a last-axis reduce): x is read once.
template <int WPR, int NQ>
__global__ void __launch_bounds__(kRThreads)
    k_max_bwd_rowreg(float* __restrict__ grad, const float* __restrict__ x, const float* __restrict__ ug,
                     int64_t nrows, int64_t B) {
    __shared__ MC ws[4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t row = WPR == 1 ? (int64_t)blockIdx.x * 4 + w : (int64_t)blockIdx.x;
    if (row >= nrows) return;  // WPR == 1: uniform per wave, and that path has no barrier
    const int tr = WPR == 1 ? lane : (int)threadIdx.x;
    constexpr int NT = 64 * WPR;
    const int64_t Bq = B >> 2;
    const float* xr = x + row * B;
    float* gr = grad + row * B;
    // One wave per row (WPR == 1): the row's x and grad quads and its ug are loaded together,
    // one wait for memory, the grad quads held in registers while the row's max and count
    // are found ([64, 512, 1024]: 47.5 -> 46.1 us). Four waves per row keep the grad loads
    // after the reduction: holding them would take 8 of 16 quads' registers and cut the
    // resident waves from 8 to 5 per SIMD ([8192, 8192] axis 1: 80.9 -> 82.1 us).
    constexpr bool PRE = WPR == 1;
    float4 v[NQ], o[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int64_t qi = tr + (int64_t)k * NT;
        if (qi < Bq) {
            v[k] = ld_nt4(xr, qi);
            if (PRE) o[k] = ld_nt4(gr, qi);
        }
    }
    const float u = PRE ? ug[row] : 0.0f;
    MC acc = RMaxCnt::init();
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int64_t qi = tr + (int64_t)k * NT;
        if (qi < Bq) {
            acc = RMaxCnt::comb(acc, RMaxCnt::lift(v[k].x));
            acc = RMaxCnt::comb(acc, RMaxCnt::lift(v[k].y));
            acc = RMaxCnt::comb(acc, RMaxCnt::lift(v[k].z));
            acc = RMaxCnt::comb(acc, RMaxCnt::lift(v[k].w));
        }
    }
    acc = wave_reduce<RMaxCnt>(acc);
    if (WPR == 4) {
        if (lane == 0) ws[w] = acc;
        __syncthreads();
        acc = RMaxCnt::comb(RMaxCnt::comb(RMaxCnt::comb(ws[0], ws[1]), ws[2]), ws[3]);
    }
    const float f = 1.0f / (float)acc.c;  // basics.mojo:609
    const float g = f * (PRE ? u : ug[row]);
    const float m = acc.m;
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int64_t qi = tr + (int64_t)k * NT;
        if (qi < Bq) {
            const float4 ok = PRE ? o[k] : ld_nt4(gr, qi);
            const float4 n = make_float4(ok.x + (v[k].x == m ? g : 0.0f), ok.y + (v[k].y == m ? g : 0.0f),
                                         ok.z + (v[k].z == m ? g : 0.0f), ok.w + (v[k].w == m ? g : 0.0f));
            if (bits_differ4(ok.x, ok.y, ok.z, ok.w, n.x, n.y, n.z, n.w)) st_nt4(gr, qi, n);  // a sparse accumulation
        }
    }
}

// MAX backward routing behind a split max-count reduction (basics.mojo:567-577, 597-613):
// grad[i] = grad[i] + (x[i] == m ? fl(1/c) * ug : 0) for the line maximum m, each grad quad
// stored only when its bits change. The reduction's first pass left each split's partial
// maximum pm (a column's rows [s * rps, (s + 1) * rps), or a row's chunk s). A split holding
// an element x[i] == m has pm == m: pm >= x[i] as the maximum of its elements, pm <= m as one
// of the values m is the maximum of, and neither is NaN (RMaxCnt keeps NaN out of the
// maximum, so x[i] == m excludes it too). A split with pm != m therefore holds no element of
// its line's maximum: every term there is +0, and its x is not read (grad + 0 still turns -0
// into +0, which the sparse store writes back). Where the partials also hold the split's count
// and the index of its maximum (RMaxCntArg), a split with pm == m and count 1 holds exactly
// one such element, at that index, and count 0 none; x is read again only in a split that
// holds several.
// Changed quads wait in registers (two of them) and are stored after the thread's loads: a
// store issued between loads would hold every later wait for loaded data until the store
// completes (vmcnt counts stores as well as loads), which cost the column route a third of
// its time. A third change in one thread stores at once.
struct PendingStores {
    int64_t q0 = 0, q1 = 0;
    float4 v0, v1;
    int n = 0;
    __device__ __forceinline__ void put(float* gr, int64_t q, float4 v) {
        if (n == 0) {
            q0 = q; v0 = v; n = 1;
        } else if (n == 1) {
            q1 = q; v1 = v; n = 2;
        } else {
            st_nt4(gr, q, v);
        }
    }
    __device__ __forceinline__ void flush(float* gr) const {
        if (n > 0) st_nt4(gr, q0, v0);
        if (n > 1) st_nt4(gr, q1, v1);
    }
};
// grad quad g plus add[j] where hit[j], else plus +0; queued when its bits change.
__device__ __forceinline__ void route_quad(PendingStores& pd, float* gr, int64_t q, float4 g, const bool (&hit)[4],
                                           const float (&add)[4]) {
    const float4 n = make_float4(g.x + (hit[0] ? add[0] : 0.0f), g.y + (hit[1] ? add[1] : 0.0f),
                                 g.z + (hit[2] ? add[2] : 0.0f), g.w + (hit[3] ? add[3] : 0.0f));
    if (bits_differ4(g.x, g.y, g.z, g.w, n.x, n.y, n.z, n.w)) pd.put(gr, q, n);
}
__device__ __forceinline__ void route_quad_x(PendingStores& pd, float* gr, int64_t q, float4 g, float4 xv, bool need,
                                             const float (&mv)[4], const float (&add)[4]) {
    const bool hit[4] = {need && xv.x == mv[0], need && xv.y == mv[1], need && xv.z == mv[2], need && xv.w == mv[3]};
    route_quad(pd, gr, q, g, hit, add);
}

// Columns (C % 4 == 0, 16-byte aligned grad and x, fewer than 2^32 elements): a thread per
// (column quad o, split s), the layout of the reduction's column launchers; two rows in
// flight. SPLIT_X: splits on grid x, column-quad blocks on grid y. pm / pc / pi hold the
// splits' maxima, counts and indices (RMaxCntArg); they, m and f are 16-byte aligned scratch:
// one quad load each.
template <bool SPLIT_X>
__global__ void __launch_bounds__(kRThreads)
    k_max_route_cols(float* __restrict__ grad, const float* __restrict__ x, const float* __restrict__ m,
                     const float* __restrict__ f, const float* __restrict__ ug, const float* __restrict__ pm,
                     const uint32_t* __restrict__ pc, const uint32_t* __restrict__ pi, int64_t A, int64_t B,
                     int64_t C, int64_t rps) {
    const int64_t AC = A * C;
    const int64_t o = ((int64_t)(SPLIT_X ? blockIdx.y : blockIdx.x) * kRThreads + threadIdx.x) * 4;
    if (o >= AC) return;
    const int64_t s = SPLIT_X ? blockIdx.x : blockIdx.y;
    const int64_t a = o / C, c = o - a * C;
    const int64_t b0 = s * rps, b1 = b0 + rps < B ? b0 + rps : B;
    const int64_t e0 = a * B * C + c;  // element of row 0, column c
    const int64_t k = s * AC + o;      // this split's partials of columns o .. o + 3
    const float4 m4 = *reinterpret_cast<const float4*>(m + o), f4 = *reinterpret_cast<const float4*>(f + o);
    const float4 p4 = *reinterpret_cast<const float4*>(pm + k);
    const uint4 c4 = *reinterpret_cast<const uint4*>(pc + k), i4 = *reinterpret_cast<const uint4*>(pi + k);
    const float u[4] = {ug[o], ug[o + 1], ug[o + 2], ug[o + 3]};
    const float mv[4] = {m4.x, m4.y, m4.z, m4.w};
    const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
    const float fv[4] = {f4.x, f4.y, f4.z, f4.w};
    const uint32_t cv[4] = {c4.x, c4.y, c4.z, c4.w}, iv[4] = {i4.x, i4.y, i4.z, i4.w};
    // column j's single maximum in this split as an element offset from (row b0, column c + j),
    // a multiple of C (x has fewer than 2^32 elements); else 0xffffffff, which no row's offset
    // r * C < 2^32 reaches
    const uint32_t eb = (uint32_t)(e0 + b0 * C);
    float add[4];
    uint32_t sel[4];
    bool xread = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        add[j] = fv[j] * u[j];
        const bool nj = pv[j] == mv[j];
        xread = xread || (nj && cv[j] >= 2u);
        sel[j] = nj && cv[j] == 1u ? iv[j] - (eb + (uint32_t)j) : 0xffffffffu;
    }
    const int64_t q0 = (e0 >> 2) + b0 * (C >> 2), qs = C >> 2;  // quad of row b0 + r: q0 + r * qs
    const int nr = (int)(b1 - b0);
    const uint32_t uc = (uint32_t)C;
    // One loop for both ways (x compared, or the row offset against sel): with a loop per way
    // in a branch that is uniform over few waves, the kernel took 61 us against 43 us here
    // ([8192, 8192], axis 0).
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    PendingStores pd;
    uint32_t rc = 0;  // r * C
    int r = 0;
    for (; r + 1 < nr; r += 2, rc += 2 * uc) {
        const int64_t qa = q0 + r * qs, qb = qa + qs;
        const float4 ga = ld_nt4(grad, qa), gb = ld_nt4(grad, qb);
        const float4 xa = xread ? ld_nt4(x, qa) : z, xb = xread ? ld_nt4(x, qb) : z;
        const uint32_t rd = rc + uc;
        const bool ha[4] = {xread ? xa.x == mv[0] : rc == sel[0], xread ? xa.y == mv[1] : rc == sel[1],
                            xread ? xa.z == mv[2] : rc == sel[2], xread ? xa.w == mv[3] : rc == sel[3]};
        const bool hb[4] = {xread ? xb.x == mv[0] : rd == sel[0], xread ? xb.y == mv[1] : rd == sel[1],
                            xread ? xb.z == mv[2] : rd == sel[2], xread ? xb.w == mv[3] : rd == sel[3]};
        route_quad(pd, grad, qa, ga, ha, add);
        route_quad(pd, grad, qb, gb, hb, add);
    }
    if (r < nr) {
        const int64_t qa = q0 + r * qs;
        const float4 ga = ld_nt4(grad, qa), xa = xread ? ld_nt4(x, qa) : z;
        const bool ha[4] = {xread ? xa.x == mv[0] : rc == sel[0], xread ? xa.y == mv[1] : rc == sel[1],
                            xread ? xa.z == mv[2] : rc == sel[2], xread ? xa.w == mv[3] : rc == sel[3]};
        route_quad(pd, grad, qa, ga, ha, add);
    }
    pd.flush(grad);
}

// Rows (C == 1, B % 4 == 0, 16-byte aligned grad and x): a block per chunk vr = r * S + s of
// kRowChunk elements (the reduction's row chunks), two quads per thread; whether the chunk
// reads x is uniform over the block.
__global__ void __launch_bounds__(kRThreads)
    k_max_route_rows(float* __restrict__ grad, const float* __restrict__ x, const float* __restrict__ m,
                     const float* __restrict__ f, const float* __restrict__ ug, const float* __restrict__ pm,
                     int64_t S, int64_t B) {
    const int64_t vr = blockIdx.x;
    const int64_t r = vr / S, s = vr - r * S;
    const int64_t rem = B - s * kRowChunk;
    const int64_t nq = (rem < kRowChunk ? rem : kRowChunk) >> 2;
    const int64_t q0 = (r * B + s * kRowChunk) >> 2;
    const float mr = m[r];
    const float ad = f[r] * ug[r];
    const float mv[4] = {mr, mr, mr, mr}, add[4] = {ad, ad, ad, ad};
    const bool need = pm[vr] == mr;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    const int t = threadIdx.x;
    static_assert(kRowChunk == 8 * kRThreads, "two quads per thread cover a chunk");
    const bool ha = t < nq, hb = t + kRThreads < nq;
    const float4 ga = ha ? ld_nt4(grad, q0 + t) : z, gb = hb ? ld_nt4(grad, q0 + t + kRThreads) : z;
    const float4 xa = ha && need ? ld_nt4(x, q0 + t) : z, xb = hb && need ? ld_nt4(x, q0 + t + kRThreads) : z;
    PendingStores pd;
    if (ha) route_quad_x(pd, grad, q0 + t, ga, xa, need, mv, add);
    if (hb) route_quad_x(pd, grad, q0 + t + kRThreads, gb, xb, need, mv, add);
    pd.flush(grad);
}

// ---------------------------------------------------------------------------------------
// tstd: one pass over x, fp64 moments
// ---------------------------------------------------------------------------------------
// The reference takes each line's mean in fp32, then sums the squared deviations from it
// (tensorutils.mojo:723-840): two passes over x. Here each line's moments about its first
// element K are accumulated in fp64 in one pass, S1 = sum(x - K) and S2 = sum((x - K)^2)
// (x - K of two fp32 values is exact in fp64), and the squared deviations from the mean are
// S2 - S1^2 / B. The fp64 rounding of that difference is about 2^-53 ((mean - K) / std)^2
// relative, far under the fp32 rounding of the reference's own two passes, so the result is
// in the sum class. The epilogue is the reference's: sqrt(f32(variance) / f32(B)).
struct Mom {
    double s1, s2;
};
constexpr int64_t kMomMaxSplit = 4096;  // row chunks per row at most (longer chunks beyond)

__device__ __forceinline__ void mom_add(Mom& m, float v, double K) {
    const double d = (double)v - K;
    m.s1 = m.s1 + d;
    m.s2 = __builtin_fma(d, d, m.s2);
}

__device__ __forceinline__ Mom mom_wave(Mom m) {
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) {
        m.s1 = m.s1 + __shfl_xor(m.s1, k);
        m.s2 = m.s2 + __shfl_xor(m.s2, k);
    }
    return m;
}

__device__ __forceinline__ float mom_std(const Mom& m, int64_t B) {
    double v = m.s2 - m.s1 * m.s1 / (double)B;
    if (v < 0.0) v = 0.0;  // rounding of a zero variance (NaN passes through)
    return __builtin_sqrtf((float)v / (float)B);
}

// tstd over rows of B % 4 == 0, B <= 16384 elements: WPR waves per row, the row's quads
// loaded together, fp64 moments (above) summed per lane in quad order, then the butterfly and
// the waves in order.
template <int WPR, int NQ>
__global__ void __launch_bounds__(kRThreads)
    k_tstd_rowreg(float* __restrict__ res, const float* __restrict__ x, int64_t nrows, int64_t B) {
    __shared__ Mom ws[4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t row = WPR == 1 ? (int64_t)blockIdx.x * 4 + w : (int64_t)blockIdx.x;
    if (row >= nrows) return;  // WPR == 1: uniform per wave, and that path has no barrier
    const int tr = WPR == 1 ? lane : (int)threadIdx.x;
    constexpr int NT = 64 * WPR;
    const int64_t Bq = B >> 2;
    const float* xr = x + row * B;
    // the row's quads load before K is needed (a quad past the row loads the last quad, then
    // holds K: x - K = 0 adds nothing to either moment), so K's load is not waited for first
    vf4 v[NQ];
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int64_t qi = tr + (int64_t)k * NT;
        v[k] = ld_ntv(xr, qi < Bq ? qi : Bq - 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    const float kf = xr[0];
    const double K = (double)kf;
#pragma unroll
    for (int k = 0; k < NQ; ++k)
        if (tr + (int64_t)k * NT >= Bq) v[k] = vf4{kf, kf, kf, kf};
    Mom m{0.0, 0.0};
#pragma unroll
    for (int k = 0; k < NQ; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) mom_add(m, v[k][j], K);
    m = mom_wave(m);
    if (WPR == 4) {
        if (lane == 0) ws[w] = m;
        __syncthreads();
        m = ws[0];
        for (int k = 1; k < 4; ++k) {
            m.s1 = m.s1 + ws[k].s1;
            m.s2 = m.s2 + ws[k].s2;
        }
    }
    if (tr == 0) res[row] = mom_std(m, B);
}

// Rows: block vr = r * S + s sums elements [s * L, min((s + 1) * L, B)) of row r (VEC: two
// quads per thread in flight), its four waves in order; S == 1 writes the row's result,
// S > 1 the partial part[vr].
template <bool VEC>
__global__ void __launch_bounds__(kRThreads)
    k_tstd_mom_rows(float* __restrict__ res, const float* __restrict__ x, int64_t B, int64_t L, int64_t S,
                    Mom* __restrict__ part) {
    __shared__ Mom ws[4];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int64_t vr = blockIdx.x;
    const int64_t r = vr / S, s = vr - r * S;
    const int64_t start = r * B + s * L;
    const int64_t rem = B - s * L;
    const int64_t len = rem < L ? rem : L;
    Mom m{0.0, 0.0};
    if (VEC) {
        // four quads in flight; element j of every quad goes to accumulator chain j, and the
        // chains are added in order (one chain had 16 dependent fp64 adds per pass of a
        // 16384-element chunk: all-element tstd over 2^26 elements took 49.9 us)
        const int64_t nq = len >> 2;
        const float* xs = x + start;
        // K (the row's first element) as a vector load, which the first quads' loads follow
        // without waiting for it: a scalar load here was waited for before any of them issued
        const float kf = __hip_atomic_load(x + r * B, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        Mom mc[4] = {Mom{0.0, 0.0}, Mom{0.0, 0.0}, Mom{0.0, 0.0}, Mom{0.0, 0.0}};
        for (int64_t q = t; q < nq; q += 4 * kRThreads) {
            // a quad past the chunk loads the chunk's last quad, then holds K: x - K = 0 adds
            // nothing to either moment
            vf4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t qi = q + u * kRThreads;
                v[u] = ld_ntv(xs, qi < nq ? qi : nq - 1);
            }
            float kq = kf;
            asm volatile("" : "+v"(kq) : : "memory");  // K's wait and conversion after the loads above
            const double K = (double)kq;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (q + u * kRThreads >= nq) v[u] = vf4{kq, kq, kq, kq};
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < 4; ++j) mom_add(mc[j], v[u][j], K);
        }
        m = mc[0];
#pragma unroll
        for (int j = 1; j < 4; ++j) {
            m.s1 = m.s1 + mc[j].s1;
            m.s2 = m.s2 + mc[j].s2;
        }
    } else {
        const double K = (double)x[r * B];
        for (int64_t j = t; j < len; j += kRThreads) mom_add(m, ld_nt(x + start + j), K);
    }
    m = mom_wave(m);
    if (lane == 0) ws[w] = m;
    __syncthreads();
    if (t == 0) {
        Mom tot = ws[0];
        for (int k = 1; k < 4; ++k) {
            tot.s1 = tot.s1 + ws[k].s1;
            tot.s2 = tot.s2 + ws[k].s2;
        }
        if (S == 1) res[r] = mom_std(tot, B);
        else part[vr] = tot;
    }
}

// Strided axis over [A, B, C]: thread = a quad (VEC) or one element of the [A, C] output,
// rows [s * rps, min((s + 1) * rps, B)) of split s in order; K is the line's element at row
// 0. S == 1 writes the result, S > 1 partials at s * (A * C) + o. SPLIT_X puts the splits on
// grid x (the column blocks on y), so the round-robin dispatch spreads each column block's
// splits over the eight XCDs instead of giving each XCD one column block of every row.
template <bool VEC, bool SPLIT_X>
__global__ void __launch_bounds__(kRThreads)
    k_tstd_mom_cols(float* __restrict__ res, const float* __restrict__ x, int64_t A, int64_t B, int64_t C,
                    int64_t rps, int64_t S, Mom* __restrict__ part) {
    constexpr int W = VEC ? 4 : 1;
    const int64_t AC = A * C;
    const int64_t o = ((int64_t)(SPLIT_X ? blockIdx.y : blockIdx.x) * kRThreads + threadIdx.x) * W;
    if (o >= AC) return;
    const int64_t a = o / C, c = o - a * C;
    const int64_t s = SPLIT_X ? blockIdx.x : blockIdx.y;
    const int64_t b0 = s * rps;
    const int64_t b1 = b0 + rps < B ? b0 + rps : B;
    const int64_t base = a * B * C + c;
    auto load = [&](int64_t b, float* v) {
        if (VEC) {
            const vf4 q = ld_ntv(x + base + b * C, 0);
#pragma unroll
            for (int j = 0; j < W; ++j) v[j] = q[j];
        } else {
            v[0] = ld_nt(x + base + b * C);
        }
    };
    // eight rows in flight, the next eight loaded before the current eight are added (about
    // one wave per SIMD runs this kernel, so no other wave's loads cover its fp64 work); row u
    // of each eight goes to accumulator chain u % 4 (the rest of the split to chain 0), and the
    // chains are added in order at the end. K (the line's row 0) loads with the first eight
    // rows (rows past the split reload its last row), not before them.
    constexpr int RU = 8, CH = 4;
    Mom m[CH][W];
#pragma unroll
    for (int h = 0; h < CH; ++h)
#pragma unroll
        for (int j = 0; j < W; ++j) m[h][j] = Mom{0.0, 0.0};
    float k0[W], v[RU][W];
    load(0, k0);
#pragma unroll
    for (int u = 0; u < RU; ++u) load(b0 + u < b1 ? b0 + u : b1 - 1, v[u]);
    double K[W];
#pragma unroll
    for (int j = 0; j < W; ++j) {
        asm volatile("" : "+v"(k0[j]) : : "memory");  // K's wait and conversion after the loads above
        K[j] = (double)k0[j];
    }
#pragma unroll
    for (int u = 0; u < RU; ++u)  // rows past a short split hold K: x - K = 0 adds nothing
        if (b0 + u >= b1)
#pragma unroll
            for (int j = 0; j < W; ++j) v[u][j] = k0[j];
    auto add_rows = [&](const float (&r)[RU][W]) {
#pragma unroll
        for (int u = 0; u < RU; ++u)
#pragma unroll
            for (int j = 0; j < W; ++j) mom_add(m[u % CH][j], r[u][j], K[j]);
    };
    // every pass of the loop issues its loads unconditionally, so the waits before the adds
    // cover the older eight rows only
    int64_t b = b0;
    for (; b + 2 * RU - 1 < b1; b += RU) {
        float w[RU][W];
#pragma unroll
        for (int u = 0; u < RU; ++u) load(b + RU + u, w[u]);
        __builtin_amdgcn_sched_barrier(0);  // the next rows' loads stay ahead of the adds
        add_rows(v);
#pragma unroll
        for (int u = 0; u < RU; ++u)
#pragma unroll
            for (int j = 0; j < W; ++j) v[u][j] = w[u][j];
    }
    add_rows(v);
    b += RU;
    for (; b < b1; ++b) {
        float v[W];
        load(b, v);
#pragma unroll
        for (int j = 0; j < W; ++j) mom_add(m[0][j], v[j], K[j]);
    }
#pragma unroll
    for (int j = 0; j < W; ++j) {
        Mom t = m[0][j];
#pragma unroll
        for (int h = 1; h < CH; ++h) {
            t.s1 = t.s1 + m[h][j].s1;
            t.s2 = t.s2 + m[h][j].s2;
        }
        if (S == 1) res[o + j] = mom_std(t, B);
        else part[s * AC + o + j] = t;
    }
}

// Combines of the split partials, in split order. Rows: one 256-thread block per row, S
// partials contiguous: thread t adds partials t, t + 256, ... (sixteen in flight, so a row of
// up to kMomMaxSplit partials waits on memory once), then the waves' butterflies and the four
// waves in order. Fewer, fuller threads shorten the serial end (butterflies of fp64 values,
// the waves' sums, the division and square root): after the moment pass over [8192, 8192]
// this ended 0.6-1.4 us sooner than 1024 threads with four partials each. Columns: partials at
// stride nlines, a block per 16 lines (below).
constexpr int kMomCombThreads = 256;
constexpr int kMomCombLoads = 16;
static_assert(kMomMaxSplit <= kMomCombLoads * kMomCombThreads, "one round of loads per thread");

__global__ void __launch_bounds__(kMomCombThreads)
    k_tstd_mom_combine_rows(float* __restrict__ res, const Mom* __restrict__ part, int64_t S, int64_t B) {
    __shared__ Mom ws[kMomCombThreads / 64];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const Mom* p = part + (int64_t)blockIdx.x * S;
    Mom m{0.0, 0.0};
    for (int64_t i = t; i < S; i += kMomCombLoads * kMomCombThreads) {  // partials in flight, added in order
        Mom q[kMomCombLoads];
#pragma unroll
        for (int u = 0; u < kMomCombLoads; ++u)
            q[u] = i + u * kMomCombThreads < S ? p[i + u * kMomCombThreads] : Mom{0.0, 0.0};
#pragma unroll
        for (int u = 0; u < kMomCombLoads; ++u) {
            m.s1 = m.s1 + q[u].s1;
            m.s2 = m.s2 + q[u].s2;
        }
    }
    m = mom_wave(m);
    if (lane == 0) ws[w] = m;
    __syncthreads();
    if (t == 0) {
        Mom tot = ws[0];
        for (int k = 1; k < kMomCombThreads / 64; ++k) {
            tot.s1 = tot.s1 + ws[k].s1;
            tot.s2 = tot.s2 + ws[k].s2;
        }
        res[blockIdx.x] = mom_std(tot, B);
    }
}

__global__ void __launch_bounds__(kRThreads)
    k_tstd_mom_combine_cols(float* __restrict__ res, const Mom* __restrict__ part, int64_t nlines, int64_t S,
                            int64_t B) {
    // a block is 16 lines x 16 partial groups; group r adds the partials
    // [r * rpg, min((r + 1) * rpg, S)) in order, eight in flight, then group 0 adds the 16
    // group sums in group order from LDS
    __shared__ Mom lds[16][16];
    const int q = threadIdx.x & 15, r = threadIdx.x >> 4;
    const int64_t l = (int64_t)blockIdx.x * 16 + q;
    const bool active = l < nlines;
    Mom m{0.0, 0.0};
    if (active) {
        const int64_t rpg = (S + 15) / 16;
        const int64_t s0 = r * rpg;
        const int64_t s1 = s0 + rpg < S ? s0 + rpg : S;
        for (int64_t s = s0; s < s1; s += 8) {
            Mom v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s + u < s1) v[u] = part[(s + u) * nlines + l];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (s + u < s1) {
                    m.s1 = m.s1 + v[u].s1;
                    m.s2 = m.s2 + v[u].s2;
                }
        }
    }
    lds[r][q] = m;
    __syncthreads();
    if (r == 0 && active) {
        for (int rr = 1; rr < 16; ++rr) {
            m.s1 = m.s1 + lds[rr][q].s1;
            m.s2 = m.s2 + lds[rr][q].s2;
        }
        res[l] = mom_std(m, B);
    }
}

// ---------------------------------------------------------------------------------------
// launch planning
// ---------------------------------------------------------------------------------------
static inline bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

struct ColSplit {
    int64_t S, rps;
    bool vec;
};
static ColSplit col_split(int64_t A, int64_t B, int64_t C, bool vec) {
    ColSplit cs;
    cs.vec = vec;
    const int64_t items = A * C / (vec ? 4 : 1);
    const int64_t bx = (items + kRThreads - 1) / kRThreads;
    const int64_t target = 8 * (int64_t)ctx().num_cus;  // blocks wanted
    int64_t S = 1;
    if (bx < target) {
        S = (target + bx - 1) / bx;
        int64_t maxS = B / 16;
        if (maxS < 1) maxS = 1;
        if (S > maxS) S = maxS;
        if (S > 65535) S = 65535;
    }
    cs.rps = (B + S - 1) / S;
    if (cs.rps < 1) cs.rps = 1;
    cs.S = (B + cs.rps - 1) / cs.rps;
    if (cs.S < 1) cs.S = 1;
    return cs;
}

// The strip kernel (C % 4 == 0, at least 32 column quads): blocks = A * nstrips * S, with S
// raising the block count to about 8 per CU while each wave keeps >= 8 rows.
static bool use_strip(int64_t C, bool vec) { return vec && C % 4 == 0 && (C >> 2) >= 32; }
static ColSplit strip_split(int64_t A, int64_t B, int64_t C, int64_t* nstrips) {
    ColSplit cs;
    cs.vec = true;
    *nstrips = ((C >> 2) + 63) / 64;
    const int64_t bx = A * *nstrips;
    const int64_t target = 8 * (int64_t)ctx().num_cus;
    int64_t S = 1;
    if (bx < target) {
        S = (target + bx - 1) / bx;
        int64_t maxS = B / 32;
        if (maxS < 1) maxS = 1;
        if (S > maxS) S = maxS;
        if (S > 65535) S = 65535;
    }
    cs.rps = (B + S - 1) / S;
    if (cs.rps < 1) cs.rps = 1;
    cs.S = (B + cs.rps - 1) / cs.rps;
    if (cs.S < 1) cs.S = 1;
    return cs;
}

// Wide strided reductions (C % 4 == 0, at least 256 column quads): one thread per column
// quad (k_cols, 2 rows in flight), about four blocks per CU (64-row splits at [8192, 8192]):
// the best of a sweep of tile shapes on gfx950 (50.4 us against 52 us for 4 rows in flight
// over 128-row splits; 8 rows in flight, whole-row blocks or strips of 64 quads were slower).
static bool use_wide_cols(int64_t C, bool vec) { return vec && C % 4 == 0 && (C >> 2) >= 256; }
static ColSplit wide_split(int64_t A, int64_t B, int64_t C) {
    ColSplit cs;
    cs.vec = true;
    const int64_t bx = (A * (C >> 2) + kRThreads - 1) / kRThreads;
    const int64_t target = 4 * (int64_t)ctx().num_cus;
    int64_t S = (target + bx - 1) / bx;
    int64_t maxS = B / 32;
    if (maxS < 1) maxS = 1;
    if (S > maxS) S = maxS;
    if (S > 65535) S = 65535;
    if (S < 1) S = 1;
    cs.rps = (B + S - 1) / S;
    cs.S = (B + cs.rps - 1) / cs.rps;
    return cs;
}

template <class R>
static constexpr int part_words() {
    return (int)(sizeof(typename R::T) / 4);
}

static inline size_t pad64(size_t v) { return (v + 63) & ~(size_t)63; }

// Rows (C == 1): B <= 64 one thread (or an LDS tile) per row, B < 2048 one wavefront per
// row, longer rows kRowChunk-element block chunks whose partials reduce again the same way.
// A pass over partials (`combine`) takes rows of up to kCombineMax elements in one block
// each (one launch for the combine instead of a chain).
constexpr int64_t kCombineMax = 32768;
static_assert(kCombineMax == 8 * 4 * kCombThreads, "k_row_comb loads eight quads per thread");
static inline bool rows_chunked(int64_t B) { return B >= 2048; }
static inline int64_t row_chunks(int64_t B, bool combine) {
    if (combine && B <= kCombineMax) return 1;
    return (B + kRowChunk - 1) / kRowChunk;
}

// Scratch floats of the row path: every level's partials, one after another.
template <class R>
static size_t row_tmp_floats(int64_t A, int64_t B, bool combine = false) {
    if (!rows_chunked(B)) return 0;
    const int64_t S = row_chunks(B, combine);
    if (S == 1) return 0;
    return pad64((size_t)(A * S) * part_words<R>()) + row_tmp_floats<R>(A, S, true);
}

// Scratch floats a reduction of [A, B, C] needs for its partials.
template <class R>
static size_t tmp_floats_t(int64_t A, int64_t B, int64_t C, bool vec_ok) {
    if (A * C == 0) return 0;
    if (C == 1) return row_tmp_floats<R>(A, B);
    // the largest split any column launcher may pick (the choice depends on alignment)
    int64_t S = 1;
    if (use_wide_cols(C, vec_ok)) {
        ColSplit cw = wide_split(A, B, C);
        S = cw.S > S ? cw.S : S;
    }
    if (use_strip(C, vec_ok)) {
        int64_t ns;
        ColSplit cs = strip_split(A, B, C, &ns);
        S = cs.S > S ? cs.S : S;
    }
    ColSplit c4 = col_split(A, B, C, vec_ok && C % 4 == 0), c1 = col_split(A, B, C, false);
    S = c4.S > S ? c4.S : S;
    S = c1.S > S ? c1.S : S;
    return S > 1 ? (size_t)(S * A * C) * part_words<R>() : 0;
}

size_t reduce_abc_tmp_floats(int op, int64_t A, int64_t B, int64_t C) {
    if (op == RED_MAXCNT) return tmp_floats_t<RMaxCnt>(A, B, C, true);
    if (op == RED_MAXCNT_ARG) return tmp_floats_t<RMaxCntArg>(A, B, C, true);
    return tmp_floats_t<RSum>(A, B, C, true);
}

template <class R>
struct PartLoader {
    using type = LdPlain<R>;
    static type make(float* p, int64_t) { return type{p}; }
};
template <>
struct PartLoader<RMaxCnt> {
    using type = LdPairs;
    static type make(float* p, int64_t n) { return LdPairs{p, reinterpret_cast<const uint32_t*>(p + n)}; }
};
template <>
struct PartLoader<RMaxCntArg> {
    using type = LdPairsArg;
    static type make(float* p, int64_t n) { return LdPairsArg{p, reinterpret_cast<const uint32_t*>(p + n)}; }
};

// nosplit: the combine stage over column-split partials runs as a single pass (tmp unused).
template <class R, class LD>
static int reduce_t(LD ld, bool vec_ok, int epi, int64_t A, int64_t B, int64_t C, float* out,
                    float* out2, float div, float* tmp, bool nosplit = false, bool combine = false,
                    RedSplit* split = nullptr) {
    if (A * C == 0) return MH_OK;
    hipStream_t st = ctx().stream;
    if (C > 1 && B <= 64 && (epi == EPI_SEQ_ACCUM || epi == EPI_SEQ_ACCUM_NEG) && A * C < kMaxGridRows) {
        const unsigned blocks = (unsigned)((A * C + kRThreads - 1) / kRThreads);
        hipLaunchKernelGGL((k_cols_seq<R, LD>), dim3(blocks), dim3(kRThreads), 0, st, ld, A, B, C, out, out2, epi,
                           div);
        return MH_OK;
    }
    if (!(C == 1 && B <= 64)) {  // serial accumulation only where one thread sums a line
        if (epi == EPI_SEQ_ACCUM) epi = EPI_ACCUM;
        else if (epi == EPI_SEQ_ACCUM_NEG) epi = EPI_ACCUM_NEG;
    }
    if (C == 1) {
        if (B <= 64) {
            if constexpr (std::is_same<LD, LdPlain<R>>::value) {
                if (B <= 32 && vec_ok && A < kMaxGridRows) {
                    const unsigned blocks = (unsigned)((A + kLdsRows - 1) / kLdsRows);
                    if (B <= 16)
                        hipLaunchKernelGGL((k_rows_lds<R, 16>), dim3(blocks), dim3(kLdsRows), 0, st, ld.x, A,
                                           (int)B, out, out2, epi, div);
                    else
                        hipLaunchKernelGGL((k_rows_lds<R, 32>), dim3(blocks), dim3(kLdsRows), 0, st, ld.x, A,
                                           (int)B, out, out2, epi, div);
                    return MH_OK;
                }
            }
            constexpr int kMaxLds = sizeof(typename R::T) == 4 ? 64 : 32;  // tile of at most 64 KB
            if (B <= kMaxLds && A < kMaxGridRows) {  // any loader: LDS-staged, element order
                const unsigned blocks = (unsigned)((A + kLdsRows - 1) / kLdsRows);
                if (B <= 16)
                    hipLaunchKernelGGL((k_rows_lds_ld<R, LD, 16>), dim3(blocks), dim3(kLdsRows), 0, st, ld, A,
                                       (int)B, out, out2, epi, div);
                else if (B <= 32)
                    hipLaunchKernelGGL((k_rows_lds_ld<R, LD, 32>), dim3(blocks), dim3(kLdsRows), 0, st, ld, A,
                                       (int)B, out, out2, epi, div);
                else if constexpr (kMaxLds == 64)
                    hipLaunchKernelGGL((k_rows_lds_ld<R, LD, 64>), dim3(blocks), dim3(kLdsRows), 0, st, ld, A,
                                       (int)B, out, out2, epi, div);
                return MH_OK;
            }
            int64_t blocks = (A + kRThreads - 1) / kRThreads;
            if (blocks > 65536) blocks = 65536;
            hipLaunchKernelGGL((k_rows_thread<R, LD>), dim3((unsigned)blocks), dim3(kRThreads), 0, st, ld, A,
                               B, out, out2, epi, div);
            return MH_OK;
        }
        const bool vec = vec_ok && B % 4 == 0;
        if (!rows_chunked(B)) {  // one wavefront per row
            dim3 g((unsigned)((A + 3) / 4)), b(kRThreads);
            if (vec) hipLaunchKernelGGL((k_rows_wave<R, LD, true>), g, b, 0, st, ld, A, (int64_t)1, B, B, out, out2, epi, div, tmp);
            else hipLaunchKernelGGL((k_rows_wave<R, LD, false>), g, b, 0, st, ld, A, (int64_t)1, B, B, out, out2, epi, div, tmp);
            return MH_OK;
        }
        const int64_t S = row_chunks(B, combine);
        if (combine && S == 1 && A <= 0x7fffffff) {  // one block per row (k_row_comb)
            dim3 g((unsigned)A), b(kCombThreads);
            if (vec) hipLaunchKernelGGL((k_row_comb<R, LD, true>), g, b, 0, st, ld, B, out, out2, epi, div);
            else hipLaunchKernelGGL((k_row_comb<R, LD, false>), g, b, 0, st, ld, B, out, out2, epi, div);
            return MH_OK;
        }
        const int64_t L = S == 1 ? B : kRowChunk;
        const int64_t nv = A * S;
        if (split && S > 1) *split = RedSplit{S, L};
        dim3 g((unsigned)nv), b(kRThreads);
        if (vec) hipLaunchKernelGGL((k_rows_block<R, LD, true>), g, b, 0, st, ld, S, B, L, out, out2, epi, div, tmp, nv);
        else hipLaunchKernelGGL((k_rows_block<R, LD, false>), g, b, 0, st, ld, S, B, L, out, out2, epi, div, tmp, nv);
        if (S > 1) {  // the chunk partials [A, S] reduce again along their rows
            using PL = PartLoader<R>;
            return reduce_t<R, typename PL::type>(PL::make(tmp, nv), true, epi, A, S, 1, out, out2, div,
                                                  tmp + pad64((size_t)nv * part_words<R>()), false, true);
        }
        return MH_OK;
    }
    // the wide layout puts the column-quad blocks on grid y (at most 65535 blocks there);
    // larger outputs take the k_cols launch below (quad blocks on x, splits on y)
    if (!nosplit && use_wide_cols(C, vec_ok) && (A * C / 4 + kRThreads - 1) / kRThreads <= 65535) {
        ColSplit cs = wide_split(A, B, C);
        const int64_t items = A * C / 4;
        if (split && cs.S > 1) *split = RedSplit{cs.S, cs.rps};
        dim3 g((unsigned)cs.S, (unsigned)((items + kRThreads - 1) / kRThreads)), b(kRThreads);
        hipLaunchKernelGGL((k_cols<R, LD, true, true>), g, b, 0, st, ld, A, B, C, cs.rps, cs.S, out, out2, epi, div,
                           tmp);
        if (cs.S > 1) {  // combine the split partials in one launch (k_parts_comb)
            using PL = PartLoader<R>;
            const int64_t n = A * C, np = cs.S * n;
            const unsigned cb = (unsigned)((n / 4 + kPcQuads - 1) / kPcQuads);
            hipLaunchKernelGGL((k_parts_comb<R, typename PL::type>), dim3(cb), dim3(kRThreads), 0, st,
                               PL::make(tmp, np), cs.S, n, (cs.S + kPcGroups - 1) / kPcGroups, out, out2, epi, div);
        }
        return MH_OK;
    }
    if (use_strip(C, vec_ok)) {
        int64_t ns;
        ColSplit cs = strip_split(A, B, C, &ns);
        if (nosplit) {
            cs.S = 1;
            cs.rps = B;
        }
        if (split && cs.S > 1) *split = RedSplit{cs.S, cs.rps};
        dim3 g((unsigned)(A * ns), (unsigned)cs.S), b(kRThreads);
        hipLaunchKernelGGL((k_cols_strip<R, LD>), g, b, 0, st, ld, A, B, C, ns, cs.rps, cs.S, out, out2, epi, div, tmp);
        if (cs.S > 1) {
            using PL = PartLoader<R>;
            const int64_t np = cs.S * A * C;
            return reduce_t<R, typename PL::type>(PL::make(tmp, np), true, epi, 1, cs.S, A * C, out, out2, div,
                                                  nullptr, true);
        }
        return MH_OK;
    }
    ColSplit cs = col_split(A, B, C, vec_ok && C % 4 == 0);
    if (nosplit) {
        cs.S = 1;
        cs.rps = B;
    }
    const int64_t items = A * C / (cs.vec ? 4 : 1);
    if (split && cs.S > 1) *split = RedSplit{cs.S, cs.rps};
    dim3 g((unsigned)((items + kRThreads - 1) / kRThreads), (unsigned)cs.S), b(kRThreads);
    if (cs.vec) hipLaunchKernelGGL((k_cols<R, LD, true>), g, b, 0, st, ld, A, B, C, cs.rps, cs.S, out, out2, epi, div, tmp);
    else hipLaunchKernelGGL((k_cols<R, LD, false>), g, b, 0, st, ld, A, B, C, cs.rps, cs.S, out, out2, epi, div, tmp);
    if (cs.S > 1) {
        using PL = PartLoader<R>;
        const int64_t np = cs.S * A * C;
        return reduce_t<R, typename PL::type>(PL::make(tmp, np), sizeof(typename R::T) == 4, epi, 1, cs.S,
                                              A * C, out, out2, div, nullptr, true);
    }
    return MH_OK;
}

int reduce_abc(int op, int epi, const float* x, int64_t A, int64_t B, int64_t C, float* out, float* out2,
               float div, float* tmp, RedSplit* split) {
    const bool al = al16(x);
    switch (op) {
        case RED_SUM:
            return reduce_t<RSum, LdPlain<RSum>>(LdPlain<RSum>{x}, al, epi, A, B, C, out, out2, div, tmp, false,
                                                 false, split);
        case RED_MAX:
            return reduce_t<RMax, LdPlain<RMax>>(LdPlain<RMax>{x}, al, epi, A, B, C, out, out2, div, tmp, false,
                                                 false, split);
        case RED_MAXCNT_ARG:
            return reduce_t<RMaxCntArg, LdArg>(LdArg{x}, al, epi, A, B, C, out, out2, div, tmp, false, false, split);
        default:
            return reduce_t<RMaxCnt, LdPlain<RMaxCnt>>(LdPlain<RMaxCnt>{x}, al, epi, A, B, C, out, out2, div, tmp,
                                                       false, false, split);
    }
}

// ---------------------------------------------------------------------------------------
// un-broadcast chain: accumulate_grad with grad broadcast to rg (tensorutils.mojo:473-487)
// ---------------------------------------------------------------------------------------
int plan_unbroadcast(const mh_shape& sgrad, const mh_shape& srg, mh_reduce_plan_info* info) {
    if (!broadcasts_to(sgrad, srg))
        return fail(MH_ERR_SHAPE, "grad shape does not broadcast to the gradient's shape");
    int64_t gst[MH_MAX_RANK];
    broadcast_strides(srg.rank, sgrad, gst);
    // groups of adjacent non-unit dims with the same class (reduced: grad stride 0)
    int64_t size[MH_MAX_RANK];
    bool red[MH_MAX_RANK];
    int ng = 0;
    for (int d = 0; d < srg.rank; ++d) {
        if (srg.dims[d] == 1) continue;
        const bool r = gst[d] == 0;
        if (ng > 0 && red[ng - 1] == r) {
            size[ng - 1] *= srg.dims[d];
        } else {
            size[ng] = srg.dims[d];
            red[ng] = r;
            ++ng;
        }
    }
    memset(info, 0, sizeof *info);
    int steps = 0;
    for (;;) {
        int j = -1;
        for (int g = ng - 1; g >= 0; --g)
            if (red[g]) {
                j = g;
                break;
            }
        if (j < 0) break;
        int64_t A = 1, C = 1;
        for (int g = 0; g < j; ++g) A *= size[g];
        for (int g = j + 1; g < ng; ++g) C *= size[g];
        info->a[steps] = A;
        info->b[steps] = size[j];
        info->c[steps] = C;
        ++steps;
        // remove group j; merge the kept neighbours that become adjacent
        for (int g = j; g + 1 < ng; ++g) {
            size[g] = size[g + 1];
            red[g] = red[g + 1];
        }
        --ng;
        if (j > 0 && j < ng && !red[j - 1] && !red[j]) {
            size[j - 1] *= size[j];
            for (int g = j; g + 1 < ng; ++g) {
                size[g] = size[g + 1];
                red[g] = red[g + 1];
            }
            --ng;
        }
    }
    info->nsteps = steps;
    return MH_OK;
}

// ---------------------------------------------------------------------------------------
// the plane form of an un-broadcast, [N, C, S] -> [C] (a per-channel bias gradient), in one
// launch
// ---------------------------------------------------------------------------------------
// One wavefront per (channel c, group of G planes n = g * G .. g * G + G - 1, chunk k of QC
// quads of each plane): lanes sum their quads of each plane in order, the planes in order
// (two planes' loads in flight together), a butterfly adds the lanes, and the partial goes to
// part[(g * K + k) * C + c] with an agent-scope store. The wave waits for the store, then
// takes a ticket on channel c's counter (one per 128-byte line); the channel's last arrival
// sums its NG * K partials in index order (lane-strided, then a butterfly) and accumulates
// grad[c] (negated for SUB's operand 1), then resets the counter. G is chosen so that each
// counter sees at most about kPlanesArrivals tickets: arrivals on one counter serialize.
constexpr int64_t kPlanesTicketStride = 32;
constexpr int64_t kPlanesArrivals = 64;
constexpr int64_t kPlanesMaxArrivals = 4096;
constexpr int64_t kPlanesMaxQuads = 1024;

template <bool NEG>
__global__ void __launch_bounds__(kRThreads)
    k_unb_planes(float* __restrict__ grad, const float* __restrict__ rg, int64_t N, int64_t C, int64_t Sq,
                 int64_t QC, int64_t K, int64_t G, int64_t nwaves, float* part, uint32_t* tickets) {
    const int lane = threadIdx.x & 63;
    const int64_t v = (int64_t)blockIdx.x * (kRThreads / 64) + (threadIdx.x >> 6);
    if (v >= nwaves) return;  // uniform per wavefront; no barrier follows
    const int64_t c = v % C, gk = v / C;
    const int64_t g = gk / K, k = gk - g * K;
    const int64_t rem = Sq - k * QC;
    const int64_t cnt = rem < QC ? rem : QC;
    const int64_t n0 = g * G, n1 = n0 + G < N ? n0 + G : N;
    // the lane's quads lane + 64 u of a 256-quad step at `base`, added in order
    auto add_step = [&](float a, const vf4 (&q)[4], int64_t base) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (base + lane + 64 * u < cnt) a = (((a + q[u].x) + q[u].y) + q[u].z) + q[u].w;
        return a;
    };
    auto load_step = [&](vf4 (&q)[4], const vf4* r, int64_t base) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (base + lane + 64 * u < cnt) q[u] = __builtin_nontemporal_load(r + base + lane + 64 * u);
    };
    auto add_rest = [&](float a, const vf4* r) {  // the plane's steps after the first
        for (int64_t base = 256; base < cnt; base += 256) {
            vf4 q[4];
            load_step(q, r, base);
            a = add_step(a, q, base);
        }
        return a;
    };
    float acc = 0.0f;
    for (int64_t n = n0; n < n1; n += 2) {  // planes in order; two planes' first steps in flight together
        const bool two = n + 1 < n1;
        const vf4* ra = reinterpret_cast<const vf4*>(rg) + (n * C + c) * Sq + k * QC;
        const vf4* rb = ra + C * Sq;
        vf4 qa[4], qb[4];
        load_step(qa, ra, 0);
        if (two) load_step(qb, rb, 0);
        acc = add_rest(add_step(acc, qa, 0), ra);
        if (two) acc = add_rest(add_step(acc, qb, 0), rb);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
    const int64_t nper = nwaves / C;  // partials per channel: NG * K
    uint32_t ticket = 0;
    if (lane == 0) {
        __hip_atomic_store(&part[gk * C + c], acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        ticket = __hip_atomic_fetch_add(&tickets[c * kPlanesTicketStride], 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    }
    ticket = __shfl(ticket, 0);
    if (ticket != (uint32_t)(nper - 1)) return;
    // acquire on the last arriver only: the partials stored before the other tickets are
    // visible to the loads below
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    // grad[c] is loaded with the partials (one memory round trip for both, not two in a row)
    const float g0 = lane == 0 ? __hip_atomic_load(&grad[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    float s = 0.0f;
    for (int64_t i = lane; i < nper; i += 64)
        s = s + __hip_atomic_load(&part[i * C + c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s = s + __shfl_xor(s, m);
    if (lane == 0) {
        grad[c] = NEG ? g0 + (-s) : g0 + s;
        __hip_atomic_store(&tickets[c * kPlanesTicketStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

struct PlaneForm {
    int64_t N, C, S, Sq, QC, K, G, NG, nwaves;
};

// The plan [N*C, S, 1] then [1, N, C] with S a multiple of 4 and at least 64.
static bool plane_form(const mh_reduce_plan_info& p, PlaneForm* f) {
    if (p.nsteps != 2 || p.c[0] != 1 || p.a[1] != 1 || p.a[0] != p.b[1] * p.c[1]) return false;
    f->N = p.b[1];
    f->C = p.c[1];
    f->S = p.b[0];
    if (f->S % 4 != 0 || f->S < 64 || f->N * f->C < 1) return false;
    f->Sq = f->S / 4;
    f->QC = f->Sq < kPlanesMaxQuads ? f->Sq : kPlanesMaxQuads;
    f->K = (f->Sq + f->QC - 1) / f->QC;
    f->G = (f->N * f->K + kPlanesArrivals - 1) / kPlanesArrivals;  // planes per wave
    if (f->G < 1) f->G = 1;
    f->NG = (f->N + f->G - 1) / f->G;
    f->nwaves = f->NG * f->K * f->C;
    return f->NG * f->K <= kPlanesMaxArrivals && (f->nwaves + 3) / 4 <= 0x7fffffff;
}

size_t unbroadcast_scratch_floats(const mh_shape& sgrad, const mh_shape& srg) {
    mh_reduce_plan_info p;
    if (plan_unbroadcast(sgrad, srg, &p) != MH_OK) return 0;
    size_t tmax = 0, bmax = 0;
    for (int i = 0; i < p.nsteps; ++i) {
        size_t t = reduce_abc_tmp_floats(RED_SUM, p.a[i], p.b[i], p.c[i]);
        if (t > tmax) tmax = t;
        size_t o = (size_t)(p.a[i] * p.c[i]);
        if (o > bmax) bmax = o;
    }
    auto pad = [](size_t v) { return (v + 63) & ~(size_t)63; };
    size_t need = pad(tmax) + 2 * pad(bmax) + 64;
    PlaneForm pf;
    if (plane_form(p, &pf)) {  // the one-launch plane form's partials
        const size_t np = pad((size_t)(pf.NG * pf.K * pf.C)) + 64;
        if (np > need) need = np;
    }
    return need;
}

int unbroadcast_accum_scratch(float* grad, const mh_shape& sgrad, const float* rg, const mh_shape& srg,
                              bool negate, float* tmp) {
    mh_reduce_plan_info p;
    MH_TRY(plan_unbroadcast(sgrad, srg, &p));
    // one reduction step: each gradient element's values are one line of rg, which the
    // thread-per-row kernels add into it in order, as the reference's serial walk does
    const int final_epi = p.nsteps <= 1 ? (negate ? EPI_SEQ_ACCUM_NEG : EPI_SEQ_ACCUM)
                                        : (negate ? EPI_ACCUM_NEG : EPI_ACCUM);
    if (p.nsteps == 0)  // only size-1 dims differ: same element order
        return reduce_abc(RED_SUM, final_epi, rg, numel(srg), 1, 1, grad, nullptr, 0.0f, nullptr);
    PlaneForm pf;
    if (al16(rg) && plane_form(p, &pf)) {  // a per-channel bias gradient: one launch
        uint32_t* tk = nullptr;
        MH_TRY(tickets(pf.C * kPlanesTicketStride, &tk));
        dim3 g((unsigned)((pf.nwaves + 3) / 4)), b(kRThreads);
        if (negate)
            hipLaunchKernelGGL(k_unb_planes<true>, g, b, 0, ctx().stream, grad, rg, pf.N, pf.C, pf.Sq, pf.QC, pf.K,
                               pf.G, pf.nwaves, tmp, tk);
        else
            hipLaunchKernelGGL(k_unb_planes<false>, g, b, 0, ctx().stream, grad, rg, pf.N, pf.C, pf.Sq, pf.QC,
                               pf.K, pf.G, pf.nwaves, tmp, tk);
        return MH_OK;
    }
    size_t tmax = 0, bmax = 0;
    for (int i = 0; i < p.nsteps; ++i) {
        size_t t = reduce_abc_tmp_floats(RED_SUM, p.a[i], p.b[i], p.c[i]);
        if (t > tmax) tmax = t;
        size_t o = (size_t)(p.a[i] * p.c[i]);
        if (o > bmax) bmax = o;
    }
    auto pad = [](size_t v) { return (v + 63) & ~(size_t)63; };
    float* part = tmp;
    float* buf[2] = {tmp + pad(tmax), tmp + pad(tmax) + pad(bmax)};
    const float* src = rg;
    for (int i = 0; i < p.nsteps; ++i) {
        const bool last = i == p.nsteps - 1;
        float* dst = last ? grad : buf[i & 1];
        MH_TRY(reduce_abc(RED_SUM, last ? final_epi : EPI_STORE, src, p.a[i], p.b[i], p.c[i], dst, nullptr,
                          0.0f, part));
        src = dst;
    }
    return MH_OK;
}

// Short rows (C == 1, B <= BMAX) of a broadcast MUL / DIV backward's un-broadcast: the block
// stages ug and the full-shape operand of rows [r0, r0 + 256) in LDS with 16-byte loads (one
// contiguous run each), then thread t adds row r0 + t's terms one at a time into its
// gradient (EPI_SEQ_ACCUM), with DIV's divisor read once per row: the terms and order of the
// generic loader path (k_rows_lds_ld over LdBinRg), so the same bits, without a row lookup
// per element. ug and the operand 16-byte aligned.
template <int OP, int ID, bool DIVS, int BMAX, bool COL1>
__global__ void __launch_bounds__(kLdsRows)
    k_rows_binrg(LdBinRg<OP, ID, DIVS, false, COL1> ld, float* __restrict__ grad, int64_t nrows, int B) {
    constexpr int QPT = BMAX / 4;  // quads per thread per operand: rows * B / 4 <= kLdsRows * QPT
    __shared__ float4 us4[kLdsRows * BMAX / 4], as4[kLdsRows * BMAX / 4];
    float* us = reinterpret_cast<float*>(us4);
    float* as = reinterpret_cast<float*>(as4);
    ld.setup();
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.x * kLdsRows;
    const int64_t rows = (nrows - r0) < kLdsRows ? (nrows - r0) : kLdsRows;
    const int64_t base = r0 * B;
    const int cnt = (int)(rows * B);
    const int nq = cnt >> 2;
    // every load of the block is issued before the barrier (the tile quads into registers,
    // the row's divisor and gradient), so a block waits for memory once
    const bool mine = t < rows;
    const int64_t row = r0 + t;
    const float d = (OP == MH_DIV && ID == 1 && !DIVS && mine) ? ld.t2[row] : 0.0f;
    float acc = mine ? grad[row] : 0.0f;  // EPI_SEQ_ACCUM
    float4 uq[QPT], aq[QPT];
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
        const int i = t + k * kLdsRows;
        if (i < nq) {
            uq[k] = ld_nt4(ld.ug + base, i);
            aq[k] = ld_nt4(ld.a + base, i);
        }
    }
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
        const int i = t + k * kLdsRows;
        if (i < nq) {
            us4[i] = uq[k];
            as4[i] = aq[k];
        }
    }
    for (int i = (nq << 2) + t; i < cnt; i += kLdsRows) {
        us[i] = ld_nt(ld.ug + base + i);
        as[i] = ld_nt(ld.a + base + i);
    }
    __syncthreads();
    if (mine) {
        for (int j = 0; j < B; ++j) acc = acc + ld.term(us[t * B + j], as[t * B + j], d);
        grad[row] = acc;
    }
}

template <int OP, int ID, bool DIVS, bool BIG, bool COL1>
static int binrg_reduce(float* grad, const float* ug, const float* a, const float* t2, int64_t A, int64_t B,
                        int64_t C, bool al, float* tmp) {
    constexpr bool DV = OP == MH_DIV && ID == 1 && !DIVS;
    LdBinRg<OP, ID, DIVS, BIG, COL1> ld{};
    ld.ug = ug;
    ld.a = a;
    ld.t2 = t2;
    ld.BC = B * C;
    ld.C = C;
    if (!BIG) {
        ld.fbc = make_fastdiv((uint32_t)(B * C > 0 ? B * C : 1));
        ld.fc = make_fastdiv((uint32_t)C);
    }
    ld.al = al;
    if constexpr (!BIG && (COL1 || !DV)) {
        if (C == 1 && B <= 32 && al && A < kMaxGridRows) {  // short rows, staged as quads
            const unsigned blocks = (unsigned)((A + kLdsRows - 1) / kLdsRows);
            if (B <= 16)
                hipLaunchKernelGGL((k_rows_binrg<OP, ID, DIVS, 16, COL1>), dim3(blocks), dim3(kLdsRows), 0,
                                   ctx().stream, ld, grad, A, (int)B);
            else
                hipLaunchKernelGGL((k_rows_binrg<OP, ID, DIVS, 32, COL1>), dim3(blocks), dim3(kLdsRows), 0,
                                   ctx().stream, ld, grad, A, (int)B);
            return MH_OK;
        }
    }
    // vec_ok: the loader reads quads at any alignment, so the kernels (and the summation
    // order) are those of a materialised, aligned rg
    return reduce_t<RSum, LdBinRg<OP, ID, DIVS, BIG, COL1>>(ld, true, EPI_SEQ_ACCUM, A, B, C, grad, nullptr, 0.0f,
                                                            tmp);
}

// COL1 only for DIV's operand 1, whose loader reads the divisor (C == 1: one per row)
template <int OP, int ID, bool DIVS, bool BIG>
static int binrg_reduce_c(float* grad, const float* ug, const float* a, const float* t2, int64_t A, int64_t B,
                          int64_t C, bool al, float* tmp) {
    if constexpr (OP == MH_DIV && ID == 1 && !DIVS) {
        if (C == 1) return binrg_reduce<OP, ID, DIVS, BIG, true>(grad, ug, a, t2, A, B, C, al, tmp);
    }
    return binrg_reduce<OP, ID, DIVS, BIG, false>(grad, ug, a, t2, A, B, C, al, tmp);
}

template <int OP, int ID, bool DIVS>
static int binrg_reduce_n(float* grad, const float* ug, const float* a, const float* t2, int64_t A, int64_t B,
                          int64_t C, bool al, float* tmp) {
    if (A * B * C < ((int64_t)1 << 32)) return binrg_reduce_c<OP, ID, DIVS, false>(grad, ug, a, t2, A, B, C, al, tmp);
    return binrg_reduce_c<OP, ID, DIVS, true>(grad, ug, a, t2, A, B, C, al, tmp);
}

int unbroadcast_binrg(int op, int id, bool divs, float* grad, const mh_shape& sgrad, const float* ug,
                      const mh_shape& sug, const float* t1, const mh_shape& s1, const float* t2,
                      const mh_shape& s2, bool* done) {
    *done = false;
    if (op != MH_MUL && op != MH_DIV) return MH_OK;
    // the operand read at every element must have the full shape
    const float* a = id == 0 ? t2 : t1;
    if (!shape_eq(id == 0 ? s2 : s1, sug)) return MH_OK;
    mh_reduce_plan_info p;
    MH_TRY(plan_unbroadcast(sgrad, sug, &p));
    if (p.nsteps > 1) return MH_OK;
    int64_t A = numel(sug), B = 1, C = 1;  // only size-1 dims differ: element for element
    if (p.nsteps == 1) {
        A = p.a[0];
        B = p.b[0];
        C = p.c[0];
    }
    float* tmp = nullptr;
    const size_t t = tmp_floats_t<RSum>(A, B, C, true);
    if (t) MH_TRY(scratch((t + 64) * sizeof(float), reinterpret_cast<void**>(&tmp)));
    const bool al = al16(ug) && al16(a);
    if (op == MH_MUL) {
        if (id == 0) MH_TRY((binrg_reduce_n<MH_MUL, 0, false>(grad, ug, a, t2, A, B, C, al, tmp)));
        else MH_TRY((binrg_reduce_n<MH_MUL, 1, false>(grad, ug, a, t2, A, B, C, al, tmp)));
    } else if (id == 0) {
        MH_TRY((binrg_reduce_n<MH_DIV, 0, false>(grad, ug, a, t2, A, B, C, al, tmp)));
    } else if (divs) {
        MH_TRY((binrg_reduce_n<MH_DIV, 1, true>(grad, ug, a, t2, A, B, C, al, tmp)));
    } else {
        MH_TRY((binrg_reduce_n<MH_DIV, 1, false>(grad, ug, a, t2, A, B, C, al, tmp)));
    }
    *done = true;
    return MH_OK;
}

// The POW backward over whole aligned quads (LdPowGrad's terms, and with gx the x gradient) in
// one-shot one-wavefront blocks, every load issued before the first quad's log and exp work.
// Each run of 64 quads (a quad per lane) adds into one partial the same way whatever the
// launch shape: a lane adds its quad's four terms as ((0 + t0) + (0 + t1)) + ((0 + t2) + (0 + t3)),
// the wave adds its lanes in a fixed order, so the exponent gradient has the same bits with and
// without the x gradient. Blocks take two such runs per thread for the exponent gradient alone
// (over 2^28 elements 374-388 us against 467-473 us at one) and one with the x gradient too
// (three streams; 671-678 us against 715-727 us at two, 0.69-0.71 ms for 256-thread blocks of
// four quads per thread, 0.73-0.75 ms for 256-thread blocks taking loads and work one quad at
// a time).
constexpr int kPowThreads = 64;
constexpr int64_t kPowStreamMinQuads = 1 << 16;
template <bool GX>
constexpr int pow_runs() { return GX ? 1 : 2; }
template <int NQ>
struct PowQuads {
    float4 xs[NQ], us[NQ], gs[NQ];
};

// every quad's loads (a quad past the end reloads the last quad, unused)
template <bool GX, int NQ>
__device__ __forceinline__ void pow_load_quads(const LdPowGrad& ld, int64_t nq, PowQuads<NQ>& t) {
    const int64_t base = (int64_t)blockIdx.x * (kPowThreads * NQ) + threadIdx.x;
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int64_t q = base + k * kPowThreads;
        const int64_t qc = q < nq ? q : nq - 1;
        t.xs[k] = ld_nt4(ld.x, qc);
        t.us[k] = ld_nt4(ld.ug, qc);
        t.gs[k] = GX ? ld_nt4(ld.gx, qc) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

__device__ __forceinline__ float pow_quad_sum(float t0, float t1, float t2, float t3) {
    return ((0.0f + t0) + (0.0f + t1)) + ((0.0f + t2) + (0.0f + t3));
}

// s[k]: the lane's sum over its quad of run k (0 past the end)
template <bool FRAC, bool GX, int NQ>
__device__ __forceinline__ void pow_block_quads(const LdPowGrad& ld, int64_t nq, PowQuads<NQ>& t, float (&s)[NQ]) {
    const int64_t base = (int64_t)blockIdx.x * (kPowThreads * NQ) + threadIdx.x;
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const int64_t q = base + k * kPowThreads;
        s[k] = 0.0f;
        if (q < nq) {
            const float4 &xq = t.xs[k], &uq = t.us[k], &g0 = t.gs[k];
            float4 g = g0;
            float r0, r1, r2, r3;
            if constexpr (FRAC) {
                // the quad's common case straight through, one wave-wide test, then elem for
                // the lanes' elements that left it
                bool o0, o1, o2, o3;
                r0 = ld.elem_frac_fast<GX>(xq.x, uq.x, g.x, o0);
                r1 = ld.elem_frac_fast<GX>(xq.y, uq.y, g.y, o1);
                r2 = ld.elem_frac_fast<GX>(xq.z, uq.z, g.z, o2);
                r3 = ld.elem_frac_fast<GX>(xq.w, uq.w, g.w, o3);
                if (__builtin_expect(!(o0 && o1 && o2 && o3), 0)) {
                    if (!o0) { g.x = g0.x; r0 = ld.elem<true, GX>(xq.x, uq.x, g.x); }
                    if (!o1) { g.y = g0.y; r1 = ld.elem<true, GX>(xq.y, uq.y, g.y); }
                    if (!o2) { g.z = g0.z; r2 = ld.elem<true, GX>(xq.z, uq.z, g.z); }
                    if (!o3) { g.w = g0.w; r3 = ld.elem<true, GX>(xq.w, uq.w, g.w); }
                }
            } else {
                r0 = ld.elem<false, GX>(xq.x, uq.x, g.x);
                r1 = ld.elem<false, GX>(xq.y, uq.y, g.y);
                r2 = ld.elem<false, GX>(xq.z, uq.z, g.z);
                r3 = ld.elem<false, GX>(xq.w, uq.w, g.w);
            }
            s[k] = pow_quad_sum(r0, r1, r2, r3);
            if constexpr (GX) st_nt4(ld.gx, q, g);
        }
    }
}

// The quads' loads go out before the exponent is read (setup): read first, every wave waited
// for that scalar load before its quads' loads issued. part[r] is run r's sum, r < nruns.
template <bool GX>
__global__ void __launch_bounds__(kPowThreads) k_pow_grad_quads(LdPowGrad ld, int64_t nq, int64_t nruns,
                                                                float* part) {
    constexpr int NQ = pow_runs<GX>();
    PowQuads<NQ> t;
    pow_load_quads<GX, NQ>(ld, nq, t);
    __builtin_amdgcn_sched_barrier(0);
    ld.setup();
    float s[NQ];
    if (ld.frac) pow_block_quads<true, GX, NQ>(ld, nq, t, s);
    else pow_block_quads<false, GX, NQ>(ld, nq, t, s);
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
        const float a = wave_reduce<RSum>(s[k]);
        const int64_t r = (int64_t)blockIdx.x * NQ + k;
        if (threadIdx.x == 0 && r < nruns) part[r] = a;
    }
}

int pow_exponent_grad(float* grad, const float* x, const float* exponent, const float* ug, int64_t n,
                      float* grad_x) {
    LdPowGrad ld{x, ug, exponent, 0.0f, grad_x, 0.0f, false};
    const bool vec = al16(x) && al16(ug) && (!grad_x || al16(grad_x));
    float* tmp = nullptr;
    if (vec && n % 4 == 0 && n / 4 >= kPowStreamMinQuads && n / 4 / kPowThreads < 0x7fffffff) {
        // run partials, then a row reduction of them into grad
        const int64_t nq = n / 4;
        const int64_t G = (nq + kPowThreads - 1) / kPowThreads;  // runs of 64 quads
        const size_t t = pad64((size_t)G) + tmp_floats_t<RSum>(1, G, 1, true);
        MH_TRY(scratch((t + 64) * sizeof(float), reinterpret_cast<void**>(&tmp)));
        if (grad_x) {
            constexpr int NQ = pow_runs<true>();
            hipLaunchKernelGGL(k_pow_grad_quads<true>, dim3((unsigned)((G + NQ - 1) / NQ)), dim3(kPowThreads), 0,
                               ctx().stream, ld, nq, G, tmp);
        } else {
            constexpr int NQ = pow_runs<false>();
            hipLaunchKernelGGL(k_pow_grad_quads<false>, dim3((unsigned)((G + NQ - 1) / NQ)), dim3(kPowThreads), 0,
                               ctx().stream, ld, nq, G, tmp);
        }
        return reduce_t<RSum, LdPlain<RSum>>(LdPlain<RSum>{tmp}, true, EPI_ACCUM, 1, G, 1, grad, nullptr, 0.0f,
                                             tmp + pad64((size_t)G), false, true);
    }
    const size_t t = tmp_floats_t<RSum>(1, n, 1, true);
    MH_TRY(scratch((t + 64) * sizeof(float), reinterpret_cast<void**>(&tmp)));
    return reduce_t<RSum, LdPowGrad>(ld, vec, EPI_ACCUM, 1, n, 1, grad, nullptr, 0.0f, tmp);
}

// elementwise helpers (mh_elementwise.hip)
int map_max_route(float* grad, const mh_shape& sx, const float* x, const mh_shape& sline, const float* m,
                  const float* f, const float* ug);
int map_scale_bcast(float* grad, const mh_shape& sx, const float* ug, const mh_shape& sug, float c, bool twice);
int map_mean_all(float* grad, int64_t n, const float* ug, float c);

static void abc_of(const mh_shape& s, int axis, int64_t* A, int64_t* B, int64_t* C) {
    if (axis < 0) {
        *A = 1;
        *B = numel(s);
        *C = 1;
        return;
    }
    int64_t a = 1, c = 1;
    for (int i = 0; i < axis; ++i) a *= s.dims[i];
    for (int i = axis + 1; i < s.rank; ++i) c *= s.dims[i];
    *A = a;
    *B = s.dims[axis];
    *C = c;
}

static int check_reduce_args(int op, const mh_shape& sx, int32_t axis) {
    if (op != MH_SUM && op != MH_MEAN && op != MH_MAX) return fail(MH_ERR_OP, "op %d is not SUM/MEAN/MAX", op);
    MH_TRY(check_shape(sx, "x"));
    if (axis < -1 || axis >= sx.rank) return fail(MH_ERR_INVALID, "axis %d outside [-1, %d)", axis, sx.rank);
    return MH_OK;
}

}  // namespace mh

using namespace mh;

extern "C" {

int mh_reduce_fwd(int op, float* res, const float* x, const mh_shape* psx, int32_t axis) {
    MH_TRACE_OP("mh_reduce_fwd", op);
    MH_SHAPE_ARG(sx);
    MH_TRY(check_reduce_args(op, sx, axis));
    int64_t A, B, C;
    abc_of(sx, axis, &A, &B, &C);
    if (A * C == 0) return MH_OK;
    if (!res || (!x && B > 0)) return fail(MH_ERR_NULL, "mh_reduce_fwd: null tensor");
    MH_TRY(require_init());
    const int epi = op == MH_MEAN ? EPI_MEAN : EPI_STORE;
    const float div = op == MH_MEAN ? (float)B : 0.0f;  // tmean: / Scalar[f32](count)
    const int rop = op == MH_MAX ? RED_MAX : RED_SUM;
    float* tmp = nullptr;
    const size_t t = reduce_abc_tmp_floats(rop, A, B, C);
    if (t) MH_TRY(scratch(t * sizeof(float), reinterpret_cast<void**>(&tmp)));
    MH_TRY(reduce_abc(rop, epi, x, A, B, C, res, nullptr, div, tmp));
    return finish("mh_reduce_fwd");
}

int mh_reduce_fwd_noalloc(int op, float* res, const float* x, const mh_shape* psx, int32_t axis) {
    MH_TRACE_OP("mh_reduce_fwd_noalloc", op);
    MH_SHAPE_ARG(sx);
    MH_TRY(check_reduce_args(op, sx, axis));
    int64_t A, B, C;
    abc_of(sx, axis, &A, &B, &C);
    if (A * C == 0) return MH_OK;
    const int rop = op == MH_MAX ? RED_MAX : RED_SUM;
    // the largest partial buffer any launcher for [A, B, C] may use, checked before anything else
    const size_t t = reduce_abc_tmp_floats(rop, A, B, C);
    if (t * sizeof(float) > kNoAllocScratchBytes)
        return fail(MH_ERR_OVERFLOW, "mh_reduce_fwd_noalloc: [%lld, %lld, %lld] needs %zu bytes of partials, more "
                    "than the %zu of the no-allocation scratch (use mh_reduce_fwd)", (long long)A, (long long)B,
                    (long long)C, t * sizeof(float), kNoAllocScratchBytes);
    if (!res || (!x && B > 0)) return fail(MH_ERR_NULL, "mh_reduce_fwd_noalloc: null tensor");
    MH_TRY(require_init());
    float* tmp = nullptr;
    if (t) MH_TRY(noalloc_scratch(t * sizeof(float), &tmp));  // partials are written before they are read
    const int epi = op == MH_MEAN ? EPI_MEAN : EPI_STORE;
    const float div = op == MH_MEAN ? (float)B : 0.0f;
    MH_TRY(reduce_abc(rop, epi, x, A, B, C, res, nullptr, div, tmp));
    return finish("mh_reduce_fwd_noalloc");
}

int mh_tstd(float* res, const float* x, const mh_shape* psx, int32_t axis) {
    MH_TRACE("mh_tstd");
    MH_SHAPE_ARG(sx);
    MH_TRY(check_shape(sx, "x"));
    if (axis < -1 || axis >= sx.rank) return fail(MH_ERR_INVALID, "mh_tstd: axis %d outside [-1, %d)", axis, sx.rank);
    int64_t A, B, C;
    abc_of(sx, axis, &A, &B, &C);
    if (A * C == 0) return MH_OK;
    if (!res || (!x && B > 0)) return fail(MH_ERR_NULL, "mh_tstd: null tensor");
    MH_TRY(require_init());
    if (C == 1 && B >= 4 && B % 4 == 0 && B <= 16384 && al16(x) && A < ((int64_t)1 << 31)) {
        // rows held in registers: one pass over x
        const int64_t Bq = B / 4;
        hipStream_t st = ctx().stream;
        if (Bq <= 64 * 16) {  // one wave per row, four rows per block
            const int nq = Bq <= 64 ? 1 : Bq <= 128 ? 2 : Bq <= 256 ? 4 : Bq <= 512 ? 8 : 16;
            dim3 g((unsigned)((A + 3) / 4)), b(kRThreads);
#define MH_TSR(NQ) hipLaunchKernelGGL((k_tstd_rowreg<1, NQ>), g, b, 0, st, res, x, A, B)
            switch (nq) {
                case 1: MH_TSR(1); break;
                case 2: MH_TSR(2); break;
                case 4: MH_TSR(4); break;
                case 8: MH_TSR(8); break;
                default: MH_TSR(16); break;
            }
#undef MH_TSR
        } else {  // one block per row
            const int nq = Bq <= 2048 ? 8 : 16;
            dim3 g((unsigned)A), b(kRThreads);
#define MH_TSR(NQ) hipLaunchKernelGGL((k_tstd_rowreg<4, NQ>), g, b, 0, st, res, x, A, B)
            if (nq == 8) MH_TSR(8);
            else MH_TSR(16);
#undef MH_TSR
        }
        return finish("mh_tstd");
    }
    if (B == 0) return mh_fill(res, __builtin_nanf(""), A * C);  // the reference divides 0 by 0
    hipStream_t st = ctx().stream;
    if (C == 1) {  // rows (all elements: one row): block chunks of kRowChunk elements or more,
                   // at most kMomMaxSplit per row so that the combine stays short
        int64_t L = kRowChunk;
        if ((B + L - 1) / L > kMomMaxSplit) L = ((B + kMomMaxSplit - 1) / kMomMaxSplit + 3) & ~(int64_t)3;
        const int64_t S = (B + L - 1) / L;
        if (S == 1) L = B;
        Mom* part = nullptr;
        if (S > 1) MH_TRY(scratch((size_t)(A * S) * sizeof(Mom), reinterpret_cast<void**>(&part)));
        const bool vec = al16(x) && B % 4 == 0;
        dim3 g((unsigned)(A * S)), b(kRThreads);
        if (vec) hipLaunchKernelGGL(k_tstd_mom_rows<true>, g, b, 0, st, res, x, B, L, S, part);
        else hipLaunchKernelGGL(k_tstd_mom_rows<false>, g, b, 0, st, res, x, B, L, S, part);
        if (S > 1)
            hipLaunchKernelGGL(k_tstd_mom_combine_rows, dim3((unsigned)A), dim3(kMomCombThreads), 0, st, res, part, S, B);
        return finish("mh_tstd");
    }
    // strided axis: a thread per column quad, about one block per CU, row splits of at least 64
    // rows, eight rows in flight over four accumulator chains. Fewer, longer splits write and
    // combine fewer fp64 partials: at [8192, 8192] axis 0 (a probe, moments + combine) 32 splits
    // took 48.1 us against 52.6 us with 64 splits of four rows in flight, one chain; 128 and
    // 256 splits took 57-60 us. In the bench (moments + combine, streamed) the splits on grid x
    // took 47.2 us against 48.9 us on y; 16 rows in flight 49.4 us, two blocks per CU 59.4 us.
    // With S > 1 there are fewer column blocks than CUs, well inside grid y's limit.
    const bool vec = al16(x) && C % 4 == 0;
    const int64_t W = vec ? 4 : 1;
    const int64_t items = A * C / W;
    const int64_t bx = (items + kRThreads - 1) / kRThreads;
    int64_t S = ((int64_t)ctx().num_cus + bx - 1) / bx;
    int64_t maxS = B / 64;
    if (maxS < 1) maxS = 1;
    if (S > maxS) S = maxS;
    if (S > 65535) S = 65535;
    if (S < 1) S = 1;
    const int64_t rps = (B + S - 1) / S;
    S = (B + rps - 1) / rps;
    Mom* part = nullptr;
    if (S > 1) MH_TRY(scratch((size_t)(S * A * C) * sizeof(Mom), reinterpret_cast<void**>(&part)));
    const dim3 b(kRThreads);
    if (S > 1) {
        const dim3 g((unsigned)S, (unsigned)bx);
        if (vec) hipLaunchKernelGGL((k_tstd_mom_cols<true, true>), g, b, 0, st, res, x, A, B, C, rps, S, part);
        else hipLaunchKernelGGL((k_tstd_mom_cols<false, true>), g, b, 0, st, res, x, A, B, C, rps, S, part);
    } else {
        const dim3 g((unsigned)bx);
        if (vec) hipLaunchKernelGGL((k_tstd_mom_cols<true, false>), g, b, 0, st, res, x, A, B, C, rps, S, part);
        else hipLaunchKernelGGL((k_tstd_mom_cols<false, false>), g, b, 0, st, res, x, A, B, C, rps, S, part);
    }
    if (S > 1)
        hipLaunchKernelGGL(k_tstd_mom_combine_cols, dim3((unsigned)((A * C + 15) / 16)), b, 0, st,
                           res, part, A * C, S, B);
    return finish("mh_tstd");
}

}  // extern "C"

// The routing pass of a MAX backward whose reduction left split partials (k_max_route_*;
// arg: RED_MAXCNT_ARG partials, which the column route needs): false where their layout does
// not fit those kernels (the caller routes every element).
static bool max_route_split(float* grad, const float* x, int64_t A, int64_t B, int64_t C, const float* m,
                            const float* f, const float* ug, float* tmp, const RedSplit& sp, bool arg) {
    if (sp.S <= 1 || !al16(x) || !al16(grad)) return false;
    hipStream_t st = ctx().stream;
    if (C == 1) {
        const int64_t nv = A * sp.S;
        if (arg || B % 4 != 0 || sp.span != kRowChunk || nv > 0x7fffffff) return false;
        hipLaunchKernelGGL(k_max_route_rows, dim3((unsigned)nv), dim3(kRThreads), 0, st, grad, x, m, f, ug, tmp,
                           sp.S, B);
        return true;
    }
    if (!arg || C % 4 != 0 || sp.S > 65535) return false;
    const int64_t np = sp.S * A * C;
    const uint32_t* pc = reinterpret_cast<const uint32_t*>(tmp + np);
    const uint32_t* pi = reinterpret_cast<const uint32_t*>(tmp + 2 * np);
    const int64_t qb = (A * C / 4 + kRThreads - 1) / kRThreads;
    const bool sx = qb <= 65535;
    if (!sx && qb > 0x7fffffff) return false;
    const dim3 g = sx ? dim3((unsigned)sp.S, (unsigned)qb) : dim3((unsigned)qb, (unsigned)sp.S), b(kRThreads);
    if (sx)
        hipLaunchKernelGGL(k_max_route_cols<true>, g, b, 0, st, grad, x, m, f, ug, tmp, pc, pi, A, B, C, sp.span);
    else
        hipLaunchKernelGGL(k_max_route_cols<false>, g, b, 0, st, grad, x, m, f, ug, tmp, pc, pi, A, B, C, sp.span);
    return true;
}

extern "C" {

int mh_reduce_bwd_accum(int op, float* grad, const float* x, const mh_shape* psx, const float* ug,
                        int32_t axis) {
    MH_TRACE_OP("mh_reduce_bwd_accum", op);
    MH_SHAPE_ARG(sx);
    MH_TRY(check_reduce_args(op, sx, axis));
    const int64_t n = numel(sx);
    if (n == 0) return MH_OK;
    if (!grad || !ug || (op == MH_MAX && !x)) return fail(MH_ERR_NULL, "mh_reduce_bwd_accum: null tensor");
    MH_TRY(require_init());
    const mh_shape sug = reduced_shape(sx, axis);
    int64_t A, B, C;
    abc_of(sx, axis, &A, &B, &C);
    if (op == MH_SUM) {  // basics.mojo:416-425
        MH_TRY(map_scale_bcast(grad, sx, ug, sug, 1.0f, shape_eq(sx, sug)));
    } else if (op == MH_MEAN) {
        if (axis < 0) {  // basics.mojo:470-487
            MH_TRY(map_mean_all(grad, n, ug, (float)(1.0 / (double)n)));
        } else {  // basics.mojo:489-506
            MH_TRY(map_scale_bcast(grad, sx, ug, sug, (float)(1.0 / (double)B), shape_eq(sx, sug)));
        }
    } else if (C == 1 && B >= 1 && B <= 32 && A < kMaxGridRows && al16(x) && al16(grad)) {
        // MAX over short last-axis rows: one pass (max, count and routing per LDS tile)
        const unsigned blocks = (unsigned)((A + kLdsRows - 1) / kLdsRows);
        const FastDiv fdB = make_fastdiv((uint32_t)B);
        if (B <= 16)
            hipLaunchKernelGGL(k_max_bwd_rows<16>, dim3(blocks), dim3(kLdsRows), 0, ctx().stream, grad, x, ug, A,
                               (int)B, fdB);
        else
            hipLaunchKernelGGL(k_max_bwd_rows<32>, dim3(blocks), dim3(kLdsRows), 0, ctx().stream, grad, x, ug, A,
                               (int)B, fdB);
    } else if (C == 1 && B % 4 == 0 && B <= 16384 && al16(x) && al16(grad) && A < ((int64_t)1 << 31)) {
        // MAX over rows held in registers: one pass
        const int64_t Bq = B / 4;
        hipStream_t st = ctx().stream;
        if (Bq <= 64 * 16) {  // one wave per row, four rows per block
            const int nq = Bq <= 64 ? 1 : Bq <= 128 ? 2 : Bq <= 256 ? 4 : Bq <= 512 ? 8 : 16;
            dim3 g((unsigned)((A + 3) / 4)), b(kRThreads);
#define MH_MBR(NQ) hipLaunchKernelGGL((k_max_bwd_rowreg<1, NQ>), g, b, 0, st, grad, x, ug, A, B)
            switch (nq) {
                case 1: MH_MBR(1); break;
                case 2: MH_MBR(2); break;
                case 4: MH_MBR(4); break;
                case 8: MH_MBR(8); break;
                default: MH_MBR(16); break;
            }
#undef MH_MBR
        } else {  // one block per row
            const int nq = Bq <= 512 ? 2 : Bq <= 1024 ? 4 : Bq <= 2048 ? 8 : 16;
            dim3 g((unsigned)A), b(kRThreads);
#define MH_MBR(NQ) hipLaunchKernelGGL((k_max_bwd_rowreg<4, NQ>), g, b, 0, st, grad, x, ug, A, B)
            switch (nq) {
                case 2: MH_MBR(2); break;
                case 4: MH_MBR(4); break;
                case 8: MH_MBR(8); break;
                default: MH_MBR(16); break;
            }
#undef MH_MBR
        }
    } else {  // MAX, basics.mojo:536-615: line max and fl(1/count), then routing
        const int64_t nl = A * C;
        const size_t pad_nl = ((size_t)nl + 63) & ~(size_t)63;
        // columns: the split partials keep each split's index of its maximum (n < 2^32)
        const bool arg = C > 1 && n < ((int64_t)1 << 32);
        const int rop = arg ? RED_MAXCNT_ARG : RED_MAXCNT;
        const size_t t = reduce_abc_tmp_floats(rop, A, B, C);
        float* base = nullptr;
        MH_TRY(scratch((2 * pad_nl + t + 64) * sizeof(float), reinterpret_cast<void**>(&base)));
        float* m = base;
        float* f = base + pad_nl;
        float* tmp = base + 2 * pad_nl;
        RedSplit sp;
        MH_TRY(reduce_abc(rop, EPI_STORE, x, A, B, C, m, f, 0.0f, tmp, &sp));
        if (!max_route_split(grad, x, A, B, C, m, f, ug, tmp, sp, arg)) MH_TRY(map_max_route(grad, sx, x, sug, m, f, ug));
    }
    return finish("mh_reduce_bwd_accum");
}

}  // extern "C"
