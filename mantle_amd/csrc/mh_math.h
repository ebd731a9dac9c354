// mh_math.h -- fp32 device math of Mantle's ops, evaluated in the reference's exact
// expression order. Compiled with -ffp-contract=off: an fma appears only where written.
//
// exp and log follow the algorithms Mantle's CPU path gets from the Mojo stdlib
// (std.math.exp / std.math.log as called at mantle/core/math_util.mojo:149-196 and
// mantle/autograd/ops/mlops.mojo:13,39,201):
//   exp: clamp to [-88.3762626647949, 88.3762626647950], k = floor(fma(x, 1/ln2, 0.5)),
//        r = fma(k, -ln2, x), degree-7 Taylor polynomial of e^r (fma Horner), times 2^k;
//   log: the Cephes logf method (S. L. Moshier, Cephes Math Library): frexp, fold below
//        sqrt(1/2), degree-8 minimax polynomial, exponent added in two parts of ln 2.
// Arguments that need special handling (exp: NaN or out of range; log: anything but a
// positive normal finite value) leave the straight-line path through one range test, so
// that the common case runs without per-element selects.
// Float pow is the stdlib's scalar rule: integral exponent -> binary exponentiation,
// negative base with fractional exponent -> NaN, otherwise exp(y * log(x)).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mh {

// exp on the clamped argument: k = floor(fma(x, 1/ln2, 0.5)), r = fma(k, -ln2, x), degree-7
// Taylor polynomial of e^r in fma-Horner form, times 2^k. ldexp rounds p * 2^k once, the
// same value as multiplying by two normal powers of two in turn (exact unless the result is
// subnormal, where both round the exact product once).
__device__ __forceinline__ float mexp_core(float xc) {
    float k = __builtin_floorf(__builtin_fmaf(xc, 1.442695040888963407359924681001892137426646f, 0.5f));
    float r = __builtin_fmaf(k, -0.69314718055966295651160180568695068359375f, xc);
    float p = 1.98412698412698412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)k);
}

__device__ __forceinline__ float mexp(float x) {
    const float lo = -88.3762626647949f, hi = 88.3762626647950f;
    // clamp without a branch: min / max return the number for a NaN operand, so a NaN x
    // evaluates the core at a bound and the select below returns x itself
    const float xc = __builtin_fminf(__builtin_fmaxf(x, lo), hi);
    const float e = mexp_core(xc);
    return x != x ? x : e;
}

// log of a positive normal finite x (Cephes logf): frexp, fold below sqrt(1/2), degree-8
// polynomial, exponent added in two parts of ln 2. eadj corrects the exponent of a
// pre-scaled subnormal. Three steps are written as fmas that give the method's bits: the
// fold's m + m - 1 and m - 1 are exact (Sterbenz), as is fma(m, 2 or 1, -1); -0.5 z is
// exact (z = m^2 is 0 or at least 2^-48), so y + (-0.5 z) is fma(-0.5, z, y); and
// 0.693359375 fe is exact (a 9-bit constant times an integer below 2^8).
__device__ __forceinline__ float mlog_core(float x, int eadj) {
    const uint32_t u = __float_as_uint(x);
    float m = __uint_as_float((u & 0x807fffffu) | 0x3f000000u);
    const bool fold = m < 0.707106781186547524f;
    // frexp's exponent of a normal x: its biased exponent - 126
    const int e = __builtin_amdgcn_frexp_expf(x) + eadj - (int)fold;
    m = __builtin_fmaf(m, fold ? 2.0f : 1.0f, -1.0f);
    float z = m * m;
    float y = 7.0376836292e-2f;
    y = y * m - 1.1514610310e-1f;
    y = y * m + 1.1676998740e-1f;
    y = y * m - 1.2420140846e-1f;
    y = y * m + 1.4249322787e-1f;
    y = y * m - 1.6668057665e-1f;
    y = y * m + 2.0000714765e-1f;
    y = y * m - 2.4999993993e-1f;
    y = y * m + 3.3333331174e-1f;
    y = y * m * z;
    const float fe = (float)e;
    y = y + -2.12194440e-4f * fe;
    y = __builtin_fmaf(-0.5f, z, y);
    const float r = m + y;
    return __builtin_fmaf(0.693359375f, fe, r);
}

// NaN, negative, zero, subnormal and infinite arguments, off the hot path.
__device__ __attribute__((noinline)) float mlog_special(float x) {
    if (x != x) return x;
    if (x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    return mlog_core(x * 33554432.0f, -25);  // subnormal: scale by 2^25 (exact)
}

__device__ __forceinline__ float mlog(float x) {
    if (__builtin_expect(!(x >= 1.17549435e-38f && x < __builtin_inff()), 0)) return mlog_special(x);
    return mlog_core(x, 0);
}

// pow(SIMD, Int): result seeded at 1, square-and-multiply, 1/res for negative n.
__device__ __forceinline__ float mpowi(float x, int64_t n) {
    uint64_t b = n < 0 ? (uint64_t)(-(n + 1)) + 1u : (uint64_t)n;
    float a = x, res = 1.0f;
    while (b > 0) {
        if (b & 1u) res = res * a;
        a = a * a;
        b >>= 1;
    }
    return n < 0 ? 1.0f / res : res;
}

__device__ __forceinline__ float mpowf(float x, float y) {
    if (y != y) return y;
    float yi = __builtin_truncf(y);
    if (yi == y && __builtin_fabsf(y) < 2147483648.0f) return mpowi(x, (int64_t)yi);
    if (x < 0.0f) return __builtin_nanf("");
    return mexp(y * mlog(x));
}

// mpowf(x, y) for a caller that already holds lgx = mlog(x): the same branches and the same
// bits, without evaluating the log a second time.
__device__ __forceinline__ float mpowf_lg(float x, float y, float lgx) {
    if (y != y) return y;
    float yi = __builtin_truncf(y);
    if (yi == y && __builtin_fabsf(y) < 2147483648.0f) return mpowi(x, (int64_t)yi);
    if (x < 0.0f) return __builtin_nanf("");
    return mexp(y * lgx);
}

__device__ __forceinline__ float msigmoid(float x) { return 1.0f / (1.0f + mexp(-x)); }

__device__ __forceinline__ float mtanh(float x) {
    float ep = mexp(x), em = mexp(-x);
    return (ep - em) / (ep + em);
}

__device__ __forceinline__ float mrelu(float x) { return x > 0.0f ? x : 0.0f; }

}  // namespace mh
