/*
 * mantle_oracle.c -- CPU restatement of Mantle's elementwise / broadcast / reduction path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker): only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library. See mantle_oracle.h for the pinning
 * status of each function; "PARITY UNPINNED" there applies to or_exp / or_log at the bit
 * level (and so to the exp/log bits inside or_powf, whose composition is pinned) and to the
 * lane-combine shape of the sums.
 *
 * Built with -ffp-contract=off: every a*b+c below rounds twice unless written as fmaf.
 * Single-threaded by construction, like the reference's elementwise, broadcast,
 * accumulate, all-element reduce and MAX-backward paths (tensorutils.mojo uses
 * vectorize only there); the axis reduce is also run on one thread here.
 */
#include "mantle_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static int g_nelts = 32;

void or_set_nelts(int nelts) {
    if (nelts >= 1 && nelts <= 64 && (nelts & (nelts - 1)) == 0) g_nelts = nelts;
}
int or_get_nelts(void) { return g_nelts; }

/* ------------------------------------------------------------------------------------ */
/* bit helpers                                                                           */
/* ------------------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* 2^e as a float for e in [-126, 127] (a normal power of two, exact). */
static inline float pow2i(int e) { return u2f((uint32_t)(e + 127) << 23); }

/* p * 2^k, exact for normal results, one rounding for subnormal results. k is split in
 * two halves so that each factor is a normal power of two (k in [-252, 254]). */
static inline float scale2(float p, int k) {
    int k1 = k >> 1;  /* floor(k/2) */
    int k2 = k - k1;
    return (p * pow2i(k1)) * pow2i(k2);
}

/* ------------------------------------------------------------------------------------ */
/* scalar math                                                                           */
/* ------------------------------------------------------------------------------------ */

/* exp for f32: restates std.math.exp as called by mantle/core/math_util.mojo:149-171 and
 * mantle/autograd/ops/mlops.mojo:13,39,201. Algorithm (Mojo stdlib, believed, unverified
 * here): clamp x to [-88.3762626647949, 88.3762626647950], k = floor(fma(x, 1/ln2, 0.5)),
 * r = fma(k, -ln2, x), degree-7 Taylor polynomial of e^r in fma-Horner form, then scale by
 * 2^k. NaN propagates. Bit-level parity with Mojo: PARITY UNPINNED. */
float or_exp(float x) {
    if (x != x) return x;
    const float lo = -88.3762626647949f, hi = 88.3762626647950f;
    float xc = x < lo ? lo : (x > hi ? hi : x);
    float k = floorf(fmaf(xc, 1.442695040888963407359924681001892137426646f, 0.5f));
    float r = fmaf(k, -0.69314718055966295651160180568695068359375f, xc);
    float p = 1.98412698412698412698e-4f;         /* 1/5040 */
    p = fmaf(p, r, 1.38888888888888888889e-3f);   /* 1/720 */
    p = fmaf(p, r, 8.33333333333333333333e-3f);   /* 1/120 */
    p = fmaf(p, r, 4.16666666666666666667e-2f);   /* 1/24 */
    p = fmaf(p, r, 1.66666666666666666667e-1f);   /* 1/6 */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return scale2(p, (int)k);
}

/* natural log for f32: restates std.math.log as called by math_util.mojo:174-196.
 * Algorithm: the Cephes logf method (S. L. Moshier, Cephes Math Library): frexp into
 * m in [0.5,1), fold m below sqrt(1/2) into [sqrt(1/2), sqrt(2)) - 1, a degree-8 minimax
 * polynomial, and the exponent added back in two parts of ln 2. Special values: log(0) =
 * -inf (POW backward relies on isinf(log 0), basics.mojo:366-370), log(x<0) = NaN,
 * log(+inf) = +inf. Bit-level parity with Mojo: PARITY UNPINNED. */
float or_log(float x) {
    if (x != x) return x;
    if (x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (x == INFINITY) return x;
    int eadj = 0;
    if (x < FLT_MIN) { x = x * 33554432.0f; eadj = -25; } /* 2^25, exact */
    uint32_t u = f2u(x);
    int e = (int)((u >> 23) & 0xffu) - 126 + eadj;
    float m = u2f((u & 0x807fffffu) | 0x3f000000u); /* [0.5, 1) */
    if (m < 0.707106781186547524f) {
        e -= 1;
        m = m + m - 1.0f;
    } else {
        m = m - 1.0f;
    }
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
    float fe = (float)e;
    y = y + -2.12194440e-4f * fe;
    y = y + -0.5f * z;
    float r = m + y;
    r = r + 0.693359375f * fe;
    return r;
}

/* pow(SIMD, Int): binary exponentiation with result seeded at 1 and 1/res for negative
 * exponents (Mojo stdlib _powi, believed). Used by elwise_pow, tensorutils.mojo:226-239,
 * and by x**2 at basics.mojo:169,199,213 and mlops.mojo:210 (n = 2 gives x*x). */
float or_powi(float x, int64_t n) {
    uint64_t b = n < 0 ? (uint64_t)(-(n + 1)) + 1u : (uint64_t)n;
    float a = x, res = 1.0f;
    while (b > 0) {
        if (b & 1u) res = res * a;
        a = a * a;
        b >>= 1;
    }
    return n < 0 ? 1.0f / res : res;
}

/* float SIMD ** SIMD (basics.mojo:353,373): the Mojo stdlib's _powf_scalar
 * (std/builtin/simd.mojo): an integral exponent goes through _powi, a negative base with a
 * fractional exponent is NaN, anything else is exp(y * log(x)) with the exp/log above. The
 * composition is pinned by test_powf_is_exp_of_y_times_log; the exp/log bits it inherits are
 * PARITY UNPINNED against Mojo. */
float or_powf(float x, float y) {
    if (y != y) return y;
    float yi = truncf(y);
    if (yi == y && fabsf(y) < 2147483648.0f) return or_powi(x, (int64_t)yi);
    if (x < 0.0f) return NAN;
    return or_exp(y * or_log(x));
}

/* SIGMOID.sigmoid, mlops.mojo:35-42: 1 / (1 + exp(-x)). */
float or_sigmoid(float x) { return 1.0f / (1.0f + or_exp(-x)); }

/* TANH.tanh, mlops.mojo:195-201: (exp(x) - exp(-x)) / (exp(x) + exp(-x)). */
float or_tanh(float x) {
    float ep = or_exp(x), em = or_exp(-x);
    return (ep - em) / (ep + em);
}

/* RELU.relu, mlops.mojo:85-90: x > 0 ? x : 0 (NaN and -0.0 give +0.0). */
float or_relu(float x) { return x > 0.0f ? x : 0.0f; }

/* ------------------------------------------------------------------------------------ */
/* shapes                                                                                */
/* ------------------------------------------------------------------------------------ */
static int64_t numel(const or_shape* s) {
    int64_t n = 1;
    for (int i = 0; i < s->rank; ++i) n *= s->dims[i];
    return n;
}
static int shape_ok(const or_shape* s) {
    if (s->rank < 1 || s->rank > OR_MAX_RANK) return 0;
    for (int i = 0; i < s->rank; ++i)
        if (s->dims[i] < 0) return 0;
    return 1;
}
static int shape_eq(const or_shape* a, const or_shape* b) {
    if (a->rank != b->rank) return 0;
    for (int i = 0; i < a->rank; ++i)
        if (a->dims[i] != b->dims[i]) return 0;
    return 1;
}
/* TensorShape(1): the "graph scalar" shape that elwise_op special-cases. */
static int is_scalar_shape(const or_shape* s) { return s->rank == 1 && s->dims[0] == 1; }

/* broadcast_shapes, tensorutils.mojo:88-127 (numpy rule, right aligned). The reference
 * prints and leaves -1 on a mismatch; here a mismatch returns OR_ERR_SHAPE. */
int or_broadcast_shapes(const or_shape* s1, const or_shape* s2, or_shape* out) {
    if (!shape_ok(s1) || !shape_ok(s2)) return OR_ERR_RANK;
    int ndim = s1->rank > s2->rank ? s1->rank : s2->rank;
    int diff = abs(s1->rank - s2->rank);
    const or_shape* big = s1->rank > s2->rank ? s1 : s2;
    const or_shape* small = s1->rank > s2->rank ? s2 : s1;
    or_shape r;
    memset(&r, 0, sizeof r);
    r.rank = ndim;
    for (int i = ndim - 1; i >= diff; --i) {
        int64_t a = big->dims[i], b = small->dims[i - diff];
        if (a == b) r.dims[i] = a;
        else if (a == 1 || b == 1) r.dims[i] = a * b;
        else return OR_ERR_SHAPE;
    }
    for (int i = diff - 1; i >= 0; --i) r.dims[i] = big->dims[i];
    *out = r;
    return OR_OK;
}

/* broadcast_calculate_strides, tensorutils.mojo:149-175: compact strides of `shape`
 * placed right-aligned in a rank-`size` space, 0 for size-1 and missing dims. */
void or_broadcast_calculate_strides(int size, const or_shape* shape, int64_t* strides) {
    int diff = size - shape->rank;
    for (int i = 0; i < size; ++i) strides[i] = 0;
    int64_t stride = 1;
    for (int i = shape->rank - 1; i >= 0; --i) {
        if (shape->dims[i] != 1) {
            strides[i + diff] = stride;
            stride *= shape->dims[i];
        }
    }
}

/* get_real_index, tensorutils.mojo:50-82: divmod chain from the last dim to the first. */
int64_t or_get_real_index(int size, const int64_t* strides, const or_shape* bshape, int64_t i) {
    int64_t index_res = 0, lin = i;
    for (int dim = 0; dim < size; ++dim) {
        int j = size - 1 - dim;
        int64_t q = lin / bshape->dims[j], r = lin % bshape->dims[j];
        index_res += r * strides[j];
        lin = q;
    }
    return index_res;
}

/* numpy-compatible "grad broadcasts to rg" check: the reference accepts some non-numpy
 * pairs (tensorutils.mojo:149-175 with :482-484) and then indexes out of bounds; here
 * those pairs are rejected. */
static int broadcasts_to(const or_shape* small, const or_shape* big) {
    or_shape r;
    if (or_broadcast_shapes(small, big, &r) != OR_OK) return 0;
    return shape_eq(&r, big);
}

/* ------------------------------------------------------------------------------------ */
/* elementwise                                                                           */
/* ------------------------------------------------------------------------------------ */
void or_fill(float* t, int64_t n, float v) { /* fill, tensorutils.mojo:29-44 */
    for (int64_t i = 0; i < n; ++i) t[i] = v;
}

/* add / sub / mul / div of math_util.mojo:37-126. */
static inline float binop(int op, float a, float b) {
    switch (op) {
        case OR_ADD: return a + b;
        case OR_SUB: return a - b;
        case OR_MUL: return a * b;
        default: return a / b;
    }
}
static int is_binary_elwise(int op) { return op >= OR_ADD && op <= OR_DIV; }

static inline float unop(int op, float x) {
    switch (op) {
        case OR_EXP: return or_exp(x);
        case OR_LOG: return or_log(x);
        case OR_SIGMOID: return or_sigmoid(x);
        case OR_RELU: return or_relu(x);
        default: return or_tanh(x);
    }
}
static int is_unary_elwise(int op) {
    return op == OR_EXP || op == OR_LOG || op == OR_SIGMOID || op == OR_RELU || op == OR_TANH;
}

/* elwise_transform, tensorutils.mojo:181-200. */
int or_elwise_transform(int op, float* res, const float* t, int64_t n) {
    if (!is_unary_elwise(op)) return OR_ERR_OP;
    for (int64_t i = 0; i < n; ++i) res[i] = unop(op, t[i]);
    return OR_OK;
}

/* elwise_pow, tensorutils.mojo:226-239. */
void or_elwise_pow(float* res, const float* t, int64_t n, int64_t x) {
    for (int64_t i = 0; i < n; ++i) res[i] = or_powi(t[i], x);
}

/* elwise_op dispatcher, tensorutils.mojo:242-274, and its four bodies :277-357. */
int or_elwise_op(int op, float* res, const float* t1, const or_shape* s1,
                 const float* t2, const or_shape* s2) {
    if (!is_binary_elwise(op)) return OR_ERR_OP;
    or_shape rs;
    int rc = or_broadcast_shapes(s1, s2, &rs);
    if (rc != OR_OK) return rc;
    if (is_scalar_shape(s2)) { /* :267 tensor (op) scalar */
        int64_t n = numel(s1);
        float b = t2[0];
        for (int64_t i = 0; i < n; ++i) res[i] = binop(op, t1[i], b);
    } else if (is_scalar_shape(s1)) { /* :269 scalar (op) tensor */
        int64_t n = numel(s2);
        float a = t1[0];
        for (int64_t i = 0; i < n; ++i) res[i] = binop(op, a, t2[i]);
    } else if (!shape_eq(s1, s2)) { /* :270-272 -> broadcast_elwise_op :321-357 */
        int64_t st1[OR_MAX_RANK], st2[OR_MAX_RANK];
        or_broadcast_calculate_strides(rs.rank, s1, st1);
        or_broadcast_calculate_strides(rs.rank, s2, st2);
        int64_t n = numel(&rs);
        for (int64_t i = 0; i < n; ++i) {
            int64_t i1 = or_get_real_index(rs.rank, st1, &rs, i);
            int64_t i2 = or_get_real_index(rs.rank, st2, &rs, i);
            res[i] = binop(op, t1[i1], t2[i2]);
        }
    } else { /* :274 same shape */
        int64_t n = numel(s1);
        for (int64_t i = 0; i < n; ++i) res[i] = binop(op, t1[i], t2[i]);
    }
    return OR_OK;
}

/* accumulate_grad, tensorutils.mojo:442-451 (same shape) and :454-487 (shape aware). */
int or_accumulate_grad(float* grad, const or_shape* sg, const float* rg, const or_shape* srg) {
    if (!shape_ok(sg) || !shape_ok(srg)) return OR_ERR_RANK;
    if (shape_eq(sg, srg)) {
        int64_t n = numel(sg);
        for (int64_t i = 0; i < n; ++i) grad[i] = grad[i] + rg[i];
    } else if (is_scalar_shape(srg)) {
        int64_t n = numel(sg);
        for (int64_t i = 0; i < n; ++i) grad[i] = grad[i] + rg[0];
    } else {
        if (!broadcasts_to(sg, srg)) return OR_ERR_SHAPE;
        int64_t st[OR_MAX_RANK];
        or_broadcast_calculate_strides(srg->rank, sg, st);
        int64_t n = numel(srg);
        for (int64_t i = 0; i < n; ++i) { /* serial, row-major order of rg */
            int64_t idx = or_get_real_index(srg->rank, st, srg, i);
            grad[idx] = grad[idx] + rg[i];
        }
    }
    return OR_OK;
}

/* accumulate_op[res_shape, t1_shape, func], tensorutils.mojo:360-393, with func = mul
 * (the only use on this path: SUM/MEAN backward). When the shapes are equal the
 * reference applies func twice (no return after :381); that is reproduced. */
static int accumulate_op_mul_bcast(float* res, const or_shape* sres, const float* t1,
                                   const or_shape* s1) {
    int64_t n = numel(sres);
    if (shape_eq(sres, s1))
        for (int64_t i = 0; i < n; ++i) res[i] = res[i] * t1[i];
    else if (!broadcasts_to(s1, sres))
        return OR_ERR_SHAPE;
    int64_t st[OR_MAX_RANK];
    or_broadcast_calculate_strides(sres->rank, s1, st);
    for (int64_t i = 0; i < n; ++i) {
        int64_t idx = or_get_real_index(sres->rank, st, sres, i);
        res[i] = res[i] * t1[idx];
    }
    return OR_OK;
}

/* ------------------------------------------------------------------------------------ */
/* reductions                                                                            */
/* ------------------------------------------------------------------------------------ */
/* max_simd, math_util.mojo:224-244: a > b ? a : b. */
static inline float max_simd(float a, float b) { return a > b ? a : b; }

/* SIMD.reduce_add / reduce_max over the nelts lanes: halving tree (lane k combined with
 * lane k + w for w = nelts/2 ... 1). The tree shape is PARITY UNPINNED (rtol class). */
static float lanes_combine(int op, float* m, int w) {
    for (w >>= 1; w >= 1; w >>= 1)
        for (int k = 0; k < w; ++k) m[k] = op == OR_MAX ? max_simd(m[k], m[k + w]) : m[k] + m[k + w];
    return m[0];
}

/* reduce (all elements), tensorutils.mojo:564-598, with tsum :694-706 (start 0) and tmax
 * :850-862 (start min_finite = -FLT_MAX). Lane k takes elements i = k (mod nelts) of the
 * full chunks; the width-1 tail goes into lane 0. MEAN is handled by the caller. */
float or_reduce_all(int op, const float* t, int64_t n) {
    float m[64];
    const int w = g_nelts;
    const float start = op == OR_MAX ? -FLT_MAX : 0.0f;
    for (int k = 0; k < w; ++k) m[k] = start;
    int64_t full = n - n % w, i = 0;
    if (op == OR_MAX) {
        for (; i < full; i += w)
            for (int k = 0; k < w; ++k) m[k] = max_simd(m[k], t[i + k]);
        for (; i < n; ++i) m[0] = max_simd(m[0], t[i]);
    } else {
        for (; i < full; i += w)
            for (int k = 0; k < w; ++k) m[k] = m[k] + t[i + k];
        for (; i < n; ++i) m[0] = m[0] + t[i];
    }
    return lanes_combine(op, m, w);
}

/* reduce (one axis), tensorutils.mojo:622-684, with tsum :746-757, tmean :760-772 (sum,
 * then accumulate_op[div] by f32(dim)) and tmax :865-876. Output i reads
 * base = (i % s) + (i / s) * (s * d), lanes over j as in or_reduce_all. */
/* Outputs [i0, i1) of an axis reduce: the body of parallel_reduce (tensorutils.mojo:651-680). */
static void reduce_axis_range(int op, float* res, const float* t, int64_t sa, int64_t d, int64_t i0, int64_t i1) {
    const int w = g_nelts;
    const int rop = op == OR_MAX ? OR_MAX : OR_SUM;
    const float start = op == OR_MAX ? -FLT_MAX : 0.0f;
    const int64_t full = d - d % w;
    for (int64_t i = i0; i < i1; ++i) {
        float m[64];
        for (int k = 0; k < w; ++k) m[k] = start;
        const int64_t base = (i % sa) + (i / sa) * (sa * d);
        int64_t j = 0;
        if (rop == OR_MAX) {
            for (; j < full; j += w)
                for (int k = 0; k < w; ++k) m[k] = max_simd(m[k], t[base + (j + k) * sa]);
            for (; j < d; ++j) m[0] = max_simd(m[0], t[base + j * sa]);
        } else {
            for (; j < full; j += w)
                for (int k = 0; k < w; ++k) m[k] = m[k] + t[base + (j + k) * sa];
            for (; j < d; ++j) m[0] = m[0] + t[base + j * sa];
        }
        res[i] = lanes_combine(rop, m, w);
    }
    if (op == OR_MEAN) { /* tmean: accumulate_op[div] by f32(dim) (tensorutils.mojo:760-772) */
        const float fd = (float)d;
        for (int64_t i = i0; i < i1; ++i) res[i] = res[i] / fd;
    }
}

static int axis_geometry(int op, const or_shape* s, int axis, int64_t* sa, int64_t* d, int64_t* nout) {
    if (!shape_ok(s)) return OR_ERR_RANK;
    if (axis < 0 || axis >= s->rank) return OR_ERR_SHAPE;
    if (op != OR_SUM && op != OR_MEAN && op != OR_MAX) return OR_ERR_OP;
    *sa = 1;
    for (int i = s->rank - 1; i > axis; --i) *sa *= s->dims[i];
    *d = s->dims[axis];
    *nout = 1;
    for (int i = 0; i < s->rank; ++i)
        if (i != axis) *nout *= s->dims[i];
    return OR_OK;
}

/* reduce along an axis (tensorutils.mojo:622-684): output i reads the line starting at
 * base = (i % s) + (i / s) * (s * d), lanes over j as in or_reduce_all. */
int or_reduce_axis(int op, float* res, const float* t, const or_shape* s, int axis) {
    int64_t sa, d, nout;
    const int rc = axis_geometry(op, s, axis, &sa, &d, &nout);
    if (rc != OR_OK) return rc;
    reduce_axis_range(op, res, t, sa, d, 0, nout);
    return OR_OK;
}

typedef struct {
    int op;
    float* res;
    const float* t;
    int64_t sa, d, i0, i1;
} axis_job;

static void* axis_worker(void* p) {
    const axis_job* j = (const axis_job*)p;
    reduce_axis_range(j->op, j->res, j->t, j->sa, j->d, j->i0, j->i1);
    return NULL;
}

/* The same reduction with its outputs spread over `nthreads` threads in contiguous blocks, as
 * parallelize[parallel_reduce](num_elements / dim(axis)) does (tensorutils.mojo:682). Every
 * output is computed exactly as by or_reduce_axis, so the results are identical. */
int or_reduce_axis_mt(int op, float* res, const float* t, const or_shape* s, int axis, int nthreads) {
    int64_t sa, d, nout;
    const int rc = axis_geometry(op, s, axis, &sa, &d, &nout);
    if (rc != OR_OK) return rc;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if ((int64_t)nthreads > nout) nthreads = nout > 0 ? (int)nout : 1;
    pthread_t th[256];
    int running[256] = {0};
    axis_job jobs[256];
    const int64_t per = (nout + nthreads - 1) / nthreads;
    int blocks = 0;
    for (int k = 0; k < nthreads; ++k) {
        const int64_t i0 = k * per, i1 = i0 + per < nout ? i0 + per : nout;
        if (i0 >= i1) break;
        jobs[k] = (axis_job){op, res, t, sa, d, i0, i1};
        blocks = k + 1;
        if (k == 0) continue; /* the calling thread takes block 0 */
        if (pthread_create(&th[k], NULL, axis_worker, &jobs[k]) == 0) running[k] = 1;
        else axis_worker(&jobs[k]); /* no thread: run the block here */
    }
    if (blocks > 0) axis_worker(&jobs[0]);
    for (int k = 1; k < blocks; ++k)
        if (running[k]) pthread_join(th[k], NULL);
    return OR_OK;
}

static int reduced_shape(const or_shape* s, int axis, or_shape* out) {
    if (axis < 0) {
        memset(out, 0, sizeof *out);
        out->rank = 1;
        out->dims[0] = 1;
        return OR_OK;
    }
    if (axis >= s->rank) return OR_ERR_SHAPE;
    *out = *s;
    out->dims[axis] = 1; /* get_reduce_shape, tensorutils.mojo:601-619 */
    return OR_OK;
}

/* ------------------------------------------------------------------------------------ */
/* forward_op / backward_op                                                              */
/* ------------------------------------------------------------------------------------ */
/* forward_op, ops.mojo:243-311, through the op structs of basics.mojo / mlops.mojo. */
int or_forward_op(int op, float* res, const float* t1, const or_shape* s1,
                  const float* t2, const or_shape* s2, int axis) {
    if (!shape_ok(s1)) return OR_ERR_RANK;
    if (is_binary_elwise(op)) return or_elwise_op(op, res, t1, s1, t2, s2);
    if (op == OR_POW) { /* POW.forward, basics.mojo:320-327: Int(t2[0]) truncates */
        if (!s2 || !is_scalar_shape(s2)) return OR_ERR_SHAPE;
        or_elwise_pow(res, t1, numel(s1), (int64_t)truncf(t2[0]));
        return OR_OK;
    }
    if (is_unary_elwise(op)) return or_elwise_transform(op, res, t1, numel(s1));
    if (op == OR_SUM || op == OR_MEAN || op == OR_MAX) {
        if (axis >= 0) return or_reduce_axis(op, res, t1, s1, axis);
        int64_t n = numel(s1);
        float v = or_reduce_all(op == OR_MAX ? OR_MAX : OR_SUM, t1, n);
        if (op == OR_MEAN) v = v / (float)n; /* tmean, tensorutils.mojo:709-720 */
        res[0] = v;
        return OR_OK;
    }
    return OR_ERR_OP;
}

/* Unary backward bodies (rg only), basics.mojo:260-309, 381-615 and mlops.mojo:27-235. */
static int unary_backward(int op, float* rg, const float* ug, const or_shape* sug,
                          const float* t, const or_shape* st, int axis) {
    const int64_t n = numel(st);
    switch (op) {
        case OR_EXP: /* basics.mojo:281-284 */
            for (int64_t i = 0; i < n; ++i) rg[i] = or_exp(t[i]) * ug[i];
            return OR_OK;
        case OR_LOG: /* basics.mojo:305-309: elwise_op[div](ug, t) */
            for (int64_t i = 0; i < n; ++i) rg[i] = ug[i] / t[i];
            return OR_OK;
        case OR_SIGMOID: /* mlops.mojo:44-74 */
            for (int64_t i = 0; i < n; ++i) {
                float s = or_sigmoid(t[i]);
                rg[i] = (s * (1.0f - s)) * ug[i];
            }
            return OR_OK;
        case OR_RELU: /* mlops.mojo:92-123 */
            for (int64_t i = 0; i < n; ++i) rg[i] = (t[i] > 0.0f ? 1.0f : 0.0f) * ug[i];
            return OR_OK;
        case OR_TANH: /* mlops.mojo:203-233: 1 - pow(tanh(x), 2) */
            for (int64_t i = 0; i < n; ++i) {
                float th = or_tanh(t[i]);
                rg[i] = (1.0f - th * th) * ug[i];
            }
            return OR_OK;
        case OR_SUM: { /* basics.mojo:416-425 */
            or_fill(rg, n, 1.0f);
            return accumulate_op_mul_bcast(rg, st, ug, sug);
        }
        case OR_MEAN:
            if (axis < 0) { /* basics.mojo:470-487 */
                float g = (float)(1.0 / (double)n);
                g = g * ug[0];
                or_fill(rg, n, g);
                return OR_OK;
            } else { /* basics.mojo:489-506 */
                float g = (float)(1.0 / (double)st->dims[axis]);
                or_fill(rg, n, g);
                return accumulate_op_mul_bcast(rg, st, ug, sug);
            }
        case OR_MAX:
            or_fill(rg, n, 0.0f); /* res_grad is zero-initialised (tensor.mojo:266) */
            if (axis < 0) { /* basics.mojo:551-577 */
                float m = or_reduce_all(OR_MAX, t, n);
                float cnt = 0.0f;
                for (int64_t i = 0; i < n; ++i)
                    if (t[i] == m) cnt = cnt + 1.0f;
                float f = 1.0f / cnt;
                for (int64_t i = 0; i < n; ++i)
                    if (t[i] == m) rg[i] = f * ug[0];
                return OR_OK;
            } else { /* basics.mojo:579-615 */
                int64_t sa = 1;
                for (int i = st->rank - 1; i > axis; --i) sa *= st->dims[i];
                const int64_t d = st->dims[axis];
                const int64_t nout = d ? n / d : 0;
                float* mx = (float*)malloc(sizeof(float) * (size_t)(nout ? nout : 1));
                if (!mx) return OR_ERR_SHAPE;
                or_reduce_axis(OR_MAX, mx, t, st, axis);
                for (int64_t i = 0; i < nout; ++i) {
                    const int64_t base = (i % sa) + (i / sa) * (sa * d);
                    float cnt = 0.0f;
                    for (int64_t j = 0; j < d; ++j)
                        if (t[base + j * sa] == mx[i]) cnt = cnt + 1.0f;
                    float f = 1.0f / cnt;
                    for (int64_t j = 0; j < d; ++j)
                        if (t[base + j * sa] == mx[i]) rg[base + j * sa] = f * ug[i];
                }
                free(mx);
                return OR_OK;
            }
        default:
            return OR_ERR_OP;
    }
}

/* Binary backward bodies (rg only), basics.mojo:28-219 and 312-378. rg has the shape of
 * ug (broadcast(t1, t2)) for ADD..DIV, of t1 for POW id0 and (1) for POW id1. */
static int binary_backward(int id, int op, float* rg, const float* ug, const or_shape* sug,
                           const float* t1, const or_shape* s1, const float* t2,
                           const or_shape* s2) {
    const int64_t n = numel(sug);
    switch (op) {
        case OR_ADD: /* basics.mojo:46-55: ug.copy() */
            memcpy(rg, ug, sizeof(float) * (size_t)n);
            return OR_OK;
        case OR_SUB: /* basics.mojo:82-91 */
            if (id == 0) memcpy(rg, ug, sizeof(float) * (size_t)n);
            else for (int64_t i = 0; i < n; ++i) rg[i] = ug[i] * -1.0f;
            return OR_OK;
        case OR_MUL: /* basics.mojo:118-129 */
            return id == 0 ? or_elwise_op(OR_MUL, rg, ug, sug, t2, s2)
                           : or_elwise_op(OR_MUL, rg, ug, sug, t1, s1);
        case OR_DIV: /* basics.mojo:155-219 */
            if (id == 0) return or_elwise_op(OR_DIV, rg, ug, sug, t2, s2);
            if (is_scalar_shape(s2)) { /* :168-180 */
                const float s = t2[0];
                const float f = -1.0f / (s * s);
                for (int64_t i = 0; i < n; ++i) rg[i] = (f * t1[i]) * ug[i];
            } else if (!shape_eq(s1, s2)) { /* :182-203 (without the OOB lanes) */
                int64_t st1[OR_MAX_RANK], st2[OR_MAX_RANK];
                or_broadcast_calculate_strides(sug->rank, s1, st1);
                or_broadcast_calculate_strides(sug->rank, s2, st2);
                for (int64_t i = 0; i < n; ++i) {
                    const float a = t1[or_get_real_index(sug->rank, st1, sug, i)];
                    const float b = t2[or_get_real_index(sug->rank, st2, sug, i)];
                    rg[i] = ((-a) / (b * b)) * ug[i];
                }
            } else { /* :205-217 */
                for (int64_t i = 0; i < n; ++i) rg[i] = ((-t1[i]) / (t2[i] * t2[i])) * ug[i];
            }
            return OR_OK;
        case OR_POW: {
            const float a = t2[0];
            const int64_t nx = numel(s1);
            if (id == 0) { /* :345-357 */
                const float am1 = a - 1.0f;
                for (int64_t i = 0; i < nx; ++i)
                    rg[i] = (a * or_powf(t1[i] + 1e-12f, am1)) * ug[i];
            } else { /* :359-376: per-chunk reduce_add added into rg[0] */
                const int w = g_nelts;
                const int64_t full = n - n % w;
                float acc = 0.0f, lanes[64];
                int64_t i = 0;
                for (; i < full; i += w) {
                    for (int k = 0; k < w; ++k) {
                        float lg = or_log(t1[i + k]);
                        if (isinf(lg)) lg = 0.0f;
                        lanes[k] = (or_powf(t1[i + k], a) * lg) * ug[i + k];
                    }
                    acc = acc + lanes_combine(OR_SUM, lanes, w);
                }
                for (; i < n; ++i) {
                    float lg = or_log(t1[i]);
                    if (isinf(lg)) lg = 0.0f;
                    acc = acc + (or_powf(t1[i], a) * lg) * ug[i];
                }
                rg[0] = acc;
            }
            return OR_OK;
        }
        default:
            return OR_ERR_OP;
    }
}

/* backward_op, ops.mojo:355-405 (unary: struct backward, then same-shape
 * accumulate_grad) and ops.mojo:408-463 (binary: struct backward, then the shape-aware
 * accumulate_grad for ADD/SUB/MUL/DIV, same-shape for POW). `grad` is accumulated into. */
int or_backward_op(int tensor_id, int op, const float* ug, const or_shape* sug,
                   const float* t1, const or_shape* s1, const float* t2, const or_shape* s2,
                   int axis, float* grad) {
    if (!shape_ok(sug) || !shape_ok(s1)) return OR_ERR_RANK;
    int rc;
    if (is_binary_elwise(op) || op == OR_POW) {
        if (!s2 || !shape_ok(s2)) return OR_ERR_RANK;
        if (tensor_id != 0 && tensor_id != 1) return OR_ERR_OP;
        or_shape rs;
        if (op == OR_POW) {
            if (!is_scalar_shape(s2) || !shape_eq(sug, s1)) return OR_ERR_SHAPE;
            rs = tensor_id == 0 ? *s1 : *s2;
        } else {
            if ((rc = or_broadcast_shapes(s1, s2, &rs)) != OR_OK) return rc;
            if (!shape_eq(&rs, sug)) return OR_ERR_SHAPE;
        }
        float* rg = (float*)malloc(sizeof(float) * (size_t)(numel(&rs) ? numel(&rs) : 1));
        if (!rg) return OR_ERR_SHAPE;
        rc = binary_backward(tensor_id, op, rg, ug, sug, t1, s1, t2, s2);
        if (rc == OR_OK) {
            if (op == OR_POW) {
                const int64_t n = numel(&rs);
                for (int64_t i = 0; i < n; ++i) grad[i] = grad[i] + rg[i];
            } else {
                rc = or_accumulate_grad(grad, tensor_id == 0 ? s1 : s2, rg, &rs);
            }
        }
        free(rg);
        return rc;
    }
    if (is_unary_elwise(op) || op == OR_SUM || op == OR_MEAN || op == OR_MAX) {
        if (is_unary_elwise(op)) {
            if (!shape_eq(sug, s1)) return OR_ERR_SHAPE;
        } else {
            or_shape red;
            if ((rc = reduced_shape(s1, axis, &red)) != OR_OK) return rc;
            if (!shape_eq(&red, sug)) return OR_ERR_SHAPE;
        }
        const int64_t n = numel(s1);
        float* rg = (float*)malloc(sizeof(float) * (size_t)(n ? n : 1));
        if (!rg) return OR_ERR_SHAPE;
        rc = unary_backward(op, rg, ug, sug, t1, s1, axis);
        if (rc == OR_OK)
            for (int64_t i = 0; i < n; ++i) grad[i] = grad[i] + rg[i];
        free(rg);
        return rc;
    }
    return OR_ERR_OP;
}

/* ------------------------------------------------------------------------------------ */
/* Adam.step, mantle/nn/optim.mojo:94-140 (the per-element body v_step, :101-132)        */
/* ------------------------------------------------------------------------------------ */
void or_adam_step(float* param, const float* grad, float* m, float* v, int64_t n, float lr,
                  float beta1, float beta2, float eps, int64_t iter) {
    /* Scalar[f32] arithmetic on the hyper-parameters: 1 - beta, and beta ** iter as Mojo's
     * SIMD ** Int (square-and-multiply, or_powi) */
    const float c1 = 1.0f - beta1;
    const float c2 = 1.0f - beta2;
    const float bc1 = 1.0f - or_powi(beta1, iter);
    const float bc2 = 1.0f - or_powi(beta2, iter);
    for (int64_t j = 0; j < n; ++j) {
        const float g = grad[j];
        float mj = beta1 * m[j] + c1 * g;          /* :109-111 */
        m[j] = mj;
        mj = mj / bc1;                             /* :116 */
        float vj = beta2 * v[j] + c2 * g * g;      /* :120-122, (c2 * g) * g */
        v[j] = vj;
        vj = vj / bc2;                             /* :127 */
        param[j] = param[j] - lr * (mj / (sqrtf(vj) + eps)); /* :130-132 */
    }
}

/* ------------------------------------------------------------------------------------ */
/* FMA, LEAKYRELU, CLIP                                                                  */
/* ------------------------------------------------------------------------------------ */
/* FMA.forward, basics.mojo:768-788: t1.fma(t2, t3), one rounding (C fmaf is exact-then-round). */
void or_fma_fwd(float* res, const float* t1, const float* t2, const float* t3, int64_t n) {
    for (int64_t i = 0; i < n; ++i) res[i] = fmaf(t1[i], t2[i], t3[i]);
}

/* FMA.backward, basics.mojo:790-817 (id 0: ug * t2, id 1: ug * t1, id 2: ug), accumulated by
 * the ternary backward_op, ops.mojo:466-497 (accumulate_grad, grad = grad + rg). */
int or_fma_bwd_accum(int tensor_id, float* grad, const float* ug, const float* t1, const float* t2, int64_t n) {
    if (tensor_id < 0 || tensor_id > 2) return OR_ERR_OP;
    for (int64_t i = 0; i < n; ++i) {
        const float rg = tensor_id == 0 ? ug[i] * t2[i] : tensor_id == 1 ? ug[i] * t1[i] : ug[i];
        grad[i] = grad[i] + rg;
    }
    return OR_OK;
}

/* LEAKYRELU, mlops.mojo:128-186: fwd x > 0 ? x : x * slope; bwd (x > 0 ? 1 : slope) * ug. */
void or_leakyrelu_fwd(float* res, const float* x, int64_t n, float slope) {
    for (int64_t i = 0; i < n; ++i) res[i] = x[i] > 0.0f ? x[i] : x[i] * slope;
}
void or_leakyrelu_bwd_accum(float* grad, const float* x, const float* ug, int64_t n, float slope) {
    for (int64_t i = 0; i < n; ++i) grad[i] = grad[i] + (x[i] > 0.0f ? 1.0f : slope) * ug[i];
}

/* min / max as LLVM minnum / maxnum: a NaN operand yields the other one; on equal operands
 * the first is returned. */
static inline float or_minnum(float a, float b) { return (b < a || a != a) ? b : a; }
static inline float or_maxnum(float a, float b) { return (b > a || a != a) ? b : a; }

/* CLIP, mlops.mojo:238-299: fwd max(min(x, hi), lo); bwd (x >= lo && x <= hi) ? ug : 0.
 * Absent attributes are min_finite / max_finite (the caller passes -FLT_MAX / FLT_MAX). */
void or_clip_fwd(float* res, const float* x, int64_t n, float lo, float hi) {
    for (int64_t i = 0; i < n; ++i) res[i] = or_maxnum(or_minnum(x[i], hi), lo);
}
void or_clip_bwd_accum(float* grad, const float* x, const float* ug, int64_t n, float lo, float hi) {
    for (int64_t i = 0; i < n; ++i) grad[i] = grad[i] + ((x[i] >= lo && x[i] <= hi) ? ug[i] : 0.0f);
}

/* ------------------------------------------------------------------------------------ */
/* tstd                                                                                  */
/* ------------------------------------------------------------------------------------ */
/* tstd (all elements), tensorutils.mojo:724-741: mu = tmean(t); variance accumulates, chunk
 * by chunk of nelts, (diff * diff).reduce_add() (width-1 tail steps one element each); the
 * result is sqrt(variance / f32(n)). */
float or_tstd_all(const float* t, int64_t n) {
    const float mu = or_reduce_all(OR_SUM, t, n) / (float)n;
    const int w = g_nelts;
    const int64_t full = n - n % w;
    float var = 0.0f, m[64];
    int64_t i = 0;
    for (; i < full; i += w) {
        for (int k = 0; k < w; ++k) {
            const float d = t[i + k] - mu;
            m[k] = d * d;
        }
        var = var + lanes_combine(OR_SUM, m, w);
    }
    for (; i < n; ++i) {
        const float d = t[i] - mu;
        var = var + d * d;
    }
    return sqrtf(var / (float)n);
}

/* tstd (one axis), tensorutils.mojo:776-840: mu = tmean(t, axis); per output line the
 * squared deviations accumulate chunk by chunk as above, then res /= f32(dim) and sqrt.
 * The reference addresses line i as sum over k != axis of (i % shape[k]) * stride[k] and
 * loads nelts contiguous elements even when the axis is not the last; both only agree with
 * the line i for a last-axis reduction of a rank-2 tensor (its tests use lines of equal
 * spread, where any line gives the expected value). This restatement reads line i as
 * tmean does: base = (i % s) + (i / s) * (s * d), elements base + j * s. */
int or_tstd_axis(float* res, const float* t, const or_shape* s, int axis) {
    if (!shape_ok(s)) return OR_ERR_RANK;
    if (axis < 0 || axis >= s->rank) return OR_ERR_SHAPE;
    int64_t sa = 1;
    for (int i = s->rank - 1; i > axis; --i) sa *= s->dims[i];
    const int64_t d = s->dims[axis];
    int64_t nout = 1;
    for (int i = 0; i < s->rank; ++i)
        if (i != axis) nout *= s->dims[i];
    float* mu = (float*)malloc(sizeof(float) * (size_t)(nout ? nout : 1));
    if (!mu) return OR_ERR_SHAPE;
    int rc = or_reduce_axis(OR_MEAN, mu, t, s, axis);
    const int w = g_nelts;
    const int64_t full = d - d % w;
    for (int64_t i = 0; rc == OR_OK && i < nout; ++i) {
        const int64_t base = (i % sa) + (i / sa) * (sa * d);
        float var = 0.0f, m[64];
        int64_t j = 0;
        for (; j < full; j += w) {
            for (int k = 0; k < w; ++k) {
                const float df = t[base + (j + k) * sa] - mu[i];
                m[k] = df * df;
            }
            var = var + lanes_combine(OR_SUM, m, w);
        }
        for (; j < d; ++j) {
            const float df = t[base + j * sa] - mu[i];
            var = var + df * df;
        }
        res[i] = sqrtf(var / (float)d);
    }
    free(mu);
    return rc;
}
