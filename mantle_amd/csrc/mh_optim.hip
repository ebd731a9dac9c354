// mh_optim.hip -- Adam.step (mantle/nn/optim.mojo:94-140) on device-resident parameters.
//
// Per element, in the reference's expression order (v_step, optim.mojo:101-132; built with
// -ffp-contract=off, so every product and sum rounds on its own):
//   m = beta1 * m + (1 - beta1) * g;           store m;   mh = m / (1 - beta1 ** iter)
//   v = beta2 * v + ((1 - beta2) * g) * g;     store v;   vh = v / (1 - beta2 ** iter)
//   p = p - lr * (mh / (sqrt(vh) + eps))
// The scalars 1 - beta and 1 - beta ** iter are Scalar[f32] arithmetic, beta ** iter being
// Mojo's SIMD ** Int (square-and-multiply); they are computed once on the host in f32.
// 28 bytes per element: p, g, m, v read; p, m, v written.
//
// mh_adam_step updates one tensor; mh_adam_step_multi updates every parameter of a model
// with one launch per 80 tensors (the reference parallelises over parameters,
// optim.mojo:140): threads walk the concatenated element quads of the launch's tensors and
// find their tensor by a wave-uniform binary search in a table passed by value, so a model of
// many small tensors costs a launch per 80 tensors, not one per tensor.
#include <cmath>

#include "mh_internal.h"

namespace mh {

constexpr int kOThreads = 64;  // one-wavefront workgroups stream fastest on gfx950

struct AdamScal {
    float lr, b1, b2, eps, c1, c2, bc1, bc2;
};

// f32 x ** n by square-and-multiply (Mojo's SIMD ** Int), n >= 0.
static float host_powi(float x, int64_t n) {
    float a = x, res = 1.0f;
    for (uint64_t b = (uint64_t)n; b > 0; b >>= 1) {
        if (b & 1u) res = res * a;
        a = a * a;
    }
    return res;
}

static AdamScal adam_scalars(float lr, float b1, float b2, float eps, int64_t iter) {
    AdamScal s;
    s.lr = lr;
    s.b1 = b1;
    s.b2 = b2;
    s.eps = eps;
    s.c1 = 1.0f - b1;
    s.c2 = 1.0f - b2;
    s.bc1 = 1.0f - host_powi(b1, iter);
    s.bc2 = 1.0f - host_powi(b2, iter);
    return s;
}

__device__ __forceinline__ void adam1(float& p, float g, float& m, float& v, const AdamScal& s) {
    float mj = s.b1 * m + s.c1 * g;
    m = mj;
    mj = mj / s.bc1;
    float vj = s.b2 * v + s.c2 * g * g;
    v = vj;
    vj = vj / s.bc2;
    p = p - s.lr * (mj / (__builtin_sqrtf(vj) + s.eps));
}

// Elements [e0, e0 + cnt) of one tensor, cnt <= 4; a full quad at a 16-byte aligned address
// moves as float4.
__device__ __forceinline__ void adam_unit(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                                          float* __restrict__ v, int64_t e0, int cnt, bool vec, const AdamScal& s) {
    if (cnt == 4 && vec) {
        float4 pp = ld_nt4(p + e0, 0);
        const float4 gg = ld_nt4(g + e0, 0);
        float4 mm = ld_nt4(m + e0, 0);
        float4 vv = ld_nt4(v + e0, 0);
        adam1(pp.x, gg.x, mm.x, vv.x, s);
        adam1(pp.y, gg.y, mm.y, vv.y, s);
        adam1(pp.z, gg.z, mm.z, vv.z, s);
        adam1(pp.w, gg.w, mm.w, vv.w, s);
        st_nt4(p + e0, 0, pp);
        st_nt4(m + e0, 0, mm);
        st_nt4(v + e0, 0, vv);
    } else {
        for (int j = 0; j < cnt; ++j) {
            float pp = p[e0 + j], mm = m[e0 + j], vv = v[e0 + j];
            adam1(pp, g[e0 + j], mm, vv, s);
            p[e0 + j] = pp;
            m[e0 + j] = mm;
            v[e0 + j] = vv;
        }
    }
}

// Units of a tensor. When the four pointers share one misalignment (the same offset into four
// aligned buffers, as a sliced arena gives), unit 0 takes the `head` = 0..3 elements before the
// first 16-byte boundary and every later unit is an aligned quad: unit k covers elements
// [max(0, 4k - sh), min(n, 4k + 4 - sh)), sh = (4 - head) & 3. Otherwise sh = 0 and units
// are scalar.
struct UnitMap {
    int sh;      // 0..3
    int vec;     // quads after the head are 16-byte aligned in all four tensors
};

__host__ __device__ __forceinline__ int64_t adam_units(int64_t n, int sh) { return (n + sh + 3) >> 2; }

__device__ __forceinline__ void adam_unit_k(float* __restrict__ p, const float* __restrict__ g,
                                            float* __restrict__ m, float* __restrict__ v, int64_t n, int64_t k,
                                            UnitMap um, const AdamScal& s) {
    const int64_t lo = 4 * k - um.sh;
    const int64_t e0 = lo < 0 ? 0 : lo;
    const int64_t e1 = (lo + 4) < n ? (lo + 4) : n;
    adam_unit(p, g, m, v, e0, (int)(e1 - e0), um.vec != 0, s);
}

static inline UnitMap unit_map(const void* p, const void* g, const void* m, const void* v) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p) & 15;
    UnitMap um{0, 0};
    if ((a & 3) == 0 && (reinterpret_cast<uintptr_t>(g) & 15) == a && (reinterpret_cast<uintptr_t>(m) & 15) == a &&
        (reinterpret_cast<uintptr_t>(v) & 15) == a) {
        um.vec = 1;
        um.sh = (int)(a >> 2);  // head = (4 - a/4) & 3 elements, so sh = a/4
    }
    return um;
}

__global__ void __launch_bounds__(kOThreads)
    k_adam(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m, float* __restrict__ v,
           int64_t n, UnitMap um, AdamScal s) {
    const int64_t units = adam_units(n, um.sh);
    const int64_t stride = (int64_t)gridDim.x * kOThreads;
    for (int64_t u = (int64_t)blockIdx.x * kOThreads + threadIdx.x; u < units; u += stride)
        adam_unit_k(p, g, m, v, n, u, um, s);
}

// The common case of k_adam (all four tensors 16-byte aligned, sh == 0): thread q takes quad q,
// with no unit arithmetic; the last n % 4 elements go to the thread after the last quad.
__global__ void __launch_bounds__(kOThreads)
    k_adam_al(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m, float* __restrict__ v,
              int64_t n, AdamScal s) {
    const int64_t q = (int64_t)blockIdx.x * kOThreads + threadIdx.x;
    const int64_t nq = n >> 2;
    if (q < nq) {
        adam_unit(p, g, m, v, 4 * q, 4, true, s);
    } else if (q == nq && (n & 3) != 0) {
        adam_unit(p, g, m, v, 4 * q, (int)(n & 3), false, s);
    }
}

// 48 bytes: the first unit of the tensor in the launch's concatenated unit space is a multiple
// of 64 (each tensor starts on a wave), so its low six bits carry the unit map: bits 0-1 sh,
// bit 2 vec.
struct AdamTensor {
    float* p;
    const float* g;
    float* m;
    float* v;
    int64_t n;
    int64_t u0m;
    __host__ __device__ int64_t unit0() const { return u0m & ~int64_t(63); }
    __host__ __device__ UnitMap um() const { return UnitMap{(int)(u0m & 3), (int)((u0m >> 2) & 1)}; }
};
static_assert(sizeof(AdamTensor) == 48, "table entry size");

// Up to kAdamPerLaunch tensors travel by value in the kernel arguments (3.8 KB of the 4 KB
// they may take), so a launch needs no device-side table. (With 56-byte entries and 64 per
// launch, 400 tensors of 1..2^18 elements took seven launches instead of five.)
constexpr int kAdamPerLaunch = 80;
struct AdamTable {
    AdamTensor t[kAdamPerLaunch];
    int32_t nt;
};

// Each tensor starts on a wave boundary of the concatenated quad space (unit0 a multiple of
// 64), so a wave belongs to one tensor: the search runs once per wave on wave-uniform values
// (scalar loads from the kernel arguments), and lanes past the tensor's end idle.
__global__ void __launch_bounds__(kOThreads) k_adam_multi(AdamTable tab, int64_t units, AdamScal s) {
    const int64_t stride = (int64_t)gridDim.x * kOThreads;
    const int wid = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = (int)(threadIdx.x & 63);
    for (int64_t uw = (int64_t)blockIdx.x * kOThreads + wid * 64; uw < units; uw += stride) {
        int lo = 0, hi = tab.nt - 1;  // the last tensor whose unit0 <= uw
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (tab.t[mid].unit0() <= uw) lo = mid;
            else hi = mid - 1;
        }
        const AdamTensor& t = tab.t[lo];
        const UnitMap um = t.um();
        const int64_t k = uw - t.unit0() + lane;
        if (k < adam_units(t.n, um.sh)) adam_unit_k(t.p, t.g, t.m, t.v, t.n, k, um, s);
    }
}

static inline unsigned grid_units(int64_t units) { return (unsigned)grid_blocks(units, kOThreads); }

// k_adam_al gives every quad, and the tail after the last one, a thread of its own with no
// loop, so it takes the aligned tensors whose quads fit one dispatch; every other tensor goes
// through k_adam, which loops over its grid.
static LaunchShape adam_shape(int64_t n, UnitMap um) {
    const int64_t al_items = (n >> 2) + 1;
    if (um.vec && um.sh == 0 && al_items <= max_grid_blocks(kOThreads) * kOThreads)
        return LaunchShape{0, kOThreads, grid_blocks(al_items, kOThreads), 1};
    return LaunchShape{1, kOThreads, grid_blocks(adam_units(n, um.sh), kOThreads), 1};
}

LaunchShape adam_launch(int64_t n, bool aligned) { return adam_shape(n, UnitMap{0, aligned ? 1 : 0}); }

static int check_hyper(const char* what, float lr, float b1, float b2, float eps, int64_t iter) {
    if (iter < 1) return fail(MH_ERR_INVALID, "%s: iter %lld (Adam.step counts from 1)", what, (long long)iter);
    if (!std::isfinite(lr) || !std::isfinite(b1) || !std::isfinite(b2) || !std::isfinite(eps))
        return fail(MH_ERR_INVALID, "%s: non-finite hyper-parameter", what);
    return MH_OK;
}

}  // namespace mh

using namespace mh;

extern "C" {

int mh_adam_step(float* param, const float* grad, float* m, float* v, int64_t n, float lr, float beta1,
                 float beta2, float eps, int64_t iter) {
    MH_TRACE("mh_adam_step");
    MH_TRY(check_hyper("mh_adam_step", lr, beta1, beta2, eps, iter));
    if (n < 0) return fail(MH_ERR_INVALID, "mh_adam_step: negative count");
    if (n == 0) return MH_OK;
    if (!param || !grad || !m || !v) return fail(MH_ERR_NULL, "mh_adam_step: null tensor");
    MH_TRY(require_init());
    const AdamScal s = adam_scalars(lr, beta1, beta2, eps, iter);
    const UnitMap um = unit_map(param, grad, m, v);
    const LaunchShape ls = adam_shape(n, um);
    if (ls.kernel == 0)
        hipLaunchKernelGGL(k_adam_al, dim3((unsigned)ls.blocks), dim3(ls.threads), 0, ctx().stream, param, grad, m, v,
                           n, s);
    else
        hipLaunchKernelGGL(k_adam, dim3((unsigned)ls.blocks), dim3(ls.threads), 0, ctx().stream, param, grad, m, v, n,
                           um, s);
    return finish("mh_adam_step");
}

int mh_adam_step_multi(int64_t ntensors, float* const* params, const float* const* grads, float* const* m,
                       float* const* v, const int64_t* sizes, float lr, float beta1, float beta2, float eps,
                       int64_t iter) {
    MH_TRACE("mh_adam_step_multi");
    MH_TRY(check_hyper("mh_adam_step_multi", lr, beta1, beta2, eps, iter));
    if (ntensors < 0) return fail(MH_ERR_INVALID, "mh_adam_step_multi: negative tensor count");
    if (ntensors == 0) return MH_OK;
    if (!params || !grads || !m || !v || !sizes) return fail(MH_ERR_NULL, "mh_adam_step_multi: null table");
    for (int64_t i = 0; i < ntensors; ++i) {  // validate everything before any launch
        if (sizes[i] < 0) return fail(MH_ERR_INVALID, "mh_adam_step_multi: negative size of tensor %lld", (long long)i);
        if (sizes[i] > 0 && (!params[i] || !grads[i] || !m[i] || !v[i]))
            return fail(MH_ERR_NULL, "mh_adam_step_multi: null pointer in tensor %lld", (long long)i);
    }
    MH_TRY(require_init());
    const AdamScal s = adam_scalars(lr, beta1, beta2, eps, iter);
    AdamTable tab;
    int64_t i = 0;
    while (i < ntensors) {
        tab.nt = 0;
        int64_t units = 0;
        for (; i < ntensors && tab.nt < kAdamPerLaunch; ++i) {
            if (sizes[i] == 0) continue;
            AdamTensor& t = tab.t[tab.nt++];
            t.p = params[i];
            t.g = grads[i];
            t.m = m[i];
            t.v = v[i];
            t.n = sizes[i];
            const UnitMap um = unit_map(t.p, t.g, t.m, t.v);
            t.u0m = units | um.sh | (um.vec << 2);  // units: a multiple of 64
            units += (adam_units(t.n, um.sh) + 63) & ~int64_t(63);  // next tensor starts on a wave
        }
        if (tab.nt > 0)
            hipLaunchKernelGGL(k_adam_multi, dim3(grid_units(units)), dim3(kOThreads), 0, ctx().stream, tab, units, s);
    }
    return finish("mh_adam_step_multi");
}

}  // extern "C"
