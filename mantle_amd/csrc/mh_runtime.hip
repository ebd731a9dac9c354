// mh_runtime.hip -- context, errors, memory, events, shape validation and launch planning.
#include <dlfcn.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <string>

#include "mh_internal.h"

// Scratch of the no-allocation entry points: 16 MiB of device memory per GPU, reserved when the
// library's code object loads on that GPU and held until the process ends. Host code never
// uses this name as an address: mh_init resolves the device's copy with hipGetSymbolAddress.
static __device__ __align__(256) float noalloc_scratch_buf[mh::kNoAllocScratchBytes / sizeof(float)];

namespace mh {

constexpr int kMaxDevices = 64;
static float* g_noalloc_ptr[kMaxDevices];  // per device: the address of noalloc_scratch_buf there

int noalloc_scratch(size_t bytes, float** out) {
    if (bytes > kNoAllocScratchBytes)
        return fail(MH_ERR_OVERFLOW, "needs %zu bytes of scratch, more than the %zu of the no-allocation scratch",
                    bytes, kNoAllocScratchBytes);
    MH_TRY(require_init());
    float* p = g_noalloc_ptr[ctx().device];
    if (!p) return fail(MH_ERR_NOT_INIT, "the no-allocation scratch was not resolved on device %d", ctx().device);
    *out = p;
    return MH_OK;
}

Context& ctx() {
    static Context c;
    return c;
}

static thread_local char g_err[512] = "";
static long g_fail_at = -2;  // -2: env not read yet, -1: no injection
static long g_hip_calls = 0;  // MH_HIP calls since the environment was last read

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

RoctxPushFn g_roctx_push = nullptr;
RoctxPopFn g_roctx_pop = nullptr;

void trace_init() {
    const char* s = getenv("MANTLE_HIP_TRACE");
    if (!s || s[0] == '\0' || s[0] == '0') {
        g_roctx_push = nullptr;
        g_roctx_pop = nullptr;
        return;
    }
    static void* h = nullptr;
    if (!h) h = dlopen("librocprofiler-sdk-roctx.so.1", RTLD_NOW | RTLD_LOCAL);
    if (!h) h = dlopen("libroctx64.so.4", RTLD_NOW | RTLD_LOCAL);
    if (!h) return;  // no roctx: tracing stays off
    auto push = reinterpret_cast<RoctxPushFn>(dlsym(h, "roctxRangePushA"));
    auto pop = reinterpret_cast<RoctxPopFn>(dlsym(h, "roctxRangePop"));
    if (push && pop) {
        g_roctx_pop = pop;
        g_roctx_push = push;
    }
}

static const char* op_name(int op) {
    switch (op) {
        case MH_ADD: return "ADD";
        case MH_SUB: return "SUB";
        case MH_MUL: return "MUL";
        case MH_DIV: return "DIV";
        case MH_EXP: return "EXP";
        case MH_LOG: return "LOG";
        case MH_POW: return "POW";
        case MH_SUM: return "SUM";
        case MH_MEAN: return "MEAN";
        case MH_MAX: return "MAX";
        case MH_SIGMOID: return "SIGMOID";
        case MH_RELU: return "RELU";
        case MH_TANH: return "TANH";
        default: return "?";
    }
}

void trace_push_op(const char* fn, int op) {
    thread_local char name[96];
    snprintf(name, sizeof(name), "%s(%s)", fn, op_name(op));
    g_roctx_push(name);
}

static void read_fail_env() {
    const char* s = getenv("MANTLE_HIP_FAIL_AT");
    g_fail_at = s ? atol(s) : -1;
    g_hip_calls = 0;
}

int hip_inject(const char* what) {
    if (g_fail_at == -2) read_fail_env();
    ++g_hip_calls;
    if (g_fail_at > 0 && g_hip_calls == g_fail_at)
        return fail(MH_ERR_HIP, "%s: injected failure (MANTLE_HIP_FAIL_AT=%ld)", what, g_fail_at);
    return MH_OK;
}

int hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(MH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return MH_OK;
}

int require_init() {
    if (!ctx().initialized) return fail(MH_ERR_NOT_INIT, "mh_init has not been called");
    return MH_OK;
}

int finish(const char* what) {
    MH_HIP(hipGetLastError());
    if (!(ctx().flags & MH_INIT_ASYNC)) {
        hipError_t e = hipStreamSynchronize(ctx().stream);
        if (e != hipSuccess) return fail(MH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    }
    return MH_OK;
}

// Gives up a library buffer that is being replaced: freed, or retired while a captured graph
// may still use it.
static int drop_buffer(void* buf) {
    Context& c = ctx();
    if (!buf) return MH_OK;
    if (c.graphs_live > 0) {
        c.retired.push_back(buf);
        return MH_OK;
    }
    int rc = hip_inject("hipStreamSynchronize");
    if (rc == MH_OK) rc = hip_check(hipStreamSynchronize(c.stream), "hipStreamSynchronize");
    if (rc == MH_OK) rc = hip_inject("hipFree");
    if (rc == MH_OK) rc = hip_check(hipFree(buf), "hipFree");
    if (rc != MH_OK) c.retired.push_back(buf);  // not freed here: mh_shutdown frees it
    return rc;
}

static int free_retired() {
    Context& c = ctx();
    if (c.retired.empty()) return MH_OK;
    if (c.stream) MH_HIP(hipStreamSynchronize(c.stream));
    int rc = MH_OK;
    for (void* p : c.retired) {
        const int r = hip_check(hipFree(p), "hipFree(retired library buffer)");
        if (rc == MH_OK) rc = r;
    }
    c.retired.clear();
    return rc;
}

void graph_retain() { ++ctx().graphs_live; }

int graph_release(uint64_t epoch) {
    Context& c = ctx();
    if (!c.initialized || epoch != c.epoch || c.graphs_live <= 0) return MH_OK;
    if (--c.graphs_live == 0) return free_retired();
    return MH_OK;
}

static int grow(void** buf, size_t* have, size_t bytes, void** out) {
    if (bytes > *have) {
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        // While a captured graph exists, the replaced buffer is retired, not freed, until the
        // last graph goes: growing at least twofold then keeps every retired buffer together
        // smaller than the live one, whatever sequence of sizes the eager calls ask for.
        if (ctx().graphs_live > 0 && want < 2 * *have) want = 2 * *have;
        want = (want + 255) & ~(size_t)255;
        if (*buf) {
            void* old = *buf;
            *buf = nullptr;
            *have = 0;
            MH_TRY(drop_buffer(old));
        }
        MH_HIP(hipMalloc(buf, want));
        *have = want;
    }
    *out = *buf;
    return MH_OK;
}

int scratch(size_t bytes, void** out) { return grow(&ctx().scratch, &ctx().scratch_bytes, bytes, out); }
int stage(size_t bytes, void** out) { return grow(&ctx().stage, &ctx().stage_bytes, bytes, out); }

static int launch_fill(float* t, float v, int64_t n);

int tickets(int64_t n, uint32_t** out) {
    Context& c = ctx();
    if (n > c.ntickets) {
        int64_t want = n < 65536 ? 65536 : n;
        if (c.graphs_live > 0 && want < 2 * c.ntickets) want = 2 * c.ntickets;  // as in grow()
        if (c.tickets) {
            void* old = c.tickets;
            c.tickets = nullptr;
            c.ntickets = 0;
            MH_TRY(drop_buffer(old));  // a retired ticket buffer stays all-zero: kernels reset what they take
        }
        uint32_t* nb = nullptr;
        MH_HIP(hipMalloc(reinterpret_cast<void**>(&nb), (size_t)want * sizeof(uint32_t)));
        // all-zero bits: a fill kernel of 0.0f (no memset node if a caller captures a graph)
        const uint64_t saved = c.flags;
        c.flags |= MH_INIT_ASYNC;
        const int rc = launch_fill(reinterpret_cast<float*>(nb), 0.0f, want);
        c.flags = saved;
        if (rc != MH_OK) {  // never keep counters that may not be zero
            (void)hipStreamSynchronize(c.stream);
            (void)hipFree(nb);
            return rc;
        }
        c.tickets = nb;
        c.ntickets = want;
    }
    *out = c.tickets;
    return MH_OK;
}

// ---------------------------------------------------------------------------------------
// shapes
// ---------------------------------------------------------------------------------------
int check_shape(const mh_shape& s, const char* name) {
    if (s.rank < 1 || s.rank > MH_MAX_RANK)
        return fail(MH_ERR_RANK, "%s: rank %d outside 1..%d", name, s.rank, MH_MAX_RANK);
    int64_t n = 1;
    for (int i = 0; i < s.rank; ++i) {
        if (s.dims[i] < 0) return fail(MH_ERR_RANK, "%s: negative dim %lld", name, (long long)s.dims[i]);
        if (s.dims[i] > 0 && n > ((int64_t)1 << 46) / s.dims[i])
            return fail(MH_ERR_OVERFLOW, "%s: element count overflows", name);
        n *= s.dims[i];
    }
    return MH_OK;
}

int64_t numel(const mh_shape& s) {
    int64_t n = 1;
    for (int i = 0; i < s.rank; ++i) n *= s.dims[i];
    return n;
}

bool shape_eq(const mh_shape& a, const mh_shape& b) {
    if (a.rank != b.rank) return false;
    for (int i = 0; i < a.rank; ++i)
        if (a.dims[i] != b.dims[i]) return false;
    return true;
}

bool is_scalar_shape(const mh_shape& s) { return s.rank == 1 && s.dims[0] == 1; }

// broadcast_shapes, tensorutils.mojo:88-127; a mismatch is an error here.
int broadcast_shapes(const mh_shape& s1, const mh_shape& s2, mh_shape* out) {
    int ndim = s1.rank > s2.rank ? s1.rank : s2.rank;
    int diff = s1.rank > s2.rank ? s1.rank - s2.rank : s2.rank - s1.rank;
    const mh_shape& big = s1.rank > s2.rank ? s1 : s2;
    const mh_shape& small = s1.rank > s2.rank ? s2 : s1;
    mh_shape r;
    memset(&r, 0, sizeof r);
    r.rank = ndim;
    for (int i = ndim - 1; i >= diff; --i) {
        int64_t a = big.dims[i], b = small.dims[i - diff];
        if (a == b) r.dims[i] = a;
        else if (a == 1 || b == 1) r.dims[i] = a * b;
        else return fail(MH_ERR_SHAPE, "shapes do not broadcast (dim %d: %lld vs %lld)", i,
                         (long long)a, (long long)b);
    }
    for (int i = diff - 1; i >= 0; --i) r.dims[i] = big.dims[i];
    *out = r;
    return MH_OK;
}

bool broadcasts_to(const mh_shape& small, const mh_shape& big) {
    if (small.rank > big.rank) return false;
    int diff = big.rank - small.rank;
    for (int i = 0; i < small.rank; ++i) {
        int64_t a = small.dims[i], b = big.dims[i + diff];
        if (a != b && a != 1) return false;
    }
    return true;
}

// broadcast_calculate_strides, tensorutils.mojo:149-175.
void broadcast_strides(int size, const mh_shape& shape, int64_t* strides) {
    int diff = size - shape.rank;
    for (int i = 0; i < size; ++i) strides[i] = 0;
    int64_t stride = 1;
    for (int i = shape.rank - 1; i >= 0; --i) {
        if (shape.dims[i] != 1) {
            strides[i + diff] = stride;
            stride *= shape.dims[i];
        }
    }
}

mh_shape reduced_shape(const mh_shape& s, int axis) {
    mh_shape r;
    memset(&r, 0, sizeof r);
    if (axis < 0) {
        r.rank = 1;
        r.dims[0] = 1;
        return r;
    }
    r = s;
    r.dims[axis] = 1;
    return r;
}

mh_shape flat_shape(int64_t n) {
    mh_shape r;
    memset(&r, 0, sizeof r);
    r.rank = 1;
    r.dims[0] = n;
    return r;
}

int build_elw_plan(const mh_shape& out, int nin, const mh_shape* in, ElwPlan* plan) {
    ElwPlan p;
    p.n = numel(out);
    p.nin = nin;
    const int r = out.rank;
    int64_t st[kMaxIn][MH_MAX_RANK];
    for (int k = 0; k < nin; ++k) {
        if (!broadcasts_to(in[k], out)) return fail(MH_ERR_SHAPE, "input %d does not broadcast to the output", k);
        broadcast_strides(r, in[k], st[k]);
    }
    // drop size-1 dims, then merge (outer, inner) pairs contiguous for every input
    int64_t dims[MH_MAX_RANK];
    int64_t cst[kMaxIn][MH_MAX_RANK];
    int cr = 0;
    for (int d = 0; d < r; ++d) {
        if (out.dims[d] == 1) continue;
        if (cr > 0) {
            bool merge = true;
            for (int k = 0; k < nin; ++k)
                if (cst[k][cr - 1] != st[k][d] * out.dims[d]) merge = false;
            if (merge) {
                dims[cr - 1] *= out.dims[d];
                for (int k = 0; k < nin; ++k) cst[k][cr - 1] = st[k][d];
                continue;
            }
        }
        dims[cr] = out.dims[d];
        for (int k = 0; k < nin; ++k) cst[k][cr] = st[k][d];
        ++cr;
    }
    if (cr == 0) {  // one element
        dims[0] = 1;
        for (int k = 0; k < nin; ++k) cst[k][0] = 0;
        cr = 1;
    }
    p.rank = cr;
    for (int d = 0; d < cr; ++d) p.dims[d] = dims[d];
    int64_t contig[MH_MAX_RANK];
    {
        int64_t s = 1;
        for (int d = cr - 1; d >= 0; --d) {
            contig[d] = s;
            s *= dims[d];
        }
    }
    p.vec_ok = (dims[cr - 1] % 4 == 0) ? 1 : 0;
    for (int k = 0; k < nin; ++k) {
        bool full = true, zero = true;
        for (int d = 0; d < cr; ++d) {
            p.st[k][d] = cst[k][d];
            if (dims[d] > 1 && cst[k][d] != contig[d]) full = false;
            if (dims[d] > 1 && cst[k][d] != 0) zero = false;
        }
        if (numel(in[k]) == 1) zero = true;
        p.kind[k] = zero ? IN_SCALAR : (full ? IN_FULL : IN_BCAST);
        if (p.kind[k] == IN_BCAST) {
            p.any_bcast = 1;
            if (cst[k][cr - 1] != 0 && cst[k][cr - 1] != 1) p.vec_ok = 0;
        }
    }
    if (p.n < ((int64_t)1 << 31))
        for (int d = 0; d < cr; ++d) p.fd[d] = make_fastdiv((uint32_t)dims[d]);
    *plan = p;
    return MH_OK;
}

// ---------------------------------------------------------------------------------------
// fill kernel (also used for zeroing: a kernel, so it can live inside captured graphs)
// ---------------------------------------------------------------------------------------
// A thread per quad, no grid loop (a launch covers at most kMaxLaunchQuads quads); the first
// thread also writes the n % 4 tail.
__global__ void __launch_bounds__(64) k_fill(float* __restrict__ t, float v, int64_t n) {
    const int64_t nq = n >> 2;
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < nq) st_nt4(t, q, make_float4(v, v, v, v));
    if (q == 0)
        for (int64_t j = nq << 2; j < n; ++j) t[j] = v;
}

__global__ void __launch_bounds__(256) k_fill_scalar(float* __restrict__ t, float v, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) t[i] = v;
}

__global__ void __launch_bounds__(64) k_copy(float4* __restrict__ dst, const float4* __restrict__ src, int64_t nq) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < nq) st_ntv(reinterpret_cast<float*>(dst), q, ld_ntv(reinterpret_cast<const float*>(src), q));
}

// Counter-based SplitMix64 (Steele, Lea & Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014): element i of stream `seed` is mix(seed * golden + (i + 1) * golden).
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void __launch_bounds__(256) k_rand(float* __restrict__ t, int64_t n, uint64_t seed, float p, float q,
                                              int normal) {
    const uint64_t g = 0x9E3779B97F4A7C15ull;
    const uint64_t base = splitmix64(seed * g + 0x632BE59BD9B4E019ull);
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint64_t r = splitmix64(base + (uint64_t)(i + 1) * g);
        if (!normal) {  // U(p, q): 24-bit uniform in [0, 1)
            const float u = (float)(uint32_t)(r >> 40) * 5.9604644775390625e-8f;
            t[i] = p + u * (q - p);
        } else {  // N(p, q): Box-Muller in fp64 on two 26-bit halves, q is the std
            const double u1 = ((double)(r >> 38) + 1.0) * 3.725290298461914e-9;  // (0, 1]
            const double u2 = (double)((r >> 12) & 0x3ffffffull) * 1.4901161193847656e-8;
            const double z = sqrt(-2.0 * log(u1)) * cospi(2.0 * u2);
            t[i] = (float)(p + q * z);
        }
    }
}

// One-wavefront workgroups. Aligned: one quad per thread, at most kMaxLaunchQuads quads per
// launch. Unaligned (k_fill_scalar): one element per thread, a grid loop beyond one dispatch.
LaunchShape fill_launch(int64_t n, bool aligned) {
    if (!aligned) return LaunchShape{1, 64, grid_blocks(n, 64), 1};
    const int64_t nq = n >> 2;
    return LaunchShape{0, 64, grid_blocks(nq < kMaxLaunchQuads ? nq : kMaxLaunchQuads, 64), launch_count(nq)};
}

// One-wavefront workgroups, one quad per thread, at most kMaxLaunchQuads quads per launch.
LaunchShape copy_launch(int64_t nquads) {
    return LaunchShape{0, 64, grid_blocks(nquads < kMaxLaunchQuads ? nquads : kMaxLaunchQuads, 64),
                       launch_count(nquads)};
}

static int launch_fill(float* t, float v, int64_t n) {
    if (n == 0) return MH_OK;
    if (!t) return fail(MH_ERR_NULL, "fill: null tensor");
    MH_TRY(require_init());
    const bool al = (reinterpret_cast<uintptr_t>(t) & 15) == 0;
    if (al) {
        for (int64_t off = 0; off < n; off += 4 * kMaxLaunchQuads) {
            const int64_t cnt = n - off < 4 * kMaxLaunchQuads ? n - off : 4 * kMaxLaunchQuads;
            const LaunchShape ls = fill_launch(cnt, true);
            hipLaunchKernelGGL(k_fill, dim3((unsigned)ls.blocks), dim3(ls.threads), 0, ctx().stream, t + off, v, cnt);
        }
    } else {
        const LaunchShape ls = fill_launch(n, false);
        hipLaunchKernelGGL(k_fill_scalar, dim3((unsigned)ls.blocks), dim3(ls.threads), 0, ctx().stream, t, v, n);
    }
    return finish("fill");
}

}  // namespace mh

using namespace mh;

extern "C" {

const char* mh_last_error(void) { return g_err; }

const char* mh_status_string(int s) {
    switch (s) {
        case MH_OK: return "ok";
        case MH_ERR_INVALID: return "invalid argument";
        case MH_ERR_SHAPE: return "shape mismatch";
        case MH_ERR_RANK: return "bad rank or dim";
        case MH_ERR_NULL: return "null pointer";
        case MH_ERR_OP: return "unsupported op";
        case MH_ERR_NOT_INIT: return "not initialised";
        case MH_ERR_HIP: return "HIP runtime error";
        case MH_ERR_NO_DEVICE: return "no usable device";
        case MH_ERR_OVERFLOW: return "size overflow";
        default: return "unknown status";
    }
}

int mh_device_count(int* count) {
    if (!count) return fail(MH_ERR_NULL, "mh_device_count: null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return MH_OK;
}

int mh_init(int device, uint64_t flags) {
    Context& c = ctx();
    read_fail_env();  // failure injection counts from here
    trace_init();
    if (c.initialized) {
        if (c.device == device) {
            c.flags = flags;
            return MH_OK;
        }
        return fail(MH_ERR_INVALID, "mh_init: already initialised on device %d", c.device);
    }
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
        return fail(MH_ERR_NO_DEVICE, "mh_init: no HIP device visible");
    if (device < 0 || device >= n) return fail(MH_ERR_NO_DEVICE, "mh_init: device %d of %d", device, n);
    MH_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    MH_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(MH_ERR_NO_DEVICE, "mh_init: device %d is %s, this library is built for gfx950",
                    device, prop.gcnArchName);
    if (device >= kMaxDevices) return fail(MH_ERR_NO_DEVICE, "mh_init: device %d beyond %d", device, kMaxDevices);
    if (!g_noalloc_ptr[device]) {  // this device's copy of the no-allocation scratch (device current)
        void* p = nullptr;
        MH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch_buf)));
        g_noalloc_ptr[device] = static_cast<float*>(p);
    }
    MH_HIP(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
    c.num_cus = prop.multiProcessorCount;
    c.device = device;
    c.flags = flags;
    ++c.epoch;
    c.initialized = true;
    return MH_OK;
}

int mh_shutdown(void) {
    Context& c = ctx();
    if (!c.initialized) return MH_OK;
    MH_HIP(hipStreamSynchronize(c.stream));
    if (c.scratch) MH_HIP(hipFree(c.scratch));
    c.scratch = nullptr;
    c.scratch_bytes = 0;
    if (c.stage) MH_HIP(hipFree(c.stage));
    c.stage = nullptr;
    c.stage_bytes = 0;
    if (c.tickets) MH_HIP(hipFree(c.tickets));
    c.tickets = nullptr;
    c.ntickets = 0;
    MH_TRY(free_retired());  // graphs captured before this point can no longer replay (epoch)
    c.graphs_live = 0;
    MH_HIP(hipStreamDestroy(c.stream));
    c.stream = nullptr;
    c.initialized = false;
    c.device = -1;
    return MH_OK;
}

int mh_sync(void) {
    MH_TRY(require_init());
    MH_HIP(hipStreamSynchronize(ctx().stream));
    return MH_OK;
}

int mh_malloc(void** dptr, size_t bytes) {
    if (!dptr) return fail(MH_ERR_NULL, "mh_malloc: null out pointer");
    *dptr = nullptr;
    MH_TRY(require_init());
    if (bytes == 0) bytes = 4;
    MH_HIP(hipMalloc(dptr, bytes));
    return MH_OK;
}

int mh_free(void* dptr) {
    if (!dptr) return MH_OK;
    MH_TRY(require_init());
    MH_HIP(hipStreamSynchronize(ctx().stream));
    MH_HIP(hipFree(dptr));
    return MH_OK;
}

int mh_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    MH_TRACE("mh_memcpy_h2d");
    if (bytes == 0) return MH_OK;
    if (!dst || !src) return fail(MH_ERR_NULL, "mh_memcpy_h2d: null pointer");
    MH_TRY(require_init());
    MH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx().stream));
    MH_HIP(hipStreamSynchronize(ctx().stream));
    return MH_OK;
}

int mh_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    MH_TRACE("mh_memcpy_d2h");
    if (bytes == 0) return MH_OK;
    if (!dst || !src) return fail(MH_ERR_NULL, "mh_memcpy_d2h: null pointer");
    MH_TRY(require_init());
    MH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx().stream));
    MH_HIP(hipStreamSynchronize(ctx().stream));
    return MH_OK;
}

int mh_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    MH_TRACE("mh_memcpy_d2d");
    if (bytes == 0) return MH_OK;
    if (!dst || !src) return fail(MH_ERR_NULL, "mh_memcpy_d2d: null pointer");
    MH_TRY(require_init());
    if (((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | bytes) & 15) == 0) {
        const int64_t nq_all = (int64_t)(bytes >> 4);
        for (int64_t off = 0; off < nq_all; off += kMaxLaunchQuads) {
            const int64_t nq = nq_all - off < kMaxLaunchQuads ? nq_all - off : kMaxLaunchQuads;
            const LaunchShape ls = copy_launch(nq);
            hipLaunchKernelGGL(k_copy, dim3((unsigned)ls.blocks), dim3(ls.threads), 0, ctx().stream,
                               reinterpret_cast<float4*>(dst) + off, reinterpret_cast<const float4*>(src) + off, nq);
        }
    } else {
        MH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx().stream));
    }
    return finish("mh_memcpy_d2d");
}

int mh_fill(float* t, float v, int64_t n) {
    MH_TRACE("mh_fill");
    if (n < 0) return fail(MH_ERR_INVALID, "mh_fill: negative count");
    return launch_fill(t, v, n);
}

int mh_zero(float* t, int64_t n) {
    MH_TRACE("mh_zero");
    if (n < 0) return fail(MH_ERR_INVALID, "mh_zero: negative count");
    return launch_fill(t, 0.0f, n);
}

int mh_rand_uniform(float* t, int64_t n, uint64_t seed, float lo, float hi) {
    MH_TRACE("mh_rand_uniform");
    if (n < 0) return fail(MH_ERR_INVALID, "mh_rand_uniform: negative count");
    if (n == 0) return MH_OK;
    if (!t) return fail(MH_ERR_NULL, "mh_rand_uniform: null tensor");
    MH_TRY(require_init());
    hipLaunchKernelGGL(k_rand, dim3(8192), dim3(256), 0, ctx().stream, t, n, seed, lo, hi, 0);
    return finish("mh_rand_uniform");
}

int mh_rand_normal(float* t, int64_t n, uint64_t seed, float mean, float std) {
    MH_TRACE("mh_rand_normal");
    if (n < 0) return fail(MH_ERR_INVALID, "mh_rand_normal: negative count");
    if (n == 0) return MH_OK;
    if (!t) return fail(MH_ERR_NULL, "mh_rand_normal: null tensor");
    MH_TRY(require_init());
    hipLaunchKernelGGL(k_rand, dim3(8192), dim3(256), 0, ctx().stream, t, n, seed, mean, std, 1);
    return finish("mh_rand_normal");
}

int mh_event_create(void** ev) {
    if (!ev) return fail(MH_ERR_NULL, "mh_event_create: null");
    MH_TRY(require_init());
    hipEvent_t e;
    MH_HIP(hipEventCreate(&e));
    *ev = (void*)e;
    return MH_OK;
}

int mh_event_destroy(void* ev) {
    if (!ev) return MH_OK;
    MH_HIP(hipEventDestroy((hipEvent_t)ev));
    return MH_OK;
}

int mh_event_record(void* ev) {
    if (!ev) return fail(MH_ERR_NULL, "mh_event_record: null");
    MH_TRY(require_init());
    MH_HIP(hipEventRecord((hipEvent_t)ev, ctx().stream));
    return MH_OK;
}

int mh_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (!ms || !start || !stop) return fail(MH_ERR_NULL, "mh_event_elapsed_ms: null");
    MH_HIP(hipEventSynchronize((hipEvent_t)stop));
    MH_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
    return MH_OK;
}

int mh_plan_binary(const mh_shape* psres, const mh_shape* psa, const mh_shape* psb, mh_plan_info* out) {
    MH_SHAPE_ARG(sres);
    MH_SHAPE_ARG(sa);
    MH_SHAPE_ARG(sb);
    if (!out) return fail(MH_ERR_NULL, "mh_plan_binary: null");
    MH_TRY(check_shape(sres, "res"));
    MH_TRY(check_shape(sa, "a"));
    MH_TRY(check_shape(sb, "b"));
    mh_shape bs;
    MH_TRY(broadcast_shapes(sa, sb, &bs));
    if (!shape_eq(bs, sres)) return fail(MH_ERR_SHAPE, "mh_plan_binary: res is not broadcast(a, b)");
    mh_shape in[2] = {sa, sb};
    ElwPlan p;
    MH_TRY(build_elw_plan(sres, 2, in, &p));
    memset(out, 0, sizeof *out);
    if (p.any_bcast) out->kind = 3;
    else if (p.kind[1] == IN_SCALAR && p.kind[0] != IN_SCALAR) out->kind = 1;
    else if (p.kind[0] == IN_SCALAR && p.kind[1] != IN_SCALAR) out->kind = 2;
    else out->kind = 0;
    out->rank = p.rank;
    for (int d = 0; d < p.rank; ++d) {
        out->dims[d] = p.dims[d];
        out->stride_a[d] = p.st[0][d];
        out->stride_b[d] = p.st[1][d];
    }
    return MH_OK;
}

int mh_plan_unbroadcast(const mh_shape* psgrad, const mh_shape* psrg, mh_reduce_plan_info* out) {
    MH_SHAPE_ARG(sgrad);
    MH_SHAPE_ARG(srg);
    if (!out) return fail(MH_ERR_NULL, "mh_plan_unbroadcast: null");
    MH_TRY(check_shape(sgrad, "grad"));
    MH_TRY(check_shape(srg, "rg"));
    return plan_unbroadcast(sgrad, srg, out);
}

int mh_plan_launch(int32_t what, int64_t n, mh_launch_info* out) {
    if (!out) return fail(MH_ERR_NULL, "mh_plan_launch: null");
    if (n < 0) return fail(MH_ERR_INVALID, "mh_plan_launch: negative count");
    LaunchShape ls;
    switch (what) {
        case MH_LAUNCH_FILL: ls = fill_launch(n, true); break;
        case MH_LAUNCH_FILL_UNALIGNED: ls = fill_launch(n, false); break;
        case MH_LAUNCH_COPY: ls = copy_launch(n >> 2); break;
        case MH_LAUNCH_SAME_SHAPE: ls = elw_same_launch(n); break;
        case MH_LAUNCH_ADAM: ls = adam_launch(n, true); break;
        case MH_LAUNCH_ADAM_UNALIGNED: ls = adam_launch(n, false); break;
        case MH_LAUNCH_ROWS16: ls = row16_launch(n); break;
        default: return fail(MH_ERR_INVALID, "mh_plan_launch: unknown launch %d", what);
    }
    out->kernel = ls.kernel;
    out->threads = ls.threads;
    out->blocks = ls.blocks;
    out->launches = ls.launches;
    return MH_OK;
}

}  // extern "C"
