// mh_fused.hip -- graph-level entry points that cover several forward_op / backward_op
// calls of one graph pattern: bias ADD followed by RELU (a Linear layer's bias + activation,
// or an NCHW per-channel bias).
//
// Forward: one pass reads x (and the small bias) and writes y = x + bias and r = relu(y):
// 12 B per element instead of the 16 B of two separate ops.
// Backward: with x viewed as [N, C, S] and the bias indexed by C alone (NCHW bias
// [1, C, 1, 1], or any bias that is constant over a contiguous inner run S), every quad
// computes gy = g_y + relu'(y) * ug and accumulates it into grad_x (and g_y when the caller
// keeps it); grad_bias takes the per-channel sum of gy in a fixed order. Planes of at least
// kBFlat quads run as one flat stream whose waves write their planes' partial sums, added per
// channel by a short second launch (k_bias_relu_bwd_flat, k_bias_partials_comb); shorter
// planes run a wavefront per (plane group, chunk), whose last arrival per channel adds the
// channel's partials in the same launch (k_bias_relu_bwd_planes). Shapes outside that form run
// the op-by-op kernels.
#include "mh_internal.h"
#include "mh_math.h"

namespace mh {

constexpr int kFThreads = 256;     // backward: four waves per workgroup, one per plane group
constexpr int kFFwdThreads = 64;  // forward: flat quad streams, one-wavefront workgroups
constexpr int64_t kTicketStride = 32;  // one 128-byte line per channel counter

static inline bool al16f(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// y = x + bias (ADD.forward, basics.mojo:36-43), r = relu(y) (RELU.forward, mlops.mojo:92-97).
// Plan inputs: 0 = x (FULL), 1 = bias (BCAST, SCALAR or FULL). y, r, x 16-byte aligned.
template <bool INNER4, bool BIG>
__global__ void __launch_bounds__(kFFwdThreads)
    k_bias_relu_fwd4(float* __restrict__ y, float* __restrict__ r, const float* __restrict__ x,
                     const float* __restrict__ bias, ElwPlan pl) {
    const int inner = pl.rank - 1;
    const int64_t dinner = pl.dims[inner];
    const int kb = pl.kind[1];
    const float sb = kb == IN_SCALAR ? bias[0] : 0.0f;
    const int64_t nq = pl.n >> 2;
    const int64_t stride = (int64_t)gridDim.x * kFFwdThreads;
    for (int64_t q = (int64_t)blockIdx.x * kFFwdThreads + threadIdx.x; q < nq; q += stride) {
        const int64_t idx = q * 4;
        float bv[4];
        if (kb == IN_SCALAR) {
            bv[0] = bv[1] = bv[2] = bv[3] = sb;
        } else if (kb == IN_FULL) {
            const float4 t = ld_nt4(bias, q);
            bv[0] = t.x; bv[1] = t.y; bv[2] = t.z; bv[3] = t.w;
        } else {
            off_type<BIG> off[4][2];
            int64_t cin = 0, cp;
            bcast_decode<2, BIG, MH_MAX_RANK>(pl, idx, off[0], &cin, &cp);
            if (INNER4) {
                if (pl.st[1][inner] == 1) {
                    const float4 t = *reinterpret_cast<const float4*>(bias + off[0][1]);
                    bv[0] = t.x; bv[1] = t.y; bv[2] = t.z; bv[3] = t.w;
                } else {
                    bv[0] = bv[1] = bv[2] = bv[3] = bias[off[0][1]];
                }
            } else {
                bv[0] = bias[off[0][1]];
#pragma unroll
                for (int j = 1; j < 4; ++j) {
                    if (cin + j < dinner) {
                        bv[j] = bias[off[0][1] + j * pl.st[1][inner]];
                    } else {
                        int64_t c2, c3;
                        bcast_decode<2, BIG, MH_MAX_RANK>(pl, idx + j, off[j], &c2, &c3);
                        bv[j] = bias[off[j][1]];
                    }
                }
            }
        }
        const float4 xv = ld_nt4(x, q);
        float yv[4], rv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            yv[j] = comp(xv, j) + bv[j];
            rv[j] = mrelu(yv[j]);
        }
        st_nt4(y, q, make_float4(yv[0], yv[1], yv[2], yv[3]));
        st_nt4(r, q, make_float4(rv[0], rv[1], rv[2], rv[3]));
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        for (int64_t i = nq << 2; i < pl.n; ++i) {
            off_type<BIG> off1[2];
            int64_t c, c2;
            bcast_decode<2, BIG, MH_MAX_RANK>(pl, i, off1, &c, &c2);
            const float b = kb == IN_SCALAR ? sb : (kb == IN_FULL ? bias[i] : bias[off1[1]]);
            const float yy = x[i] + b;
            y[i] = yy;
            r[i] = mrelu(yy);
        }
    }
}

// Forward over [N, C, S] planes (S % 4 == 0, fewer than 2^31 elements; the bias indexed by C,
// or a scalar with C == 1): one quad per thread in flat order, its channel
// (q / (S / 4)) mod C from two fast divisions. No grid loop: one launch covers the tensor.
__global__ void __launch_bounds__(kFFwdThreads)
    k_bias_relu_fwd_planes(float* __restrict__ y, float* __restrict__ r, const float* __restrict__ x,
                           const float* __restrict__ bias, int64_t nq, uint32_t C, FastDiv fsq, FastDiv fc) {
    const int64_t q = (int64_t)blockIdx.x * kFFwdThreads + threadIdx.x;
    if (q < nq) {
        const uint32_t p = fdiv((uint32_t)q, fsq);
        const float bv = bias[p - fdiv(p, fc) * C];
        const vf4 xv = ld_ntv(x, q);
        vf4 yv, rv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            yv[j] = xv[j] + bv;  // ADD.forward
            rv[j] = mrelu(yv[j]);  // RELU.forward
        }
        st_ntv(y, q, yv);
        st_ntv(r, q, rv);
    }
}

// Backward over [N, C, S] planes, S % 4 == 0. One wavefront per (channel c, group g of G
// planes n = g * G .. g * G + G - 1, chunk k of QC quads of each plane, QC <= 1024), wave
// v = blockIdx.x * 4 + wave with c = v % C, g * K + k = v / C; the planes in order, four quads
// per lane in flight per stream:
//   rg = (y > 0 ? 1 : 0) * ug            RELU.backward (mlops.mojo:118-123)
//   g  = g_y + rg  (0 + rg without g_y)  accumulate_grad into the grad of y (ops.mojo:405)
//   grad_x = grad_x + g                  ADD backward_op, operand 0 (ops.mojo:457-461)
//   part[(g * K + k) * C + c] = sum of g over the wave's quads: each lane sums its quads in
//   order, plane by plane, then a butterfly across the wave.
// The bias gradient (ADD's operand-1 un-broadcast) completes in the same launch: every wave
// publishes its partial with an agent-scope store, waits for that store to complete, then
// takes a ticket on its channel; the wave that takes the channel's last ticket reads the
// channel's NG * K partials with agent-scope loads, adds them in a fixed order into
// grad_bias[c] and resets the ticket. No wave waits for another. G keeps the tickets per
// channel counter near kArrivals (arrivals on one counter serialize).
constexpr int64_t kArrivals = 64;

template <bool HAS_GY, bool HAS_GX, bool HAS_PART>
__global__ void __launch_bounds__(kFThreads)
    k_bias_relu_bwd_planes(float* __restrict__ gy, float* __restrict__ gx, const float* __restrict__ y,
                           const float* __restrict__ ug, int64_t N, int64_t C, int64_t Sq, int64_t QC, int64_t K,
                           int64_t G, int64_t nwaves, float* part, uint32_t* tickets, float* grad_bias) {
    const int lane = threadIdx.x & 63;
    const int64_t v = (int64_t)blockIdx.x * (kFThreads / 64) + (threadIdx.x >> 6);
    if (v >= nwaves) return;  // uniform per wavefront; no barrier follows
    const int64_t c = v % C, gk = v / C;
    const int64_t g = gk / K, k = gk - g * K;
    const int64_t rem = Sq - k * QC;
    const int64_t cnt = rem < QC ? rem : QC;
    const int64_t n0 = g * G, n1 = n0 + G < N ? n0 + G : N;
    constexpr int U = 4;
    float acc = 0.0f;
    for (int64_t n = n0; n < n1; ++n) {
        const int64_t q0 = (n * C + c) * Sq + k * QC;
        for (int64_t base = 0; base < cnt; base += 64 * U) {  // the lane's quads in ascending order
            vf4 yv[U], uv[U], gv[U], xv[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t i = base + lane + 64 * u;
                gv[u] = xv[u] = vf4{0.f, 0.f, 0.f, 0.f};
                if (i < cnt) {
                    yv[u] = ld_ntv(y, q0 + i);
                    uv[u] = ld_ntv(ug, q0 + i);
                    if (HAS_GY) gv[u] = ld_ntv(gy, q0 + i);
                    if (HAS_GX) xv[u] = ld_ntv(gx, q0 + i);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t i = base + lane + 64 * u;
                if (i >= cnt) continue;
                vf4 gg, o;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float rg = (yv[u][j] > 0.0f ? 1.0f : 0.0f) * uv[u][j];
                    gg[j] = gv[u][j] + rg;
                    o[j] = xv[u][j] + gg[j];
                }
                if (HAS_GY) st_ntv(gy, q0 + i, gg);
                if (HAS_GX) st_ntv(gx, q0 + i, o);
                if (HAS_PART) acc = (((acc + gg[0]) + gg[1]) + gg[2]) + gg[3];
            }
        }
    }
    if (HAS_PART) {
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
        const int64_t nper = nwaves / C;  // partials per channel: NG * K
        uint32_t ticket = 0;
        if (lane == 0) {
            // The partial is an agent-scope store (coherent across XCDs by itself), so the
            // ticket needs only to follow its completion, not a release of every earlier
            // store (which would write back this XCD's whole L2 once per wave).
            __hip_atomic_store(&part[gk * C + c], acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
            ticket = __hip_atomic_fetch_add(&tickets[c * kTicketStride], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        ticket = __shfl(ticket, 0);
        if (ticket == (uint32_t)(nper - 1)) {  // the channel's last partial: sum them all
            // acquire: the other waves' partials (stored before their tickets) are visible
            // to the loads below; one cache invalidate, on the last arriver only
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            const float gb =  // in flight with the partials (a vector load, not a scalar one waited for first)
                lane == 0 ? __hip_atomic_load(&grad_bias[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
            float s = 0.0f;
            for (int64_t i = lane; i < nper; i += 64)
                s = s + __hip_atomic_load(&part[i * C + c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int m = 32; m >= 1; m >>= 1) s = s + __shfl_xor(s, m);
            if (lane == 0) {
                grad_bias[c] = gb + s;
                __hip_atomic_store(&tickets[c * kTicketStride], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// Backward over [N, C, S] planes of at least 64 quads, as one flat stream: thread q owns quad q
// (one-wavefront workgroups), computes
//   rg = (y > 0 ? 1 : 0) * ug;  g = g_y + rg (0 + rg without g_y);  grad_x = grad_x + g
// (RELU backward_op, then ADD backward_op operand 0) and adds its quad's g in order. A wave
// covers 64 consecutive quads, so at most two planes (a plane has >= 64 quads): the wave sums
// the lanes of its first plane and those of the next plane, each with an xor butterfly. With
// SLOTS, planes span at most kPlaneSlots waves and the partials go to a slot table [C][N][8]:
// the first plane's partial to slot (wave - the plane's first wave), the next plane's to its
// slot 0 (this wave is that plane's first). Without SLOTS they go to part[2 w] and
// part[2 w + 1] (+0 when there is no next plane). k_bias_partials_comb (or _comb8 for the slot
// table) then adds every plane's wave partials into grad_bias in a fixed order.
constexpr int kBFlat = 64;
constexpr int kPlaneSlots = 8;  // a plane of Sq quads spans at most (Sq + 126) / 64 waves

template <bool HAS_GY, bool HAS_GX, bool HAS_PART, bool SLOTS>
__global__ void __launch_bounds__(kBFlat)
    k_bias_relu_bwd_flat(float* __restrict__ gy, float* __restrict__ gx, const float* __restrict__ y,
                         const float* __restrict__ ug, int64_t nq, uint32_t Sq, FastDiv fsq, float* part,
                         uint32_t N, uint32_t C, FastDiv fc) {
    const int lane = threadIdx.x;
    const int64_t q = (int64_t)blockIdx.x * kBFlat + lane;
    float sum = 0.0f;
    uint32_t plane = 0;
    if (q < nq) {
        const vf4 yv = ld_ntv(y, q), uv = ld_ntv(ug, q);
        vf4 gv = vf4{0.f, 0.f, 0.f, 0.f}, xv = gv;
        if (HAS_GY) gv = ld_ntv(gy, q);
        if (HAS_GX) xv = ld_ntv(gx, q);
        vf4 gg, o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float rg = (yv[j] > 0.0f ? 1.0f : 0.0f) * uv[j];  // RELU.backward (mlops.mojo:118-123)
            gg[j] = gv[j] + rg;                                    // accumulate into the grad of y
            o[j] = xv[j] + gg[j];                                  // ADD backward_op, operand 0
        }
        if (HAS_GY) st_ntv(gy, q, gg);
        if (HAS_GX) st_ntv(gx, q, o);
        sum = ((gg[0] + gg[1]) + gg[2]) + gg[3];
        plane = fdiv((uint32_t)q, fsq);
    }
    if (HAS_PART) {
        const uint32_t first = fdiv((uint32_t)((int64_t)blockIdx.x * kBFlat), fsq);
        float s0 = plane == first ? sum : 0.0f;
        float s1 = plane == first ? 0.0f : sum;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            s0 = s0 + __shfl_xor(s0, m);
            s1 = s1 + __shfl_xor(s1, m);
        }
        if (lane == 0) {
            if (SLOTS) {
                const uint32_t w = blockIdx.x;
                const uint32_t n0 = fdiv(first, fc), c0 = first - n0 * C;
                const uint32_t k0 = w - (uint32_t)(((uint64_t)first * Sq) / kBFlat);  // first plane's slot
                part[((size_t)c0 * N + n0) * kPlaneSlots + k0] = s0;
                const uint32_t next = first + 1;
                if ((uint64_t)next * Sq < (uint64_t)(w + 1) * kBFlat && (uint64_t)next * Sq < (uint64_t)nq) {
                    const uint32_t n1 = fdiv(next, fc), c1 = next - n1 * C;
                    part[((size_t)c1 * N + n1) * kPlaneSlots] = s1;
                }
            } else {
                part[2 * (int64_t)blockIdx.x] = s0;
                part[2 * (int64_t)blockIdx.x + 1] = s1;
            }
        }
    }
}

// grad_bias[c] += the sum of channel c's plane partials written by k_bias_relu_bwd_flat: one
// 256-thread workgroup per channel; thread t takes the channel's planes n = t, t + 256, ...,
// loading each plane's wave partials (at most 8 in flight, more one by one) and adding them in
// wave order; the plane sums add up per thread in order, then per wave (xor butterfly) and
// across the four waves in order.
constexpr int kCombPlaneWaves = 8;

__global__ void __launch_bounds__(256)
    k_bias_partials_comb(float* __restrict__ grad_bias, const float* __restrict__ part, int64_t N, int64_t C,
                         int64_t Sq) {
    __shared__ float ws[4];
    const int64_t c = blockIdx.x;
    // grad_bias[c] is loaded with the partials, not after them (a vector load: a scalar one
    // would be waited for before the partials' loads issue)
    const float gb =
        threadIdx.x == 0 ? __hip_atomic_load(&grad_bias[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    float acc = 0.0f;
    for (int64_t n = threadIdx.x; n < N; n += 256) {
        const int64_t p = n * C + c;
        const int64_t q0 = p * Sq;  // the plane's first quad; its waves are w0 .. w1
        const int64_t w0 = q0 / kBFlat, w1 = (q0 + Sq - 1) / kBFlat;
        // slot 0 where the wave begins inside the plane (w * 64 >= q0), else slot 1: the wave
        // began in the plane before (only w0 can); no integer division on the load path
        // every load issued before any add: a slot past w1 reloads w1's (in bounds) and adds 0
        float v[kCombPlaneWaves];
#pragma unroll
        for (int k = 0; k < kCombPlaneWaves; ++k) {
            const int64_t w = w0 + k <= w1 ? w0 + k : w1;
            v[k] = part[2 * w + (w * kBFlat >= q0 ? 0 : 1)];
        }
        __builtin_amdgcn_sched_barrier(0);  // keep the adds (and their waits) after every load
        float sp = 0.0f;
#pragma unroll
        for (int k = 0; k < kCombPlaneWaves; ++k) sp = sp + (w0 + k <= w1 ? v[k] : 0.0f);
        for (int64_t w = w0 + kCombPlaneWaves; w <= w1; ++w) sp = sp + part[2 * w + (w * kBFlat >= q0 ? 0 : 1)];
        acc = acc + sp;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) grad_bias[c] = gb + (((ws[0] + ws[1]) + ws[2]) + ws[3]);
}

// The same sums over the slot table [C][N][kPlaneSlots] that k_bias_relu_bwd_flat<.., SLOTS>
// writes: thread t reads plane (n = t, c)'s slots with two 16-byte loads (contiguous across the
// workgroup) and adds its cnt wave partials in wave order, then +0 for each unused slot, which
// is the order and the bits of k_bias_partials_comb.
__global__ void __launch_bounds__(256)
    k_bias_partials_comb8(float* __restrict__ grad_bias, const float* __restrict__ part, int64_t N, int64_t C,
                          int64_t Sq) {
    static_assert(kPlaneSlots == 8, "two quads per plane");
    __shared__ float ws[4];
    const int64_t c = blockIdx.x;
    // grad_bias[c] is loaded with the partials, not after them (a vector load: a scalar one
    // would be waited for before the partials' loads issue)
    const float gb =
        threadIdx.x == 0 ? __hip_atomic_load(&grad_bias[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0f;
    float acc = 0.0f;
    for (int64_t n = threadIdx.x; n < N; n += 256) {
        const vf4* src = reinterpret_cast<const vf4*>(part + (c * N + n) * kPlaneSlots);
        const vf4 a = src[0], b = src[1];
        const int64_t q0 = (n * C + c) * Sq;
        const int64_t cnt = (q0 + Sq - 1) / kBFlat - q0 / kBFlat + 1;  // waves of the plane
        const float v[kPlaneSlots] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
        float sp = 0.0f;
#pragma unroll
        for (int k = 0; k < kPlaneSlots; ++k) sp = sp + (k < cnt ? v[k] : 0.0f);
        acc = acc + sp;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc = acc + __shfl_xor(acc, m);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) grad_bias[c] = gb + (((ws[0] + ws[1]) + ws[2]) + ws[3]);
}

// [N, C, S] form of x with the bias indexed by C alone, from the collapsed plan of
// (x, bias); false when the shapes have another form.
static bool plane_form(const ElwPlan& pl, int64_t* N, int64_t* C, int64_t* S) {
    if (pl.kind[1] == IN_SCALAR) {
        *N = 1; *C = 1; *S = pl.n;
        return true;
    }
    if (pl.kind[1] != IN_BCAST) return false;
    if (pl.rank == 3 && pl.st[1][0] == 0 && pl.st[1][1] == 1 && pl.st[1][2] == 0) {
        *N = pl.dims[0]; *C = pl.dims[1]; *S = pl.dims[2];
        return true;
    }
    if (pl.rank == 2 && pl.st[1][0] == 1 && pl.st[1][1] == 0) {
        *N = 1; *C = pl.dims[0]; *S = pl.dims[1];
        return true;
    }
    return false;
}

}  // namespace mh

using namespace mh;

extern "C" {

int mh_bias_relu_fwd(float* y, float* r, const float* x, const mh_shape* psx, const float* bias,
                     const mh_shape* psbias) {
    MH_TRACE("mh_bias_relu_fwd");
    MH_SHAPE_ARG(sx);
    MH_SHAPE_ARG(sbias);
    MH_TRY(check_shape(sx, "x"));
    MH_TRY(check_shape(sbias, "bias"));
    mh_shape bs;
    MH_TRY(broadcast_shapes(sx, sbias, &bs));
    if (!shape_eq(bs, sx)) return fail(MH_ERR_SHAPE, "mh_bias_relu_fwd: bias must broadcast to x");
    const int64_t n = numel(sx);
    if (n == 0) return MH_OK;
    if (!y || !r || !x || !bias) return fail(MH_ERR_NULL, "mh_bias_relu_fwd: null tensor");
    MH_TRY(require_init());
    mh_shape in[2] = {sx, sbias};
    ElwPlan pl;
    MH_TRY(build_elw_plan(sx, 2, in, &pl));
    const bool al = al16f(y) && al16f(r) && al16f(x) && (pl.kind[1] != IN_FULL || al16f(bias));
    if (!al) {  // unaligned views: the two forward_op calls
        MH_TRY(mh_binary_fwd(MH_ADD, y, &sx, x, &sx, bias, &sbias));  // ADD.forward
        return mh_unary_fwd(MH_RELU, r, y, n);                       // RELU.forward
    }
    const bool big = n >= ((int64_t)1 << 31);
    const bool inner4 = pl.vec_ok && al16f(bias);
    // the plane kernel (below 2^31 elements) covers every quad with this grid; k_bias_relu_fwd4
    // loops over it beyond one dispatch
    dim3 g((unsigned)grid_blocks(n >> 2, kFFwdThreads)), b(kFFwdThreads);
    hipStream_t st = ctx().stream;
    int64_t N = 0, C = 0, S = 0;
    if (!big && pl.kind[1] != IN_FULL && plane_form(pl, &N, &C, &S) && S % 4 == 0) {
        hipLaunchKernelGGL(k_bias_relu_fwd_planes, g, b, 0, st, y, r, x, bias, n >> 2, (uint32_t)C,
                           make_fastdiv((uint32_t)(S / 4)), make_fastdiv((uint32_t)C));
        return finish("mh_bias_relu_fwd");
    }
    if (inner4) {
        if (big) hipLaunchKernelGGL((k_bias_relu_fwd4<true, true>), g, b, 0, st, y, r, x, bias, pl);
        else hipLaunchKernelGGL((k_bias_relu_fwd4<true, false>), g, b, 0, st, y, r, x, bias, pl);
    } else {
        if (big) hipLaunchKernelGGL((k_bias_relu_fwd4<false, true>), g, b, 0, st, y, r, x, bias, pl);
        else hipLaunchKernelGGL((k_bias_relu_fwd4<false, false>), g, b, 0, st, y, r, x, bias, pl);
    }
    return finish("mh_bias_relu_fwd");
}

int mh_bias_relu_bwd_accum(float* g_y, float* grad_x, float* grad_bias, const float* y, const float* ug,
                           const mh_shape* psx, const mh_shape* psbias) {
    MH_TRACE("mh_bias_relu_bwd_accum");
    MH_SHAPE_ARG(sx);
    MH_SHAPE_ARG(sbias);
    MH_TRY(check_shape(sx, "x"));
    MH_TRY(check_shape(sbias, "bias"));
    mh_shape bs;
    MH_TRY(broadcast_shapes(sx, sbias, &bs));
    if (!shape_eq(bs, sx)) return fail(MH_ERR_SHAPE, "mh_bias_relu_bwd_accum: bias must broadcast to x");
    const int64_t n = numel(sx);
    if (n == 0) return MH_OK;
    if (!y || !ug) return fail(MH_ERR_NULL, "mh_bias_relu_bwd_accum: null tensor");
    MH_TRY(require_init());
    mh_shape in[2] = {sx, sbias};
    ElwPlan pl;
    MH_TRY(build_elw_plan(sx, 2, in, &pl));
    int64_t N = 0, C = 0, S = 0;
    const bool al = al16f(y) && al16f(ug) && (!g_y || al16f(g_y)) && (!grad_x || al16f(grad_x));
    // planes of at least 64 elements (16 quads), so that a block has work for its waves
    const bool planes = al && plane_form(pl, &N, &C, &S) && S % 4 == 0 && S >= 64;
    const int64_t Sq = S / 4;
    const int64_t QC = Sq < 1024 ? Sq : 1024;  // quads per plane chunk
    const int64_t K = planes ? (Sq + QC - 1) / QC : 0;
    const int64_t G = planes ? (N * K + kArrivals - 1) / kArrivals : 0;  // planes per wavefront
    const int64_t NG = planes ? (N + G - 1) / G : 0;
    const int64_t nwaves = NG * K * C;
    const int64_t nblocks = (nwaves + 3) / 4;
    const int64_t nqf = n >> 2;
    // the flat stream: every wave spans at most two planes, and the combine's threads read at
    // most a few thousand partials each
    if (planes && Sq >= kBFlat && n < ((int64_t)1 << 31) && (N + 255) / 256 * (Sq / kBFlat + 2) <= 4096) {
        const int64_t nw = (nqf + kBFlat - 1) / kBFlat;
        float* part = nullptr;
        const bool has_part = grad_bias != nullptr;
        const bool slots = (Sq + 2 * kBFlat - 2) / kBFlat <= kPlaneSlots;  // every plane within 8 waves
        const size_t part_floats = slots ? (size_t)(N * C) * kPlaneSlots : (size_t)(2 * nw);
        if (has_part) MH_TRY(scratch((part_floats + 64) * sizeof(float), reinterpret_cast<void**>(&part)));
        hipStream_t st = ctx().stream;
        dim3 g((unsigned)nw), b(kBFlat);
        const FastDiv fsq = make_fastdiv((uint32_t)Sq), fc = make_fastdiv((uint32_t)C);
#define MH_BRF(GY, GX, PT)                                                                                      \
    do {                                                                                                        \
        if (slots)                                                                                              \
            hipLaunchKernelGGL((k_bias_relu_bwd_flat<GY, GX, PT, true>), g, b, 0, st, g_y, grad_x, y, ug, nqf,  \
                               (uint32_t)Sq, fsq, part, (uint32_t)N, (uint32_t)C, fc);                          \
        else                                                                                                    \
            hipLaunchKernelGGL((k_bias_relu_bwd_flat<GY, GX, PT, false>), g, b, 0, st, g_y, grad_x, y, ug, nqf, \
                               (uint32_t)Sq, fsq, part, (uint32_t)N, (uint32_t)C, fc);                          \
    } while (0)
        const int sel = (g_y ? 4 : 0) | (grad_x ? 2 : 0) | (has_part ? 1 : 0);
        switch (sel) {
            case 0: return MH_OK;  // nothing to produce
            case 1: MH_BRF(false, false, true); break;
            case 2: MH_BRF(false, true, false); break;
            case 3: MH_BRF(false, true, true); break;
            case 4: MH_BRF(true, false, false); break;
            case 5: MH_BRF(true, false, true); break;
            case 6: MH_BRF(true, true, false); break;
            default: MH_BRF(true, true, true); break;
        }
#undef MH_BRF
        if (has_part && slots)
            hipLaunchKernelGGL(k_bias_partials_comb8, dim3((unsigned)C), dim3(256), 0, st, grad_bias, part, N, C, Sq);
        else if (has_part)
            hipLaunchKernelGGL(k_bias_partials_comb, dim3((unsigned)C), dim3(256), 0, st, grad_bias, part, N, C, Sq);
        return finish("mh_bias_relu_bwd_accum");
    }
    if (planes && nblocks <= 0x7fffffff) {
        float* part = nullptr;
        uint32_t* tk = nullptr;
        const bool has_part = grad_bias != nullptr;
        if (has_part) {
            MH_TRY(scratch(((size_t)nwaves + 64) * sizeof(float), reinterpret_cast<void**>(&part)));
            MH_TRY(tickets(C * kTicketStride, &tk));
        }
        hipStream_t st = ctx().stream;
        dim3 g((unsigned)nblocks), b(kFThreads);
#define MH_BRB(GY, GX, PT)                                                                                       \
    hipLaunchKernelGGL((k_bias_relu_bwd_planes<GY, GX, PT>), g, b, 0, st, g_y, grad_x, y, ug, N, C, Sq, QC, K, G, \
                       nwaves, part, tk, grad_bias)
        const int sel = (g_y ? 4 : 0) | (grad_x ? 2 : 0) | (has_part ? 1 : 0);
        switch (sel) {
            case 0: return MH_OK;  // nothing to produce
            case 1: MH_BRB(false, false, true); break;
            case 2: MH_BRB(false, true, false); break;
            case 3: MH_BRB(false, true, true); break;
            case 4: MH_BRB(true, false, false); break;
            case 5: MH_BRB(true, false, true); break;
            case 6: MH_BRB(true, true, false); break;
            default: MH_BRB(true, true, true); break;
        }
#undef MH_BRB
        return finish("mh_bias_relu_bwd_accum");
    }
    // other shapes (a Linear layer's [rows, features] bias, unaligned views): op by op
    float* gy = g_y;
    if (!gy) {  // the grad of y starts at zero: stage it
        MH_TRY(stage((size_t)n * sizeof(float), reinterpret_cast<void**>(&gy)));
        MH_TRY(mh_zero(gy, n));
    }
    MH_TRY(mh_unary_bwd_accum(MH_RELU, gy, y, ug, n));  // RELU backward_op
    if (grad_x) MH_TRY(mh_binary_bwd_accum(MH_ADD, 0, grad_x, &sx, gy, &sx, y, &sx, y, &sbias));
    if (grad_bias) MH_TRY(mh_binary_bwd_accum(MH_ADD, 1, grad_bias, &sbias, gy, &sx, y, &sx, y, &sbias));
    return MH_OK;
}

}  // extern "C"
