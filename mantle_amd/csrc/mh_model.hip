// mh_model.hip -- Mantle's Graph builder (mantle/autograd/graph.mojo:33-217) and Model
// executor (mantle/nn/model.mojo:55-340) with its two Collections (tensors and grads,
// mantle/autograd/collection.mojo:24-224, mantle/nn/parameters.mojo) held in device memory.
//
// A graph records symbols (inputs, parameters, node outputs) and nodes in creation order,
// which is a topological order (graph.mojo:448-451). A model built from it places every
// symbol in one device arena and every trainable symbol's gradient in a second one, each
// tensor on a 256-byte boundary so the float4 paths apply, and runs forward / backward as
// back-to-back launches on the library stream with one synchronisation at the end (none
// under MH_INIT_ASYNC). Inputs enter by copy into their slots, as Collection.__setitem__
// does (collection.mojo:202-209); everything else stays on the device.
//
// Optional fusion: an ADD whose output feeds only the RELU node right after it runs as the
// fused bias + RELU kernels (MH_MODEL_FUSE_BIAS_RELU), and the node runs of nn.Softmax,
// nn.LogSoftmax, CrossEntropyLoss and the Softmax -> LOG -> MUL -> MEAN head run as the
// row-fused kernels (MH_MODEL_FUSE_ROWS). Every tensor and gradient slot holds what the
// op-by-op execution writes there, so the fusion is not observable in results.
// mh_model_capture records a pass (forward, backward, or zero_grad + forward + backward) as
// one HIP graph that mh_model_replay launches. While a captured graph exists, a library
// buffer that grows is retired rather than freed, so the addresses the graph holds stay
// valid until the graph is released or the library shuts down (a replay after mh_shutdown is
// refused).
#include <new>
#include <vector>

#include "mh_internal.h"

struct mh_graph {
    struct Sym {
        mh_shape shape;
        int trainable;
        int kind;          // MH_SYM_INPUT / MH_SYM_PARAM / MH_SYM_NODE
        int64_t init_off;  // parameter data in init_data, or -1 (zero-initialised)
    };
    struct Node {
        int op;
        int nin;
        int32_t in[3];
        int32_t out;
        mh_attrs attrs;
    };
    std::vector<Sym> syms;
    std::vector<float> init_data;
    std::vector<int32_t> inputs, params, outputs;
    int32_t loss = -1;
    std::vector<Node> nodes;
};

struct mh_model {
    mh_graph g;
    uint64_t flags = 0;
    float* arena = nullptr;
    float* grad_arena = nullptr;
    size_t arena_floats = 0, grad_floats = 0;
    std::vector<float*> t;  // per symbol: its tensor slot
    std::vector<float*> gr;  // per symbol: its gradient slot (nullptr if not trainable)
    int32_t n_inference = -1;
    size_t param_span = 0;  // floats of the trainable-parameter span at the start of both arenas
    std::vector<int> fuse;  // per node: kFuseAdd / kFuseRelu (bias + RELU), kFuseRow (row group)
    struct RowGroup {
        int graph;  // 0 head (Softmax, LOG, MUL, MEAN), 1 cross entropy, 2 Softmax, 3 LogSoftmax
        int first, last;
        int32_t x, target, out;
        int64_t rows, K;
        float scale;  // cross entropy: the graph scalar of its last MUL
    };
    std::vector<RowGroup> rows;
    std::vector<int> row_of;  // per node: its RowGroup, or -1
    hipGraphExec_t graph[3] = {nullptr, nullptr, nullptr};  // captured passes (MH_PASS_FORWARD / _BACKWARD / _STEP)
    uint64_t graph_epoch[3] = {0, 0, 0};                     // the mh_init epoch each was captured in
};

namespace mh {

static int op_arity(int op) {
    switch (op) {
        case MH_ADD: case MH_SUB: case MH_MUL: case MH_DIV: case MH_POW: return 2;
        case MH_EXP: case MH_LOG: case MH_SIGMOID: case MH_RELU: case MH_TANH:
        case MH_SUM: case MH_MEAN: case MH_MAX: case MH_CLIP: case MH_LEAKYRELU: return 1;
        case MH_FMA: return 3;
        default: return 0;
    }
}

static int axis_of(const mh_attrs& a) { return (a.flags & MH_ATTR_AXIS) ? a.axis : -1; }
static bool is_binary(int op) { return op >= MH_ADD && op <= MH_DIV; }
static bool is_unary(int op) {
    return op == MH_EXP || op == MH_LOG || op == MH_SIGMOID || op == MH_RELU || op == MH_TANH;
}
static bool is_reduce(int op) { return op == MH_SUM || op == MH_MEAN || op == MH_MAX; }
static float clip_lo(const mh_attrs& a) { return (a.flags & MH_ATTR_MIN) ? a.min_val : -3.40282347e38f; }
static float clip_hi(const mh_attrs& a) { return (a.flags & MH_ATTR_MAX) ? a.max_val : 3.40282347e38f; }

// static_result_shape (ops.mojo:104-218) for the ops of this path.
static int result_shape(const mh_graph& g, int op, int nin, const int32_t* in, const mh_attrs& at, mh_shape* out) {
    const mh_shape& s1 = g.syms[in[0]].shape;
    if (is_binary(op)) return broadcast_shapes(s1, g.syms[in[1]].shape, out);
    if (op == MH_POW) {
        if (!is_scalar_shape(g.syms[in[1]].shape))
            return fail(MH_ERR_SHAPE, "POW: the exponent must be a shape-(1) symbol (basics.mojo:317)");
        *out = s1;
        return MH_OK;
    }
    if (is_reduce(op)) {
        const int ax = axis_of(at);
        if (ax < -1 || ax >= s1.rank) return fail(MH_ERR_INVALID, "reduce: axis %d outside [-1, %d)", ax, s1.rank);
        *out = reduced_shape(s1, ax);
        return MH_OK;
    }
    if (op == MH_FMA) {
        if (!shape_eq(s1, g.syms[in[1]].shape) || !shape_eq(s1, g.syms[in[2]].shape))
            return fail(MH_ERR_SHAPE, "FMA: the three operands must have one shape (basics.mojo:759-766)");
    }
    if (op == MH_LEAKYRELU && !(at.flags & MH_ATTR_NEGATIVE_SLOPE))
        return fail(MH_ERR_INVALID, "LEAKYRELU needs the negative_slope attribute (mlops.mojo:145)");
    (void)nin;
    *out = s1;
    return MH_OK;
}

static int add_symbol(mh_graph* g, const mh_shape& s, int trainable, int kind, int32_t* sym) {
    MH_TRY(check_shape(s, "symbol"));
    if (g->syms.size() >= 0x7fffffff) return fail(MH_ERR_INVALID, "too many symbols");
    mh_graph::Sym y;
    y.shape = s;
    y.trainable = trainable ? 1 : 0;
    y.kind = kind;
    y.init_off = -1;
    g->syms.push_back(y);
    *sym = (int32_t)(g->syms.size() - 1);
    return MH_OK;
}

static int check_sym(const mh_graph* g, int32_t sym) {
    if (sym < 0 || (size_t)sym >= g->syms.size()) return fail(MH_ERR_INVALID, "unknown symbol %d", sym);
    return MH_OK;
}

static size_t slot_floats(const mh_shape& s) {
    const size_t n = (size_t)numel(s);
    return (n + 63) & ~(size_t)63;  // 256-byte slots
}

// Sets MH_INIT_ASYNC for the ops of one model pass; synchronises once at the end when the
// caller did not ask for asynchronous calls.
struct PassScope {
    uint64_t saved;
    PassScope() : saved(ctx().flags) { ctx().flags |= MH_INIT_ASYNC; }
    ~PassScope() { ctx().flags = saved; }
    int end(const char* what) {
        ctx().flags = saved;
        return finish(what);
    }
};

static int copy_in(float* dst, const float* src, size_t n, int where) {
    if (n == 0) return MH_OK;
    if (!src) return fail(MH_ERR_NULL, "null input tensor");
    const hipMemcpyKind k = where == MH_FROM_HOST ? hipMemcpyHostToDevice : hipMemcpyDeviceToDevice;
    MH_HIP(hipMemcpyAsync(dst, src, n * sizeof(float), k, ctx().stream));
    return MH_OK;
}

// n_inference_nodes (model.mojo:39-48): one past the last node that writes a graph output.
static int32_t inference_nodes(const mh_graph& g) {
    for (int32_t i = (int32_t)g.nodes.size() - 1; i >= 0; --i)
        for (int32_t o : g.outputs)
            if (g.nodes[i].out == o) return i + 1;
    return -1;
}

constexpr int kFuseAdd = 1, kFuseRelu = 2, kFuseRow = 3;
constexpr int64_t kRowMaxClasses = 2047;  // the fused row kernels' limit

// Row groups (MH_MODEL_FUSE_ROWS): consecutive nodes that nn.Softmax / nn.LogSoftmax /
// nn.CrossEntropyLoss emit (activations.mojo:74-108, loss.mojo:45-61), or the config-5 head
// (Softmax, LOG, MUL by a target, MEAN), over the last axis, whose intermediates are read by
// the group alone and are neither graph outputs nor the loss.
static void plan_row_groups(mh_model* m) {
    const mh_graph& g = m->g;
    const size_t nn = g.nodes.size();
    std::vector<std::vector<int>> users(g.syms.size());
    for (size_t j = 0; j < nn; ++j)
        for (int k = 0; k < g.nodes[j].nin; ++k) users[g.nodes[j].in[k]].push_back((int)j);
    auto exported = [&](int32_t sym) {
        if (g.loss == sym) return true;
        for (int32_t o : g.outputs)
            if (o == sym) return true;
        return false;
    };
    // every reader of `sym` lies in [first, last], and it is not exported
    auto local = [&](int32_t sym, int first, int last) {
        if (exported(sym)) return false;
        for (int j : users[sym])
            if (j < first || j > last) return false;
        return true;
    };
    auto node_is = [&](size_t j, int op) { return j < nn && g.nodes[j].op == op && m->fuse[j] == 0; };
    auto axis_last = [&](const mh_graph::Node& nd, const mh_shape& s) {
        return (nd.attrs.flags & MH_ATTR_AXIS) && nd.attrs.axis == s.rank - 1;
    };
    for (size_t i = 0; i + 4 < nn; ++i) {
        const mh_graph::Node& n0 = g.nodes[i];
        if (!node_is(i, MH_MAX)) continue;
        const int32_t x = n0.in[0];
        const mh_shape& sx = g.syms[x].shape;
        if (!axis_last(n0, sx)) continue;
        const int64_t K = sx.dims[sx.rank - 1];
        if (K < 1 || K > kRowMaxClasses) continue;
        const mh_graph::Node &n1 = g.nodes[i + 1], &n2 = g.nodes[i + 2], &n3 = g.nodes[i + 3];
        if (!node_is(i + 1, MH_SUB) || n1.in[0] != x || n1.in[1] != n0.out) continue;
        if (!node_is(i + 2, MH_EXP) || n2.in[0] != n1.out) continue;
        if (!node_is(i + 3, MH_SUM) || n3.in[0] != n2.out || !axis_last(n3, sx)) continue;
        mh_model::RowGroup rg{};
        rg.x = x;
        rg.rows = numel(sx) / K;
        rg.K = K;
        rg.first = (int)i;
        const mh_graph::Node& n4 = g.nodes[i + 4];
        int32_t core_out;
        if (node_is(i + 4, MH_DIV) && n4.in[0] == n2.out && n4.in[1] == n3.out) {
            rg.graph = 2;  // Softmax
            rg.last = (int)i + 4;
        } else if (node_is(i + 4, MH_LOG) && n4.in[0] == n3.out && node_is(i + 5, MH_SUB) &&
                   g.nodes[i + 5].in[0] == n1.out && g.nodes[i + 5].in[1] == n4.out) {
            rg.graph = 3;  // LogSoftmax
            rg.last = (int)i + 5;
        } else {
            continue;
        }
        core_out = g.nodes[rg.last].out;
        rg.out = core_out;
        // a loss on top: the head (Softmax, LOG, MUL(target), MEAN) or the cross entropy
        // (LogSoftmax, MUL(target), SUM, MUL(scalar)), target not trainable, x of rank 2 for
        // the cross entropy (its axis 1)
        auto mul_target = [&](size_t j, int32_t v, int32_t* t) {
            if (!node_is(j, MH_MUL)) return false;
            const mh_graph::Node& nd = g.nodes[j];
            const int32_t o = nd.in[0] == v ? nd.in[1] : nd.in[1] == v ? nd.in[0] : -1;
            if (o < 0 || o == v || g.syms[o].trainable || !shape_eq(g.syms[o].shape, sx)) return false;
            *t = o;
            return true;
        };
        int32_t t = -1;
        const size_t L = (size_t)rg.last;
        if (rg.graph == 2 && node_is(L + 1, MH_LOG) && g.nodes[L + 1].in[0] == core_out &&
            mul_target(L + 2, g.nodes[L + 1].out, &t) && node_is(L + 3, MH_MEAN) &&
            g.nodes[L + 3].in[0] == g.nodes[L + 2].out && !(g.nodes[L + 3].attrs.flags & MH_ATTR_AXIS)) {
            mh_model::RowGroup h = rg;
            h.graph = 0;
            h.last = (int)L + 3;
            h.target = t;
            h.out = g.nodes[L + 3].out;
            if (local(core_out, h.first, h.last) && local(g.nodes[L + 1].out, h.first, h.last) &&
                local(g.nodes[L + 2].out, h.first, h.last))
                rg = h;
        } else if (rg.graph == 3 && sx.rank == 2 && mul_target(L + 1, core_out, &t) && node_is(L + 2, MH_SUM) &&
                   g.nodes[L + 2].in[0] == g.nodes[L + 1].out && !(g.nodes[L + 2].attrs.flags & MH_ATTR_AXIS) &&
                   node_is(L + 3, MH_MUL) && g.nodes[L + 3].in[0] == g.nodes[L + 2].out) {
            const int32_t c = g.nodes[L + 3].in[1];
            const mh_graph::Sym& cs = g.syms[c];
            if (cs.kind == MH_SYM_PARAM && !cs.trainable && cs.init_off >= 0 && is_scalar_shape(cs.shape)) {
                mh_model::RowGroup h = rg;
                h.graph = 1;
                h.last = (int)L + 3;
                h.target = t;
                h.out = g.nodes[L + 3].out;
                h.scale = g.init_data[(size_t)cs.init_off];
                if (local(core_out, h.first, h.last) && local(g.nodes[L + 1].out, h.first, h.last) &&
                    local(g.nodes[L + 2].out, h.first, h.last))
                    rg = h;
            }
        }
        // the core's intermediates: MAX, SUB, EXP, SUM (and LOG of LogSoftmax) outputs
        bool ok = true;
        for (int j = rg.first; j < (rg.graph == 3 || rg.graph == 1 ? rg.first + 5 : rg.first + 4) && ok; ++j)
            ok = local(g.nodes[j].out, rg.first, rg.last);
        if (!ok) continue;
        const int id = (int)m->rows.size();
        m->rows.push_back(rg);
        for (int j = rg.first; j <= rg.last; ++j) {
            m->fuse[j] = kFuseRow;
            m->row_of[j] = id;
        }
        i = (size_t)rg.last;
    }
}

static void plan_fusion(mh_model* m) {
    const mh_graph& g = m->g;
    m->fuse.assign(g.nodes.size(), 0);
    m->row_of.assign(g.nodes.size(), -1);
    m->rows.clear();
    if (m->flags & MH_MODEL_FUSE_ROWS) plan_row_groups(m);
    if (!(m->flags & MH_MODEL_FUSE_BIAS_RELU)) return;
    for (size_t i = 0; i + 1 < g.nodes.size(); ++i) {
        const mh_graph::Node& a = g.nodes[i];
        const mh_graph::Node& r = g.nodes[i + 1];
        if (a.op != MH_ADD || r.op != MH_RELU || r.in[0] != a.out || m->fuse[i] || m->fuse[i + 1]) continue;
        // the ADD output is read by this RELU only, and is not a graph output or the loss
        bool only = g.loss != a.out;
        for (size_t j = 0; j < g.nodes.size() && only; ++j)
            for (int k = 0; k < g.nodes[j].nin; ++k)
                if (j != i + 1 && g.nodes[j].in[k] == a.out) only = false;
        for (int32_t o : g.outputs)
            if (o == a.out) only = false;
        if (!only) continue;
        // x + bias with x of the output shape and bias broadcast into it (never the reverse)
        const mh_shape& sx = g.syms[a.in[0]].shape;
        const mh_shape& sb = g.syms[a.in[1]].shape;
        const mh_shape& sy = g.syms[a.out].shape;
        if (!shape_eq(sx, sy) || shape_eq(sb, sy) || !broadcasts_to(sb, sy)) continue;
        m->fuse[i] = kFuseAdd;
        m->fuse[i + 1] = kFuseRelu;
    }
}

static int run_forward_node(mh_model* m, size_t i) {
    const mh_graph& g = m->g;
    const mh_graph::Node& nd = g.nodes[i];
    float* res = m->t[nd.out];
    const mh_shape& so = g.syms[nd.out].shape;
    const float* a = m->t[nd.in[0]];
    const mh_shape& sa = g.syms[nd.in[0]].shape;
    const int64_t n = numel(so);
    if (m->fuse[i] == kFuseRow) {  // a row group runs as one kernel at its first node
        const mh_model::RowGroup& r = m->rows[m->row_of[i]];
        if ((int)i != r.first) return MH_OK;
        switch (r.graph) {
            case 0: return mh_softmax_log_mul_mean_fwd(m->t[r.out], m->t[r.x], m->t[r.target], r.rows, r.K);
            case 1: return cross_entropy_fwd_c(m->t[r.out], m->t[r.x], m->t[r.target], r.rows, r.K, r.scale);
            case 2: return mh_softmax_fwd(m->t[r.out], m->t[r.x], r.rows, r.K);
            default: return mh_logsoftmax_fwd(m->t[r.out], m->t[r.x], r.rows, r.K);
        }
    }
    if (m->fuse[i] == kFuseAdd) {  // ADD + the RELU after it: writes both outputs
        const mh_graph::Node& r = g.nodes[i + 1];
        return mh_bias_relu_fwd(res, m->t[r.out], a, &sa, m->t[nd.in[1]], &g.syms[nd.in[1]].shape);
    }
    if (m->fuse[i] == kFuseRelu) return MH_OK;
    if (is_binary(nd.op)) return mh_binary_fwd(nd.op, res, &so, a, &sa, m->t[nd.in[1]], &g.syms[nd.in[1]].shape);
    if (nd.op == MH_POW) return mh_pow_fwd(res, a, n, m->t[nd.in[1]]);
    if (is_unary(nd.op)) return mh_unary_fwd(nd.op, res, a, n);
    if (is_reduce(nd.op)) return mh_reduce_fwd(nd.op, res, a, &sa, axis_of(nd.attrs));
    if (nd.op == MH_FMA) return mh_fma_fwd(res, a, m->t[nd.in[1]], m->t[nd.in[2]], n);
    if (nd.op == MH_LEAKYRELU) return mh_leakyrelu_fwd(res, a, n, nd.attrs.negative_slope);
    return mh_clip_fwd(res, a, n, clip_lo(nd.attrs), clip_hi(nd.attrs));
}

// Model.backward's per-node step (model.mojo:214-330): backward_op for every trainable
// operand, in operand order, each accumulating into that operand's gradient.
static int run_backward_node(mh_model* m, size_t i) {
    const mh_graph& g = m->g;
    const mh_graph::Node& nd = g.nodes[i];
    const float* ug = m->gr[nd.out];
    if (!ug) return MH_OK;  // no trainable operand
    const mh_shape& so = g.syms[nd.out].shape;
    const int32_t* in = nd.in;
    if (m->fuse[i] == kFuseRow) {  // a row group's backward runs at its last node
        const mh_model::RowGroup& r = m->rows[m->row_of[i]];
        if ((int)i != r.last) return MH_OK;
        float* gx = m->gr[r.x];
        switch (r.graph) {
            case 0: return mh_softmax_log_mul_mean_bwd_accum(gx, m->t[r.x], m->t[r.target], ug, r.rows, r.K);
            case 1: return cross_entropy_bwd_c(gx, m->t[r.x], m->t[r.target], ug, r.rows, r.K, r.scale);
            case 2: return mh_softmax_bwd_accum(gx, m->t[r.x], ug, r.rows, r.K);
            default: return mh_logsoftmax_bwd_accum(gx, m->t[r.x], ug, r.rows, r.K);
        }
    }
    if (m->fuse[i] == kFuseRelu) {  // RELU, then the ADD before it
        const mh_graph::Node& a = g.nodes[i - 1];
        float* gy = m->gr[a.out];
        float* gx = m->gr[a.in[0]];
        float* gb = m->gr[a.in[1]];
        return mh_bias_relu_bwd_accum(gy, gx, gb, m->t[a.out], ug, &so, &g.syms[a.in[1]].shape);
    }
    if (m->fuse[i] == kFuseAdd) return MH_OK;
    const float* t1 = m->t[in[0]];
    const mh_shape& s1 = g.syms[in[0]].shape;
    const int64_t n1 = numel(s1);
    if (is_binary(nd.op)) {
        const float* t2 = m->t[in[1]];
        const mh_shape& s2 = g.syms[in[1]].shape;
        float* g1 = m->gr[in[0]];
        float* g2 = m->gr[in[1]];
        // same result, one pass (also for one symbol used twice: one gradient, id 0's part first)
        if (g1 && g2 && shape_eq(s1, s2) && shape_eq(s1, so))
            return mh_binary_bwd_accum2(nd.op, g1, g2, ug, t1, t2, &s1);
        if (g1) MH_TRY(mh_binary_bwd_accum(nd.op, 0, g1, &s1, ug, &so, t1, &s1, t2, &s2));
        if (g2) MH_TRY(mh_binary_bwd_accum(nd.op, 1, g2, &s2, ug, &so, t1, &s1, t2, &s2));
        return MH_OK;
    }
    if (nd.op == MH_POW)  // both operand gradients in one pass where both are trainable
        return mh_pow_bwd_accum2(m->gr[in[0]], m->gr[in[1]], t1, m->t[in[1]], ug, n1);
    if (nd.op == MH_FMA) {
        for (int j = 0; j < 3; ++j)
            if (m->gr[in[j]]) MH_TRY(mh_fma_bwd_accum(j, m->gr[in[j]], ug, t1, m->t[in[1]], n1));
        return MH_OK;
    }
    float* g1 = m->gr[in[0]];
    if (!g1) return MH_OK;
    if (is_unary(nd.op)) return mh_unary_bwd_accum(nd.op, g1, t1, ug, n1);
    if (is_reduce(nd.op)) return mh_reduce_bwd_accum(nd.op, g1, t1, &s1, ug, axis_of(nd.attrs));
    if (nd.op == MH_LEAKYRELU) return mh_leakyrelu_bwd_accum(g1, t1, ug, n1, nd.attrs.negative_slope);
    return mh_clip_bwd_accum(g1, t1, ug, n1, clip_lo(nd.attrs), clip_hi(nd.attrs));
}

static int write_inputs(mh_model* m, int32_t ninputs, const float* const* inputs, int where) {
    const mh_graph& g = m->g;
    if (ninputs != (int32_t)g.inputs.size())
        return fail(MH_ERR_INVALID, "%d inputs given, the graph has %zu", ninputs, g.inputs.size());
    if (ninputs > 0 && !inputs) return fail(MH_ERR_NULL, "null input table");
    if (where != MH_FROM_HOST && where != MH_FROM_DEVICE) return fail(MH_ERR_INVALID, "bad input location %d", where);
    for (int32_t k = 0; k < ninputs; ++k) {
        const int32_t s = g.inputs[k];
        MH_TRY(copy_in(m->t[s], inputs[k], (size_t)numel(g.syms[s].shape), where));
    }
    if (where == MH_FROM_HOST && ninputs > 0) MH_HIP(hipStreamSynchronize(ctx().stream));  // pageable sources
    return MH_OK;
}

// The ops of one pass, enqueued on the library stream (no synchronisation): forward = every
// node; backward = the loss gradient seeded with 1.0, then every node in reverse.
static int check_pass(const mh_model* m, int pass) {
    if (pass == MH_PASS_FORWARD) return MH_OK;
    if (pass != MH_PASS_BACKWARD && pass != MH_PASS_STEP) return fail(MH_ERR_INVALID, "unknown pass %d", pass);
    if (m->g.loss < 0) return fail(MH_ERR_INVALID, "backward pass: the graph has no loss symbol");
    if (!m->gr[m->g.loss]) return fail(MH_ERR_INVALID, "backward pass: the loss is not trainable");
    return MH_OK;
}

static int enqueue_pass(mh_model* m, int pass) {
    const mh_graph& g = m->g;
    if (pass == MH_PASS_STEP && m->grad_arena)  // parameters.grads.set_zero (collection.mojo:221-224)
        MH_TRY(mh_zero(m->grad_arena, (int64_t)m->grad_floats));
    if (pass == MH_PASS_FORWARD || pass == MH_PASS_STEP)
        for (size_t i = 0; i < g.nodes.size(); ++i) MH_TRY(run_forward_node(m, i));
    if (pass == MH_PASS_FORWARD) return MH_OK;
    MH_TRY(mh_fill(m->gr[g.loss], 1.0f, numel(g.syms[g.loss].shape)));  // model.mojo:176-180
    for (size_t k = g.nodes.size(); k-- > 0;) MH_TRY(run_backward_node(m, k));
    return MH_OK;
}

static void drop_graphs(mh_model* m) {
    for (int p = 0; p < 3; ++p) {
        if (m->graph[p]) {
            (void)hipGraphExecDestroy(m->graph[p]);
            (void)graph_release(m->graph_epoch[p]);
        }
        m->graph[p] = nullptr;
    }
}

static int execute(mh_model* m, int32_t nodes, const char* what) {
    PassScope ps;
    for (int32_t i = 0; i < nodes; ++i) MH_TRY(run_forward_node(m, (size_t)i));
    return ps.end(what);
}

}  // namespace mh

using namespace mh;

extern "C" {

// ---------------------------------------------------------------------------------------
// Graph (graph.mojo:33-217)
// ---------------------------------------------------------------------------------------
int mh_graph_create(mh_graph** out) {
    if (!out) return fail(MH_ERR_NULL, "mh_graph_create: null out");
    *out = new (std::nothrow) mh_graph();
    if (!*out) return fail(MH_ERR_INVALID, "mh_graph_create: out of host memory");
    return MH_OK;
}

int mh_graph_destroy(mh_graph* g) {
    delete g;
    return MH_OK;
}

int mh_graph_input(mh_graph* g, const mh_shape* pshape, int trainable, int32_t* sym) {
    if (!g || !sym) return fail(MH_ERR_NULL, "mh_graph_input: null argument");
    MH_SHAPE_ARG(shape);
    MH_TRY(add_symbol(g, shape, trainable, MH_SYM_INPUT, sym));
    g->inputs.push_back(*sym);
    return MH_OK;
}

int mh_graph_param(mh_graph* g, const mh_shape* pshape, int trainable, const float* data, int64_t ndata,
                   int32_t* sym) {
    if (!g || !sym) return fail(MH_ERR_NULL, "mh_graph_param: null argument");
    MH_SHAPE_ARG(shape);
    MH_TRY(check_shape(shape, "param"));
    if (ndata < 0 || (ndata > 0 && !data)) return fail(MH_ERR_INVALID, "mh_graph_param: bad init data");
    if (ndata > 0 && ndata != numel(shape))
        return fail(MH_ERR_SHAPE, "mh_graph_param: %lld init values for %lld elements", (long long)ndata,
                    (long long)numel(shape));
    MH_TRY(add_symbol(g, shape, trainable, MH_SYM_PARAM, sym));
    if (ndata > 0) {
        g->syms.back().init_off = (int64_t)g->init_data.size();
        g->init_data.insert(g->init_data.end(), data, data + ndata);
    }
    g->params.push_back(*sym);
    return MH_OK;
}

int mh_graph_scalar(mh_graph* g, float value, int32_t* sym) {
    const mh_shape s = flat_shape(1);
    return mh_graph_param(g, &s, 0, &value, 1, sym);
}

int mh_graph_op(mh_graph* g, int op, int32_t noperands, const int32_t* operands, const mh_attrs* attrs,
                int32_t* sym) {
    if (!g || !sym || (noperands > 0 && !operands)) return fail(MH_ERR_NULL, "mh_graph_op: null argument");
    const int ar = op_arity(op);
    if (ar == 0) return fail(MH_ERR_OP, "mh_graph_op: operator %d is not on this path", op);
    if (noperands != ar) return fail(MH_ERR_INVALID, "mh_graph_op: operator %d takes %d operands, got %d", op, ar, noperands);
    for (int k = 0; k < ar; ++k) MH_TRY(check_sym(g, operands[k]));
    mh_attrs at{};
    if (attrs) at = *attrs;
    mh_shape rs;
    MH_TRY(result_shape(*g, op, ar, operands, at, &rs));
    int tr = 0;  // result_trainable (graph.mojo:212-217)
    for (int k = 0; k < ar; ++k) tr |= g->syms[operands[k]].trainable;
    MH_TRY(add_symbol(g, rs, tr, MH_SYM_NODE, sym));
    mh_graph::Node nd;
    nd.op = op;
    nd.nin = ar;
    for (int k = 0; k < 3; ++k) nd.in[k] = k < ar ? operands[k] : -1;
    nd.out = *sym;
    nd.attrs = at;
    g->nodes.push_back(nd);
    return MH_OK;
}

int mh_graph_out(mh_graph* g, int32_t sym) {
    if (!g) return fail(MH_ERR_NULL, "mh_graph_out: null graph");
    MH_TRY(check_sym(g, sym));
    g->outputs.push_back(sym);
    return MH_OK;
}

int mh_graph_loss(mh_graph* g, int32_t sym) {
    if (!g) return fail(MH_ERR_NULL, "mh_graph_loss: null graph");
    MH_TRY(check_sym(g, sym));
    g->loss = sym;
    return MH_OK;
}

int mh_graph_symbol(const mh_graph* g, int32_t sym, mh_shape* shape, int* trainable, int* kind) {
    if (!g) return fail(MH_ERR_NULL, "mh_graph_symbol: null graph");
    MH_TRY(check_sym(g, sym));
    if (shape) *shape = g->syms[sym].shape;
    if (trainable) *trainable = g->syms[sym].trainable;
    if (kind) *kind = g->syms[sym].kind;
    return MH_OK;
}

int mh_graph_counts(const mh_graph* g, int32_t* nsymbols, int32_t* nnodes, int32_t* ninputs, int32_t* nparams,
                    int32_t* noutputs) {
    if (!g) return fail(MH_ERR_NULL, "mh_graph_counts: null graph");
    if (nsymbols) *nsymbols = (int32_t)g->syms.size();
    if (nnodes) *nnodes = (int32_t)g->nodes.size();
    if (ninputs) *ninputs = (int32_t)g->inputs.size();
    if (nparams) *nparams = (int32_t)g->params.size();
    if (noutputs) *noutputs = (int32_t)g->outputs.size();
    return MH_OK;
}

// ---------------------------------------------------------------------------------------
// Model (model.mojo:55-340)
// ---------------------------------------------------------------------------------------
int mh_model_create(const mh_graph* g, uint64_t flags, mh_model** out) {
    if (!g || !out) return fail(MH_ERR_NULL, "mh_model_create: null argument");
    *out = nullptr;
    MH_TRY(require_init());
    mh_model* m = new (std::nothrow) mh_model();
    if (!m) return fail(MH_ERR_INVALID, "mh_model_create: out of host memory");
    m->g = *g;
    m->flags = flags;
    const size_t ns = g->syms.size();
    std::vector<size_t> toff(ns), goff(ns, (size_t)-1);
    // allocate_tensor_memory / allocate_grad_memory. The trainable parameters come first in
    // both arenas, in the same order with the same slot sizes, so that parameters and their
    // gradients form two parallel spans an optimizer updates in one launch; then every other
    // symbol in creation order.
    auto is_tparam = [&](size_t s) { return g->syms[s].kind == MH_SYM_PARAM && g->syms[s].trainable; };
    for (int pass = 0; pass < 2; ++pass) {
        for (size_t s = 0; s < ns; ++s) {
            if (is_tparam(s) != (pass == 0)) continue;
            toff[s] = m->arena_floats;
            m->arena_floats += slot_floats(g->syms[s].shape);
            if (g->syms[s].trainable) {
                goff[s] = m->grad_floats;
                m->grad_floats += slot_floats(g->syms[s].shape);
            }
        }
        if (pass == 0) m->param_span = m->arena_floats;
    }
    int rc = MH_OK;
    if (m->arena_floats) rc = mh_malloc(reinterpret_cast<void**>(&m->arena), m->arena_floats * sizeof(float));
    if (rc == MH_OK && m->grad_floats)
        rc = mh_malloc(reinterpret_cast<void**>(&m->grad_arena), m->grad_floats * sizeof(float));
    if (rc == MH_OK) {
        m->t.resize(ns);
        m->gr.assign(ns, nullptr);
        for (size_t s = 0; s < ns; ++s) {
            m->t[s] = m->arena + toff[s];
            if (goff[s] != (size_t)-1) m->gr[s] = m->grad_arena + goff[s];
        }
        // Tensor[f32](shape) is zero-initialised (tensor.mojo:266); parameters with data
        // get it copied in (model.mojo:353-370)
        PassScope ps;
        if (m->arena) rc = mh_zero(m->arena, (int64_t)m->arena_floats);
        if (rc == MH_OK && m->grad_arena) rc = mh_zero(m->grad_arena, (int64_t)m->grad_floats);
        for (size_t s = 0; s < ns && rc == MH_OK; ++s) {
            const mh_graph::Sym& y = g->syms[s];
            if (y.kind == MH_SYM_PARAM && y.init_off >= 0)
                rc = copy_in(m->t[s], g->init_data.data() + y.init_off, (size_t)numel(y.shape), MH_FROM_HOST);
        }
        // the host init data is pageable: wait for its copies whatever the caller's flags
        if (rc == MH_OK) rc = hip_check(hipStreamSynchronize(ctx().stream), "mh_model_create");
        (void)ps;
    }
    if (rc != MH_OK) {
        if (m->arena) mh_free(m->arena);
        if (m->grad_arena) mh_free(m->grad_arena);
        delete m;
        return rc;
    }
    m->n_inference = inference_nodes(m->g);
    plan_fusion(m);
    *out = m;
    return MH_OK;
}

int mh_model_destroy(mh_model* m) {
    if (!m) return MH_OK;
    drop_graphs(m);
    int rc = MH_OK;
    if (m->arena) rc = mh_free(m->arena);
    if (m->grad_arena) {
        const int r2 = mh_free(m->grad_arena);
        if (rc == MH_OK) rc = r2;
    }
    delete m;
    return rc;
}

int mh_model_forward(mh_model* m, int32_t ninputs, const float* const* inputs, int where) {
    MH_TRACE("mh_model_forward");
    if (!m) return fail(MH_ERR_NULL, "mh_model_forward: null model");
    MH_TRY(require_init());
    MH_TRY(write_inputs(m, ninputs, inputs, where));
    return execute(m, (int32_t)m->g.nodes.size(), "mh_model_forward");
}

int mh_model_inference(mh_model* m, int32_t ninputs, const float* const* inputs, int where) {
    MH_TRACE("mh_model_inference");
    if (!m) return fail(MH_ERR_NULL, "mh_model_inference: null model");
    if (m->n_inference < 0) return fail(MH_ERR_INVALID, "mh_model_inference: the graph has no output");
    MH_TRY(require_init());
    MH_TRY(write_inputs(m, ninputs, inputs, where));
    int32_t nodes = m->n_inference;
    // a fused ADD + RELU pair is never split by the inference cut
    if (nodes > 0 && nodes < (int32_t)m->fuse.size() && m->fuse[nodes - 1] == kFuseAdd) ++nodes;
    if (nodes > 0 && nodes < (int32_t)m->fuse.size() && m->fuse[nodes - 1] == kFuseRow)
        nodes = m->rows[m->row_of[nodes - 1]].last + 1;  // never cut a row group
    return execute(m, nodes, "mh_model_inference");
}

int mh_model_backward(mh_model* m, int32_t nupper, const float* const* upper_grads, int where) {
    MH_TRACE("mh_model_backward");
    if (!m) return fail(MH_ERR_NULL, "mh_model_backward: null model");
    MH_TRY(require_init());
    const mh_graph& g = m->g;
    if (g.nodes.empty()) return MH_OK;
    PassScope ps;
    if (nupper == 0) {  // model.mojo:176-180: seed the loss gradient with 1.0
        if (g.loss < 0) return fail(MH_ERR_INVALID, "mh_model_backward: no loss symbol and no upper grads");
        if (!m->gr[g.loss]) return fail(MH_ERR_INVALID, "mh_model_backward: the loss is not trainable");
        MH_TRY(mh_fill(m->gr[g.loss], 1.0f, numel(g.syms[g.loss].shape)));
    } else {  // model.mojo:181-193: the last node's output gradient is a copy of the given one
        if (!upper_grads) return fail(MH_ERR_NULL, "mh_model_backward: null upper grads");
        if (where != MH_FROM_HOST && where != MH_FROM_DEVICE)
            return fail(MH_ERR_INVALID, "bad upper-grad location %d", where);
        const int32_t last = g.nodes.back().out;
        if (!m->gr[last]) return fail(MH_ERR_INVALID, "mh_model_backward: the last node output is not trainable");
        MH_TRY(copy_in(m->gr[last], upper_grads[0], (size_t)numel(g.syms[last].shape), where));
    }
    for (size_t k = g.nodes.size(); k-- > 0;) MH_TRY(run_backward_node(m, k));
    if (nupper != 0 && where == MH_FROM_HOST) {  // pageable source: wait whatever the flags
        MH_HIP(hipStreamSynchronize(ctx().stream));
    }
    return ps.end("mh_model_backward");
}

int mh_model_capture(mh_model* m, int pass) {
    MH_TRACE("mh_model_capture");
    if (!m) return fail(MH_ERR_NULL, "mh_model_capture: null model");
    MH_TRY(require_init());
    MH_TRY(check_pass(m, pass));
    hipStream_t st = ctx().stream;
    {  // run the pass once: library buffers reach the sizes the pass needs before capture
        PassScope ps;
        MH_TRY(enqueue_pass(m, pass));
        MH_HIP(hipStreamSynchronize(st));
    }
    PassScope ps;
    MH_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue_pass(m, pass);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(st, &graph);
    if (rc != MH_OK || e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc != MH_OK ? rc : hip_check(e, "mh_model_capture: hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t e2 = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    MH_HIP(e2);
    if (m->graph[pass]) {
        (void)hipGraphExecDestroy(m->graph[pass]);
        (void)graph_release(m->graph_epoch[pass]);
    }
    graph_retain();
    m->graph[pass] = exec;
    m->graph_epoch[pass] = ctx().epoch;
    return MH_OK;
}

int mh_model_replay(mh_model* m, int pass) {
    MH_TRACE("mh_model_replay");
    if (!m) return fail(MH_ERR_NULL, "mh_model_replay: null model");
    MH_TRY(require_init());
    if (pass != MH_PASS_FORWARD && pass != MH_PASS_BACKWARD && pass != MH_PASS_STEP)
        return fail(MH_ERR_INVALID, "unknown pass %d", pass);
    if (!m->graph[pass]) return fail(MH_ERR_INVALID, "mh_model_replay: pass %d has not been captured", pass);
    if (m->graph_epoch[pass] != ctx().epoch)
        return fail(MH_ERR_INVALID, "mh_model_replay: pass %d was captured before the last mh_shutdown; capture it again",
                    pass);
    MH_HIP(hipGraphLaunch(m->graph[pass], ctx().stream));
    return finish("mh_model_replay");
}

int mh_model_tensor(mh_model* m, int32_t sym, float** dptr) {
    if (!m || !dptr) return fail(MH_ERR_NULL, "mh_model_tensor: null argument");
    MH_TRY(check_sym(&m->g, sym));
    *dptr = m->t[sym];
    return MH_OK;
}

int mh_model_grad(mh_model* m, int32_t sym, float** dptr) {
    if (!m || !dptr) return fail(MH_ERR_NULL, "mh_model_grad: null argument");
    MH_TRY(check_sym(&m->g, sym));
    if (!m->gr[sym]) return fail(MH_ERR_INVALID, "mh_model_grad: symbol %d is not trainable", sym);
    *dptr = m->gr[sym];
    return MH_OK;
}

int mh_model_zero_grad(mh_model* m) {
    MH_TRACE("mh_model_zero_grad");
    if (!m) return fail(MH_ERR_NULL, "mh_model_zero_grad: null model");
    if (!m->grad_arena) return MH_OK;
    return mh_zero(m->grad_arena, (int64_t)m->grad_floats);
}

int mh_model_param_span(mh_model* m, float** params, float** grads, int64_t* n) {
    if (!m || !params || !grads || !n) return fail(MH_ERR_NULL, "mh_model_param_span: null argument");
    *params = m->param_span ? m->arena : nullptr;
    *grads = m->param_span ? m->grad_arena : nullptr;
    *n = (int64_t)m->param_span;
    return MH_OK;
}

int mh_model_info(const mh_model* m, int32_t* n_inference_nodes, int64_t* tensor_bytes, int64_t* grad_bytes,
                  int32_t* fused_groups) {
    if (!m) return fail(MH_ERR_NULL, "mh_model_info: null model");
    if (n_inference_nodes) *n_inference_nodes = m->n_inference;
    if (tensor_bytes) *tensor_bytes = (int64_t)(m->arena_floats * sizeof(float));
    if (grad_bytes) *grad_bytes = (int64_t)(m->grad_floats * sizeof(float));
    if (fused_groups) {
        int32_t c = 0;
        for (int f : m->fuse) c += f == kFuseAdd;
        c += (int32_t)m->rows.size();
        *fused_groups = c;
    }
    return MH_OK;
}

}  // extern "C"
