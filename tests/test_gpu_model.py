"""The native Graph / Model executor (mh_graph_*, mh_model_*; mantle/autograd/graph.mojo,
mantle/nn/model.mojo, mantle/autograd/collection.mojo) against the CPU oracle running the same
graph one forward_op / backward_op at a time in Model's node order and trainable gating
(model.mojo:113-330, restated by util.Graph): every tensor and gradient slot holds the oracle's
bits, except sums whose order differs (named per test), which are in the rtol class."""
import numpy as np
import pytest

from mantle_amd import synth
from util import (FMA, O, OPS, GpuEngine, Graph, Mag64Engine, OracleEngine, assert_bitexact, assert_order_close,
                  assert_sum_close, config5_nodes, cross_entropy_nodes, load_fixtures, logsoftmax_nodes, native_graph,
                  softmax_nodes, spec_to_array)

pytestmark = pytest.mark.gpu
ORC = OracleEngine()


@pytest.fixture(scope="module")
def gpu():
    return GpuEngine()


@pytest.fixture(autouse=True)
def _nelts():
    O.set_nelts(32)
    yield


def _sum_ref(vals, grads, spec):
    """(fp64 value, fp64 sum of |terms|) of a sum-class slot: spec = (source, axes, kind, grads?)
    with kind "sum" or "mean" over `axes` (None: every element) of the source slot."""
    src, axes, kind, of_grads = spec
    terms = np.asarray((grads if of_grads else vals)[src], np.float64)
    ex = terms.sum(axis=axes)
    ab = np.abs(terms).sum(axis=axes)
    if kind == "mean":
        n = terms.size if axes is None else int(np.prod([terms.shape[a] for a in np.atleast_1d(axes)]))
        ex, ab = ex / n, ab / n
    return ex, ab


def _compare(gpu, nodes, values, trainable, params=(), seed=None, fuse=False, what="", sums=None):
    """Runs the graph on the native Model and on the oracle (util.Graph, one engine call per
    node) and compares every slot. `sums` = {slot: (source, axes, "sum"|"mean", of_grads)}:
    slots that are sums over `axes` of another slot (a tensor, or a gradient when of_grads) in
    another fixed order (a loss, a long un-broadcast, the fused bias gradient); they are checked
    in the rtol class against the fp64 sum. Returns (model, symbols, oracle values, grads)."""
    m = gpu.m
    sums = sums or {}
    ref = Graph(nodes, trainable)
    vals = ref.forward(ORC, values)
    grads = ref.backward(ORC, vals, seed)
    g, syms, inputs = native_graph(m, nodes, values, trainable, params)
    last = nodes[-1][3]
    if seed is None:
        g.loss(syms[last])
    g.out(syms[last])
    model = m.Model(g, fuse_bias_relu=fuse)
    ins = [values[n] for n in inputs]
    if seed is None:
        model.forward(*ins)
        model.backward()
    else:
        model.inference(*ins)
        model.backward(seed)

    def check(got, refv, key, label):
        if key in sums:
            ex, ab = _sum_ref(vals, grads, sums[key])
            shape = got.shape
            assert_sum_close(got, refv, np.reshape(ex, shape), label, terms_abs=np.reshape(ab, shape))
        else:
            assert_bitexact(got, refv, label)

    for name, sym in syms.items():
        got = model.parameters.tensors[sym].to_numpy().reshape(np.shape(vals[name]))
        check(got, vals[name], name, f"{what} tensor {name}")
        if not sym.trainable:
            continue
        got = model.parameters.grads[sym].to_numpy().reshape(np.shape(grads[name]))
        check(got, grads[name], "grad " + name, f"{what} grad {name}")
    return model, syms, vals, grads


def _bias_relu_nodes():
    return [(OPS["ADD"], ["x", "bias"], None, "y"), (OPS["RELU"], ["y"], None, "r")]


@pytest.mark.parametrize("fuse", [False, True])
@pytest.mark.parametrize("xshape,bshape", [((32, 32), (1, 32)), ((16, 32, 28, 28), (1, 32, 1, 1))])
def test_model_bias_relu_configs(gpu, fuse, xshape, bshape):
    """Configs 1 and 3: ADD(x, bias) -> RELU with an upper gradient, x a trainable input and
    bias a trainable parameter, fused or not, against the oracle. Config 1's bias gradient
    (32-row columns) adds each row into the gradient in order, as accumulate_grad's serial walk
    does (tensorutils.mojo:473-487): bit-exact unfused. Config 3's (200 704 terms per channel),
    and the fused kernel's, sum in another order: rtol class."""
    values = {"x": synth.normal(xshape, 0, 1, 1200), "bias": synth.normal(bshape, 0, 0.1, 1201)}
    seed = synth.normal(xshape, 0, 1, 1202)
    axes = tuple(i for i, d in enumerate(bshape) if d == 1)
    long_lines = int(np.prod(xshape)) // int(np.prod(bshape)) > 64
    sums = {"grad bias": ("y", axes, "sum", True)} if (fuse or long_lines) else None
    model, *_ = _compare(gpu, _bias_relu_nodes(), values, ["x", "bias"], params=["bias"], seed=seed, fuse=fuse,
                         what=f"fuse={fuse}", sums=sums)
    assert model.info()["fused_groups"] == (1 if fuse else 0)


def test_model_config5_chain(gpu):
    """Config 5's graph (10-class rows) against the oracle: row sums of 10 terms add in element
    order on both sides, so every slot is bit-exact but the loss (an all-element MEAN, rtol);
    the loss gradient is seeded with 1.0, so no gradient depends on the loss sum."""
    rows, classes = 4099, 10
    logits = synth.normal((rows, classes), 0, 2, 1210)
    cls = np.floor(synth.uniform((rows,), 0, 1, 1211) * classes).astype(np.int64)
    onehot = np.zeros((rows, classes), np.float32)
    onehot[np.arange(rows), cls] = 1
    _compare(gpu, config5_nodes(), {"logits": logits, "onehot": onehot}, ["logits"], what="c5",
             sums={"loss": ("t", None, "mean", False)})


def _every_op_reference(E, x, w):
    """The every-op graph one engine call per node in Model.backward's order (model.mojo:194-330):
    (loss, grads of x, w, b, e, t)."""
    va = E.forward(OPS["MUL"], x, w)
    vb = E.forward(OPS["ADD"], va, x)
    vc = E.forward(OPS["TANH"], vb)
    vd = E.forward(OPS["SIGMOID"], vc)
    ve = E.forward(OPS["FMA"], vc, vd, t3=vb)
    vf = E.forward(OPS["LEAKYRELU"], ve, attrs={"negative_slope": 0.2})
    vh = E.forward(OPS["CLIP"], vf, attrs={"min": -0.5, "max": 1.5})
    vk = E.forward(OPS["MAX"], vh, axis=1)
    vq = E.forward(OPS["SUB"], vh, vk)
    vr = E.forward(OPS["EXP"], vq)
    two = np.array([2.0], np.float32)
    vs = E.forward(OPS["POW"], vr, two)
    vsum = E.forward(OPS["SUM"], vs, axis=0)
    vt = E.forward(OPS["DIV"], vs, vsum)
    vu = E.forward(OPS["MUL"], vt, vt)
    vl = E.forward(OPS["MEAN"], vu)
    z = lambda v: np.zeros(np.shape(v), np.float32)  # noqa: E731
    gl = np.ones(1, np.float32)
    gu = E.backward(0, OPS["MEAN"], gl, vu, grad=z(vu))
    gt = E.backward(0, OPS["MUL"], gu, vt, vt, grad=z(vt))
    gt = E.backward(1, OPS["MUL"], gu, vt, vt, grad=gt)
    gs = E.backward(0, OPS["DIV"], gt, vs, vsum, grad=z(vs))
    gsum = E.backward(1, OPS["DIV"], gt, vs, vsum, grad=z(vsum))
    gs = E.backward(0, OPS["SUM"], gsum, vs, axis=0, grad=gs)
    gr = E.backward(0, OPS["POW"], gs, vr, two, grad=z(vr))
    gq = E.backward(0, OPS["EXP"], gr, vq, grad=z(vq))
    gh = E.backward(0, OPS["SUB"], gq, vh, vk, grad=z(vh))
    gk = E.backward(1, OPS["SUB"], gq, vh, vk, grad=z(vk))
    gh = E.backward(0, OPS["MAX"], gk, vh, axis=1, grad=gh)
    gf = E.backward(0, OPS["CLIP"], gh, vf, grad=z(vf), attrs={"min": -0.5, "max": 1.5})
    ge = E.backward(0, OPS["LEAKYRELU"], gf, ve, grad=z(ve), attrs={"negative_slope": 0.2})
    gc = E.backward(0, FMA, ge, vc, vd, grad=z(vc))
    gd = E.backward(1, FMA, ge, vc, vd, grad=z(vd))
    gb = E.backward(2, FMA, ge, vc, vd, grad=z(vb))
    gc = E.backward(0, OPS["SIGMOID"], gd, vc, grad=gc)
    gb = E.backward(0, OPS["TANH"], gc, vb, grad=gb)
    ga = E.backward(0, OPS["ADD"], gb, va, x, grad=z(va))
    gx = E.backward(1, OPS["ADD"], gb, va, x, grad=z(x))
    gx = E.backward(0, OPS["MUL"], ga, x, w, grad=gx)
    gw = E.backward(1, OPS["MUL"], ga, x, w, grad=z(w))
    return vl, vu, {"x": gx, "w": gw, "b": gb, "e": ge, "t": gt}


@pytest.mark.parametrize("rows", [20, 37])
def test_model_every_op(gpu, rows):
    """One graph over every op of the path (broadcast, scalar, reduce, POW, FMA, CLIP,
    LEAKYRELU) with trainable parameters, a shared operand and one symbol as both operands of
    a MUL, against the oracle op by op. With 20 rows the column SUM adds its 20 terms in element
    order on both sides (fewer than the oracle's 32 lanes), so every gradient is bit-exact and
    only the loss (an all-element MEAN) is in the rtol class. With 37 rows the oracle's column
    sums run lane-striped: the slots are bit-exact against the GPU's own op-by-op calls and in
    the fp64 sum class against the oracle (assert_order_close: the fp64 magnitude engine
    carries the order of the column sums through the DIV and every gradient after it)."""
    m = gpu.m
    x = synth.normal((rows, 20), 0, 1, 1220)
    w = synth.normal((1, 20), 0, 1, 1221)
    g = m.Graph()
    sx = g.input((rows, 20), trainable=True)
    sw = g.param((1, 20), init=w)
    a = g.op(m.OP.MUL, sx, sw)
    b = g.op(m.OP.ADD, a, sx)                    # sx used twice
    c = g.op(m.OP.TANH, b)
    d = g.op(m.OP.SIGMOID, c)
    e = g.op(m.OP.FMA, c, d, b)
    f = g.op(m.OP.LEAKYRELU, e, attributes={"negative_slope": 0.2})
    h = g.op(m.OP.CLIP, f, attributes={"min": -0.5, "max": 1.5})
    k = g.op(m.OP.MAX, h, attributes={"axis": 1})
    q = g.op(m.OP.SUB, h, k)
    r = g.op(m.OP.EXP, q)
    s = g.op(m.OP.POW, r, 2.0)
    t = g.op(m.OP.DIV, s, g.op(m.OP.SUM, s, attributes={"axis": 0}))
    u = g.op(m.OP.MUL, t, t)                     # same symbol twice
    loss = g.op(m.OP.MEAN, u)
    g.loss(loss)
    g.out(loss)
    model = m.Model(g)
    got = model.forward(x).to_numpy()
    model.backward()
    P = model.parameters
    slots = {"x": P.grads[sx], "w": P.grads[sw], "b": P.grads[b], "e": P.grads[e], "t": P.grads[t]}
    ol, ou, og = _every_op_reference(ORC, x, w)
    u64 = ou.astype(np.float64)
    assert_sum_close(got, ol, np.array([u64.mean()]), "loss vs oracle", terms_abs=np.array([np.abs(u64).mean()]))
    if rows <= 31:
        for k, v in og.items():
            assert_bitexact(slots[k].to_numpy(), v, f"grad {k} vs oracle")
        return
    _, _, og64 = _every_op_reference(Mag64Engine(), x, w)
    for k, v in og.items():
        assert_order_close(slots[k].to_numpy(), v, og64[k], f"grad {k} vs oracle")
    gl, _, gg = _every_op_reference(gpu, x, w)
    assert_bitexact(got, gl, "loss")
    for k, v in gg.items():
        assert_bitexact(slots[k].to_numpy(), v, f"grad {k} vs GPU op by op")


@pytest.mark.parametrize("shape", [(37, 20), (4099, 7)])
def test_model_pow_both_operands_trainable(gpu, shape):
    """POW with a trainable exponent parameter: Model.backward's two POW backward_op calls
    (model.mojo:233-270) run as one pass (mh_pow_bwd_accum2). x's gradient holds the oracle's
    bits; the exponent's gradient is in the sum class against the oracle and bit-identical to
    the GPU's own two separate calls. Two backward passes check that both slots accumulate."""
    m = gpu.m
    x = synth.uniform(shape, 0.1, 4, 1300 + shape[0])
    e = np.array([2.37], np.float32)
    g = m.Graph()
    sx = g.input(shape, trainable=True)
    se = g.param((1,), init=e)
    p = g.op(m.OP.POW, sx, se)
    loss = g.op(m.OP.MEAN, p)
    g.loss(loss)
    g.out(loss)
    model = m.Model(g)
    model.forward(x)
    model.backward()
    P = model.parameters
    pv = ORC.forward(OPS["POW"], x, e)
    gp = ORC.backward(0, OPS["MEAN"], np.ones(1, np.float32), pv)
    ox = ORC.backward(0, OPS["POW"], gp, x, e)
    oe = ORC.backward(1, OPS["POW"], gp, x, e)
    assert_bitexact(P.grads[sx].to_numpy(), ox, "grad x vs oracle")
    X = x.astype(np.float64)
    terms = X ** np.float64(e[0]) * np.log(X) * gp.astype(np.float64)
    got_e = P.grads[se].to_numpy()
    assert_sum_close(got_e, oe, np.array([terms.sum()]), "grad exponent vs oracle",
                     terms_abs=np.array([np.abs(terms).sum()]))
    ge_sep = gpu.backward(1, OPS["POW"], gp, x, e)
    assert_bitexact(got_e, ge_sep, "grad exponent vs the separate GPU call")
    # a second pass clears nothing: the loss seed is set to 1.0 again, p's gradient becomes
    # 2 gp, and both POW gradients add the terms of that upper gradient
    model.backward()
    gp2 = ORC.backward(0, OPS["MEAN"], np.ones(1, np.float32), pv, grad=gp)
    assert_bitexact(P.grads[sx].to_numpy(), ORC.backward(0, OPS["POW"], gp2, x, e, grad=ox), "grad x, second pass")
    assert_bitexact(P.grads[se].to_numpy(), gpu.backward(1, OPS["POW"], gp2, x, e, grad=got_e),
                    "grad exponent, second pass")


def test_model_grads_accumulate_until_zero_grad(gpu):
    m = gpu.m
    values = {"x": synth.normal((64, 48), 0, 1, 1230), "bias": synth.normal((1, 48), 0, 0.1, 1231)}
    nodes = _bias_relu_nodes() + [(OPS["MEAN"], ["r"], None, "l")]
    g, syms, inputs = native_graph(m, nodes, values, ["x", "bias"], params=["bias"])
    g.loss(syms["l"])
    model = m.Model(g)
    model.forward(values["x"])
    model.backward()
    g1 = model.parameters.grads[syms["bias"]].to_numpy()
    model.backward()
    g2 = model.parameters.grads[syms["bias"]].to_numpy()
    # nothing clears the intermediate gradients either (model.mojo:176-180 refills only the
    # loss gradient): grads[r] becomes 2c, grads[y] 3c', and the bias gradient g1 + 3 g1
    np.testing.assert_allclose(g2, 4 * g1, rtol=1e-5)
    model.parameters.grads.set_zero()
    assert not model.parameters.grads[syms["bias"]].to_numpy().any()
    model.backward()
    assert_bitexact(model.parameters.grads[syms["bias"]].to_numpy(), g1, "after zero_grad")


def test_model_inference_stops_at_last_output(gpu):
    m = gpu.m
    x = synth.normal((10, 6), 0, 1, 1240)
    g = m.Graph()
    sx = g.input((10, 6))
    a = g.op(m.OP.EXP, sx)
    g.out(a)
    b = g.op(m.OP.SUM, a)  # after the last output: not run by inference
    g.loss(b)
    model = m.Model(g)
    outs = model.inference(x)
    assert_bitexact(outs[0].to_numpy(), O.elwise_transform(OPS["EXP"], x), "inference output")
    assert not model.parameters.tensors[b].to_numpy().any()
    assert model.info()["n_inference_nodes"] == 1
    model.forward(x)
    assert model.parameters.tensors[b].to_numpy()[0] != 0


def test_model_device_inputs_and_errors(gpu):
    m = gpu.m
    x = synth.normal((8, 8), 0, 1, 1250)
    g = m.Graph()
    sx = g.input((8, 8), trainable=True)
    l = g.op(m.OP.SUM, g.op(m.OP.RELU, sx))
    g.loss(l)
    model = m.Model(g)
    a = model.forward(m.Tensor.from_numpy(x)).to_numpy()
    b = model.forward(x).to_numpy()
    assert_bitexact(a, b, "device and host inputs")
    with pytest.raises(m.MantleHipError):
        model.forward()
    with pytest.raises(m.MantleHipError):
        model.forward(np.zeros(63, np.float32))
    g2 = m.Graph()
    s2 = g2.input((4,))
    g2.op(m.OP.EXP, s2)
    m2 = m.Model(g2, inference_only=True)
    with pytest.raises(m.MantleHipError):
        m2.inference(np.zeros(4, np.float32))  # no graph output
    with pytest.raises(m.MantleHipError):
        m2.backward()  # no loss


def test_model_training_with_adam(gpu):
    """Model + Adam(model.parameters): three training steps against the same steps on the oracle
    (util.Graph over forward_op / backward_op, then Adam.step, optim.mojo:94-140). With 32 rows
    the weight and bias gradients (un-broadcasts over 32 rows) add each row in order on both
    sides, so every step's parameters are bit-exact."""
    m = gpu.m
    x = synth.normal((32, 32), 0, 1, 1260)
    w0 = synth.normal((1, 32), 0, 0.5, 1261)
    b0 = synth.normal((1, 32), 0, 0.1, 1262)
    g = m.Graph()
    sx = g.input((32, 32))
    sw = g.param((1, 32), init=w0)
    sb = g.param((1, 32), init=b0)
    h = g.op(m.OP.RELU, g.op(m.OP.ADD, g.op(m.OP.MUL, sx, sw), sb))
    l = g.op(m.OP.MEAN, g.op(m.OP.MUL, h, h))
    g.loss(l)
    model = m.Model(g)
    opt = m.Adam(model.parameters, lr=0.01)
    nodes = [(OPS["MUL"], ["x", "w"], None, "a"), (OPS["ADD"], ["a", "b"], None, "y"), (OPS["RELU"], ["y"], None, "h"),
             (OPS["MUL"], ["h", "h"], None, "hh"), (OPS["MEAN"], ["hh"], None, "l")]
    ref = Graph(nodes, ["w", "b"])
    st = {k: [v.copy(), np.zeros_like(v), np.zeros_like(v)] for k, v in (("w", w0), ("b", b0))}
    for it in range(1, 4):
        opt.zero_grad()
        model.forward(x)
        model.backward()
        opt.step()
        vals = ref.forward(ORC, {"x": x, "w": st["w"][0], "b": st["b"][0]})
        grads = ref.backward(ORC, vals)
        for k in ("w", "b"):
            st[k] = list(O.adam_step(st[k][0], grads[k], st[k][1], st[k][2], it, lr=0.01))
        assert_bitexact(model.parameters.tensors[sw].to_numpy(), st["w"][0], f"w step {it}")
        assert_bitexact(model.parameters.tensors[sb].to_numpy(), st["b"][0], f"b step {it}")
    assert opt.iter == 3


def test_model_param_span_layout_and_single_launch_adam(gpu):
    """Trainable parameters sit first in the tensor arena and their grads first in the grad
    arena, at the same offsets; Adam over the span matches Adam per tensor, and the padding
    between slots stays zero."""
    m = gpu.m
    g = m.Graph()
    x = g.input((6, 7))
    shapes = [(3, 7), (1, 7), (2, 3, 7)]
    ps = [g.param(s, init=synth.normal(s, 0, 1, 1270 + i)) for i, s in enumerate(shapes)]
    frozen = g.param((1, 7), init=np.ones(7, np.float32), trainable=False)
    a = g.op(m.OP.MUL, x, ps[1])
    b = g.op(m.OP.ADD, a, frozen)
    c = g.op(m.OP.MEAN, g.op(m.OP.MUL, b, b))
    d = g.op(m.OP.SUM, g.op(m.OP.MUL, ps[0], ps[0]))
    e = g.op(m.OP.MEAN, g.op(m.OP.TANH, ps[2]))
    loss = g.op(m.OP.ADD, g.op(m.OP.ADD, c, d), e)
    g.loss(loss)
    model = m.Model(g)
    span_p, span_g, n = model.parameters.param_span()
    P = model.parameters
    offs = []
    for s in ps:
        tp, tg = P.tensors[s].ptr, P.grads[s].ptr
        assert span_p <= tp < span_p + 4 * n and tg - span_g == tp - span_p
        offs.append((tp - span_p) // 4)
    assert not (span_p <= P.tensors[frozen].ptr < span_p + 4 * n)
    opt = m.Adam(model.parameters, lr=0.05)
    # the same updates through per-tensor Adam on copies
    cp = [m.Tensor.from_numpy(P.tensors[s].to_numpy()) for s in ps]
    cg = [m.Tensor(m.TensorShape(*s.shape.dims)) for s in ps]
    ref = m.Adam(list(zip(cp, cg)), lr=0.05)
    xv = synth.normal((6, 7), 0, 1, 1280)
    for it in range(3):
        opt.zero_grad()
        model.forward(xv)
        model.backward()
        for s, t in zip(ps, cg):
            m._lib.call("mh_memcpy_d2d", t.ptr, P.grads[s].ptr, s.shape.num_elements() * 4)
        opt.step()
        ref.step()
        for s, t in zip(ps, cp):
            assert_bitexact(P.tensors[s].to_numpy(), t.to_numpy(), f"param {s} step {it}")
    whole = m.Tensor(m.TensorShape(n), _ptr=span_p, _owner=model).to_numpy()
    used = np.zeros(n, bool)
    for s, o in zip(ps, offs):
        used[o:o + s.shape.num_elements()] = True
    assert not whole[~used].any(), "padding between parameter slots changed"


@pytest.mark.parametrize("which", ["bias_relu_fused", "config5"])
def test_model_graph_replay_matches_eager(gpu, which):
    """Captured forward / backward passes and the whole-step graph (zero_grad, forward, backward)
    replayed in turn with new inputs and host reads between replays; every replay bit-identical
    to an eager model."""
    m = gpu.m
    if which == "bias_relu_fused":
        nodes = _bias_relu_nodes() + [(OPS["MEAN"], ["r"], None, "l")]
        shape = (64, 32, 7, 7)
        values = {"x": synth.normal(shape, 0, 1, 1290), "bias": synth.normal((1, 32, 1, 1), 0, 0.1, 1291)}
        trainable, params, fuse = ["x", "bias"], ["bias"], True
        new_inputs = lambda it: {"x": synth.normal(shape, 0, 1, 1300 + it)}  # noqa: E731
    else:
        nodes = config5_nodes()
        rows = 4099
        onehot = np.zeros((rows, 10), np.float32)
        onehot[np.arange(rows), synth.integers((rows,), 0, 10, 1292)] = 1
        values = {"logits": synth.normal((rows, 10), 0, 2, 1293), "onehot": onehot}
        trainable, params, fuse = ["logits"], [], False
        new_inputs = lambda it: {"logits": synth.normal((rows, 10), 0, 2, 1310 + it), "onehot": onehot}  # noqa: E731
    models = []
    for _ in range(2):
        g, syms, inputs = native_graph(m, nodes, values, trainable, params)
        g.loss(syms[nodes[-1][3]])
        models.append((g, syms, inputs, m.Model(g, fuse_bias_relu=fuse)))
    (_, syms_a, inputs, eager), (_, syms_b, _, graphed) = models
    graphed.capture("forward")
    graphed.capture("backward")
    graphed.capture("step")
    for it in range(6):
        iv = new_inputs(it)
        eager.parameters.grads.set_zero()
        la = eager.forward(*[iv[n] for n in inputs]).to_numpy()
        eager.backward()
        for n in inputs:
            graphed.parameters.tensors[syms_b[n]] = iv[n]
        if it % 2 == 0:  # the two pass graphs, zero_grad eager between them
            graphed.parameters.grads.set_zero()
            lb = graphed.replay("forward").to_numpy()
            graphed.replay("backward")
        else:  # the whole step as one graph (zero_grad inside)
            lb = graphed.replay("step").to_numpy()
        assert_bitexact(lb, la, f"{which} loss, replay {it}")
        for name, sa in syms_a.items():
            sb = syms_b[name]
            assert_bitexact(graphed.parameters.tensors[sb].to_numpy(), eager.parameters.tensors[sa].to_numpy(),
                            f"{which} tensor {name}, replay {it}")
            if sa.trainable:
                assert_bitexact(graphed.parameters.grads[sb].to_numpy(), eager.parameters.grads[sa].to_numpy(),
                                f"{which} grad {name}, replay {it}")


def test_model_replay_requires_capture(gpu):
    m = gpu.m
    g = m.Graph()
    x = g.input((4, 4), trainable=True)
    g.loss(g.op(m.OP.SUM, x))
    model = m.Model(g)
    with pytest.raises(m.MantleHipError):
        model.replay("forward")



def _ce_graph(m, rows, classes, x_tr=True, extra=False):
    """nn.CrossEntropyLoss's nodes (loss.mojo:45-61) over x [rows, classes] (with `extra`, a
    second use of the Softmax output keeps that group unfused in its loss form)."""
    g = m.Graph()
    x = g.input((rows, classes), trainable=x_tr)
    t = g.input((rows, classes))
    mx = g.op(m.OP.MAX, x, attributes={"axis": 1})
    xm = g.op(m.OP.SUB, x, mx)
    e = g.op(m.OP.EXP, xm)
    s = g.op(m.OP.SUM, e, attributes={"axis": 1})
    ls = g.op(m.OP.LOG, s)
    lsm = g.op(m.OP.SUB, xm, ls)
    tl = g.op(m.OP.MUL, t, lsm)
    ret = g.op(m.OP.SUM, tl)
    loss = g.op(m.OP.MUL, ret, -1.0 / rows)
    if extra:
        loss = g.op(m.OP.ADD, loss, g.op(m.OP.MEAN, g.op(m.OP.MUL, lsm, lsm)))
    g.loss(loss)
    return g, x, t


def _oracle_row_graph(build, xv, tv):
    """(loss, grad_x, the loss's fp64 value and sum of |terms|, grad_x in fp64 with its
    magnitudes) of a row graph on the oracle, one forward_op / backward_op per node
    (util.Graph), and on the fp64 magnitude engine."""
    rows = xv.shape[0]
    if build == "head":
        nodes, vals0 = config5_nodes(), {"logits": xv, "onehot": tv}
        xname, tname, scale = "logits", "t", 1.0 / tv.size
    else:
        nodes = cross_entropy_nodes("x", "target")
        vals0 = {"x": xv, "target": tv, "cN": np.array([np.float32(-1.0 / rows)], np.float32)}
        xname, tname, scale = "x", "tl", float(np.float32(-1.0 / rows))
        if build == "ce_extra":
            nodes = nodes + [(OPS["MUL"], ["lsm", "lsm"], None, "sq"), (OPS["MEAN"], ["sq"], None, "msq"),
                             (OPS["ADD"], ["loss", "msq"], None, "total")]
    gr = Graph(nodes, [xname])
    v = gr.forward(ORC, vals0)
    gd = gr.backward(ORC, v)
    f64 = Mag64Engine()
    gx64 = gr.backward(f64, gr.forward(f64, vals0))[xname]
    terms = v[tname].astype(np.float64)
    ex, ab = terms.sum() * scale, np.abs(terms).sum() * abs(scale)
    if build == "ce_extra":
        sq = v["sq"].astype(np.float64)
        ex, ab = ex + sq.mean(), ab + np.abs(sq).mean()
    return v[nodes[-1][3]], gd[xname], ex, ab, gx64


@pytest.mark.parametrize("rows,classes", [(4099, 10), (300, 130), (64, 1000), (7, 1)])
def test_model_fused_rows_cross_entropy_and_head(gpu, rows, classes):
    """MH_MODEL_FUSE_ROWS: the cross-entropy group (and the config-5 head), fused and op by op,
    against the oracle: the loss in the sum class; grad_x bit-exact for rows shorter than the
    oracle's 32 SIMD lanes (row sums in element order on both sides), else in the fp64 sum
    class against the oracle (assert_order_close) and bit-identical between the fused and
    op-by-op models."""
    m = gpu.m
    xv = synth.normal((rows, classes), 0, 2, 1400)
    tv = synth.uniform((rows, classes), 0, 1, 1401)
    for build in ("ce", "ce_extra", "head"):
        results = []
        for fuse in (False, True):
            if build == "head":
                g, syms, inputs = native_graph(m, config5_nodes(), {"logits": xv, "onehot": tv}, ["logits"])
                g.loss(syms["loss"])
                x = syms["logits"]
                feed = [xv, tv]
            else:
                g, x, _ = _ce_graph(m, rows, classes, extra=build == "ce_extra")
                feed = [xv, tv]
            model = m.Model(g, fuse_rows=fuse)
            loss = model.forward(*feed).to_numpy()
            model.backward()
            results.append((loss, model.parameters.grads[x].to_numpy(), model.info()["fused_groups"]))
        (l0, g0, f0), (l1, g1, f1) = results
        assert f0 == 0 and f1 == 1, (build, f0, f1)
        ol, og, ex, ab, gx64 = _oracle_row_graph(build, xv, tv)
        for lv, gv, label in ((l0, g0, "op by op"), (l1, g1, "fused")):
            assert_sum_close(lv, ol, np.array([ex]), f"{build} {label} loss", terms_abs=np.array([ab]))
            if classes < 32:
                assert_bitexact(gv, og, f"{build} {label} grad_x vs oracle")
            else:
                assert_order_close(gv, og, gx64, f"{build} {label} grad_x vs oracle")
        assert_bitexact(g1, g0, f"{build} grad_x fused vs op by op")


@pytest.mark.parametrize("classes", [10, 257])
def test_model_fused_rows_softmax_inside_a_graph(gpu, classes):
    """A Softmax group whose output feeds later nodes: the output slot and every gradient
    outside the group are bit-identical to the unfused model."""
    m = gpu.m
    rows = 513
    xv = synth.normal((rows, classes), 0, 2, 1410)
    wv = synth.normal((1, classes), 0, 1, 1411)
    outs = []
    for fuse in (False, True):
        g = m.Graph()
        x = g.input((rows, classes), trainable=True)
        w = g.param((1, classes), init=wv)
        h = g.op(m.OP.MUL, x, w)
        mx = g.op(m.OP.MAX, h, attributes={"axis": 1})
        e = g.op(m.OP.EXP, g.op(m.OP.SUB, h, mx))
        sm = g.op(m.OP.DIV, e, g.op(m.OP.SUM, e, attributes={"axis": 1}))
        loss = g.op(m.OP.SUM, g.op(m.OP.TANH, sm))
        g.loss(loss)
        g.out(sm)
        model = m.Model(g, fuse_rows=fuse)
        l = model.forward(xv).to_numpy()
        model.backward()
        P = model.parameters
        outs.append((l, P.tensors[sm].to_numpy(), P.grads[x].to_numpy(), P.grads[w].to_numpy(),
                     model.info()["fused_groups"], model.inference(xv)[0].to_numpy()))
    (l0, s0, gx0, gw0, f0, i0), (l1, s1, gx1, gw1, f1, i1) = outs
    assert (f0, f1) == (0, 1)
    assert_bitexact(s1, s0, "softmax output")
    assert_bitexact(l1, l0, "loss")
    assert_bitexact(gx1, gx0, "grad x")
    assert_bitexact(gw1, gw0, "grad w")
    assert_bitexact(i1, i0, "inference output")
    # the same graph on the oracle: bit-exact below 32 classes (row sums in element order),
    # else rtol; the loss (all-element SUM) and grad w (un-broadcast over 513 rows) are sums
    nodes = [(OPS["MUL"], ["x", "w"], None, "h"), (OPS["MAX"], ["h"], 1, "mx"), (OPS["SUB"], ["h", "mx"], None, "hm"),
             (OPS["EXP"], ["hm"], None, "e"), (OPS["SUM"], ["e"], 1, "s"), (OPS["DIV"], ["e", "s"], None, "sm"),
             (OPS["TANH"], ["sm"], None, "th"), (OPS["SUM"], ["th"], None, "loss")]
    ref = Graph(nodes, ["x", "w"])
    v = ref.forward(ORC, {"x": xv, "w": wv})
    gd = ref.backward(ORC, v)
    th = v["th"].astype(np.float64)
    assert_sum_close(l1, v["loss"], np.array([th.sum()]), "loss vs oracle", terms_abs=np.array([np.abs(th).sum()]))
    # grad w sums 513 terms ug * x; from 32 classes its terms (grad h) also carry the order of
    # the row sums: the fp64 magnitude engine bounds both
    f64 = Mag64Engine()
    v64 = ref.forward(f64, {"x": xv, "w": wv})
    gd64 = ref.backward(f64, v64)
    if classes < 32:
        rgw = (gd["h"] * xv).astype(np.float64)
        assert_sum_close(gw1, gd["w"], rgw.sum(axis=0, keepdims=True), "grad w vs oracle",
                         terms_abs=np.abs(rgw).sum(axis=0, keepdims=True))
    else:
        assert_order_close(gw1, gd["w"], gd64["w"], "grad w vs oracle")
    for got, exp, e64, what in ((s1, v["sm"], v64["sm"], "softmax output"), (gx1, gd["x"], gd64["x"], "grad x")):
        if classes < 32:
            assert_bitexact(got, exp, f"{what} vs oracle")
        else:
            assert_order_close(got, exp, e64, f"{what} vs oracle")


GRAPH_FIXTURES = [c for c in load_fixtures() if c["kind"] == "graph"]


def _fixture_nodes(case):
    """(nodes, values, trainable, params) of a reference graph fixture: Softmax / LogSoftmax
    (activations.mojo:74-108), MSE (loss.mojo:25-38), CrossEntropyLoss (loss.mojo:45-61)."""
    t1 = spec_to_array(case["t1"])
    kind = case["graph"]
    if kind in ("softmax", "logsoftmax"):
        nodes = (softmax_nodes if kind == "softmax" else logsoftmax_nodes)("x", case["axis"])
        return nodes, {"x": t1}, ["x"], []
    t2 = spec_to_array(case["t2"])
    if kind == "mse":
        nodes = [(OPS["SUB"], ["yt", "yp"], None, "d"), (OPS["POW"], ["d", "two"], None, "p"),
                 (OPS["MEAN"], ["p"], None, "loss")]
        return nodes, {"yp": t1, "yt": t2, "two": np.array([2.0], np.float32)}, ["yp"], ["two"]
    nodes = logsoftmax_nodes("yp", 1) + [(OPS["MUL"], ["yt", "lsm"], None, "tl"), (OPS["SUM"], ["tl"], None, "s2"),
                                         (OPS["MUL"], ["s2", "negn"], None, "loss")]
    negn = np.array([np.float32(-1.0 / float(t1.shape[0]))], np.float32)
    return nodes, {"yp": t1, "yt": t2, "negn": negn}, ["yp"], ["negn"]


@pytest.mark.parametrize("fuse", [False, True])
@pytest.mark.parametrize("case", GRAPH_FIXTURES, ids=lambda c: c["id"])
def test_model_reference_graph_fixtures(gpu, case, fuse):
    """The reference's activation and loss tests (test_activations.mojo:105-140,
    test_loss.mojo:9-171) on the native Model, with row fusion off and on (Softmax / LogSoftmax
    over the last axis and CrossEntropyLoss then run as one row kernel each way): the output
    matches the tests' expected values at their tolerance, and the input gradient (from a
    seeded upper gradient, or the loss seed 1.0) is bit-exact against the oracle."""
    m = gpu.m
    nodes, values, trainable, params = _fixture_nodes(case)
    g, syms, inputs = native_graph(m, nodes, values, trainable, params)
    last = nodes[-1][3]
    is_loss = case["graph"] in ("mse", "crossentropy")
    if is_loss:
        g.loss(syms[last])
    g.out(syms[last])
    model = m.Model(g, fuse_rows=fuse)
    row_group = case["graph"] == "crossentropy" or (case.get("axis") == np.ndim(values["x" if "x" in values else "yp"]) - 1)
    assert model.info()["fused_groups"] == (1 if fuse and row_group else 0)
    out = model.inference(*[values[n] for n in inputs])[0].to_numpy()
    exp = spec_to_array(case["expected"])
    if case["tol"] == "almost6":
        np.testing.assert_allclose(out.reshape(exp.shape), exp, rtol=1e-5, atol=1e-8, err_msg=case["id"])
    else:
        np.testing.assert_allclose(out.reshape(exp.shape), exp, rtol=1e-5, atol=1e-5, err_msg=case["id"])
    ref = Graph(nodes, trainable)
    v = ref.forward(ORC, values)
    seed = None if is_loss else synth.normal(np.shape(v[last]), 0, 1, 1500)
    gd = ref.backward(ORC, v, seed)
    if is_loss:
        model.forward(*[values[n] for n in inputs])
        model.backward()
    else:
        model.backward(seed)
    xs = syms[trainable[0]]
    assert_bitexact(model.parameters.grads[xs].to_numpy().reshape(np.shape(gd[trainable[0]])), gd[trainable[0]],
                    f"{case['id']} grad")


@pytest.mark.parametrize("case", [c for c in GRAPH_FIXTURES if c["graph"] in ("softmax", "logsoftmax", "crossentropy")
                                  and c.get("axis", 1) == len(c["t1"]["shape"]) - 1], ids=lambda c: c["id"])
def test_fused_row_entry_points_reference_fixtures(gpu, case):
    """The reference's last-axis Softmax / LogSoftmax and CrossEntropyLoss fixtures through the
    fused entry points themselves (mh_softmax_*, mh_logsoftmax_*, mh_cross_entropy_*): forward
    against the expected values, backward (accumulated into a non-zero gradient) bit-exact
    against the oracle's graph backward."""
    m = gpu.m
    nodes, values, trainable, params = _fixture_nodes(case)
    xname = trainable[0]
    x = values[xname]
    rows, classes = int(np.prod(x.shape[:-1])), x.shape[-1]
    x2 = x.reshape(rows, classes)
    tx = gpu.T(x2)
    exp = spec_to_array(case["expected"])
    g0 = synth.normal((rows, classes), 0, 1, 1510)
    ref = Graph(nodes, trainable)
    v = ref.forward(ORC, values)
    if case["graph"] == "crossentropy":
        tt = gpu.T(values["yt"])
        loss = m.Tensor(m.TensorShape(1))
        m.cross_entropy_forward(loss, tx, tt)
        np.testing.assert_allclose(loss.to_numpy(), exp.reshape(-1), rtol=1e-5, atol=1e-8, err_msg=case["id"])
        seed = np.array([0.7], np.float32)
        gd = ref.backward(ORC, v, seed, init={xname: g0})
        tg = gpu.T(g0)
        m.cross_entropy_backward(tg, tx, tt, gpu.T(seed))
    else:
        fwd, bwd = ((m.softmax_forward, m.softmax_backward) if case["graph"] == "softmax"
                    else (m.logsoftmax_forward, m.logsoftmax_backward))
        out = m.Tensor(m.TensorShape(rows, classes))
        fwd(out, tx)
        np.testing.assert_allclose(out.to_numpy().reshape(exp.shape), exp, rtol=1e-5, atol=1e-5, err_msg=case["id"])
        assert_bitexact(out.to_numpy().reshape(exp.shape), v[nodes[-1][3]], f"{case['id']} output vs oracle")
        seed = synth.normal(x.shape, 0, 1, 1511)
        gd = ref.backward(ORC, v, seed, init={xname: g0.reshape(x.shape)})
        tg = gpu.T(g0)
        bwd(tg, tx, gpu.T(seed.reshape(rows, classes)))
    assert_bitexact(tg.to_numpy().reshape(x.shape), gd[xname], f"{case['id']} backward vs oracle")
