"""Shared test helpers: fixture specs, comparators, the two engines (CPU oracle and the HIP
library) behind one interface, and a small graph executor that drives forward_op /
backward_op in the node order and trainable gating of Mantle's Model
(mantle/nn/model.mojo:113-330)."""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402  (test infrastructure: the checker)

OPS = {"ADD": 0, "SUB": 1, "MUL": 2, "DIV": 3, "EXP": 4, "LOG": 5, "POW": 6, "SUM": 8, "MEAN": 9,
       "MAX": 10, "SIGMOID": 13, "RELU": 14, "TANH": 15, "FMA": 19, "CLIP": 20, "LEAKYRELU": 28}
FMA, CLIP, LEAKYRELU = 19, 20, 28
BINARY = (0, 1, 2, 3)
UNARY = (4, 5, 13, 14, 15)
REDUCE = (8, 9, 10)


# ---------------------------------------------------------------------------------------
# fixtures
# ---------------------------------------------------------------------------------------
def load_fixtures():
    with open(os.path.join(ROOT, "tests", "golden", "reference_fixtures.json")) as f:
        return json.load(f)["cases"]


def spec_to_array(spec):
    if spec is None:
        return None
    shape = tuple(spec["shape"])
    n = int(np.prod(shape))
    if "fill" in spec:
        a = np.full(n, spec["fill"], dtype=np.float32)
    elif spec.get("arange1"):
        a = np.arange(1, n + 1, dtype=np.float32)
    else:
        a = np.asarray(spec["data"], dtype=np.float32).reshape(-1)
    for k, v in spec.get("set", {}).items():
        a[int(k)] = v
    return a.reshape(shape)


# ---------------------------------------------------------------------------------------
# comparators
# ---------------------------------------------------------------------------------------
def ordered(a: np.ndarray) -> np.ndarray:
    """float32 -> int64 with the same order (for ulp distances)."""
    i = np.asarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    return np.where(i < 0, -(i & 0x7FFFFFFF), i)


def ulp_dist(a, b) -> np.ndarray:
    return np.abs(ordered(a) - ordered(b))


def assert_bitexact(got, ref, what=""):
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    if not same.all():
        bad = np.flatnonzero(~same.reshape(-1))
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {got.size} differ; first at {i}: "
                             f"{got.reshape(-1)[i]!r} vs {ref.reshape(-1)[i]!r}")


def assert_ulp(got, ref, max_ulp, what=""):
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    both_nan = np.isnan(got) & np.isnan(ref)
    d = np.where(both_nan, 0, ulp_dist(got, ref))
    if d.max(initial=0) > max_ulp:
        i = int(np.argmax(d.reshape(-1)))
        raise AssertionError(f"{what}: max {d.max()} ulp > {max_ulp} at {i}: "
                             f"{got.reshape(-1)[i]!r} vs {ref.reshape(-1)[i]!r}")


def assert_sum_close(got, ref, exact64, what="", rtol=1e-5, terms_abs=None):
    """The rtol-1e-5 class for sums whose order differs: pass where |got - ref| <= rtol*|ref|,
    or where got is no farther from the fp64 sum than the reference is, or (if given) where
    |got - exact| <= rtol * sum|terms| (the conditioning bound for cancelling sums)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    ex = np.asarray(exact64, dtype=np.float64)
    ok = np.abs(got - ref) <= rtol * np.abs(ref)
    ok |= np.abs(got - ex) <= np.abs(ref - ex)
    if terms_abs is not None:
        ok |= np.abs(got - ex) <= rtol * np.asarray(terms_abs, dtype=np.float64)
    ok |= (got == ref)
    if not ok.all():
        i = int(np.flatnonzero(~ok.reshape(-1))[0])
        raise AssertionError(f"{what}: {int((~ok).sum())} sums out of tolerance; first at {i}: "
                             f"got {got.reshape(-1)[i]!r} ref {ref.reshape(-1)[i]!r} "
                             f"fp64 {ex.reshape(-1)[i]!r}")


def _ulp32(v) -> np.ndarray:
    return np.spacing(np.abs(np.asarray(v, np.float64)).astype(np.float32)).astype(np.float64)


def assert_order_close(got, ref, exact, what="", rtol=1e-5):
    """The sum class for values that depend on sums whose order differs (the GPU's fixed order
    against the reference's lane-striped one). `exact` is an Mag64 value: the fp64 evaluation of
    the same graph and, per element, the first-order magnitude M of everything a different
    order of its sums can change. An element passes when it equals the reference, or is no
    farther from fp64 than the reference is (plus 2 ulp), or lies within rtol * M of fp64 or of
    the reference (the last covers values that both float32 evaluations share a larger error
    in, such as subnormal intermediates)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    ex = np.asarray(exact.v, dtype=np.float64).reshape(got.shape)
    mag = np.asarray(exact.M, dtype=np.float64).reshape(got.shape)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    with np.errstate(invalid="ignore"):
        ok = (got == ref) | (np.isnan(got) & np.isnan(ref))
        ok |= np.abs(got - ex) <= np.abs(ref - ex) + 2 * _ulp32(ex)
        ok |= np.abs(got - ex) <= rtol * mag
        ok |= np.abs(got - ref) <= rtol * mag
    if not ok.all():
        i = int(np.flatnonzero(~ok.reshape(-1))[0])
        raise AssertionError(f"{what}: {int((~ok).sum())} of {ok.size} out of the sum class; first at {i}: "
                             f"got {got.reshape(-1)[i]!r} ref {ref.reshape(-1)[i]!r} fp64 {ex.reshape(-1)[i]!r} "
                             f"M {mag.reshape(-1)[i]!r}")


def assert_almost(got, ref, what="", rtol=1e-5, atol=1e-5):
    """testing_utils.mojo:16-27 'almost': rtol = atol = 1e-5 per element."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    ok = np.abs(got - ref) <= atol + rtol * np.abs(ref)
    if not ok.all():
        i = int(np.flatnonzero(~ok.reshape(-1))[0])
        raise AssertionError(f"{what}: {got.reshape(-1)[i]!r} vs {ref.reshape(-1)[i]!r} at {i}")


# ---------------------------------------------------------------------------------------
# engines
# ---------------------------------------------------------------------------------------
def _clip_bounds(attrs):
    attrs = attrs or {}
    return float(attrs.get("min", -O.FLT_MAX)), float(attrs.get("max", O.FLT_MAX))


class OracleEngine:
    name = "oracle"

    def forward(self, op, t1, t2=None, axis=None, attrs=None, t3=None):
        if op == FMA:
            return O.fma_fwd(t1, t2, t3)
        if op == LEAKYRELU:
            return O.leakyrelu_fwd(t1, attrs["negative_slope"])
        if op == CLIP:
            return O.clip_fwd(t1, *_clip_bounds(attrs))
        return O.forward_op(op, t1, t2, axis)

    def backward(self, tensor_id, op, ug, t1, t2=None, axis=None, grad=None, attrs=None):
        if op in (FMA, LEAKYRELU, CLIP):
            g = np.zeros(np.shape(t1), np.float32) if grad is None else grad
            if op == FMA:
                return O.fma_bwd_accum(tensor_id, g, ug, t1, t2)
            if op == LEAKYRELU:
                return O.leakyrelu_bwd_accum(g, t1, ug, attrs["negative_slope"])
            return O.clip_bwd_accum(g, t1, ug, *_clip_bounds(attrs))
        return O.backward_op(tensor_id, op, ug, t1, t2, grad=grad, axis=axis)

    def tstd(self, t1, axis=None):
        return O.tstd(t1, axis)



class Mag64:
    """A value of the fp64 magnitude engine: v, the fp64 evaluation, and M, the first-order
    magnitude of what the order of sums can change in it (Sum |terms| through every sum,
    carried through each op by its derivative, plus |v| for the op's own rounding). Arrays
    compare and reshape through `v`, so the graph executor handles these like numpy arrays."""
    __slots__ = ("v", "M")

    def __init__(self, v, M=None):
        self.v = np.asarray(v, np.float64)
        self.M = np.zeros(self.v.shape) if M is None else np.broadcast_to(np.asarray(M, np.float64), self.v.shape)

    @property
    def shape(self):
        return self.v.shape

    def __array__(self, dtype=None, copy=None):
        return self.v if dtype is None else self.v.astype(dtype)


def _mag(a):
    if a is None or isinstance(a, Mag64):
        return a
    return Mag64(np.asarray(a, np.float64))


def _pm(*factors):
    """Product of the factors' magnitudes, with 0 * inf = 0: a term whose derivative vanishes
    (a clamped exp, a relu below zero) carries nothing, even from an infinite operand."""
    out = np.ones(())
    zero = np.zeros((), bool)
    for f in factors:
        f = np.abs(np.asarray(f, np.float64))
        zero = zero | (f == 0)
        with np.errstate(invalid="ignore", over="ignore"):
            out = out * f
    return np.where(zero, 0.0, out)


_FLT_MIN = float(np.finfo(np.float32).tiny)


def _own(v):
    """The magnitude of one float32 rounding of v: |v|, or FLT_MIN for a subnormal result
    (its rounding error is absolute, 2^-150, not relative)."""
    return np.maximum(np.abs(v), _FLT_MIN)


def _unbroadcast_mag(v, M, shape):
    """Sums v (and M + |v|, a sum's own magnitude) over the axes that broadcast `shape` to v's."""
    while v.ndim > len(shape):
        M, v = (M + np.abs(v)).sum(axis=0), v.sum(axis=0)
    for ax, d in enumerate(shape):
        if d == 1 and v.shape[ax] != 1:
            M, v = (M + np.abs(v)).sum(axis=ax, keepdims=True), v.sum(axis=ax, keepdims=True)
    return v, M


_EXP_LO, _EXP_HI = float(np.float32(-88.3762626647949)), float(np.float32(88.3762626647950))


class Mag64Engine:
    """The path's ops in fp64 with first-order magnitudes (see Mag64), behind the engines'
    forward / backward interface. Each value is the reference expression in exact arithmetic
    (exp clamps its argument to +-88.376 as the reference's exp does, POW truncates its
    exponent as POW.forward does, MAX splits ties as fl(1/c) * ug with the same count, CLIP and
    LEAKYRELU keep the oracle's boundary rules); M bounds, to first order, how far two float32
    evaluations that differ only in the order of their sums can move apart (in units of the
    relative rounding error)."""
    name = "fp64"

    @staticmethod
    def _unary(op, a, attrs):
        """(value, its derivative, the factor the reference's backward multiplies ug by, that
        factor's derivative) of a unary op at a. The factor is the derivative except for exp
        beyond its clamp, where the reference's backward still multiplies by E(x)."""
        if op == OPS["EXP"]:
            e = np.exp(np.clip(a, _EXP_LO, _EXP_HI))
            d = np.where((a >= _EXP_LO) & (a <= _EXP_HI), e, 0.0)  # flat beyond the clamp
            return e, d, e, d
        if op == OPS["LOG"]:
            with np.errstate(divide="ignore", invalid="ignore"):
                return np.log(a), 1 / a, 1 / a, -1 / (a * a)
        if op == OPS["TANH"]:
            t = np.tanh(a)
            d = 1 - t * t
            return t, d, d, -2 * t * d
        if op == OPS["SIGMOID"]:
            s = 1 / (1 + np.exp(-a))
            d = s * (1 - s)
            return s, d, d, d * (1 - 2 * s)
        zero = np.zeros(a.shape)
        if op == OPS["RELU"]:
            d = (a > 0).astype(np.float64)
            return np.where(a > 0, a, 0.0), d, d, zero
        if op == LEAKYRELU:
            d = np.where(a > 0, 1.0, float(np.float32(attrs["negative_slope"])))
            return a * d, d, d, zero
        if op == CLIP:
            lo, hi = _clip_bounds(attrs)
            d = ((a >= lo) & (a <= hi)).astype(np.float64)
            return np.clip(a, lo, hi), d, d, zero
        raise AssertionError(f"fp64 engine: op {op}")

    def forward(self, op, t1, t2=None, axis=None, attrs=None, t3=None):
        A, B = _mag(t1), _mag(t2)
        a, Ma = A.v, A.M
        if op in REDUCE:
            if op == OPS["MAX"]:
                if axis is None:
                    return Mag64([a.max()], [Ma.max()])
                return Mag64(a.max(axis=axis, keepdims=True), Ma.max(axis=axis, keepdims=True))
            n = a.size if axis is None else a.shape[axis]
            sc = 1.0 / n if op == OPS["MEAN"] else 1.0
            if axis is None:
                return Mag64([a.sum() * sc], [(Ma + np.abs(a)).sum() * sc])
            return Mag64(a.sum(axis=axis, keepdims=True) * sc, (Ma + np.abs(a)).sum(axis=axis, keepdims=True) * sc)
        with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
            if op == FMA:
                C = _mag(t3)
                b, Mb = B.v, B.M
                v = a * b + C.v
                return Mag64(v, _pm(Ma, b) + _pm(a, Mb) + C.M + _own(v))
            if op == OPS["POW"]:
                p = float(np.trunc(B.v.reshape(-1)[0]))
                v = a ** p
                return Mag64(v, (_pm(p * a ** (p - 1), Ma) if p else 0.0) + _own(v))
            if op in BINARY:
                b, Mb = B.v, B.M
                if op == OPS["ADD"]:
                    v, M = a + b, Ma + Mb
                elif op == OPS["SUB"]:
                    v, M = a - b, Ma + Mb
                elif op == OPS["MUL"]:
                    v, M = a * b, _pm(Ma, b) + _pm(a, Mb)
                else:
                    v, M = a / b, _pm(Ma, 1 / b) + _pm(a, Mb, 1 / (b * b))
                return Mag64(v, M + _own(v))
            v, d1, _, _ = self._unary(op, a, attrs)
            return Mag64(v, _pm(d1, Ma) + _own(v))

    def backward(self, tensor_id, op, ug, t1, t2=None, axis=None, grad=None, attrs=None):
        U, A, B = _mag(ug), _mag(t1), _mag(t2)
        u, Mu, a, Ma = U.v, U.M, A.v, A.M
        tshape = a.shape if tensor_id != 1 or B is None else B.v.shape
        with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
            if op in REDUCE:
                n = a.size if axis is None else a.shape[axis]
                uu, MM = (u, Mu) if axis is not None else (u.reshape(-1)[0], Mu.reshape(-1)[0])
                if op == OPS["MAX"]:
                    m = a.max(axis=axis, keepdims=axis is not None)
                    eq = a == m
                    c = eq.sum(axis=axis, keepdims=axis is not None)
                    rg = np.where(eq, uu / c, 0.0)
                    M = np.where(eq, MM / c, 0.0) + _own(rg)
                else:
                    sc = 1.0 / n if op == OPS["MEAN"] else 1.0
                    rg = np.broadcast_to(uu * sc, a.shape)
                    M = np.broadcast_to(MM * sc, a.shape)
            elif op in BINARY or op == FMA:
                b, Mb = B.v, B.M
                if op == OPS["ADD"] or (op == FMA and tensor_id == 2):
                    rg, M = u, Mu
                elif op == OPS["SUB"]:
                    rg, M = (u, Mu) if tensor_id == 0 else (-u, Mu)
                elif op in (OPS["MUL"], FMA):
                    o, Mo = (b, Mb) if tensor_id == 0 else (a, Ma)
                    rg = u * o
                    M = _pm(Mu, o) + _pm(u, Mo) + _own(rg)
                elif tensor_id == 0:
                    rg = u / b
                    M = _pm(Mu, 1 / b) + _pm(u, Mb, 1 / (b * b)) + _own(rg)
                else:
                    rg = u * (-a / (b * b))
                    M = _pm(Mu, a, 1 / (b * b)) + _pm(u, Ma, 1 / (b * b)) + 2 * _pm(u, a, Mb, 1 / (b * b * b)) \
                        + _own(rg)
            elif op == OPS["POW"]:
                if tensor_id != 0:
                    raise AssertionError("fp64 engine: POW exponent gradient")
                p = float(B.v.reshape(-1)[0])
                d1, d2 = p * a ** (p - 1), p * (p - 1) * a ** (p - 2)
                rg = u * d1
                M = _pm(Mu, d1) + _pm(u, d2, Ma) + _own(rg)
            else:
                _, _, f, df = self._unary(op, a, attrs)
                rg = u * f
                M = _pm(Mu, f) + _pm(u, df, Ma) + _own(rg)
            rg, M = _unbroadcast_mag(np.asarray(rg, np.float64), np.asarray(M, np.float64), tshape)
            G = _mag(np.zeros(tshape) if grad is None else grad)
            v = G.v + rg
            return Mag64(v, G.M + M + _own(v))


# MANTLE_TEST_ASYNC=1 runs the GPU tests with the library in MH_INIT_ASYNC mode (no stream
# synchronisation at the end of each call, as bench.py runs it): every host boundary must
# synchronise by itself for the results to hold.
TEST_ASYNC = os.environ.get("MANTLE_TEST_ASYNC") == "1"


class GpuEngine:
    """Runs each op through mantle_amd (libmantle_hip.so) with host round trips (tests only)."""
    name = "gpu"

    def __init__(self):
        import mantle_amd
        self.m = mantle_amd
        mantle_amd.init(0, asynchronous=TEST_ASYNC)

    def T(self, a):
        return self.m.Tensor.from_numpy(np.asarray(a, dtype=np.float32))

    @staticmethod
    def _attrs(axis, attrs):
        if axis is None and not attrs:
            return None
        d = dict(attrs or {})
        if axis is not None:
            d["axis"] = axis
        return d

    def forward(self, op, t1, t2=None, axis=None, attrs=None, t3=None):
        m = self.m
        a = self.T(t1)
        b = self.T(t2) if t2 is not None else None
        c = self.T(t3) if t3 is not None else None
        shapes = [x.shape() for x in (a, b, c) if x is not None]
        at = self._attrs(axis, attrs)
        res = m.Tensor(m.static_result_shape(op, *shapes, attributes=at))
        m.forward_op(op, res, a, b, attributes=at, t3=c)
        return res.to_numpy()

    def backward(self, tensor_id, op, ug, t1, t2=None, axis=None, grad=None, attrs=None):
        m = self.m
        a = self.T(t1)
        b = self.T(t2) if t2 is not None else None
        u = self.T(ug)
        gshape = np.asarray(t1 if tensor_id != 1 or t2 is None else t2).shape or (1,)
        g = self.T(np.zeros(gshape, np.float32) if grad is None else grad)
        m.backward_op(tensor_id, op, u, a, b, g, attributes=self._attrs(axis, attrs))
        return g.to_numpy()

    def tstd(self, t1, axis=None):
        return self.m.tstd(self.T(t1), -1 if axis is None else axis).to_numpy()


# ---------------------------------------------------------------------------------------
# graph executor (Model semantics on numpy arrays, one engine call per node)
# ---------------------------------------------------------------------------------------
class Graph:
    """nodes: (op, [input names], axis, output name). Symbols not produced by a node are
    inputs; `trainable` names those with a grad. Node outputs are trainable when any operand
    is (graph.mojo:212-217)."""

    def __init__(self, nodes, trainable=()):
        self.nodes = nodes
        self.trainable = set(trainable)
        for op, ins, ax, out in nodes:
            if any(i in self.trainable for i in ins):
                self.trainable.add(out)

    def forward(self, eng, values):
        vals = dict(values)
        for op, ins, ax, out in self.nodes:
            t1 = vals[ins[0]]
            t2 = vals[ins[1]] if len(ins) > 1 else None
            vals[out] = eng.forward(op, t1, t2, ax)
        return vals

    def backward(self, eng, vals, seed=None, init=None):
        """Model.backward (model.mojo:173-330): seed the last node's grad (1.0 for a loss, else
        `seed`), then reverse node order, operands gated on trainable. `init` gives starting
        values of chosen grads (zero otherwise)."""
        grads = {k: np.zeros(np.asarray(v).shape, np.float32) for k, v in vals.items() if k in self.trainable}
        for k, v in (init or {}).items():
            grads[k] = np.asarray(v, np.float32).copy()
        last = self.nodes[-1][3]
        grads[last] = np.ones(np.asarray(vals[last]).shape, np.float32) if seed is None else \
            np.asarray(seed, np.float32).copy()
        for op, ins, ax, out in reversed(self.nodes):
            t1 = vals[ins[0]]
            t2 = vals[ins[1]] if len(ins) > 1 else None
            for k, name in enumerate(ins):
                if name in self.trainable:
                    grads[name] = eng.backward(k, op, grads[out], t1, t2, ax, grad=grads[name])
        return grads


def native_graph(m, nodes, values, trainable=(), params=()):
    """The util Graph node list as a mantle_amd.Graph: names not produced by a node become
    inputs (in order of first use), or parameters holding their value when listed in
    `params`; node outputs are op symbols. Returns (graph, {name: Symbol}, [input names])."""
    g = m.Graph()
    syms, inputs = {}, []
    produced = {n[3] for n in nodes}
    for op, ins, ax, out in nodes:
        for name in ins:
            if name in syms or name in produced:
                continue
            shape = np.asarray(values[name]).shape or (1,)
            if name in params:
                syms[name] = g.param(shape, init=values[name], trainable=name in trainable)
            else:
                syms[name] = g.input(shape, trainable=name in trainable)
                inputs.append(name)
        attrs = {"axis": ax} if ax is not None else None
        syms[out] = g.op(op, *[syms[i] for i in ins], attributes=attrs)
    return g, syms, inputs


def softmax_nodes(x, axis, prefix=""):
    """Softmax graph, mantle/nn/activations.mojo:74-87."""
    p = prefix
    return [(OPS["MAX"], [x], axis, p + "max"), (OPS["SUB"], [x, p + "max"], None, p + "xm"),
            (OPS["EXP"], [p + "xm"], None, p + "e"), (OPS["SUM"], [p + "e"], axis, p + "s"),
            (OPS["DIV"], [p + "e", p + "s"], None, p + "sm")]


def cross_entropy_nodes(x, target, prefix=""):
    """CrossEntropyLoss graph, mantle/nn/loss.mojo:45-61: LogSoftmax(axis 1), MUL(target, .),
    SUM, MUL(., cN) with cN the graph scalar f32(-1 / rows)."""
    p = prefix
    return logsoftmax_nodes(x, 1, p) + [(OPS["MUL"], [target, p + "lsm"], None, p + "tl"),
                                        (OPS["SUM"], [p + "tl"], None, p + "ret"),
                                        (OPS["MUL"], [p + "ret", p + "cN"], None, p + "loss")]


def config5_nodes():
    """Config 5: MAX(ax1) -> SUB -> EXP -> SUM(ax1) -> DIV -> LOG -> MUL(onehot) -> MEAN."""
    return softmax_nodes("logits", 1) + [(OPS["LOG"], ["sm"], None, "lp"), (OPS["MUL"], ["lp", "onehot"], None, "t"),
                                         (OPS["MEAN"], ["t"], None, "loss")]


def logsoftmax_nodes(x, axis, prefix=""):
    """LogSoftmax graph, mantle/nn/activations.mojo:94-108."""
    p = prefix
    return [(OPS["MAX"], [x], axis, p + "max"), (OPS["SUB"], [x, p + "max"], None, p + "xm"),
            (OPS["EXP"], [p + "xm"], None, p + "e"), (OPS["SUM"], [p + "e"], axis, p + "s"),
            (OPS["LOG"], [p + "s"], None, p + "ls"), (OPS["SUB"], [p + "xm", p + "ls"], None, p + "lsm")]


def run_fixture_graph(eng, case):
    kind = case["graph"]
    t1 = spec_to_array(case["t1"])
    if kind in ("softmax", "logsoftmax"):
        nodes = (softmax_nodes if kind == "softmax" else logsoftmax_nodes)("x", case["axis"])
        vals = Graph(nodes).forward(eng, {"x": t1})
        return vals[nodes[-1][3]]
    t2 = spec_to_array(case["t2"])
    if kind == "mse":  # mantle/nn/loss.mojo:25-38: SUB(y_true, y_pred) -> POW 2 -> MEAN
        two = np.array([2.0], np.float32)
        nodes = [(OPS["SUB"], ["yt", "yp"], None, "d"), (OPS["POW"], ["d", "two"], None, "p"),
                 (OPS["MEAN"], ["p"], None, "loss")]
        return Graph(nodes).forward(eng, {"yp": t1, "yt": t2, "two": two})["loss"]
    # crossentropy, mantle/nn/loss.mojo:45-61: -1/N * SUM(y_true * logsoftmax(y_pred, 1))
    negn = np.array([np.float32(-1.0 / float(t1.shape[0]))], np.float32)
    nodes = logsoftmax_nodes("yp", 1) + [(OPS["MUL"], ["yt", "lsm"], None, "tl"),
                                         (OPS["SUM"], ["tl"], None, "s2"),
                                         (OPS["MUL"], ["s2", "negn"], None, "loss")]
    return Graph(nodes).forward(eng, {"yp": t1, "yt": t2, "negn": negn})["loss"]


def check_fixture(eng, case):
    """Runs one reference fixture on `eng` and checks it against its expected values."""
    tol = case["tol"]

    def cmp(got, exp, what):
        if tol == "exact":
            np.testing.assert_array_equal(np.asarray(got, np.float32), exp, err_msg=what)
        elif tol == "almost6":
            assert_almost(got, exp, what, rtol=1e-5, atol=1e-8)
        else:
            assert_almost(got, exp, what)

    kind = case["kind"]
    attrs = case.get("attrs")
    if kind == "forward":
        op = OPS[case["op"]]
        got = eng.forward(op, spec_to_array(case["t1"]), spec_to_array(case["t2"]), case["axis"], attrs=attrs,
                          t3=spec_to_array(case.get("t3")))
        cmp(got, spec_to_array(case["expected"]), case["id"])
    elif kind == "backward":
        op = OPS[case["op"]]
        t1, t2, ug = spec_to_array(case["t1"]), spec_to_array(case["t2"]), spec_to_array(case["ug"])
        g1 = eng.backward(0, op, ug, t1, t2, case["axis"], attrs=attrs)
        cmp(g1, spec_to_array(case["grad1"]), case["id"] + " grad1")
        if case.get("grad2") is not None:
            g2 = eng.backward(1, op, ug, t1, t2, case["axis"], attrs=attrs)
            cmp(g2, spec_to_array(case["grad2"]), case["id"] + " grad2")
    elif kind == "tstd":
        cmp(eng.tstd(spec_to_array(case["t1"]), case["axis"]), spec_to_array(case["expected"]), case["id"])
    elif kind == "graph":
        cmp(run_fixture_graph(eng, case), spec_to_array(case["expected"]), case["id"])
    else:
        raise AssertionError(f"unknown fixture kind {kind}")
