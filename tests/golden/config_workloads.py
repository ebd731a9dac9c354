"""The five configurations of BASELINE.json at their full sizes, as named outputs computed
through an engine of tests/util.py (OracleEngine for the committed golden fixture,
GpuEngine for the GPU test that checks the HIP path against it).

Inputs come from mantle_amd.synth (numpy SFC64 streams keyed by tensor id), so both sides
draw the same bytes. Every backward accumulates into a zeroed gradient, as the reference's
test harness does (tests/mojo/testing_utils.mojo:30-177). Each config is a generator of
(name, output, kind, exact, terms_abs):
  kind "bit": the output must match bit for bit (SHA-256 of the full array);
  kind "sum": a sum whose order differs between engines (the rtol class); `exact` is its
              fp64 value and `terms_abs` the fp64 sum of the terms' magnitudes.
"""
from __future__ import annotations

import numpy as np

from mantle_amd import synth

ADD, SUB, MUL, DIV, EXP, LOG, POW, SUM, MEAN, MAX, SIGMOID, RELU, TANH = 0, 1, 2, 3, 4, 5, 6, 8, 9, 10, 13, 14, 15
N2 = 1 << 28  # config 2: 2^28 elements per tensor


def _bit(name, out):
    return name, out, "bit", None, None


def _sum(name, out, exact, terms_abs):
    return name, out, "sum", exact, terms_abs


def config1(eng):
    """X [32,32] + bias [1,32] -> RELU; backward from ug ~ N(0,1)."""
    x = synth.normal((32, 32), 0, 1, 5001)
    bias = synth.normal((1, 32), 0, 0.1, 5002)
    ug = synth.normal((32, 32), 0, 1, 5003)
    y = eng.forward(ADD, x, bias)
    yield _bit("y", y)
    yield _bit("r", eng.forward(RELU, y))
    gy = eng.backward(0, RELU, ug, y)
    yield _bit("grad_y", gy)
    yield _bit("grad_x", eng.backward(0, ADD, gy, x, bias))
    g64 = gy.astype(np.float64)
    yield _sum("grad_bias", eng.backward(1, ADD, gy, x, bias), g64.sum(axis=0, keepdims=True),
               np.abs(g64).sum(axis=0, keepdims=True))


def config2_inputs():
    u = synth.uniform((1,), 0, 1, 5018)
    expo = np.array([np.float32(0.5) + np.float32(2.5) * u[0]], np.float32)
    return {"a": synth.uniform((N2,), -1, 1, 5011), "b": synth.uniform((N2,), 0.5, 2, 5012),
            "ug": synth.normal((N2,), 0, 1, 5013), "EXP": synth.uniform((N2,), -10, 10, 5014),
            "LOG": synth.uniform((N2,), 1e-3, 10, 5015), "ACT": synth.normal((N2,), 0, 3, 5016),
            "POW": synth.uniform((N2,), 0.1, 4, 5017), "expo": expo}


def config2(eng, inp, part):
    """2^28-element elementwise ops, forward and backward of each operand; `part` selects
    "binary", "unary" or "pow" (the GPU test runs them as separate tests)."""
    a, b, ug = inp["a"], inp["b"], inp["ug"]
    if part == "binary":
        for name, op in (("ADD", ADD), ("SUB", SUB), ("MUL", MUL), ("DIV", DIV)):
            yield _bit(f"{name}.fwd", eng.forward(op, a, b))
            yield _bit(f"{name}.bwd0", eng.backward(0, op, ug, a, b))
            yield _bit(f"{name}.bwd1", eng.backward(1, op, ug, a, b))
    elif part == "unary":
        for name, op, x in (("EXP", EXP, inp["EXP"]), ("LOG", LOG, inp["LOG"]), ("TANH", TANH, inp["ACT"]),
                            ("SIGMOID", SIGMOID, inp["ACT"]), ("RELU", RELU, inp["ACT"])):
            yield _bit(f"{name}.fwd", eng.forward(op, x))
            yield _bit(f"{name}.bwd", eng.backward(0, op, ug, x))
    else:
        x, e = inp["POW"], inp["expo"]
        yield _bit("POW.fwd", eng.forward(POW, x, e))
        for ev in (0.5, 1.5, 2.5):  # the Int(e) sweep 0, 1, 2
            yield _bit(f"POW.fwd.e{ev}", eng.forward(POW, x, np.array([ev], np.float32)))
        yield _bit("POW.bwd_x", eng.backward(0, POW, ug, x, e))
        a64, x64, u64 = np.float64(e[0]), x.astype(np.float64), ug.astype(np.float64)
        terms = np.power(x64, a64) * np.log(x64) * u64
        yield _sum("POW.bwd_exp", eng.backward(1, POW, ug, x, e), np.array([terms.sum()]),
                   np.array([np.abs(terms).sum()]))


def config3(eng):
    """x [256,32,28,28] + bias [1,32,1,1] -> RELU; backward from ug ~ N(0,1)."""
    shape, bshape = (256, 32, 28, 28), (1, 32, 1, 1)
    x = synth.normal(shape, 0, 1, 5021)
    bias = synth.normal(bshape, 0, 0.1, 5022)
    ug = synth.normal(shape, 0, 1, 5023)
    y = eng.forward(ADD, x, bias)
    yield _bit("y", y)
    yield _bit("r", eng.forward(RELU, y))
    gy = eng.backward(0, RELU, ug, y)
    yield _bit("grad_y", gy)
    yield _bit("grad_x", eng.backward(0, ADD, gy, x, bias))
    g64 = gy.astype(np.float64)
    yield _sum("grad_bias", eng.backward(1, ADD, gy, x, bias), g64.sum(axis=(0, 2, 3), keepdims=True),
               np.abs(g64).sum(axis=(0, 2, 3), keepdims=True))


C4_CASES = [("8192x8192", (8192, 8192), 0, "n"), ("8192x8192", (8192, 8192), 1, "n"),
            ("8192x8192", (8192, 8192), None, "n"), ("64x512x1024", (64, 512, 1024), 2, "u")]


def config4(eng, case):
    """SUM / MEAN / MAX forward and backward over one axis (or all elements) of a tie-injected
    tensor: half of the lines hold an exact copy of their maximum."""
    tag, shape, axis, dist = case
    x = synth.normal(shape, 0, 1, 5031) if dist == "n" else synth.uniform(shape, -1, 1, 5032)
    if axis is not None:
        synth.inject_ties(x, axis, 5033)
    else:
        x.reshape(-1)[x.size // 2] = x.max()
    red = (1,) if axis is None else tuple(1 if i == axis else d for i, d in enumerate(shape))
    d = x.size if axis is None else shape[axis]
    x64 = x.astype(np.float64)
    kd = dict(axis=axis, keepdims=True) if axis is not None else {}
    ex = np.asarray(x64.sum(**kd)).reshape(red)
    mag = np.asarray(np.abs(x64).sum(**kd)).reshape(red)
    del x64
    yield _sum("SUM.fwd", eng.forward(SUM, x, axis=axis), ex, mag)
    yield _sum("MEAN.fwd", eng.forward(MEAN, x, axis=axis), ex / d, mag / d)
    yield _bit("MAX.fwd", eng.forward(MAX, x, axis=axis))
    ug = synth.normal(red, 0, 1, 5034)
    for name, op in (("SUM", SUM), ("MEAN", MEAN), ("MAX", MAX)):
        yield _bit(f"{name}.bwd", eng.backward(0, op, ug, x, axis=axis))


def config5(eng):
    """The classifier head on logits [2^20, 10] ~ N(0, 2) and one-hot targets, forward and
    backward from the loss gradient 1.0, through the graph executor of tests/util.py."""
    from util import Graph, config5_nodes
    rows = 1 << 20
    logits = synth.normal((rows, 10), 0, 2, 5051)
    cls = synth.integers((rows,), 0, 10, 5052)
    onehot = np.zeros((rows, 10), np.float32)
    onehot[np.arange(rows), cls] = 1.0
    g = Graph(config5_nodes(), ["logits"])
    v = g.forward(eng, {"logits": logits, "onehot": onehot})
    for k in ("max", "xm", "e", "s", "sm", "lp", "t"):
        yield _bit(k, v[k])
    t64 = v["t"].astype(np.float64)
    yield _sum("loss", v["loss"], np.array([t64.mean()]), np.array([np.abs(t64).mean()]))
    gr = g.backward(eng, v, np.array([1.0], np.float32))
    for k in ("logits", "max", "xm", "e", "s", "sm", "lp", "t"):
        yield _bit(f"grad_{k}", gr[k])


def workloads():
    """(config, part) pairs in fixture order, with the generator that produces each."""
    return [("c1", None), ("c2", "binary"), ("c2", "unary"), ("c2", "pow"), ("c3", None)] + \
           [("c4", f"{c[0]}.{'all' if c[2] is None else 'ax%d' % c[2]}") for c in C4_CASES] + [("c5", None)]


def run(eng, config, part, cache):
    """Outputs of one workload; `cache` holds config 2's inputs between its parts."""
    if config == "c1":
        return config1(eng)
    if config == "c2":
        if "c2" not in cache:
            cache["c2"] = config2_inputs()
        return config2(eng, cache["c2"], part)
    if config == "c3":
        return config3(eng)
    if config == "c4":
        case = [c for c in C4_CASES if f"{c[0]}.{'all' if c[2] is None else 'ax%d' % c[2]}" == part][0]
        return config4(eng, case)
    return config5(eng)


SLICE = 256


def slice_idx(size: int, key: str) -> np.ndarray:
    """Seeded sample of indices (all of them for outputs of at most SLICE elements)."""
    if size <= SLICE:
        return np.arange(size)
    seed = int.from_bytes(key.encode(), "little") % (1 << 31)
    return np.sort(np.random.default_rng(seed).choice(size, SLICE, replace=False))
