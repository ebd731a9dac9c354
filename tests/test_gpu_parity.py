"""GPU parity: the HIP path (libmantle_hip.so through the C ABI) against the CPU oracle on the
same seeded inputs, at sizes the oracle finishes in seconds, plus the reference fixtures.

Bars (written per assertion): bit-exact for add/sub/mul/div, relu, max, broadcast gathers and
every backward that is a single expression per element; <= 2 ulp for exp/log/sigmoid/tanh/pow
(the kernels use the same algorithm as the oracle, so these are expected bit-exact too); the
rtol 1e-5 class with the condition-aware comparator for sums whose order differs."""
import numpy as np
import pytest

from mantle_amd import synth
from util import (O, OPS, GpuEngine, Graph, Mag64Engine, OracleEngine, config5_nodes, assert_bitexact,
                  assert_order_close, assert_sum_close, assert_ulp, check_fixture, load_fixtures)

pytestmark = pytest.mark.gpu

ORC = OracleEngine()


@pytest.fixture(scope="module")
def gpu():
    print("\n[gpu] init device 0", flush=True)
    return GpuEngine()


# ---------------------------------------------------------------------------------------
# reference fixtures
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", [c for c in load_fixtures() if c["kind"] != "accumulate"], ids=lambda c: c["id"])
def test_reference_fixture_on_gpu(gpu, case):
    check_fixture(gpu, case)


def test_accumulate_fixture_on_gpu(gpu):
    m = gpu.m
    g = m.Tensor(m.TensorShape(2, 1, 1))
    rg = gpu.T(np.full((2, 3, 4), 3.0, np.float32))
    m.accumulate_grad(g, rg)
    np.testing.assert_array_equal(g.to_numpy(), np.full((2, 1, 1), 36.0, np.float32))
    with pytest.raises(m.MantleHipError):
        m.accumulate_grad(m.Tensor(m.TensorShape(2, 1)), rg)


# ---------------------------------------------------------------------------------------
# binary ops: forward bit-exact, backward per operand
# ---------------------------------------------------------------------------------------
BIN_SHAPES = [((37, 63, 107), (37, 63, 107)), ((37, 63, 107), (37, 63, 1)), ((37, 63, 1), (37, 63, 107)),
              ((2, 3, 4), (5, 2, 1, 4)), ((1001,), (1,)), ((1,), (1001,)), ((32, 32), (1, 32)),
              ((4, 32, 7, 7), (1, 32, 1, 1)), ((4099, 10), (4099, 1)), ((8, 1, 5), (1, 6, 1)),
              ((3,), (3,)), ((1,), (1,)), ((7, 5), (5,)), ((2, 1, 3, 1, 5), (1, 4, 3, 6, 1)),
              ((5, 3), (5, 1)), ((7, 2), (1, 2)), ((9, 1, 3), (9, 4, 1)), ((1023, 6), (1023, 1)),
              ((65, 4), (65, 1)), ((1001, 5), (1001, 1)), ((6, 2, 13), (6, 2, 1)),
              # a full and a broadcast operand in both orders through the column, plane and
              # general engines (their compile-time kind pairs)
              ((1, 32), (32, 32)), ((4, 32, 8, 8), (1, 32, 1, 1)), ((1, 32, 1, 1), (4, 32, 8, 8)),
              ((6, 5, 16), (6, 1, 16)), ((6, 1, 16), (6, 5, 16)), ((1, 5, 16), (6, 5, 16))]


def _dim(rng, big):
    """A dimension: often tiny (1-9, where the short-row and LDS forms apply), else 10-300 or,
    for one axis of a case, up to `big` (row chunks, wide and strip column splits)."""
    u = rng.random()
    if u < 0.35:
        return int(rng.integers(1, 10))
    if u < 0.8:
        return int(rng.integers(10, 301))
    return int(rng.integers(301, big + 1))


def _seeded_bin_shapes(count, seed):
    """Broadcast pairs drawn with a fixed seed: an output of rank 1-5 and up to 2^18 elements,
    each operand a copy with some axes set to 1 and, sometimes, leading axes dropped."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        r = int(rng.integers(1, 6))
        shape = [_dim(rng, 3000) for _ in range(r)]
        if int(np.prod(shape)) > (1 << 18):
            continue
        ops = []
        for _ in range(2):
            sh = [d if rng.random() < 0.6 else 1 for d in shape]
            drop = int(rng.integers(0, r)) if rng.random() < 0.3 else 0
            ops.append(tuple(sh[drop:]) or (1,))
        if tuple(np.broadcast_shapes(*ops)) != tuple(shape) and rng.random() < 0.5:
            continue  # keep most pairs at the full output shape
        out.append((ops[0], ops[1]))
    return out


# seeded shapes beside the chosen ones: launch forms in combinations nobody picked by hand
BIN_SHAPES += _seeded_bin_shapes(20, 20261202)


def _binary_inputs(sa, sb, seed):
    a = synth.uniform(sa, -1, 1, seed)
    b = synth.uniform(sb, 0.5, 2, seed + 1)
    return a, b


@pytest.mark.parametrize("op", [0, 1, 2, 3], ids=["ADD", "SUB", "MUL", "DIV"])
@pytest.mark.parametrize("sa,sb", BIN_SHAPES, ids=[f"{a}x{b}" for a, b in BIN_SHAPES])
def test_binary_fwd_bwd_parity(gpu, op, sa, sb):
    a, b = _binary_inputs(sa, sb, 100 + op)
    assert_bitexact(gpu.forward(op, a, b), ORC.forward(op, a, b), f"fwd op{op}")
    out_shape = np.broadcast_shapes(sa, sb)
    ug = synth.normal(out_shape, 0, 1, 200 + op)
    for k, shape in ((0, sa), (1, sb)):
        g0 = synth.normal(shape, 0, 1, 300 + k)  # accumulate into a non-zero grad
        got = gpu.backward(k, op, ug, a, b, grad=g0)
        ref = ORC.backward(k, op, ug, a, b, grad=g0)
        if tuple(shape) == tuple(out_shape):
            assert_bitexact(got, ref, f"bwd op{op} id{k}")
        else:  # un-broadcast: a sum over the broadcast axes in a different order
            A, B, U = (v.astype(np.float64) for v in (a, b, ug))
            rg = {0: U, 1: (U if k == 0 else -U), 2: (U * B if k == 0 else U * A),
                  3: (U / B if k == 0 else -A / (B * B) * U)}[op]
            red = tuple(i for i in range(len(out_shape)) if i >= len(out_shape) - len(shape) and
                        shape[i - (len(out_shape) - len(shape))] == 1 and out_shape[i] != 1) + \
                tuple(range(len(out_shape) - len(shape)))
            ex = (rg.sum(axis=red, keepdims=True).reshape(shape) + g0.astype(np.float64))
            mag = np.abs(rg).sum(axis=red, keepdims=True).reshape(shape) + np.abs(g0)
            assert_sum_close(got, ref, ex, f"bwd op{op} id{k}", terms_abs=mag)


# (full shape, broadcast operand): un-broadcasts that are one reduction along lines of at
# most 64 elements -- rows, columns, and middle axes
SEQ_UNB_CASES = [((1, 1), (1, 1)), ((255, 3), (255, 1)), ((257, 4), (257, 1)), ((4099, 10), (4099, 1)),
                 ((300, 16), (300, 1)), ((513, 17), (513, 1)), ((1000, 31), (1000, 1)), ((7, 5), (7, 1)),
                 ((300, 64), (300, 1)), ((32, 32), (1, 32)), ((7, 2), (1, 2)), ((64, 1000), (1, 1000)),
                 ((9, 4, 3), (9, 1, 3)), ((5, 33, 257), (5, 1, 257)), ((40, 4096), (4096,)), ((3, 7), (7,))]


@pytest.mark.parametrize("op", [0, 1, 2, 3], ids=["ADD", "SUB", "MUL", "DIV"])
@pytest.mark.parametrize("full,small", SEQ_UNB_CASES, ids=[f"{f}-{s}" for f, s in SEQ_UNB_CASES])
def test_short_line_unbroadcast_bitexact(gpu, op, full, small):
    """full (op) small in both operand orders: the broadcast operand's gradient is an
    un-broadcast along lines of at most 64 elements, which the reference's accumulate_grad
    adds into the gradient one value at a time in row-major order, as the GPU's
    thread-per-line kernels do -- so every gradient is bit-exact against the oracle."""
    for sa, sb in ((full, small), (small, full)):
        a, b = _binary_inputs(sa, sb, 700 + op + len(full))
        ug = synth.normal(full, 0, 1, 710 + full[0])
        for tid, shape in ((0, sa), (1, sb)):
            g0 = synth.normal(shape, 0, 1, 720 + tid)
            got = gpu.backward(tid, op, ug, a, b, grad=g0)
            assert_bitexact(got, ORC.backward(tid, op, ug, a, b, grad=g0), f"{sa}x{sb} op{op} id{tid}")


@pytest.mark.parametrize("op", [0, 1, 2, 3], ids=["ADD", "SUB", "MUL", "DIV"])
def test_binary_bwd_both_operands_fused(gpu, op):
    m = gpu.m
    n = (1 << 20) + 3
    a, b = _binary_inputs((n,), (n,), 400 + op)
    ug = synth.normal((n,), 0, 1, 401)
    g1, g2 = synth.normal((n,), 0, 1, 402), synth.normal((n,), 0, 1, 403)
    ta, tb, tu, tg1, tg2 = (gpu.T(v) for v in (a, b, ug, g1, g2))
    m.backward_op_both(op, tu, ta, tb, tg1, tg2)
    assert_bitexact(tg1.to_numpy(), ORC.backward(0, op, ug, a, b, grad=g1), "fused id0")
    assert_bitexact(tg2.to_numpy(), ORC.backward(1, op, ug, a, b, grad=g2), "fused id1")


_SPECIAL32 = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-45, -1e-40, 1.17549435e-38, 1.0, -1.0, 0.5, 2.0,
                       3.4e38, -3.4e38, 1e20, -1e-20, 3.0, -7.0], np.float32)


@pytest.mark.parametrize("op", [0, 1, 2, 3], ids=["ADD", "SUB", "MUL", "DIV"])
def test_binary_special_values_bitexact(gpu, op):
    """Every pair of special operands (NaN, infinities, signed zeros, subnormals, values near
    the float limit, and ordinary ones), same shape and with each operand a scalar: the
    forward, each operand's gradient and the fused two-gradient pass bit-identical to the
    oracle (NaN matching NaN), accumulated into gradients that hold special values too."""
    m = gpu.m
    s = _SPECIAL32
    a = np.repeat(s, s.size).astype(np.float32)
    b = np.tile(s, s.size).astype(np.float32)
    n = a.size
    ug = np.tile(np.array([1.0, -0.0, np.nan, 2.5e38, -3.0, 1e-42], np.float32), -(-n // 6))[:n].copy()
    g1 = np.tile(np.array([0.0, -0.0, 1.0, np.inf, -2.0], np.float32), -(-n // 5))[:n].copy()
    g2 = np.tile(np.array([-0.0, 3.0, np.nan, 0.0, -1e38, 7.0, 1e-44], np.float32), -(-n // 7))[:n].copy()
    assert_bitexact(gpu.forward(op, a, b), ORC.forward(op, a, b), f"fwd op{op}")
    for k, g0 in ((0, g1), (1, g2)):
        assert_bitexact(gpu.backward(k, op, ug, a, b, grad=g0), ORC.backward(k, op, ug, a, b, grad=g0),
                        f"bwd op{op} id{k}")
    ta, tb, tu, tg1, tg2 = (gpu.T(v) for v in (a, b, ug, g1, g2))
    m.backward_op_both(op, tu, ta, tb, tg1, tg2)
    assert_bitexact(tg1.to_numpy(), ORC.backward(0, op, ug, a, b, grad=g1), f"fused op{op} id0")
    assert_bitexact(tg2.to_numpy(), ORC.backward(1, op, ug, a, b, grad=g2), f"fused op{op} id1")
    for sv in (np.float32(-0.0), np.float32(np.inf), np.float32(np.nan), np.float32(1e-40)):
        sc = np.array([sv], np.float32)
        assert_bitexact(gpu.forward(op, a, sc), ORC.forward(op, a, sc), f"fwd op{op} tensor-scalar {sv}")
        assert_bitexact(gpu.forward(op, sc, b), ORC.forward(op, sc, b), f"fwd op{op} scalar-tensor {sv}")
        assert_bitexact(gpu.backward(0, op, ug, a, sc, grad=g1), ORC.backward(0, op, ug, a, sc, grad=g1),
                        f"bwd op{op} id0 tensor-scalar {sv}")


# the broadcast engines: per-row and per-column operands, a per-channel NCHW operand, and a
# general broadcast (both operands broadcast)
BCAST_SPECIAL = [((18, 20), (18, 1)), ((20, 18), (1, 18)), ((2, 18, 20), (1, 18, 1)), ((18, 1, 20), (1, 3, 20))]


@pytest.mark.parametrize("op", [0, 1, 2, 3], ids=["ADD", "SUB", "MUL", "DIV"])
@pytest.mark.parametrize("sa,sb", BCAST_SPECIAL, ids=[f"{a}x{b}" for a, b in BCAST_SPECIAL])
def test_broadcast_special_values(gpu, op, sa, sb):
    """Special operands (NaN, infinities, signed zeros, subnormals, near-limit values) through
    the row, column, plane and general broadcast engines, in both operand orders: the forward
    and the full-shape operand's gradient bit for bit against the oracle; the broadcast
    operand's gradient (a sum over the broadcast axes) NaN / +-inf exactly where the oracle's
    is and in the sum class elsewhere."""
    s = _SPECIAL32
    for x_shape, y_shape in ((sa, sb), (sb, sa)):
        a = np.resize(s, int(np.prod(x_shape))).reshape(x_shape).astype(np.float32)
        b = np.resize(s[::-1], int(np.prod(y_shape))).reshape(y_shape).astype(np.float32)
        assert_bitexact(gpu.forward(op, a, b), ORC.forward(op, a, b), f"fwd op{op} {x_shape}x{y_shape}")
        out_shape = np.broadcast_shapes(x_shape, y_shape)
        ug = synth.normal(out_shape, 0, 1, 790 + op)
        ug.reshape(-1)[::11] = np.float32(-0.0)
        for k, shape in ((0, x_shape), (1, y_shape)):
            g0 = synth.normal(shape, 0, 1, 795 + k)
            got = gpu.backward(k, op, ug, a, b, grad=g0)
            ref = ORC.backward(k, op, ug, a, b, grad=g0)
            what = f"bwd op{op} id{k} {x_shape}x{y_shape}"
            if tuple(shape) == tuple(out_shape):
                assert_bitexact(got, ref, what)
                continue
            A, B, U = (v.astype(np.float64) for v in np.broadcast_arrays(a, b, ug))
            with np.errstate(all="ignore"):
                rg = {0: U, 1: (U if k == 0 else -U), 2: (U * B if k == 0 else U * A),
                      3: (U / B if k == 0 else -A / (B * B) * U)}[op]
            red = tuple(i for i in range(len(out_shape)) if i >= len(out_shape) - len(shape) and
                        shape[i - (len(out_shape) - len(shape))] == 1 and out_shape[i] != 1) + \
                tuple(range(len(out_shape) - len(shape)))
            rgf = np.where(np.isfinite(rg), rg, 0.0)
            ex = rgf.sum(axis=red, keepdims=True).reshape(shape) + g0.astype(np.float64)
            mag = np.abs(rgf).sum(axis=red, keepdims=True).reshape(shape) + np.abs(g0)
            # where the finite terms' magnitudes stay below the float limit no partial sum can
            # overflow, so whether a sum is NaN or infinite does not depend on its order
            safe = mag < 1e38
            assert (np.isnan(got) == np.isnan(ref))[safe].all(), what
            assert (np.isinf(got) == np.isinf(ref))[safe].all(), what
            inf = np.isinf(ref) & safe
            assert (np.sign(got[inf]) == np.sign(ref[inf])).all(), what
            fin = np.isfinite(ref) & safe
            assert_sum_close(got[fin], ref[fin], ex[fin], what, terms_abs=mag[fin])


@pytest.mark.parametrize("n", [(1 << 16) + 3, 5, 4096])
@pytest.mark.parametrize("op", [0, 1, 2, 3], ids=["ADD", "SUB", "MUL", "DIV"])
def test_binary_bwd_both_operands_one_symbol(gpu, op, n):
    """x + x, x * x ...: both operands are one symbol, so Model.backward's two backward_op calls
    (model.mojo:233-270) accumulate into one gradient, operand 0's first. The fused entry point
    given the same gradient twice must match those two calls on the oracle bit for bit; so must
    two gradient views that overlap without being equal (one element apart), which run as the
    two calls in order."""
    m = gpu.m
    x = synth.uniform((n,), 0.5, 2, 410 + op)
    ug = synth.normal((n,), 0, 1, 411)
    g0 = synth.normal((n,), 0, 1, 412)
    exp = ORC.backward(1, op, ug, x, x, grad=ORC.backward(0, op, ug, x, x, grad=g0))
    tx, tu, tg = gpu.T(x), gpu.T(ug), gpu.T(g0)
    m.backward_op_both(op, tu, tx, tx, tg, tg)
    assert_bitexact(tg.to_numpy(), exp, "one gradient for both operands")
    # overlapping views: grad1 = buf[0:n], grad2 = buf[1:n+1]
    buf0 = synth.normal((n + 1,), 0, 1, 413)
    buf = gpu.T(buf0)
    v1 = m.Tensor(m.TensorShape(n), _ptr=buf.ptr, _owner=buf)
    v2 = m.Tensor(m.TensorShape(n), _ptr=buf.ptr + 4, _owner=buf)
    m.backward_op_both(op, tu, tx, tx, v1, v2)
    e = buf0.copy()
    e[:n] = ORC.backward(0, op, ug, x, x, grad=e[:n])
    e[1:] = ORC.backward(1, op, ug, x, x, grad=e[1:])
    assert_bitexact(buf.to_numpy(), e, "overlapping gradient views")


# ---------------------------------------------------------------------------------------
# unary ops and POW on the config-2 distributions
# ---------------------------------------------------------------------------------------
UNARY_DIST = {"EXP": ("u", -10, 10), "LOG": ("u", 1e-3, 10), "TANH": ("n", 0, 3), "SIGMOID": ("n", 0, 3),
              "RELU": ("n", 0, 3)}


def _dist(name, n, seed):
    kind, p, q = UNARY_DIST[name]
    return synth.uniform((n,), p, q, seed) if kind == "u" else synth.normal((n,), p, q, seed)


@pytest.mark.parametrize("name", list(UNARY_DIST))
def test_unary_fwd_bwd_parity(gpu, name):
    op = OPS[name]
    n = (1 << 20) + 5
    x = _dist(name, n, 500 + op)
    ug = synth.normal((n,), 0, 1, 501)
    g0 = synth.normal((n,), 0, 1, 502)
    fwd = gpu.forward(op, x)
    ref = ORC.forward(op, x)
    if name == "RELU":
        assert_bitexact(fwd, ref, "relu fwd")
        assert_bitexact(gpu.backward(0, op, ug, x, grad=g0), ORC.backward(0, op, ug, x, grad=g0), "relu bwd")
        return
    assert_ulp(fwd, ref, 2, f"{name} fwd")
    exact = np.mean(fwd.view(np.uint32) == ref.view(np.uint32))
    print(f"[gpu] {name} fwd bit-exact fraction {exact:.6f}", flush=True)
    bwd = gpu.backward(0, op, ug, x, grad=g0)
    assert_ulp(bwd, ORC.backward(0, op, ug, x, grad=g0), 2, f"{name} bwd")


def _special_inputs(seed):
    """Arguments around every branch of the device exp/log: NaN, +-inf, +-0, the exp clamp
    bounds and just beyond, results that underflow to subnormal, subnormal and tiny log
    arguments, negative log arguments, and a dense sweep of ordinary values."""
    f32 = np.float32
    lo, hi = f32(-88.3762626647949), f32(88.3762626647950)
    pts = [np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0, 2.0, 0.5, 1e-45, 1e-40, 1.17549435e-38, 3e-38,
           float(lo), float(hi), float(np.nextafter(lo, f32(-1e9))), float(np.nextafter(hi, f32(1e9))), -100.0, 100.0,
           -87.0, -87.5, -88.0, 88.0, 3.4e38, -3.4e38, 0.7071067, 0.70710677, 0.7071068]
    sweep = synth.uniform((20000,), -104, 90, seed)
    tiny = (synth.uniform((4000,), 0, 1, seed + 1) * f32(1.2e-38)).astype(f32)
    return np.concatenate([np.array(pts, f32), sweep, tiny, -tiny]).astype(f32)


@pytest.mark.parametrize("name", ["EXP", "LOG", "SIGMOID", "TANH"])
def test_device_math_matches_oracle_bitwise(gpu, name):
    """The device exp/log and the oracle's restatement are the same algorithm: the GPU must
    reproduce the oracle's bits on every branch (the north-star bar against Mantle itself is
    2 ulp; this is the stricter internal check)."""
    x = _special_inputs(900 + OPS[name])
    assert_bitexact(gpu.forward(OPS[name], x), ORC.forward(OPS[name], x), f"{name} special inputs")


@pytest.mark.parametrize("name", ["LOG", "EXP"])
def test_device_math_float_sweep_bitwise(gpu, name):
    """The device log and exp against the oracle over every 251st 32-bit pattern: about 17 M
    floats of both signs and every exponent and class (zeros, subnormals, normals, infinities,
    NaNs), bit for bit. The device log writes three of the method's steps as fmas (the fold,
    -0.5 z and the second part of ln 2, all exact) and takes the exponent with frexp; the
    sweep shows the bits stay the method's across the whole domain."""
    x = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32).view(np.float32)
    assert_bitexact(gpu.forward(OPS[name], x), ORC.forward(OPS[name], x), f"{name} float sweep")


@pytest.mark.parametrize("name", ["EXP", "LOG", "SIGMOID", "TANH", "RELU"])
def test_unary_backward_special_values_bitexact(gpu, name):
    """The unary backward passes on the same special arguments, with NaN, infinite, signed-zero
    and subnormal values in the upstream gradient and in the gradient they accumulate into:
    bit-identical to the oracle (NaN matching NaN)."""
    x = _special_inputs(960 + OPS[name])
    n = x.size
    ug = synth.normal((n,), 0, 1, 961)
    ug[::7] = np.float32(-0.0)
    ug[1::11] = np.float32(np.nan)
    ug[2::13] = np.float32(np.inf)
    ug[3::17] = np.float32(1e-42)
    ug[4::19] = np.float32(-3.0e38)
    g0 = synth.normal((n,), 0, 1, 962)
    g0[::5] = np.float32(-0.0)
    g0[1::9] = np.float32(-np.inf)
    g0[2::23] = np.float32(np.nan)
    assert_bitexact(gpu.backward(0, OPS[name], ug, x, grad=g0), ORC.backward(0, OPS[name], ug, x, grad=g0),
                    f"{name} backward, special values")


def test_device_pow_matches_oracle_bitwise(gpu):
    x = np.abs(_special_inputs(950))
    ug = synth.normal(x.shape, 0, 1, 951)
    for e in (2.37, 0.5, -0.75, 3.0, 0.0, -2.0):
        t2 = np.array([e], np.float32)
        assert_bitexact(gpu.forward(OPS["POW"], x, t2), ORC.forward(OPS["POW"], x, t2), f"pow fwd {e}")
        g0 = np.zeros_like(x)
        assert_bitexact(gpu.backward(0, OPS["POW"], ug, x, t2, grad=g0), ORC.backward(0, OPS["POW"], ug, x, t2, grad=g0),
                        f"pow bwd x {e}")


def test_elwise_pow_integer_exponents(gpu):
    """mh_powi_fwd (elwise_pow with a given Int exponent) bit-exact against the oracle's
    square-and-multiply, negative exponents included, on a ragged length with 0, +-inf, NaN
    and negative bases."""
    m = gpu.m
    x = synth.uniform((4099,), -3, 3, 1150)
    x[:6] = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0], np.float32)
    tx = gpu.T(x)
    for n in (-3, -1, 0, 1, 2, 3, 5, 17, 40):
        res = m.Tensor(tx.shape())
        m.elwise_pow(res, tx, n)
        assert_bitexact(res.to_numpy(), O.elwise_pow(x, n), f"x^{n}")
    with pytest.raises(ValueError):
        m.elwise_pow(m.Tensor(tx.shape()), tx, 1 << 40)


@pytest.mark.parametrize("e", [2.37, 0.61, 1.0, 2.0, -1.5, 3.9])
def test_pow_parity(gpu, e):
    n = (1 << 18) + 7
    x = synth.uniform((n,), 0.1, 4, 600)
    t2 = np.array([e], np.float32)
    ug = synth.normal((n,), 0, 1, 601)
    assert_bitexact(gpu.forward(OPS["POW"], x, t2), ORC.forward(OPS["POW"], x, t2), f"pow fwd {e}")
    g0 = synth.normal((n,), 0, 1, 602)
    assert_ulp(gpu.backward(0, OPS["POW"], ug, x, t2, grad=g0), ORC.backward(0, OPS["POW"], ug, x, t2, grad=g0), 2,
               f"pow bwd x {e}")
    got = gpu.backward(1, OPS["POW"], ug, x, t2)
    ref = ORC.backward(1, OPS["POW"], ug, x, t2)
    X, U = x.astype(np.float64), ug.astype(np.float64)
    terms = X ** np.float64(t2[0]) * np.log(X) * U
    assert_sum_close(got, ref, np.array([terms.sum()]), f"pow bwd exponent {e}", terms_abs=np.array([np.abs(terms).sum()]))


@pytest.mark.parametrize("n", [1, 3, 4, 63, 64, 65, 2047, 2048, 2052, 4099, (1 << 18) + 4, (1 << 20) + 3,
                               (1 << 23) + 20])
def test_pow_bwd_both_operands_fused(gpu, n):
    """mh_pow_bwd_accum2 (x's and the exponent's gradient in one pass) against the two
    mh_pow_bwd_accum calls bit for bit: the x gradient element by element, the exponent gradient
    through the same reduction kernels in the same order (every reduction shape the length
    selects: LDS rows, one wavefront, block chunks with a combine, and for aligned lengths of
    2^16 whole quads or more the one-shot quad kernel, a 64-quad run per block with the x
    gradient and two without, with a ragged last run). Bases include values where
    x + 1e-12 is not x (0, 1e-13, a subnormal), a negative base, NaN and inf; exponents integral
    and fractional; x, ug and the gradients also as unaligned views. The x gradient also matches
    the oracle bit for bit and the exponent gradient the oracle's in the sum class."""
    m = gpu.m
    pw = OPS["POW"]
    x = synth.uniform((n,), 0.1, 4, 610 + n % 97)
    specials = np.array([0.0, 1e-13, 3e-6, 1e-40, -2.0, np.nan, np.inf, 1.0], np.float32)
    ug = synth.normal((n,), 0, 1, 611)
    g0 = synth.normal((n,), 0, 1, 612)
    for e in (2.37, 3.0, -1.5, 0.5):
        t2 = np.array([e], np.float32)
        ge0 = np.array([0.25], np.float32)
        for xs, label in ((x, "clean"), (np.concatenate([specials, x])[:n], "specials")):
            for off in (0, 1):
                def view(v, off=off):
                    buf = gpu.T(np.concatenate([np.zeros(off, np.float32), v]))
                    return m.Tensor(m.TensorShape(*v.shape), _ptr=buf.ptr + 4 * off, _owner=buf)
                tx, tu, te = view(xs), view(ug), gpu.T(t2)
                sx, se = view(g0), gpu.T(ge0)
                m.backward_op(0, pw, tu, tx, te, sx)
                m.backward_op(1, pw, tu, tx, te, se)
                fx, fe = view(g0), gpu.T(ge0)
                m.backward_op_both(pw, tu, tx, te, fx, fe)
                what = f"n={n} e={e} {label} off={off}"
                assert_bitexact(fx.to_numpy(), sx.to_numpy(), f"fused x grad {what}")
                assert_bitexact(fe.to_numpy(), se.to_numpy(), f"fused exponent grad {what}")
                if label == "clean" and off == 0:
                    assert_ulp(fx.to_numpy(), ORC.backward(0, pw, ug, xs, t2, grad=g0), 2, f"x grad vs oracle {what}")
                    ref = ORC.backward(1, pw, ug, xs, t2, grad=ge0)
                    X, U = xs.astype(np.float64), ug.astype(np.float64)
                    terms = X ** np.float64(e) * np.log(X) * U
                    assert_sum_close(fe.to_numpy(), ref, np.array([0.25 + terms.sum()]), f"exponent grad {what}",
                                     terms_abs=np.array([0.25 + np.abs(terms).sum()]))
    # one null gradient: only the other part runs
    tx, tu, te = gpu.T(x), gpu.T(ug), gpu.T(np.array([2.37], np.float32))
    fx = gpu.T(g0)
    m.backward_op_both(pw, tu, tx, te, fx, None)
    sx = gpu.T(g0)
    m.backward_op(0, pw, tu, tx, te, sx)
    assert_bitexact(fx.to_numpy(), sx.to_numpy(), "x grad alone")


def _pow_band_edge_bases(e):
    """Positive bases whose x^(e-1) or x^e lies at the edges of [FLT_MIN, 2e38] (the band in
    which the one-pass POW backward takes x^e as x * (x + 1e-12)^(e-1) and that power's exp
    without its clamp), near exp's clamp (e^+-88.376, about 2.4e38 and 4.2e-39) and beyond
    it, each with its two float neighbours."""
    a = np.float64(np.float32(e))
    out = []
    for target in (5e-39, 1.0e-38, 1.1754944e-38, 1.3e-38, 1.0e38, 1.99e38, 2.0e38, 2.01e38, 2.3e38, 2.45e38,
                   3.3e38):
        for y in (a - 1.0, a):
            r = target ** (1.0 / y)
            if 1e-37 < r < 3e38:  # a normal float base
                v = np.float32(r)
                out += [v, np.nextafter(v, np.float32(np.inf)), np.nextafter(v, np.float32(0))]
    return np.array(out, np.float32)


@pytest.mark.parametrize("e", [2.37, 1.5, -1.5, 3.9])
def test_pow_bwd_band_edges(gpu, e):
    """The one-pass POW backward (mh_pow_bwd_accum2, the one-wavefront kernel at 2^18
    elements) at the edges of its shared-power band: the x gradient holds the oracle's bits at
    every edge base (the unclamped exp is used only where its bits are exp's), and each base's
    exponent-gradient term, alone in its call (a one-hot upstream gradient, every other base
    1.0), is in the sum class against the oracle and bit-identical to the exponent-only call."""
    m = gpu.m
    pw = OPS["POW"]
    n = 1 << 18
    bases = _pow_band_edge_bases(e)
    t2 = np.array([e], np.float32)
    x = np.ones(n, np.float32)
    x[:bases.size] = bases
    ug = synth.normal((n,), 0, 1, 1400)
    g0 = synth.normal((n,), 0, 1, 1401)
    fx, fe = gpu.T(g0), gpu.T(np.zeros(1, np.float32))
    m.backward_op_both(pw, gpu.T(ug), gpu.T(x), gpu.T(t2), fx, fe)
    assert_bitexact(fx.to_numpy(), ORC.backward(0, pw, ug, x, t2, grad=g0), f"x grad at the band edges, e={e}")
    te = gpu.T(t2)
    for k, v in enumerate(bases):
        xk = np.ones(n, np.float32)
        xk[k] = v
        uk = np.zeros(n, np.float32)
        uk[k] = 1.0
        tx, tu = gpu.T(xk), gpu.T(uk)
        fx, fe = gpu.T(np.zeros(n, np.float32)), gpu.T(np.zeros(1, np.float32))
        m.backward_op_both(pw, tu, tx, te, fx, fe)
        sep = gpu.backward(1, pw, uk, xk, t2)
        what = f"e={e} base {v!r}"
        assert_bitexact(fe.to_numpy(), sep, f"fused vs exponent-only term, {what}")
        ref = ORC.backward(1, pw, uk, xk, t2)
        exact = np.float64(v) ** np.float64(t2[0]) * np.log(np.float64(v))
        with np.errstate(invalid="ignore"):  # a term that overflows is inf on both sides
            assert_sum_close(fe.to_numpy(), ref, np.array([exact]), f"exponent term, {what}",
                             terms_abs=np.array([abs(exact)]))


# ---------------------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------------------
RED_CASES = [((87, 73, 107), 0), ((87, 73, 107), 1), ((87, 73, 107), 2), ((87, 73, 107), None),
             ((1024, 1024), 0), ((1024, 1024), 1), ((64, 512, 1024), 2), ((4099, 10), 1), ((3, 1, 5), 1),
             ((1,), None), ((5,), 0), ((2, 70000), 1), ((70000, 3), 0), ((1 << 22,), None), ((6, 33, 2), 1),
             ((1000, 20), 1), ((513, 32), 1), ((1001, 3), 1), ((300, 1), 1), ((257, 16), 1), ((40, 33), 1),
             ((30,), None), ((2, 3, 17), 2), ((5, 16384), 1), ((3, 4100), 1), ((7, 2052), 1), ((16, 36), 1),
             ((300, 256), 0), ((33, 512, 128), 1), ((4, 8, 1024), 0), ((2, 5000, 132), 1), ((9000, 64), 0),
             ((3, 12000), None),
             # chunk-partial combines of 16386 (odd quads: the scalar pass) and 20000 partials, and
             # a wide column split whose last partial group is short
             ((2048 * 16385 + 4,), None), ((2048 * 20000,), None), ((3, 3000, 1024), 1)]


def _seeded_red_cases(count, seed):
    """Reduction cases drawn with a fixed seed: rank 1-4, up to 1.5 M elements, every axis and
    all elements; a third of them strided over rows of 128-4096 columns in quads (the wide,
    strip and per-quad column forms with their row splits)."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        if len(out) % 3 == 2:
            r = int(rng.integers(2, 4))
            shape = tuple(_dim(rng, 600) for _ in range(r - 1)) + (4 * int(rng.integers(32, 1025)),)
            axis = int(rng.integers(0, r - 1))
        else:
            r = int(rng.integers(1, 5))
            shape = tuple(_dim(rng, 40000) for _ in range(r))
            axis = int(rng.integers(-1, r))
        if int(np.prod(shape)) > 1_500_000 or int(np.prod(shape)) < 2:
            continue
        out.append((shape, None if axis < 0 else axis))
    return out


RED_CASES += _seeded_red_cases(30, 20261203)


@pytest.mark.parametrize("shape,axis", RED_CASES, ids=[f"{s}-ax{a}" for s, a in RED_CASES])
def test_reduce_fwd_bwd_parity(gpu, shape, axis):
    x = synth.normal(shape, 0, 1, 700)
    if axis is not None and shape[axis] > 1:
        synth.inject_ties(x, axis, 701)
    elif x.size > 1:
        x.reshape(-1)[x.size // 2] = x.max()
    red_shape = (1,) if axis is None else tuple(1 if i == axis else d for i, d in enumerate(shape))
    kd = dict(axis=axis, keepdims=True) if axis is not None else {}
    ex = x.astype(np.float64).sum(**kd).reshape(red_shape)
    mag = np.abs(x.astype(np.float64)).sum(**kd).reshape(red_shape)
    d = x.size if axis is None else shape[axis]
    s = gpu.forward(OPS["SUM"], x, axis=axis)
    assert_sum_close(s, ORC.forward(OPS["SUM"], x, axis=axis), ex, "sum", terms_abs=mag)
    mn = gpu.forward(OPS["MEAN"], x, axis=axis)
    assert_sum_close(mn, ORC.forward(OPS["MEAN"], x, axis=axis), ex / d, "mean", terms_abs=mag / d)
    assert_bitexact(gpu.forward(OPS["MAX"], x, axis=axis), ORC.forward(OPS["MAX"], x, axis=axis), "max")
    ug = synth.normal(red_shape, 0, 1, 702)
    g0 = synth.normal(shape, 0, 1, 703)
    for name in ("SUM", "MEAN", "MAX"):
        got = gpu.backward(0, OPS[name], ug, x, axis=axis, grad=g0)
        assert_bitexact(got, ORC.backward(0, OPS[name], ug, x, axis=axis, grad=g0), f"{name} bwd")


SUM_SPECIAL_CASES = [((4099, 10), 1), ((300, 257), 0), ((64, 5000), 1), ((37, 63, 107), 1), ((9000, 64), 0),
                     (((1 << 20) + 3,), None), ((3, 12000), None)]


@pytest.mark.parametrize("shape,axis", SUM_SPECIAL_CASES, ids=[f"{s}-ax{a}" for s, a in SUM_SPECIAL_CASES])
def test_sum_mean_special_values(gpu, shape, axis):
    """SUM and MEAN over lines holding +inf, both infinities, NaN, only -0 (which sum to +0, as
    a sum from +0 does), only positive values near the float limit (which overflow in any
    order), signed zeros and subnormals: a line's result is NaN / +-inf exactly where the
    oracle's is, +0 bit for bit on the -0 lines, and in the sum class elsewhere; the backward
    passes (a scaled broadcast of an upstream gradient holding special values) bit-identical."""
    x = synth.normal(shape, 0, 1, 760)
    lines = np.moveaxis(x, axis, -1) if axis is not None else x.reshape(1, -1)
    flat = lines.reshape(-1, lines.shape[-1])  # a view for contiguous moves, else a copy
    L = flat.shape[0]
    special = [(0, "inf"), (1, "both"), (2, "nan"), (3, "negzero"), (4, "huge")] if L >= 5 else [(0, "nan")]
    for li, kind in special:
        row = flat[li]
        if kind == "inf":
            row[row.size // 3] = np.inf
        elif kind == "both":
            row[0], row[-1] = np.inf, -np.inf
        elif kind == "nan":
            row[row.size // 2] = np.nan
        elif kind == "negzero":
            row[:] = np.float32(-0.0)
        else:
            row[:] = np.abs(row) + np.float32(1.0)
            row[: max(2, row.size // 4)] = np.float32(3.0e38)
    if L > 6:
        flat[5, ::3] = np.float32(-0.0)
        flat[6, 1::4] = np.float32(1e-41)
    if not np.shares_memory(flat, x):
        lines[...] = flat.reshape(lines.shape)  # lines is a view of x
    red_shape = (1,) if axis is None else tuple(1 if i == axis else d for i, d in enumerate(shape))
    d = x.size if axis is None else shape[axis]
    for name in ("SUM", "MEAN"):
        got = gpu.forward(OPS[name], x, axis=axis)
        ref = ORC.forward(OPS[name], x, axis=axis)
        assert (np.isnan(got) == np.isnan(ref)).all(), f"{name}: NaN lines"
        assert (np.isinf(got) == np.isinf(ref)).all() and (np.sign(got[np.isinf(got)]) == np.sign(ref[np.isinf(ref)])).all(), \
            f"{name}: infinite lines"
        fin = np.isfinite(ref)
        if L >= 5:  # line 3 holds only -0: the sum from +0 is +0
            assert_bitexact(got.reshape(-1)[3:4], ref.reshape(-1)[3:4], f"{name}: a line of -0")
            assert ref.reshape(-1)[3].tobytes() == np.float32(0.0).tobytes()
        x64 = np.where(np.isfinite(x), x, 0).astype(np.float64)
        kd = dict(axis=axis, keepdims=True) if axis is not None else {}
        ex = x64.sum(**kd).reshape(red_shape) / (d if name == "MEAN" else 1)
        mag = np.abs(x64).sum(**kd).reshape(red_shape) / (d if name == "MEAN" else 1)
        assert_sum_close(got[fin], ref[fin], ex[fin], name, terms_abs=mag[fin])
        ug = synth.normal(red_shape, 0, 1, 761)
        ug.reshape(-1)[0] = np.float32(-0.0)
        if ug.size > 2:
            ug.reshape(-1)[1], ug.reshape(-1)[2] = np.float32(np.inf), np.float32(np.nan)
        g0 = synth.normal(shape, 0, 1, 762)
        g0.reshape(-1)[::97] = np.float32(-0.0)
        got = gpu.backward(0, OPS[name], ug, x, axis=axis, grad=g0)
        assert_bitexact(got, ORC.backward(0, OPS[name], ug, x, axis=axis, grad=g0), f"{name} bwd")


MAX_SPARSE_CASES = [((1024, 1024), 0), ((4099, 10), 1), ((300, 20), 1), ((64, 512), 1), ((9, 2052), 1),
                    ((87, 73, 107), None), ((87, 73, 107), 1), ((4, 8, 1024), 0), ((2, 5000, 132), 1),
                    # split routes: row chunks (all elements, a short last chunk), the strip and
                    # thread-per-quad column splits, a wide split over three slabs
                    ((1 << 20,), None), ((3, 12000), None), ((300, 256), 0), ((9000, 64), 0),
                    ((3, 3000, 1024), 1)]


@pytest.mark.parametrize("shape,axis", MAX_SPARSE_CASES, ids=[f"{s}-ax{a}" for s, a in MAX_SPARSE_CASES])
def test_max_backward_sparse_stores_keep_every_bit(gpu, shape, axis):
    """MAX backward stores only the quads whose bits change (it adds +0 away from the line
    maxima). The gradient it accumulates into holds -0 (which + 0 turns into +0, so those
    quads must be stored), +0 and NaN away from the maxima: bit-exact against the oracle on
    every routing path (column, short-row, register-row, all-element and generic forms)."""
    x = synth.normal(shape, 0, 1, 710)
    if axis is not None and shape[axis] > 1:
        synth.inject_ties(x, axis, 711)
    else:
        x.reshape(-1)[x.size // 2] = x.max()
    red_shape = (1,) if axis is None else tuple(1 if i == axis else d for i, d in enumerate(shape))
    ug = synth.normal(red_shape, 0, 1, 712)
    g0 = synth.normal(shape, 0, 1, 713).reshape(-1)
    g0[::3] = np.float32(-0.0)
    g0[1::7] = np.float32(0.0)
    g0[2::11] = np.float32(np.nan)
    g0 = g0.reshape(shape)
    got = gpu.backward(0, OPS["MAX"], ug, x, axis=axis, grad=g0)
    ref = ORC.backward(0, OPS["MAX"], ug, x, axis=axis, grad=g0)
    assert_bitexact(got, ref, "MAX bwd")  # bits, so the sign of every zero too
    r3 = ref.reshape(-1)[::3]
    assert ((r3 == 0) & ~np.signbit(r3)).any(), "no -0 turned into +0: the case is not exercised"


ROUTE_CASES = [((1024, 1024), 0), ((300, 256), 0), ((9000, 64), 0), ((3, 3000, 1024), 1), ((1 << 20,), None),
               ((3, 12000), None), ((5, 70000), 1)]


@pytest.mark.parametrize("shape,axis", ROUTE_CASES, ids=[f"{s}-ax{a}" for s, a in ROUTE_CASES])
def test_max_backward_split_route_special_values(gpu, shape, axis):
    """A MAX backward whose line maxima come from a split reduction reads x again only in the
    splits whose partial maximum equals the line's. Lines here hold their maximum as +0 and -0
    in far-apart splits (equal as floats: both route), -inf elements, only -inf (maximum
    -FLT_MAX, count 0: nothing routes), a maximum repeated across many splits (one per split:
    routed at the split's recorded index) and one on every third row (several per split:
    routed by comparing x); the
    gradient holds -0 (turned into +0 in the splits that skip x too), +0 and NaN. Bit-exact
    against the oracle; the forward maximum equal as floats (the sign of a maximum that is a
    zero tie follows the order the maxima are combined in, the reference's SIMD lanes or the
    GPU's splits: the routing is the same for either)."""
    n = int(np.prod(shape))
    ax = 0 if axis is None else axis
    lead = () if axis is None else tuple(d for i, d in enumerate(shape) if i != ax)
    B = n if axis is None else shape[ax]
    L = synth.normal((n // B, B), 0, 1, 720)  # one line per row
    L[0::4] = -np.abs(L[0::4]) - 1.0
    L[0::4, 5::17] = -np.inf
    L[0::4, B // 7] = 0.0
    L[0::4, B - 3] = -0.0
    if L.shape[0] > 1:
        L[1::4] = -np.inf
        L[2::4, ::97] = L[2::4].max(axis=1, keepdims=True) + np.float32(1.0)
        # the maximum on every third row: several in every split, whose routing reads x
        L[3::4, ::3] = L[3::4].max(axis=1, keepdims=True) + np.float32(1.0)
    if axis is None:
        x = L.reshape(shape)
    else:
        x = np.ascontiguousarray(np.moveaxis(L.reshape(lead + (B,)), -1, ax))
    red_shape = (1,) if axis is None else tuple(1 if i == ax else d for i, d in enumerate(shape))
    ug = synth.normal(red_shape, 0, 1, 721)
    g0 = synth.normal(shape, 0, 1, 722).reshape(-1)
    g0[::3] = np.float32(-0.0)
    g0[1::7] = np.float32(0.0)
    g0[2::11] = np.float32(np.nan)
    g0 = g0.reshape(shape)
    np.testing.assert_array_equal(gpu.forward(OPS["MAX"], x, axis=axis), ORC.forward(OPS["MAX"], x, axis=axis))
    got = gpu.backward(0, OPS["MAX"], ug, x, axis=axis, grad=g0)
    assert_bitexact(got, ORC.backward(0, OPS["MAX"], ug, x, axis=axis, grad=g0), "MAX bwd")


NAN_MAX_CASES = [((64, 10), 1), ((70, 33), 1), ((64, 1000), 1), ((3, 40000), 1), ((1 << 16,), None),
                 ((1024, 1024), 0), ((300, 256), 0), ((9000, 64), 0), ((70, 3), 0), ((5, 6, 7), 1)]


@pytest.mark.parametrize("shape,axis", NAN_MAX_CASES, ids=[f"{s}-ax{a}" for s, a in NAN_MAX_CASES])
def test_max_backward_nan_elements_are_not_counted(gpu, shape, axis):
    """MAX backward over lines holding NaN elements: the line maximum is the largest non-NaN
    element (-FLT_MAX when there is none), the count the elements equal to it (c = #(x == m),
    basics.mojo:551-577, 597-613; NaN equals nothing), so grad + (x == m ? fl(1/c) * ug : +0)
    follows in float32. The reference's own maximum depends on where a NaN meets its SIMD
    lanes (outside parity), so this pins the GPU's defined behaviour on every routing path:
    short rows, register rows, row chunks, all elements, and the wide, strip, per-quad and
    generic column forms."""
    n = int(np.prod(shape))
    ax = 0 if axis is None else axis
    B = n if axis is None else shape[ax]
    lead = () if axis is None else tuple(d for i, d in enumerate(shape) if i != ax)
    L = synth.normal((n // B, B), 0, 1, 730)  # one line per row
    L[:, 1::5] = np.nan
    L[0::3] = np.where(np.arange(B) % 2 == 0, np.float32(np.nan), L[0::3])  # NaN-heavy lines
    if L.shape[0] > 2:
        L[2] = np.nan  # a line of NaN only: maximum -FLT_MAX, count 0, nothing routes
    if axis is None:
        x = L.reshape(shape)
    else:
        x = np.ascontiguousarray(np.moveaxis(L.reshape(lead + (B,)), -1, ax))
    red_shape = (1,) if axis is None else tuple(1 if i == ax else d for i, d in enumerate(shape))
    ug = synth.normal(red_shape, 0, 1, 731)
    g0 = synth.normal(shape, 0, 1, 732)
    got = gpu.backward(0, OPS["MAX"], ug, x, axis=axis, grad=g0)
    # the expected gradient, line by line in float32
    fmax = np.float32(np.finfo(np.float32).max)
    m = np.maximum(np.where(np.isnan(L), -np.inf, L).max(axis=1), -fmax).astype(np.float32)
    eq = L == m[:, None]
    c = eq.sum(axis=1).astype(np.float32)
    with np.errstate(divide="ignore"):
        f = (np.float32(1.0) / c).astype(np.float32)
    U = ug.reshape(-1) if axis is None else np.moveaxis(ug, ax, -1).reshape(-1)
    G = g0.reshape(1, -1) if axis is None else np.moveaxis(g0, ax, -1).reshape(-1, B)
    add = (f * U).astype(np.float32)
    E = (G + np.where(eq, add[:, None], np.float32(0.0))).astype(np.float32)
    exp = E.reshape(shape) if axis is None else np.moveaxis(E.reshape(lead + (B,)), -1, ax)
    assert_bitexact(got, np.ascontiguousarray(exp), "MAX bwd with NaN elements")


RANK8_A, RANK8_B = (2, 1, 3, 1, 2, 1, 2, 5), (1, 2, 1, 2, 1, 3, 1, 5)


@pytest.mark.parametrize("op", [0, 1, 2, 3], ids=["ADD", "SUB", "MUL", "DIV"])
def test_rank8_broadcast(gpu, op):
    """MAX_RANK = 8 (core/tensor.mojo:20): a broadcast over every other axis of two rank-8
    operands, forward bit-exact and both operands' gradients (un-broadcast over four axes)."""
    a, b = _binary_inputs(RANK8_A, RANK8_B, 160 + op)
    assert_bitexact(gpu.forward(op, a, b), ORC.forward(op, a, b), f"rank-8 fwd op{op}")
    out_shape = np.broadcast_shapes(RANK8_A, RANK8_B)
    ug = synth.normal(out_shape, 0, 1, 170 + op)
    for k, shape in ((0, RANK8_A), (1, RANK8_B)):
        g0 = synth.normal(shape, 0, 1, 180 + k)
        got = gpu.backward(k, op, ug, a, b, grad=g0)
        ref = ORC.backward(k, op, ug, a, b, grad=g0)
        A, B, U = (v.astype(np.float64) for v in (a, b, ug))
        rg = {0: U, 1: (U if k == 0 else -U), 2: (U * B if k == 0 else U * A),
              3: (U / B if k == 0 else -A / (B * B) * U)}[op]
        red = tuple(i for i, d in enumerate(shape) if d == 1 and out_shape[i] != 1)
        ex = rg.sum(axis=red, keepdims=True) + g0.astype(np.float64)
        mag = np.abs(rg).sum(axis=red, keepdims=True) + np.abs(g0)
        assert_sum_close(got, ref, ex, f"rank-8 bwd op{op} id{k}", terms_abs=mag)


@pytest.mark.parametrize("axis", [0, 3, 6, 7, None])
def test_rank8_reductions(gpu, axis):
    """SUM / MEAN / MAX forward and backward and tstd over one axis (or all) of a rank-8
    tensor with ties injected."""
    shape = (2, 3, 2, 3, 2, 3, 2, 7)
    x = synth.normal(shape, 0, 1, 190)
    if axis is not None:
        synth.inject_ties(x, axis, 191)
    red = (1,) if axis is None else tuple(1 if i == axis else d for i, d in enumerate(shape))
    kd = dict(axis=axis, keepdims=True) if axis is not None else {}
    x64 = x.astype(np.float64)
    ex = np.asarray(x64.sum(**kd)).reshape(red)
    mag = np.asarray(np.abs(x64).sum(**kd)).reshape(red)
    d = x.size if axis is None else shape[axis]
    assert_sum_close(gpu.forward(OPS["SUM"], x, axis=axis), ORC.forward(OPS["SUM"], x, axis=axis), ex, "sum",
                     terms_abs=mag)
    assert_sum_close(gpu.forward(OPS["MEAN"], x, axis=axis), ORC.forward(OPS["MEAN"], x, axis=axis), ex / d, "mean",
                     terms_abs=mag / d)
    assert_bitexact(gpu.forward(OPS["MAX"], x, axis=axis), ORC.forward(OPS["MAX"], x, axis=axis), "max")
    ug = synth.normal(red, 0, 1, 192)
    g0 = synth.normal(shape, 0, 1, 193)
    for name in ("SUM", "MEAN", "MAX"):
        assert_bitexact(gpu.backward(0, OPS[name], ug, x, axis=axis, grad=g0),
                        ORC.backward(0, OPS[name], ug, x, axis=axis, grad=g0), f"{name} bwd")
    sd = np.asarray(x64.std(**kd)).reshape(red)
    assert_sum_close(gpu.tstd(x, axis), ORC.tstd(x, axis), sd, "tstd")


def test_reductions_are_deterministic(gpu):
    m = gpu.m
    x = gpu.T(synth.normal((4096, 4096), 0, 1, 710))
    for ax in (0, 1, -1):
        r1 = m.tsum(x, ax).to_numpy()
        r2 = m.tsum(x, ax).to_numpy()
        assert_bitexact(r1, r2, f"sum twice axis {ax}")


# ---------------------------------------------------------------------------------------
# ragged, tiny and unaligned inputs
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 63, 65, 1023, 4097])
def test_ragged_sizes(gpu, n):
    a, b = _binary_inputs((n,), (n,), 800)
    for op in (0, 3):
        assert_bitexact(gpu.forward(op, a, b), ORC.forward(op, a, b), f"op{op} n={n}")
    x = _dist("EXP", n, 801)
    assert_ulp(gpu.forward(OPS["EXP"], x), ORC.forward(OPS["EXP"], x), 2, f"exp n={n}")
    assert_bitexact(gpu.forward(OPS["MAX"], x), ORC.forward(OPS["MAX"], x), f"max n={n}")


def test_unaligned_device_pointers(gpu):
    m = gpu.m
    n = 10007
    a, b = _binary_inputs((n,), (n,), 810)
    base_a, base_b, base_r = gpu.T(np.concatenate([[0], a])), gpu.T(np.concatenate([[0], b])), m.Tensor(n + 1)
    va = m.Tensor(m.TensorShape(n), _ptr=base_a.ptr + 4, _owner=base_a)
    vb = m.Tensor(m.TensorShape(n), _ptr=base_b.ptr + 4, _owner=base_b)
    vr = m.Tensor(m.TensorShape(n), _ptr=base_r.ptr + 4, _owner=base_r)
    m.forward_op(m.OP.MUL, vr, va, vb)
    assert_bitexact(vr.to_numpy(), a * b, "unaligned mul")
    # broadcast path with an unaligned operand
    x = synth.normal((101, 40), 0, 1, 811)
    bias = synth.normal((1, 40), 0, 0.1, 812)
    bx = gpu.T(np.concatenate([[0], x.reshape(-1)]))
    vx = m.Tensor(m.TensorShape(101, 40), _ptr=bx.ptr + 4, _owner=bx)
    r = m.Tensor(m.TensorShape(101, 40))
    m.forward_op(m.OP.ADD, r, vx, gpu.T(bias))
    assert_bitexact(r.to_numpy(), x + bias, "unaligned bcast add")


@pytest.mark.parametrize("shape,axis", [((1000, 256), 0), ((256, 1000), 1), ((70001,), None), ((40, 1000), 1)])
def test_unaligned_reduction_input(gpu, shape, axis):
    """x starting 4 bytes into its allocation: the scalar launchers, whose split partials
    must still fit the library scratch."""
    m = gpu.m
    x = synth.normal(shape, 0, 1, 820)
    base = gpu.T(np.concatenate([[0], x.reshape(-1)]).astype(np.float32))
    vx = m.Tensor(m.TensorShape(*shape), _ptr=base.ptr + 4, _owner=base)
    ax = -1 if axis is None else axis
    kd = dict(axis=axis, keepdims=True) if axis is not None else {}
    red = (1,) if axis is None else tuple(1 if i == axis else d for i, d in enumerate(shape))
    ex = x.astype(np.float64).sum(**kd).reshape(red)
    mag = np.abs(x.astype(np.float64)).sum(**kd).reshape(red)
    assert_sum_close(m.tsum(vx, ax).to_numpy(), ORC.forward(OPS["SUM"], x, axis=axis), ex, "unaligned sum",
                     terms_abs=mag)
    assert_bitexact(m.tmax(vx, ax).to_numpy(), ORC.forward(OPS["MAX"], x, axis=axis), "unaligned max")
    g = m.Tensor(m.TensorShape(*shape))
    ug = synth.normal(red, 0, 1, 821)
    m.backward_op(0, m.OP.MAX, gpu.T(ug), vx, None, g, attributes=None if axis is None else {"axis": axis})
    assert_bitexact(g.to_numpy(), ORC.backward(0, OPS["MAX"], ug, x, axis=axis, grad=np.zeros(shape, np.float32)),
                    "unaligned max bwd")


def test_empty_tensors_are_noops(gpu):
    m = gpu.m
    lib = m.lib()
    S = m._lib.make_shape
    assert lib.mh_binary_fwd(0, None, S((0, 4)), None, S((0, 4)), None, S((1, 4))) == 0
    assert lib.mh_reduce_fwd(8, None, None, S((0, 4)), 1) == 0


# ---------------------------------------------------------------------------------------
# graphs: config 1 (bias + RELU), config 3 (NCHW bias + RELU) and config 5 (classifier head)
# ---------------------------------------------------------------------------------------
def _graph_parity(gpu, nodes, inputs, trainable, seed=None, exact=()):
    g = Graph(nodes, trainable)
    vg = g.forward(gpu, inputs)
    vo = g.forward(ORC, inputs)
    gg = g.backward(gpu, vg, seed)
    go = g.backward(ORC, vo, seed)
    return vg, vo, gg, go


def test_config1_mlp_bias_relu_chain(gpu):
    x = synth.normal((32, 32), 0, 1, 1)
    bias = synth.normal((1, 32), 0, 0.1, 2)
    ug = synth.normal((32, 32), 0, 1, 3)
    nodes = [(OPS["ADD"], ["x", "b"], None, "y"), (OPS["RELU"], ["y"], None, "r")]
    vg, vo, gg, go = _graph_parity(gpu, nodes, {"x": x, "b": bias}, ["x", "b"], seed=ug)
    assert_bitexact(vg["r"], vo["r"], "r")
    assert_bitexact(gg["x"], go["x"], "grad x")
    assert_bitexact(gg["y"], go["y"], "grad y")
    ex = np.where(vo["y"] > 0, ug, 0).astype(np.float64).sum(axis=0, keepdims=True)
    assert_sum_close(gg["b"], go["b"], ex, "grad bias", terms_abs=np.abs(ug).sum(axis=0, keepdims=True))


def test_config3_nchw_bias_relu_small(gpu):
    x = synth.normal((8, 32, 28, 28), 0, 1, 11)
    bias = synth.normal((1, 32, 1, 1), 0, 0.1, 12)
    ug = synth.normal((8, 32, 28, 28), 0, 1, 13)
    nodes = [(OPS["ADD"], ["x", "b"], None, "y"), (OPS["RELU"], ["y"], None, "r")]
    vg, vo, gg, go = _graph_parity(gpu, nodes, {"x": x, "b": bias}, ["x", "b"], seed=ug)
    assert_bitexact(vg["r"], vo["r"], "r")
    assert_bitexact(gg["x"], go["x"], "grad x")
    gy = np.where(vo["y"] > 0, ug, 0).astype(np.float64)
    assert_sum_close(gg["b"], go["b"], gy.sum(axis=(0, 2, 3), keepdims=True), "grad bias",
                     terms_abs=np.abs(gy).sum(axis=(0, 2, 3), keepdims=True))


def test_fused_bias_relu_matches_op_by_op(gpu):
    m = gpu.m
    x = synth.normal((8, 32, 28, 28), 0, 1, 21)
    bias = synth.normal((1, 32, 1, 1), 0, 0.1, 22)
    ug = synth.normal((8, 32, 28, 28), 0, 1, 23)
    tx, tb, tu = gpu.T(x), gpu.T(bias), gpu.T(ug)
    y, r = m.Tensor(tx.shape()), m.Tensor(tx.shape())
    S = m._lib
    S.call("mh_bias_relu_fwd", y.ptr, r.ptr, tx.ptr, tx.shape().c(), tb.ptr, tb.shape().c())
    y_ref = ORC.forward(OPS["ADD"], x, bias)
    assert_bitexact(y.to_numpy(), y_ref, "y")
    assert_bitexact(r.to_numpy(), ORC.forward(OPS["RELU"], y_ref), "r")
    gx, gb = m.Tensor(tx.shape()), m.Tensor(tb.shape())
    S.call("mh_bias_relu_bwd_accum", None, gx.ptr, gb.ptr, y.ptr, tu.ptr, tx.shape().c(), tb.shape().c())
    gy = ORC.backward(0, OPS["RELU"], ug, y_ref)
    assert_bitexact(gx.to_numpy(), ORC.backward(0, OPS["ADD"], gy, x, bias), "fused grad x")
    gyd = gy.astype(np.float64)
    assert_sum_close(gb.to_numpy(), ORC.backward(1, OPS["ADD"], gy, x, bias), gyd.sum(axis=(0, 2, 3), keepdims=True),
                     "fused grad bias", terms_abs=np.abs(gyd).sum(axis=(0, 2, 3), keepdims=True))


FUSED_SHAPES = [((8, 32, 28, 28), (1, 32, 1, 1)), ((2, 3, 64), (3, 1)), ((5, 300), (5, 1)), ((4, 6, 96), (1,)),
                ((3, 7, 10), (1, 7, 1)), ((64, 40), (1, 40)), ((2, 3, 4, 80), (1, 3, 4, 1)), ((3, 2, 20000), (1, 2, 1)),
                ((100, 3, 64), (1, 3, 1)), ((33, 2, 5000), (1, 2, 1)), ((7, 5, 260), (1, 5, 1)),
                ((3, 4, 256), (1, 4, 1)),
                # planes of 449 quads: the slot table's bound, planes starting at every offset of a
                # wave, so some span all eight slots; 450 quads: the two-slots-per-wave layout
                ((22, 3, 1796), (1, 3, 1)), ((5, 3, 1800), (1, 3, 1))]


@pytest.mark.parametrize("sx,sb", FUSED_SHAPES, ids=[f"{a}+{b}" for a, b in FUSED_SHAPES])
@pytest.mark.parametrize("keep_gy", [False, True], ids=["no_gy", "gy"])
def test_fused_bias_relu_shapes(gpu, sx, sb, keep_gy):
    """mh_bias_relu_fwd / _bwd_accum against the op-by-op oracle, accumulating into non-zero
    grads (plane-form shapes take the fused kernels, the others the op-by-op path)."""
    m = gpu.m
    x = synth.normal(sx, 0, 1, 31)
    bias = synth.normal(sb, 0, 0.1, 32)
    ug = synth.normal(sx, 0, 1, 33)
    gy0, gx0, gb0 = synth.normal(sx, 0, 1, 34), synth.normal(sx, 0, 1, 35), synth.normal(sb, 0, 1, 36)
    tx, tb, tu = gpu.T(x), gpu.T(bias), gpu.T(ug)
    y, r = m.Tensor(tx.shape()), m.Tensor(tx.shape())
    S = m._lib
    S.call("mh_bias_relu_fwd", y.ptr, r.ptr, tx.ptr, tx.shape().c(), tb.ptr, tb.shape().c())
    y_ref = ORC.forward(OPS["ADD"], x, bias)
    assert_bitexact(y.to_numpy(), y_ref, "y")
    assert_bitexact(r.to_numpy(), ORC.forward(OPS["RELU"], y_ref), "r")
    tgy, tgx, tgb = gpu.T(gy0), gpu.T(gx0), gpu.T(gb0)
    S.call("mh_bias_relu_bwd_accum", tgy.ptr if keep_gy else None, tgx.ptr, tgb.ptr, y.ptr, tu.ptr, tx.shape().c(),
           tb.shape().c())
    gy = ORC.backward(0, OPS["RELU"], ug, y_ref, grad=gy0 if keep_gy else np.zeros(sx, np.float32))
    if keep_gy:
        assert_bitexact(tgy.to_numpy(), gy, "fused grad y")
    assert_bitexact(tgx.to_numpy(), ORC.backward(0, OPS["ADD"], gy, x, bias, grad=gx0), "fused grad x")
    red = tuple(i for i in range(len(sx)) if i < len(sx) - len(sb) or sb[i - (len(sx) - len(sb))] == 1)
    gyd = gy.astype(np.float64)
    ex = gyd.sum(axis=red).reshape(sb) + gb0.astype(np.float64)
    mag = np.abs(gyd).sum(axis=red).reshape(sb) + np.abs(gb0)
    assert_sum_close(tgb.to_numpy(), ORC.backward(1, OPS["ADD"], gy, x, bias, grad=gb0), ex, "fused grad bias",
                     terms_abs=mag)


FUSED_SPECIAL_SHAPES = [((8, 32, 28, 28), (1, 32, 1, 1)), ((22, 3, 1796), (1, 3, 1)), ((3, 7, 10), (1, 7, 1)),
                        ((64, 40), (1, 40))]


@pytest.mark.parametrize("sx,sb", FUSED_SPECIAL_SHAPES, ids=[f"{a}+{b}" for a, b in FUSED_SPECIAL_SHAPES])
@pytest.mark.parametrize("nonfinite", [False, True], ids=["finite", "nonfinite"])
def test_fused_bias_relu_special_values(gpu, sx, sb, nonfinite):
    """mh_bias_relu_fwd / _bwd_accum against the op-by-op oracle where y = x + bias is a signed
    zero (RELU's gradient at -0 and +0), near the float limit, subnormal, and (nonfinite) NaN
    or infinite, with such values in the upstream gradient too: y, r, grad_y and grad_x
    bit-identical (NaN matching NaN); the bias gradient in the sum class, or NaN / infinite
    exactly where the oracle's is."""
    m = gpu.m
    print(f"\n[fused bias relu special] {sx}+{sb} nonfinite={nonfinite}", flush=True)
    x = synth.normal(sx, 0, 1, 41)
    bias = synth.normal(sb, 0, 0.1, 42)
    bias.reshape(-1)[0] = np.float32(-0.0)
    ug = synth.normal(sx, 0, 1, 43)
    u = synth.uniform(sx, 0, 1, 44)
    x[u < 0.04] = np.float32(-0.0)
    x[(u >= 0.04) & (u < 0.08)] = np.float32(0.0)
    x[(u >= 0.08) & (u < 0.09)] = np.float32(3.0e38)
    x[(u >= 0.09) & (u < 0.10)] = np.float32(-3.0e38)
    x[(u >= 0.10) & (u < 0.11)] = np.float32(1.0e-40)
    ug[(u >= 0.11) & (u < 0.13)] = np.float32(-0.0)
    ug[(u >= 0.13) & (u < 0.14)] = np.float32(2.0e38)
    if nonfinite:
        x[(u >= 0.14) & (u < 0.15)] = np.float32(np.nan)
        x[(u >= 0.15) & (u < 0.16)] = np.float32(np.inf)
        x[(u >= 0.16) & (u < 0.17)] = np.float32(-np.inf)
        ug[(u >= 0.17) & (u < 0.18)] = np.float32(np.nan)
        ug[(u >= 0.18) & (u < 0.19)] = np.float32(np.inf)
    gy0, gx0, gb0 = synth.normal(sx, 0, 1, 45), synth.normal(sx, 0, 1, 46), synth.normal(sb, 0, 1, 47)
    tx, tb, tu = gpu.T(x), gpu.T(bias), gpu.T(ug)
    y, r = m.Tensor(tx.shape()), m.Tensor(tx.shape())
    S = m._lib
    S.call("mh_bias_relu_fwd", y.ptr, r.ptr, tx.ptr, tx.shape().c(), tb.ptr, tb.shape().c())
    y_ref = ORC.forward(OPS["ADD"], x, bias)
    assert_bitexact(y.to_numpy(), y_ref, "y")
    assert_bitexact(r.to_numpy(), ORC.forward(OPS["RELU"], y_ref), "r")
    tgy, tgx, tgb = gpu.T(gy0), gpu.T(gx0), gpu.T(gb0)
    S.call("mh_bias_relu_bwd_accum", tgy.ptr, tgx.ptr, tgb.ptr, y.ptr, tu.ptr, tx.shape().c(), tb.shape().c())
    gy = ORC.backward(0, OPS["RELU"], ug, y_ref, grad=gy0)
    assert_bitexact(tgy.to_numpy(), gy, "fused grad y")
    assert_bitexact(tgx.to_numpy(), ORC.backward(0, OPS["ADD"], gy, x, bias, grad=gx0), "fused grad x")
    ref = ORC.backward(1, OPS["ADD"], gy, x, bias, grad=gb0)
    got = tgb.to_numpy()
    fin = np.isfinite(ref)
    assert (np.isnan(got) == np.isnan(ref)).all() and (np.isinf(got) == np.isinf(ref)).all(), "bias grad non-finite"
    red = tuple(i for i in range(len(sx)) if i < len(sx) - len(sb) or sb[i - (len(sx) - len(sb))] == 1)
    gyd = gy.astype(np.float64)
    ex = gyd.sum(axis=red).reshape(sb) + gb0.astype(np.float64)
    mag = np.abs(gyd).sum(axis=red).reshape(sb) + np.abs(gb0)
    assert_sum_close(got[fin], ref[fin], ex[fin], "fused grad bias", terms_abs=mag[fin])


def config5_inputs(n, seed=0):
    logits = synth.normal((n, 10), 0, 2, 31 + seed)
    cls = synth.integers((n,), 0, 10, 32 + seed)
    onehot = np.zeros((n, 10), np.float32)
    onehot[np.arange(n), cls] = 1.0
    return logits, onehot


def test_config5_classifier_chain_small(gpu):
    logits, onehot = config5_inputs(4099)
    vg, vo, gg, go = _graph_parity(gpu, config5_nodes(), {"logits": logits, "onehot": onehot}, ["logits"])
    assert_bitexact(vg["max"], vo["max"], "max")
    assert_bitexact(vg["xm"], vo["xm"], "xm")
    assert_ulp(vg["e"], vo["e"], 2, "exp")
    # 10-term row sums run sequentially on both sides: same order, same bits
    assert_bitexact(vg["s"], vo["s"], "row sums")
    for k in ("sm", "lp", "t"):
        assert_ulp(vg[k], vo[k], 2, k)
    t64 = vo["t"].astype(np.float64)
    assert_sum_close(vg["loss"], vo["loss"], np.array([t64.mean()]), "loss",
                     terms_abs=np.array([np.abs(t64).mean()]))
    # the loss grad is seeded with 1.0, so no backward value depends on the loss sum
    for k in ("logits", "max", "xm", "e", "s", "sm", "lp", "t"):
        assert_ulp(gg[k], go[k], 2, f"grad {k}")


# every class count up to 16 has a kernel of its own: each appears at least once
SMLM_CASES = [(4099, 10), (1, 1), (3, 2), (257, 3), (1000, 16), (513, 17), (300, 32), (64, 1), (7, 5), (2048, 10),
              (40, 33), (20, 64), (9, 65), (8, 128), (5, 130), (3, 1000), (2, 2047), (777, 47), (1500, 27),
              (513, 63)] + \
             [(259 + k, k) for k in (4, 6, 7, 8, 9, 11, 12, 13, 14, 15)]


def _check_fused_head(gpu, logits, onehot, ugv):
    """The fused config-5 head (mh_softmax_log_mul_mean_fwd / _bwd_accum) against the op-by-op
    graph: the loss in the sum class (both NaN where the graph's is), the gradient bit-exact,
    accumulated into a non-zero grad_x and from zero. Rows shorter than the oracle's 32 SIMD
    lanes sum in element order on every path, so the oracle is the reference; from 32 classes
    its row sums follow the lane order, so the bit-exact reference is the GPU op-by-op chain
    and the oracle is met within the sum class (the fp64 magnitude comparator); up to 64
    classes that chain sums every row in element order and matches the oracle at nelts = 1
    bit for bit."""
    m = gpu.m
    rows, classes = logits.shape
    g = Graph(config5_nodes(), ["logits"])
    seed = np.array([ugv], np.float32)
    vo = g.forward(ORC, {"logits": logits, "onehot": onehot})
    go = g.backward(ORC, vo, seed)
    ref_eng, vr, gr = ORC, vo, go
    if classes >= 32:
        ref_eng = gpu
        vr = g.forward(gpu, {"logits": logits, "onehot": onehot})
        gr = g.backward(gpu, vr, seed)
        fin = np.isfinite(go["logits"])
        assert (np.isfinite(gr["logits"]) == fin).all()
        f64 = Mag64Engine()
        gx64 = g.backward(f64, g.forward(f64, {"logits": logits, "onehot": onehot}), seed)["logits"]
        gx64 = type(gx64)(gx64.v[fin], gx64.M[fin])
        assert_order_close(gr["logits"][fin], go["logits"][fin], gx64, "op-by-op grad vs oracle, reference order")
        if classes <= 64:
            O.set_nelts(1)
            try:
                g1 = g.backward(ORC, g.forward(ORC, {"logits": logits, "onehot": onehot}), seed)
            finally:
                O.set_nelts(32)
            assert_bitexact(gr["logits"], g1["logits"], "op-by-op grad vs oracle, element order")
    tl, to = gpu.T(logits), gpu.T(onehot)
    loss = m.Tensor(m.TensorShape(1))
    m.softmax_log_mul_mean_forward(loss, tl, to)
    if np.isnan(vo["loss"]).any():
        assert np.isnan(loss.to_numpy()).all(), "fused loss should be NaN"
    else:
        t64 = vo["t"].astype(np.float64)
        assert_sum_close(loss.to_numpy(), vo["loss"], np.array([t64.mean()]), "fused loss",
                         terms_abs=np.array([np.abs(t64).mean()]))
    g0 = synth.normal((rows, classes), 0, 1, 64)
    tg = gpu.T(g0)
    m.softmax_log_mul_mean_backward(tg, tl, to, gpu.T(seed))
    exp = ref_eng.backward(0, OPS["SUB"], gr["xm"], logits, vr["max"], grad=g0)
    exp = ref_eng.backward(0, OPS["MAX"], gr["max"], logits, axis=1, grad=exp)
    assert_bitexact(tg.to_numpy(), exp, "fused grad, accumulated")
    tz = m.Tensor(m.TensorShape(rows, classes))
    m.softmax_log_mul_mean_backward(tz, tl, to, gpu.T(seed))
    assert_bitexact(tz.to_numpy(), gr["logits"], "fused grad from zero")


@pytest.mark.parametrize("rows,classes", SMLM_CASES, ids=[f"{r}x{c}" for r, c in SMLM_CASES])
@pytest.mark.parametrize("ugv", [1.0, -0.37])
def test_fused_softmax_log_mul_mean(gpu, rows, classes, ugv):
    """The fused head on one-hot targets (ties injected) against the op-by-op graph."""
    logits = synth.normal((rows, classes), 0, 2, 61)
    if classes > 1:
        synth.inject_ties(logits, 1, 62)
    cls = synth.integers((rows,), 0, classes, 63)
    onehot = np.zeros((rows, classes), np.float32)
    onehot[np.arange(rows), cls] = 1.0
    _check_fused_head(gpu, logits, onehot, ugv)


HEAD_SKIP_CASES = [(4099, 10), (1000, 16), (513, 17), (300, 40), (301, 47), (9, 130), (3, 1000)]


@pytest.mark.parametrize("rows,classes", HEAD_SKIP_CASES, ids=[f"{r}x{c}" for r, c in HEAD_SKIP_CASES])
@pytest.mark.parametrize("case", ["sparse", "tiny_e", "clamped", "nan", "inf_ug"])
def test_fused_head_zero_target_shortcut(gpu, rows, classes, case):
    """The fused head skips the divisions and log of zero-target elements whose e is at least
    2^-100. Targets here are sparse with +0 and -0 zeros, non-unit nonzero values, all-zero and
    dense rows; "tiny_e" puts elements 60-95 below the row max (e on both sides of 2^-100, down
    to subnormal), "clamped" 110 below it and -inf (exp's argument clamp: e is the subnormal
    exp(-88.376...)), "nan" NaN logits (NaN rows and a NaN loss), "inf_ug" an infinite loss
    gradient (g_t not finite: no skipping)."""
    logits = synth.normal((rows, classes), 0, 2, 71)
    u = synth.uniform((rows, classes), 0, 1, 72)
    onehot = np.where(u < 0.08, np.float32(1.0), np.where(u < 0.12, np.float32(-0.0), np.float32(0.0)))
    onehot = onehot.astype(np.float32)
    onehot[u > 0.97] = np.float32(0.3)
    onehot[u < 0.01] = np.float32(-2.0)
    onehot[::7] = 0.0          # all-zero rows
    onehot[3::11] = u[3::11]   # dense rows
    if case in ("tiny_e", "clamped", "nan"):
        mx = logits.max(axis=1)
        cols = synth.integers((rows,), 0, classes, 73)
        gaps = {"tiny_e": [60.0, 69.0, 69.4, 70.0, 80.0, 95.0], "clamped": [110.0, np.inf],
                "nan": [np.nan]}[case]
        for k, r in enumerate(range(0, rows, 2)):
            gap = gaps[k % len(gaps)]
            c = int(cols[r])
            if logits[r, c] == mx[r]:
                continue  # keep the row max in place
            logits[r, c] = np.float32(mx[r] - gap)
    ugv = np.float32(np.inf) if case == "inf_ug" else 0.61
    _check_fused_head(gpu, logits, onehot, ugv)


def test_fused_row_graphs_reject_wide_rows(gpu):
    m = gpu.m
    x = gpu.T(np.zeros((2, 2048), np.float32))
    with pytest.raises(m.MantleHipError):
        m.softmax_log_mul_mean_forward(m.Tensor(m.TensorShape(1)), x, x)
    with pytest.raises(m.MantleHipError):
        m.cross_entropy_forward(m.Tensor(m.TensorShape(1)), x, x)
    with pytest.raises(m.MantleHipError):
        m.softmax_forward(m.Tensor(m.TensorShape(2, 2048)), x)


# Row lengths around every engine boundary: 1-64 one thread per row (element-order sums),
# 65-2047 one wavefront per row (the row-reduction kernel's order; multiples of 4 and not);
# every class count up to 16 (a kernel of its own each) appears.
ROW_CASES = [(300, 1), (7, 2), (257, 3), (100, 10), (33, 31), (65, 32), (40, 33), (17, 63), (16, 64), (9, 65),
             (11, 66), (8, 100), (6, 128), (5, 130), (4, 257), (3, 1000), (2, 1024), (3, 1025), (2, 2044),
             (2, 2047), (1000, 10), (2000, 20), (1500, 48), (777, 47), (1200, 64)] + \
            [(259 + k, k) for k in (4, 5, 6, 7, 8, 9, 11, 12, 13, 14, 15, 16)]


def _seeded_row_cases(count, seed):
    """(rows, classes) drawn with a fixed seed over every row engine: 1-16 classes (the
    pipelined kernels), 17-64 (the thread and multi-lane engines, quad rows or not) and
    65-2047 (a wavefront per row), up to 600 K elements."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        lo, hi = [(1, 17), (17, 65), (65, 2048)][i % 3]
        k = int(rng.integers(lo, hi))
        rows = int(rng.integers(1, max(2, min(3000, 600_000 // k))))
        out.append((rows, k))
    return out


ROW_CASES += _seeded_row_cases(12, 20261204)


@pytest.mark.parametrize("rows,classes", ROW_CASES, ids=[f"{r}x{c}" for r, c in ROW_CASES])
def test_fused_row_graphs(gpu, rows, classes):
    """Softmax, LogSoftmax and CrossEntropyLoss fused (one kernel each way) against the
    op-by-op graphs on the GPU: outputs and gradients bit-identical, accumulated into a
    non-zero grad_x; the cross-entropy loss in the sum class."""
    from util import cross_entropy_nodes, logsoftmax_nodes, softmax_nodes
    m = gpu.m
    x = synth.normal((rows, classes), 0, 2, 1300)
    if classes > 1:
        synth.inject_ties(x, 1, 1301)
    g0 = synth.normal((rows, classes), 0, 1, 1302)
    gout = synth.normal((rows, classes), 0, 1, 1303)
    tx = gpu.T(x)
    for name, nodes, out_name, fwd, bwd in [
            ("softmax", softmax_nodes("x", 1), "sm", m.softmax_forward, m.softmax_backward),
            ("logsoftmax", logsoftmax_nodes("x", 1), "lsm", m.logsoftmax_forward, m.logsoftmax_backward)]:
        g = Graph(nodes, ["x"])
        v = g.forward(gpu, {"x": x})
        out = m.Tensor(m.TensorShape(rows, classes))
        fwd(out, tx)
        assert_bitexact(out.to_numpy(), v[out_name], f"{name} forward")
        gr = g.backward(gpu, v, seed=gout, init={"x": g0})
        tg = gpu.T(g0)
        bwd(tg, tx, gpu.T(gout))
        assert_bitexact(tg.to_numpy(), gr["x"], f"{name} backward")
    # cross entropy with soft targets and a non-unit loss gradient
    target = synth.uniform((rows, classes), 0, 1, 1304)
    cn = np.array([np.float32(-1.0 / rows)], np.float32)
    g = Graph(cross_entropy_nodes("x", "target"), ["x"])
    v = g.forward(gpu, {"x": x, "target": target, "cN": cn})
    loss = m.Tensor(m.TensorShape(1))
    m.cross_entropy_forward(loss, tx, gpu.T(target))
    tl64 = v["tl"].astype(np.float64)
    assert_sum_close(loss.to_numpy(), v["loss"], np.array([tl64.sum() * float(cn[0])]), "cross-entropy loss",
                     terms_abs=np.array([np.abs(tl64).sum() * abs(float(cn[0]))]))
    seed = np.array([0.7], np.float32)
    gr = g.backward(gpu, v, seed=seed, init={"x": g0})
    tg = gpu.T(g0)
    m.cross_entropy_backward(tg, tx, gpu.T(target), gpu.T(seed))
    assert_bitexact(tg.to_numpy(), gr["x"], "cross-entropy backward")


SPECIAL_ROW_CASES = [(64, 1), (131, 3), (200, 10), (129, 16), (70, 20), (65, 33), (40, 100)]


def _special_rows(rows, classes, nonfinite):
    """Logits with signed zeros, magnitudes near the float limit, subnormals and exact ties
    (and with `nonfinite`, NaN and infinities), plus whole rows of one value."""
    x = synth.normal((rows, classes), 0, 2, 1500)
    if classes > 1:
        synth.inject_ties(x, 1, 1501)
    u = synth.uniform((rows, classes), 0, 1, 1502)
    x[u < 0.05] = np.float32(-0.0)
    x[(u >= 0.05) & (u < 0.08)] = np.float32(0.0)
    x[(u >= 0.08) & (u < 0.10)] = np.float32(3.0e38)
    x[(u >= 0.10) & (u < 0.12)] = np.float32(-3.0e38)
    x[(u >= 0.12) & (u < 0.14)] = np.float32(1.0e-40)
    x[1] = np.float32(-3.0e38)
    x[2] = np.float32(-0.0)
    if nonfinite:
        x[(u >= 0.14) & (u < 0.16)] = np.float32(np.nan)
        x[(u >= 0.16) & (u < 0.18)] = np.float32(np.inf)
        x[(u >= 0.18) & (u < 0.20)] = np.float32(-np.inf)
        x[3] = np.float32(-np.inf)
        x[4] = np.float32(np.inf)
    return x


@pytest.mark.parametrize("rows,classes", SPECIAL_ROW_CASES, ids=[f"{r}x{c}" for r, c in SPECIAL_ROW_CASES])
@pytest.mark.parametrize("nonfinite", [False, True], ids=["finite", "nonfinite"])
def test_fused_row_graphs_special_values(gpu, rows, classes, nonfinite):
    """Softmax, LogSoftmax and CrossEntropyLoss fused against the op-by-op graphs on the GPU
    at row lengths of every engine (one-shot and pipelined up to 16 classes, thread and
    multi-lane up to 64, wavefront beyond), on logits with signed zeros, near-limit
    magnitudes, subnormals, ties and whole rows of one value, and (nonfinite) NaN and
    infinities: outputs and gradients bit-identical (NaN matching NaN), the loss in the sum
    class or non-finite where the graph's is."""
    from util import cross_entropy_nodes, logsoftmax_nodes, softmax_nodes
    m = gpu.m
    print(f"\n[special rows] {rows}x{classes} nonfinite={nonfinite}", flush=True)
    x = _special_rows(rows, classes, nonfinite)
    g0 = synth.normal((rows, classes), 0, 1, 1503)
    gout = synth.normal((rows, classes), 0, 1, 1504)
    gout[0] = np.float32(-0.0)
    tx = gpu.T(x)
    for name, nodes, out_name, fwd, bwd in [
            ("softmax", softmax_nodes("x", 1), "sm", m.softmax_forward, m.softmax_backward),
            ("logsoftmax", logsoftmax_nodes("x", 1), "lsm", m.logsoftmax_forward, m.logsoftmax_backward)]:
        g = Graph(nodes, ["x"])
        v = g.forward(gpu, {"x": x})
        out = m.Tensor(m.TensorShape(rows, classes))
        fwd(out, tx)
        assert_bitexact(out.to_numpy(), v[out_name], f"{name} forward")
        gr = g.backward(gpu, v, seed=gout, init={"x": g0})
        tg = gpu.T(g0)
        bwd(tg, tx, gpu.T(gout))
        assert_bitexact(tg.to_numpy(), gr["x"], f"{name} backward")
    target = synth.uniform((rows, classes), 0, 1, 1505)
    target[0] = np.float32(0.0)
    cn = np.array([np.float32(-1.0 / rows)], np.float32)
    g = Graph(cross_entropy_nodes("x", "target"), ["x"])
    v = g.forward(gpu, {"x": x, "target": target, "cN": cn})
    loss = m.Tensor(m.TensorShape(1))
    ttg = gpu.T(target)
    m.cross_entropy_forward(loss, tx, ttg)
    got, ref = loss.to_numpy(), v["loss"]
    if np.isfinite(ref).all():
        tl64 = v["tl"].astype(np.float64)
        assert_sum_close(got, ref, np.array([tl64.sum() * float(cn[0])]), "cross-entropy loss",
                         terms_abs=np.array([np.abs(tl64).sum() * abs(float(cn[0]))]))
    else:
        assert (np.isnan(got) == np.isnan(ref)).all() and (np.isinf(got) == np.isinf(ref)).all(), (got, ref)
    seed = np.array([0.7], np.float32)
    gr = g.backward(gpu, v, seed=seed, init={"x": g0})
    tg = gpu.T(g0)
    m.cross_entropy_backward(tg, tx, ttg, gpu.T(seed))
    assert_bitexact(tg.to_numpy(), gr["x"], "cross-entropy backward")


# Row counts whose one-shot loss partials (one per 64 rows) the one-block combine sums in three
# rounds with a partial count that is not a multiple of four (2999999 rows: 46875 partials), in
# exactly its largest count (64 * 65536 rows), and one past it, where the multi-block
# all-element reduction takes the partials instead.
LOSS_PARTIAL_CASES = [(2_999_999, 2), (64 * 65536, 3), (64 * 65536 + 1, 2)]


@pytest.mark.parametrize("rows,classes", LOSS_PARTIAL_CASES, ids=[f"{r}x{c}" for r, c in LOSS_PARTIAL_CASES])
def test_fused_loss_sums_over_many_block_partials(gpu, rows, classes):
    """The config-5 head and CrossEntropyLoss losses at row counts that take every way the
    block partials of the loss engines are summed, against the op-by-op graphs on the GPU
    (whose per-element terms are the oracle's bits) in the sum class; the cross-entropy
    backward at the same size bit-identical to the op-by-op graph."""
    from util import cross_entropy_nodes
    m = gpu.m
    print(f"\n[loss partials] rows {rows} classes {classes}", flush=True)
    x = synth.normal((rows, classes), 0, 2, 1400)
    cls = synth.integers((rows,), 0, classes, 1401)
    onehot = np.zeros((rows, classes), np.float32)
    onehot[np.arange(rows), cls] = 1.0
    tx = gpu.T(x)
    g = Graph(config5_nodes(), ["logits"])
    v = g.forward(gpu, {"logits": x, "onehot": onehot})
    loss = m.Tensor(m.TensorShape(1))
    m.softmax_log_mul_mean_forward(loss, tx, gpu.T(onehot))
    t64 = v["t"].astype(np.float64)
    assert_sum_close(loss.to_numpy(), v["loss"], np.array([t64.mean()]), "head loss",
                     terms_abs=np.array([np.abs(t64).mean()]))
    target = synth.uniform((rows, classes), 0, 1, 1402)
    cn = np.array([np.float32(-1.0 / rows)], np.float32)
    g = Graph(cross_entropy_nodes("x", "target"), ["x"])
    v = g.forward(gpu, {"x": x, "target": target, "cN": cn})
    ttg = gpu.T(target)
    m.cross_entropy_forward(loss, tx, ttg)
    tl64 = v["tl"].astype(np.float64)
    assert_sum_close(loss.to_numpy(), v["loss"], np.array([tl64.sum() * float(cn[0])]), "cross-entropy loss",
                     terms_abs=np.array([np.abs(tl64).sum() * abs(float(cn[0]))]))
    seed = np.array([0.7], np.float32)
    g0 = synth.normal((rows, classes), 0, 1, 1403)
    gr = g.backward(gpu, v, seed=seed, init={"x": g0})
    tg = gpu.T(g0)
    m.cross_entropy_backward(tg, tx, ttg, gpu.T(seed))
    assert_bitexact(tg.to_numpy(), gr["x"], "cross-entropy backward")


ORACLE_ROW_CASES = [(513, 17), (300, 24), (1000, 31), (40, 33), (777, 47), (1200, 64), (500, 32), (280, 20), (150, 28),
                    (333, 36)]
_rng_oracle_rows = np.random.default_rng(20261202)
ORACLE_ROW_CASES += [(int(_rng_oracle_rows.integers(1, 1500)), int(_rng_oracle_rows.integers(17, 65))) for _ in range(6)]


@pytest.mark.parametrize("rows,classes", ORACLE_ROW_CASES, ids=[f"{r}x{c}" for r, c in ORACLE_ROW_CASES])
def test_fused_rows_17_to_64_classes_against_the_oracle(gpu, rows, classes):
    """The thread, multi-lane and (whole quads of 20-32 classes) one-shot row engines through
    mh_softmax_*, mh_logsoftmax_* and mh_cross_entropy_* against the oracle's op-by-op graphs
    (activations.mojo:74-108, loss.mojo:45-61), ties injected, backward accumulated into a
    non-zero grad_x:
    - bit-exact against the oracle with nelts = 1, whose row sums run in element order, the
      order these engines use: only the order of the sums separates them from the reference;
    - against the reference's lane order (nelts = 32): bit-exact below 32 classes (both orders
      are the element order there), else every element in the fp64 sum class
      (assert_order_close with the fp64 magnitude engine);
    - the cross-entropy loss (an all-element sum in the kernel's own order) in that class."""
    from util import cross_entropy_nodes, logsoftmax_nodes, softmax_nodes
    m = gpu.m
    x = synth.normal((rows, classes), 0, 2, 1300)
    synth.inject_ties(x, 1, 1301)
    g0 = synth.normal((rows, classes), 0, 1, 1302)
    gout = synth.normal((rows, classes), 0, 1, 1303)
    target = synth.uniform((rows, classes), 0, 1, 1304)
    cn = np.array([np.float32(-1.0 / rows)], np.float32)
    seed = np.array([0.7], np.float32)
    tx, tt = gpu.T(x), gpu.T(target)
    f64 = Mag64Engine()

    def graph(eng, nodes, vals, out, ug):
        g = Graph(nodes, ["x"])
        v = g.forward(eng, vals)
        return v[out], g.backward(eng, v, seed=ug, init={"x": g0})["x"]

    cases = []
    for name, nodes, out, fwd, bwd in [
            ("softmax", softmax_nodes("x", 1), "sm", m.softmax_forward, m.softmax_backward),
            ("logsoftmax", logsoftmax_nodes("x", 1), "lsm", m.logsoftmax_forward, m.logsoftmax_backward)]:
        res = m.Tensor(m.TensorShape(rows, classes))
        fwd(res, tx)
        tg = gpu.T(g0)
        bwd(tg, tx, gpu.T(gout))
        cases.append((name, nodes, out, {"x": x}, gout, res.to_numpy(), tg.to_numpy(), True))
    loss = m.Tensor(m.TensorShape(1))
    m.cross_entropy_forward(loss, tx, tt)
    tg = gpu.T(g0)
    m.cross_entropy_backward(tg, tx, tt, gpu.T(seed))
    cases.append(("cross_entropy", cross_entropy_nodes("x", "target"), "loss", {"x": x, "target": target, "cN": cn},
                  seed, loss.to_numpy(), tg.to_numpy(), False))
    try:
        for name, nodes, out, vals, ug, got_f, got_b, fwd_rows in cases:
            O.set_nelts(1)
            e1 = graph(ORC, nodes, vals, out, ug)
            O.set_nelts(32)
            e32 = graph(ORC, nodes, vals, out, ug)
            ex = graph(f64, nodes, vals, out, ug)
            if fwd_rows:
                assert_bitexact(got_f, e1[0], f"{name} forward vs oracle, element order")
            assert_bitexact(got_b, e1[1], f"{name} backward vs oracle, element order")
            for got, ref, e, what in ((got_f, e32[0], ex[0], "forward"), (got_b, e32[1], ex[1], "backward")):
                if classes < 32 and (fwd_rows or what == "backward"):
                    assert_bitexact(got, ref, f"{name} {what} vs oracle, reference order")
                assert_order_close(got, ref, e, f"{name} {what} vs oracle, reference order")
    finally:
        O.set_nelts(32)


def test_fused_cross_entropy_matches_reference_fixtures(gpu):
    """test_loss.mojo:86-171: 0.76794958 and 1.31794953 (its 'almost6' tolerance)."""
    m = gpu.m
    x = np.array([[0.1, 0.2, 0.7], [0.7, 0.2, 0.1]], np.float32)
    for t, exp in [([[0, 0, 1], [1, 0, 0]], 0.76794958), ([[0, 1, 0], [0, 0, 1]], 1.31794953)]:
        loss = m.Tensor(m.TensorShape(1))
        m.cross_entropy_forward(loss, gpu.T(x), gpu.T(np.array(t, np.float32)))
        np.testing.assert_allclose(loss.to_numpy()[0], exp, rtol=1e-5, atol=1e-8)


# ---------------------------------------------------------------------------------------
# Adam.step (mantle/nn/optim.mojo:94-140)
# ---------------------------------------------------------------------------------------
ADAM_HP = dict(lr=0.01, beta1=0.9, beta2=0.999, eps=1e-8)


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 65537])
def test_adam_step_single(gpu, n):
    m = gpu.m
    p = synth.normal((n,), 0, 1, 70)
    mo, vo = np.zeros(n, np.float32), np.zeros(n, np.float32)
    tp, tm, tv = gpu.T(p), m.Tensor(m.TensorShape(n)), m.Tensor(m.TensorShape(n))
    L = m.lib()
    for it in range(1, 5):
        g = synth.normal((n,), 0, 0.1, 71 + it)
        tg = gpu.T(g)
        m._lib.check(L.mh_adam_step(tp.ptr, tg.ptr, tm.ptr, tv.ptr, n, ADAM_HP["lr"], ADAM_HP["beta1"],
                                    ADAM_HP["beta2"], ADAM_HP["eps"], it))
        p, mo, vo = O.adam_step(p, g, mo, vo, it, ADAM_HP["lr"], ADAM_HP["beta1"], ADAM_HP["beta2"], ADAM_HP["eps"])
        assert_bitexact(tm.to_numpy(), mo, f"m it {it}")
        assert_bitexact(tv.to_numpy(), vo, f"v it {it}")
        assert_bitexact(tp.to_numpy(), p, f"param it {it}")
    assert L.mh_adam_step(tp.ptr, tp.ptr, tm.ptr, tv.ptr, n, 0.01, 0.9, 0.999, 1e-8, 0) == m._lib.ERR_INVALID


def test_adam_step_multi_and_optimizer(gpu):
    """90 tensors (two launches of the 80-tensor table), sizes 0..5000 with ragged tails and one
    unaligned view, through mantle_amd.Adam (step counts iter, zero_grad clears)."""
    m = gpu.m
    sizes = [0, 1, 2, 3, 4, 5, 7, 8, 33, 64, 100, 257, 1000, 4099, 5000] + [int(s) for s in synth.integers((75,), 1, 3000, 75)]
    params, grads, ps, owners = [], [], [], []
    for i, n in enumerate(sizes):
        p = synth.normal((max(n, 1),), 0, 1, 100 + i)[:n] if n else np.zeros(0, np.float32)
        ps.append(p.copy())
        if i == 20 and n > 0:  # an unaligned view
            base = gpu.T(np.concatenate([[0], p]).astype(np.float32))
            owners.append(base)
            tp = m.Tensor(m.TensorShape(n), _ptr=base.ptr + 4, _owner=base)
        else:
            tp = gpu.T(p) if n else m.Tensor(m.TensorShape(0))
        params.append(tp)
        grads.append(m.Tensor(m.TensorShape(n)))
    opt = m.Adam(list(zip(params, grads)), lr=ADAM_HP["lr"])
    mos = [np.zeros(n, np.float32) for n in sizes]
    vos = [np.zeros(n, np.float32) for n in sizes]
    for it in range(1, 4):
        gs = []
        for i, n in enumerate(sizes):
            g = synth.normal((max(n, 1),), 0, 0.1, 300 + 10 * i + it)[:n]
            gs.append(g)
            if n:
                m._lib.call("mh_memcpy_h2d", grads[i].ptr, np.ascontiguousarray(g).ctypes.data, n * 4)
        opt.step()
        assert opt.iter == it
        for i, n in enumerate(sizes):
            ps[i], mos[i], vos[i] = O.adam_step(ps[i], gs[i], mos[i], vos[i], it, ADAM_HP["lr"])
            if n:
                assert_bitexact(params[i].to_numpy(), ps[i], f"param {i} it {it}")
                assert_bitexact(opt.momentum_grads[i].to_numpy(), mos[i], f"m {i} it {it}")
                assert_bitexact(opt.rms_grads[i].to_numpy(), vos[i], f"v {i} it {it}")
    opt.zero_grad()
    assert all(not g.to_numpy().any() for g in grads)


@pytest.mark.parametrize("off", [(1, 1, 1, 1), (2, 2, 2, 2), (3, 3, 3, 3), (1, 0, 2, 3)])
@pytest.mark.parametrize("n", [1, 2, 5, 1001])
def test_adam_step_misaligned_views(gpu, off, n):
    """Views at element offsets into aligned buffers: a shared offset takes the head-then-quads
    path, mixed offsets the scalar one."""
    m = gpu.m
    L = m.lib()
    p = synth.normal((n,), 0, 1, 80)
    mo, vo = np.zeros(n, np.float32), np.zeros(n, np.float32)
    views, owners = [], []
    for j, init in enumerate([p, None, mo, vo]):
        base = gpu.T(np.zeros(n + off[j], np.float32) if init is None else np.concatenate([np.zeros(off[j], np.float32), init]))
        owners.append(base)
        views.append(base.ptr + 4 * off[j])
    for it in range(1, 4):
        g = synth.normal((n,), 0, 0.1, 81 + it)
        m._lib.call("mh_memcpy_h2d", views[1], np.ascontiguousarray(g).ctypes.data, n * 4)
        m._lib.check(L.mh_adam_step(views[0], views[1], views[2], views[3], n, 0.01, 0.9, 0.999, 1e-8, it))
        p, mo, vo = O.adam_step(p, g, mo, vo, it, 0.01, 0.9, 0.999, 1e-8)
        got = [owners[j].to_numpy()[off[j]:] for j in (0, 2, 3)]
        assert_bitexact(got[0], p, f"param it {it}")
        assert_bitexact(got[1], mo, f"m it {it}")
        assert_bitexact(got[2], vo, f"v it {it}")
        for j in (0, 2, 3):  # nothing written before the view
            assert not owners[j].to_numpy()[:off[j]].any()


# ---------------------------------------------------------------------------------------
# FMA (basics.mojo:759-817), LEAKYRELU (mlops.mojo:128-186), CLIP (mlops.mojo:238-299)
# ---------------------------------------------------------------------------------------
ADJ_SIZES = [1, 3, 4, 5, 1023, 65537, 1 << 20]


def _adj_inputs(n, seed):
    x = synth.normal((n,), 0, 3, seed)
    x[: min(n, 7)] = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.1, -1.1], np.float32)[: min(n, 7)]
    return x


@pytest.mark.parametrize("n", ADJ_SIZES)
def test_fma_parity(gpu, n):
    a, b, c = (synth.normal((n,), 0, 1, 1100 + k) for k in range(3))
    assert_bitexact(gpu.forward(OPS["FMA"], a, b, t3=c), O.fma_fwd(a, b, c), "fma fwd")
    ug, g0 = synth.normal((n,), 0, 1, 1104), synth.normal((n,), 0, 1, 1105)
    for tid in range(3):
        m = gpu.m
        g = gpu.T(g0)
        m.backward_op(tid, m.OP.FMA, gpu.T(ug), gpu.T(a), gpu.T(b), g, t3=gpu.T(c))
        assert_bitexact(g.to_numpy(), O.fma_bwd_accum(tid, g0, ug, a, b), f"fma bwd {tid}")


@pytest.mark.parametrize("n", ADJ_SIZES)
def test_leakyrelu_clip_parity(gpu, n):
    x, ug, g0 = _adj_inputs(n, 1110), synth.normal((n,), 0, 1, 1111), synth.normal((n,), 0, 1, 1112)
    for slope in (0.1, 0.0, -0.5):
        at = {"negative_slope": slope}
        assert_bitexact(gpu.forward(OPS["LEAKYRELU"], x, attrs=at), O.leakyrelu_fwd(x, slope), f"leaky {slope}")
        assert_bitexact(gpu.backward(0, OPS["LEAKYRELU"], ug, x, grad=g0, attrs=at),
                        O.leakyrelu_bwd_accum(g0, x, ug, slope), f"leaky bwd {slope}")
    for at in ({}, {"min": -1.1}, {"max": 1.1}, {"min": -1.1, "max": 1.1}, {"min": 0.0, "max": 0.0}):
        lo, hi = at.get("min", -O.FLT_MAX), at.get("max", O.FLT_MAX)
        assert_bitexact(gpu.forward(OPS["CLIP"], x, attrs=at), O.clip_fwd(x, lo, hi), f"clip {at}")
        assert_bitexact(gpu.backward(0, OPS["CLIP"], ug, x, grad=g0, attrs=at),
                        O.clip_bwd_accum(g0, x, ug, lo, hi), f"clip bwd {at}")


def test_adjacent_ops_unaligned_and_errors(gpu):
    m = gpu.m
    n = 10007
    x = _adj_inputs(n, 1120)
    base = gpu.T(np.concatenate([[0], x]).astype(np.float32))
    vx = m.Tensor(m.TensorShape(n), _ptr=base.ptr + 4, _owner=base)
    r = m.Tensor(m.TensorShape(n))
    m.forward_op(m.OP.CLIP, r, vx, attributes={"min": -2.0, "max": 0.5})
    assert_bitexact(r.to_numpy(), O.clip_fwd(x, -2.0, 0.5), "unaligned clip")
    m.forward_op(m.OP.FMA, r, vx, vx, t3=vx)
    assert_bitexact(r.to_numpy(), O.fma_fwd(x, x, x), "unaligned fma")
    L = m.lib()
    assert L.mh_fma_bwd_accum(3, r.ptr, r.ptr, r.ptr, r.ptr, n) == m._lib.ERR_INVALID
    with pytest.raises(m.MantleHipError):
        m.forward_op(m.OP.LEAKYRELU, r, vx)  # negative_slope is required


# ---------------------------------------------------------------------------------------
# tstd (tensorutils.mojo:724-741, 776-840)
# ---------------------------------------------------------------------------------------
TSTD_CASES = [((87, 73, 107), 0), ((87, 73, 107), 1), ((87, 73, 107), 2), ((87, 73, 107), None),
              ((1024, 1024), 0), ((1024, 1024), 1), ((64, 512, 1024), 2), ((4099, 10), 1), ((2, 10), 0),
              ((3, 4, 5), 1), ((1,), None), ((5,), 0), ((2, 70000), 1), ((70000, 3), 0), ((1 << 22,), None),
              ((1000, 20), 1), ((513, 32), 1), ((40, 33), 1), ((3, 4100), 1), ((300, 256), 0),
              ((33, 512, 128), 1), ((9000, 64), 0), ((5, 1, 7), 1), ((7, 4), 1), ((9, 8), 1), ((6, 4096), 1),
              ((5, 16384), 1), ((3, 12000), 1), ((2, 3, 16388), 2),
              # strided splits of 65 rows whose last split is shorter than one group of eight
              # rows (5 / 10 rows), column quads and single columns
              ((16385, 4), 0), ((16385, 3), 0), ((16390, 8), 0)]


@pytest.mark.parametrize("shape,axis", TSTD_CASES, ids=[f"{s}-ax{a}" for s, a in TSTD_CASES])
def test_tstd_parity(gpu, shape, axis):
    x = synth.normal(shape, 1.5, 2, 1130)
    red = (1,) if axis is None else tuple(1 if i == axis else d for i, d in enumerate(shape))
    ex = (x.astype(np.float64).std() if axis is None else x.astype(np.float64).std(axis=axis, keepdims=True))
    ex = np.asarray(ex).reshape(red)
    got = gpu.tstd(x, axis)
    assert got.shape == red
    assert_sum_close(got, ORC.tstd(x, axis), ex, f"tstd {shape} axis {axis}")


TSTD_OFFSET_CASES = [((1000, 256), 0), ((1000, 256), 1), ((1000, 256), None), ((37, 63, 107), 1),
                     ((3, 40000), 1), ((2, 3, 20002), 2), ((16385, 4), 0)]


@pytest.mark.parametrize("shape,axis", TSTD_OFFSET_CASES, ids=[f"{s}-ax{a}" for s, a in TSTD_OFFSET_CASES])
def test_tstd_large_mean_small_spread(gpu, shape, axis):
    """Lines whose mean is 10^5 of their spread (mean 1000, std 0.01): the one-pass fp64
    moments about each line's first element against the oracle's fp32 two passes, in the sum
    class (which accepts the result closer to the fp64 standard deviation of the same fp32
    values)."""
    x = synth.normal(shape, 1000.0, 0.01, 1140)
    red = (1,) if axis is None else tuple(1 if i == axis else d for i, d in enumerate(shape))
    ex = (x.astype(np.float64).std() if axis is None else x.astype(np.float64).std(axis=axis, keepdims=True))
    ex = np.asarray(ex).reshape(red)
    got = gpu.tstd(x, axis)
    assert_sum_close(got, ORC.tstd(x, axis), ex, f"tstd {shape} axis {axis}")
    np.testing.assert_allclose(got, ex, rtol=1e-4)


def test_tstd_of_empty_lines_is_nan(gpu):
    """Lines of length 0: the reference divides 0 by 0 (tensorutils.mojo:735-744, 836-838)."""
    for shape, axis in (((3, 0), 1), ((0,), None), ((2, 0, 5), 1)):
        x = np.zeros(shape, np.float32)
        ref = ORC.tstd(x, axis)
        got = gpu.tstd(x, axis)
        assert got.shape == ref.shape and np.isnan(ref).all() and np.isnan(got).all(), (shape, axis)


def test_tstd_unaligned(gpu):
    m = gpu.m
    x = synth.normal((1000, 256), 0, 1, 1131)
    base = gpu.T(np.concatenate([[0], x.reshape(-1)]).astype(np.float32))
    vx = m.Tensor(m.TensorShape(1000, 256), _ptr=base.ptr + 4, _owner=base)
    for ax in (0, 1, -1):
        a = None if ax < 0 else ax
        ex = np.asarray(x.astype(np.float64).std(axis=a, keepdims=a is not None)).reshape(ORC.tstd(x, a).shape)
        assert_sum_close(m.tstd(vx, ax).to_numpy(), ORC.tstd(x, a), ex, f"unaligned tstd axis {ax}")


@pytest.mark.parametrize("xshape", [(16, 32, 8, 8), (8, 32, 28, 28), (3, 5, 16, 4), (300, 3, 64, 1)])
def test_bias_gradient_plane_form(gpu, xshape):
    """Broadcast backward into a per-channel operand [1, C, 1, 1] (the one-launch plane form
    of the un-broadcast when H*W is a multiple of 4 and at least 64): every binary op's
    operand-1 gradient against the oracle in the sum class, called twice in a row (the
    arrival counters start at zero again), and accumulate_grad directly."""
    m = gpu.m
    C = xshape[1]
    bshape = (1, C) + (1,) * (len(xshape) - 2)
    x = synth.normal(xshape, 0, 1, 1500)
    b = synth.uniform(bshape, 0.5, 2, 1501)
    ug = synth.normal(xshape, 0, 1, 1502)
    g0 = synth.normal(bshape, 0, 1, 1503)
    red = tuple(i for i in range(len(xshape)) if bshape[i] == 1)
    rg = {"ADD": ug, "SUB": -ug, "MUL": ug * x, "DIV": ((-x) / (b * b)) * ug}
    for name in ("ADD", "SUB", "MUL", "DIV"):
        exp = O.backward_op(1, OPS[name], ug, x, b, grad=g0)
        r64 = rg[name].astype(np.float64)
        ex = r64.sum(axis=red, keepdims=True) + g0
        mag = np.abs(r64).sum(axis=red, keepdims=True) + np.abs(g0)
        for rep in range(2):
            got = gpu.backward(1, OPS[name], ug, x, b, grad=g0)
            assert_sum_close(got, exp, ex, f"{name} bias grad {xshape} call {rep}", terms_abs=mag)
    tg = gpu.T(g0)
    m.accumulate_grad(tg, gpu.T(ug))
    assert_sum_close(tg.to_numpy(), O.accumulate_grad(g0, ug),
                     ug.astype(np.float64).sum(axis=red, keepdims=True) + g0, "accumulate_grad",
                     terms_abs=np.abs(ug.astype(np.float64)).sum(axis=red, keepdims=True) + np.abs(g0))
