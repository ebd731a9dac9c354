"""Pins the CPU oracle (oracle/liboracle.so) before it is trusted as the parity checker:
against the closed-form cases of Mantle's own tests, and against what the mathematics fixes
(fp64 results, exact small-integer sums, brute force on tiny inputs, symmetries)."""
import math

import numpy as np
import pytest

from util import (O, OPS, Graph, Mag64Engine, OracleEngine, assert_bitexact, assert_order_close,
                  assert_sum_close, check_fixture, cross_entropy_nodes, load_fixtures, logsoftmax_nodes,
                  softmax_nodes, spec_to_array, ulp_dist)

FIXTURES = load_fixtures()
ENG = OracleEngine()


@pytest.fixture(autouse=True)
def _nelts():
    O.set_nelts(32)
    yield
    O.set_nelts(32)


@pytest.mark.parametrize("case", [c for c in FIXTURES if c["kind"] != "accumulate"], ids=lambda c: c["id"])
def test_reference_fixture(case):
    check_fixture(ENG, case)


def test_accumulate_fixtures():
    ok = [c for c in FIXTURES if c["kind"] == "accumulate" and "reject" not in c]
    for c in ok:
        g = O.accumulate_grad(np.zeros(c["grad_shape"], np.float32), spec_to_array(c["rg"]))
        np.testing.assert_array_equal(g, spec_to_array(c["expected"]))
    # (2,1) <- (2,3,4) is accepted by the reference only by indexing out of bounds
    bad = [c for c in FIXTURES if "reject" in c]
    assert bad
    for c in bad:
        assert O.accumulate_grad_rc(tuple(c["grad_shape"]), spec_to_array(c["rg"])) == -2


# ---------------------------------------------------------------------------------------
# shapes and broadcasting (tests/python/test_broadcast_shapes.mojo checks numpy agreement)
# ---------------------------------------------------------------------------------------
def _rand_shapes(rng, n):
    out = []
    for _ in range(n):
        r = int(rng.integers(1, 6))
        base = [int(rng.integers(1, 5)) for _ in range(r)]
        other = [d if rng.random() < 0.6 else (1 if rng.random() < 0.8 else int(rng.integers(1, 5))) for d in base]
        cut = int(rng.integers(0, r))
        out.append((tuple(base), tuple(other[cut:]) or (1,)))
    return out


def test_broadcast_shapes_vs_numpy():
    rng = np.random.default_rng(1)
    for a, b in _rand_shapes(rng, 400):
        try:
            ref = np.broadcast_shapes(a, b)
        except ValueError:
            ref = None
        assert O.broadcast_shapes(a, b) == ref, (a, b)
        assert O.broadcast_shapes(b, a) == ref, (b, a)


def test_get_real_index_matches_numpy_broadcast_view():
    # index of the compact operand element feeding each output element
    for small, big in [((1, 32), (32, 32)), ((1, 32, 1, 1), (4, 32, 3, 3)), ((5, 2, 1, 4), (5, 2, 3, 4)),
                       ((2, 3, 4), (5, 2, 3, 4)), ((7, 1), (7, 10)), ((1,), (3, 4))]:
        ids = np.arange(int(np.prod(small)), dtype=np.int64).reshape(small)
        expect = np.broadcast_to(ids, big).reshape(-1)
        st = O.broadcast_calculate_strides(len(big), small)
        got = [O.get_real_index(st, big, i) for i in range(int(np.prod(big)))]
        np.testing.assert_array_equal(got, expect)


# ---------------------------------------------------------------------------------------
# elementwise forward: single IEEE ops, bit-exact against numpy's float32 arithmetic
# ---------------------------------------------------------------------------------------
BIN_NP = {0: np.add, 1: np.subtract, 2: np.multiply, 3: np.divide}


@pytest.mark.parametrize("op", [0, 1, 2, 3])
@pytest.mark.parametrize("sa,sb", [((37, 63, 107), (37, 63, 107)), ((37, 63, 107), (37, 63, 1)),
                                   ((37, 63, 1), (37, 63, 107)), ((2, 3, 4), (5, 2, 1, 4)),
                                   ((33,), (1,)), ((1,), (33,)), ((8, 1, 5), (1, 6, 1))])
def test_binary_forward_bitexact(op, sa, sb):
    rng = np.random.default_rng(op)
    a = rng.uniform(-1, 1, sa).astype(np.float32)
    b = rng.uniform(0.5, 2, sb).astype(np.float32)
    with np.errstate(all="ignore"):
        ref = BIN_NP[op](a, b)
    assert_bitexact(ENG.forward(op, a, b), ref, f"op {op} {sa} {sb}")


def test_relu_signed_zero_and_nan():
    x = np.array([-0.0, 0.0, -1.0, 2.0, np.nan, -np.inf, np.inf], np.float32)
    r = O.elwise_transform(O.RELU, x)
    np.testing.assert_array_equal(r.view(np.uint32), np.array([0, 0, 0, 2.0, 0, 0, np.inf], np.float32).view(np.uint32))
    # backward into a zero grad: 0 * (negative ug) = -0.0, then 0 + -0.0 = +0.0 (ops.mojo:405)
    g = O.backward_op(0, O.RELU, np.full(7, -3.0, np.float32), x)
    assert not np.signbit(g[[0, 1, 2, 4, 5]]).any()


# ---------------------------------------------------------------------------------------
# transcendental functions: bounds against fp64
# ---------------------------------------------------------------------------------------
def _ulps_vs64(got32, ref64):
    ref32 = ref64.astype(np.float32)
    return np.abs(got32.astype(np.float64) - ref64) / np.spacing(np.abs(ref32)).astype(np.float64)


def test_exp_within_2ulp_of_fp64_on_config_domains():
    rng = np.random.default_rng(7)
    for lo, hi, bound in [(-10, 10, 2.0), (-30, 30, 2.0), (-88, 88, 6.0)]:
        x = rng.uniform(lo, hi, 200_000).astype(np.float32)
        e = _ulps_vs64(O.elwise_transform(O.EXP, x), np.exp(x.astype(np.float64)))
        assert e.max() <= bound, (lo, hi, e.max())
    sp = O.elwise_transform(O.EXP, np.array([0.0, -0.0, np.nan], np.float32))
    assert sp[0] == 1.0 and sp[1] == 1.0 and np.isnan(sp[2])


def test_log_within_2ulp_of_fp64_and_special_values():
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.uniform(1e-3, 10, 200_000), np.exp(rng.uniform(-87, 88, 100_000)),
                        rng.uniform(1e-44, 1e-38, 1000)]).astype(np.float32)
    x = x[x > 0]
    e = _ulps_vs64(O.elwise_transform(O.LOG, x), np.log(x.astype(np.float64)))
    assert e.max() <= 2.0, e.max()
    sp = O.elwise_transform(O.LOG, np.array([1.0, 0.0, -1.0, np.inf, np.nan], np.float32))
    assert sp[0] == 0.0 and sp[1] == -np.inf and np.isnan(sp[2]) and sp[3] == np.inf and np.isnan(sp[4])


def test_sigmoid_bound_and_special_points():
    rng = np.random.default_rng(9)
    x = (rng.standard_normal(200_000) * 3).astype(np.float32)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert _ulps_vs64(O.elwise_transform(O.SIGMOID, x), ref).max() <= 3.0
    assert O.lib().or_sigmoid(0.0) == 0.5


def test_tanh_formula_bound_and_symmetry():
    # (e^x - e^-x)/(e^x + e^-x) cancels near 0: bounded in absolute terms, exactly odd
    rng = np.random.default_rng(10)
    x = (rng.standard_normal(200_000) * 3).astype(np.float32)
    t = O.elwise_transform(O.TANH, x)
    assert np.abs(t.astype(np.float64) - np.tanh(x.astype(np.float64))).max() <= 4e-7
    assert_bitexact(O.elwise_transform(O.TANH, -x), -t, "tanh odd")
    assert O.lib().or_tanh(0.0) == 0.0
    # the sign is right and |t| <= 1
    assert (np.sign(t) == np.sign(x)).all() and (np.abs(t) <= 1).all()


def _exp_rn(v):
    """exp correctly rounded to float32 (fp64 exp, then one rounding)."""
    return np.exp(np.asarray(v, np.float64)).astype(np.float32)


def test_tanh_is_the_exp_cancellation_formula():
    """TANH.tanh, mlops.mojo:195-201, is (e^x - e^-x) / (e^x + e^-x) in float32, not a library
    tanh. Two properties fix that formula independently of the oracle's code:
    - for x in (2^-20, 2^-13), e^x rounds to 1 + k 2^-23 and e^-x to 1 - j 2^-24, their sum to
      exactly 2, so the result is an exact multiple of 2^-25 (a correctly rounded tanh, ~x, is
      one in about 1 of 2^5..2^12 cases only by chance);
    - wherever the oracle's exp is the correctly rounded exp at both x and -x, its tanh has the
      bits of that formula evaluated in numpy float32 arithmetic over np.exp's values."""
    rng = np.random.default_rng(12)
    x = np.exp2(rng.uniform(-20, -13, 100_000)).astype(np.float32)
    t = O.elwise_transform(O.TANH, x)
    q = t.astype(np.float64) * 2.0 ** 25
    assert (q == np.round(q)).all(), "tanh near 0 is not quantised to 2^-25"
    lib = np.tanh(x.astype(np.float64)).astype(np.float32).astype(np.float64) * 2.0 ** 25
    assert (lib == np.round(lib)).mean() < 0.01  # the signature tells the two apart
    assert np.abs(t.astype(np.float64) - np.tanh(x.astype(np.float64))).max() <= 2.0 ** -24
    for xs in (x, (rng.standard_normal(400_000) * 3).astype(np.float32),
               rng.uniform(-12, 12, 200_000).astype(np.float32)):
        xs = np.concatenate([xs, -xs])
        ts = O.elwise_transform(O.TANH, xs)
        ep, em = _exp_rn(xs), _exp_rn(-xs)
        with np.errstate(over="ignore", invalid="ignore"):
            formula = (ep - em) / (ep + em)
        same = (O.elwise_transform(O.EXP, xs) == ep) & (O.elwise_transform(O.EXP, -xs) == em)
        assert same.mean() > 0.5, same.mean()
        assert_bitexact(ts[same], formula[same], "tanh vs the reference formula")


def test_powi_is_square_and_multiply():
    rng = np.random.default_rng(11)
    x = rng.uniform(0.1, 4, 1000).astype(np.float32)
    assert_bitexact(O.elwise_pow(x, 0), np.ones_like(x), "x^0")
    assert_bitexact(O.elwise_pow(x, 1), x, "x^1")
    assert_bitexact(O.elwise_pow(x, 2), x * x, "x^2")
    assert_bitexact(O.elwise_pow(x, 3), x * (x * x), "x^3")
    assert_bitexact(O.elwise_pow(x, 5), x * ((x * x) * (x * x)), "x^5")
    assert_bitexact(O.elwise_pow(x, -2), np.float32(1) / (x * x), "x^-2")
    # POW.forward truncates the float exponent toward zero (basics.mojo:327)
    for e, n in [(2.9, 2), (0.7, 0), (-1.5, -1), (1.0, 1)]:
        got = O.forward_op(O.POW, x, np.array([e], np.float32))
        assert_bitexact(got, O.elwise_pow(x, n), f"trunc {e}")


def test_powf_bound_and_rules():
    rng = np.random.default_rng(12)
    x = rng.uniform(0.1, 4, 20_000).astype(np.float32)
    for y in (0.5, 1.37, 2.71, -0.5):
        got = np.array([O.powf_scalar(v, y) for v in x], np.float32)
        ref = x.astype(np.float64) ** np.float64(np.float32(y))
        # exp(y*log x) carries |y log x| * 2^-24 relative error from the product rounding
        assert _ulps_vs64(got, ref).max() <= 8.0, y
    assert O.powf_scalar(0.0, 0.0) == 1.0  # integral exponent: _powi (0^0 = 1)
    assert O.powf_scalar(3.0, 2.0) == 9.0
    assert math.isnan(O.powf_scalar(-2.0, 0.5))
    assert O.powf_scalar(-2.0, 3.0) == -8.0


def _pow_composition_signature(powfn, x, y32):
    """Share of eligible samples where powfn(x, y) has the bits of RN(exp(fl32(y * RN(log x)))),
    and the share of them where that composition differs from the correctly rounded x^y.
    Eligible: the oracle's log is correctly rounded at x and its exp at p = fl32(y * RN(log x)),
    so the composition's value is fixed by fp64 numpy alone, not by the oracle's code."""
    l_rn = np.log(x.astype(np.float64)).astype(np.float32)
    p = (y32 * l_rn).astype(np.float32)  # one float32 rounding of the product
    e_rn = _exp_rn(p)
    ok = (O.elwise_transform(O.LOG, x) == l_rn) & (O.elwise_transform(O.EXP, p) == e_rn)
    got = np.asarray(powfn(x, y32), np.float32)
    same = (got[ok].view(np.uint32) == e_rn[ok].view(np.uint32)).mean()
    pow_rn = (x.astype(np.float64) ** np.float64(y32)).astype(np.float32)
    differs = (e_rn[ok] != pow_rn[ok]).mean()
    return ok.mean(), same, differs


def test_powf_is_exp_of_y_times_log():
    """Float SIMD ** SIMD (basics.mojo:353 `** (a - 1)`, :373 `** a`) restated as the Mojo
    stdlib's `_powf_scalar` (std/builtin/simd.mojo): an integral exponent through `_powi`, a
    negative base with a fractional exponent NaN, otherwise `exp(y * log(x))` over the stdlib's
    f32 exp and log. Where the oracle's log and exp are correctly rounded, its pow must have
    exactly the bits of that composition evaluated in fp64 numpy; the composition differs from
    a correctly rounded x^y (what a library powf returns) in a large share of those samples, so
    a library powf in its place fails the check (the second loop shows it does)."""
    rng = np.random.default_rng(21)
    x = rng.uniform(0.1, 4, 30_000).astype(np.float32)
    oracle_pow = lambda xs, y: [O.powf_scalar(v, y) for v in xs]  # noqa: E731
    library_pow = lambda xs, y: (xs.astype(np.float64) ** np.float64(y)).astype(np.float32)  # noqa: E731
    # config 2's exponent (the exponent gradient's `** a`), its `a - 1`, and a third point
    for y in (2.4349, 1.4349, 2.9):
        y32 = np.float32(y)
        eligible, same, differs = _pow_composition_signature(oracle_pow, x, y32)
        assert eligible > 0.7, (y, eligible)
        assert same == 1.0, (y, same)
        assert differs > 0.3, (y, differs)
        # negative control: a correctly rounded pow misses the composition's bits
        _, lib_same, _ = _pow_composition_signature(library_pow, x, y32)
        assert lib_same < 0.7, (y, lib_same)


# ---------------------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------------------
def test_reduce_all_nelts1_is_sequential():
    rng = np.random.default_rng(13)
    x = rng.standard_normal(1001).astype(np.float32)
    O.set_nelts(1)
    acc = np.float32(0)
    for v in x:
        acc = np.float32(acc + v)
    assert O.reduce_all(O.SUM, x) == acc


@pytest.mark.parametrize("nelts", [1, 8, 32])
def test_small_integer_sums_are_exact_in_any_order(nelts):
    O.set_nelts(nelts)
    rng = np.random.default_rng(14)
    x = rng.integers(-50, 50, (13, 37, 11)).astype(np.float32)
    for ax in (None, 0, 1, 2):
        got = ENG.forward(OPS["SUM"], x, axis=ax)
        ref = x.sum(axis=ax, keepdims=True).astype(np.float32) if ax is not None else np.array([x.sum()], np.float32)
        np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("shape,axis", [((87, 73, 107), 0), ((87, 73, 107), 1), ((87, 73, 107), 2),
                                        ((87, 73, 107), None), ((4096, 3), 0)])
def test_sum_mean_max_vs_fp64(shape, axis):
    rng = np.random.default_rng(15)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    kd = dict(axis=axis, keepdims=True) if axis is not None else {}
    ex = x.astype(np.float64).sum(**kd).reshape(-1)
    s = ENG.forward(OPS["SUM"], x, axis=axis).reshape(-1)
    assert_sum_close(s, ex.astype(np.float32), ex, "sum", terms_abs=np.abs(x.astype(np.float64)).sum(**kd).reshape(-1))
    d = x.shape[axis] if axis is not None else x.size
    m = ENG.forward(OPS["MEAN"], x, axis=axis).reshape(-1)
    np.testing.assert_array_equal(m, (s / np.float32(d)).astype(np.float32))
    mx = ENG.forward(OPS["MAX"], x, axis=axis).reshape(-1)
    np.testing.assert_array_equal(mx, x.max(**kd).reshape(-1) if axis is not None else [x.max()])


def test_max_of_all_neg_inf_is_min_finite():
    x = np.full((3, 4), -np.inf, np.float32)
    assert ENG.forward(OPS["MAX"], x)[0] == -np.finfo(np.float32).max


# ---------------------------------------------------------------------------------------
# backward
# ---------------------------------------------------------------------------------------
def test_binary_backward_matches_derivatives():
    rng = np.random.default_rng(16)
    a = rng.uniform(-1, 1, (5, 7, 9)).astype(np.float32)
    b = rng.uniform(0.5, 2, (5, 7, 9)).astype(np.float32)
    ug = rng.standard_normal((5, 7, 9)).astype(np.float32)
    A, B, U = (v.astype(np.float64) for v in (a, b, ug))
    d = {(0, 0): U, (0, 1): U, (1, 0): U, (1, 1): -U, (2, 0): U * B, (2, 1): U * A,
         (3, 0): U / B, (3, 1): -A / (B * B) * U}
    for (op, k), ref in d.items():
        g = ENG.backward(k, op, ug, a, b)
        assert ulp_dist(g, ref.astype(np.float32)).max() <= 3, (op, k)
    # exact ones: pure copies and single products
    assert_bitexact(ENG.backward(0, 0, ug, a, b), ug + np.float32(0), "add")
    assert_bitexact(ENG.backward(1, 1, ug, a, b), np.float32(0) + ug * np.float32(-1), "sub id1")
    assert_bitexact(ENG.backward(0, 2, ug, a, b), np.float32(0) + ug * b, "mul id0")


@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_unbroadcast_backward_sums_over_broadcast_axes(op):
    rng = np.random.default_rng(17 + op)
    a = rng.uniform(-1, 1, (6, 5, 4)).astype(np.float32)
    b = rng.uniform(0.5, 2, (1, 5, 1)).astype(np.float32)
    ug = rng.standard_normal((6, 5, 4)).astype(np.float32)
    A, B, U = (v.astype(np.float64) for v in (a, b, ug))
    rg = {0: U, 1: -U, 2: U * A, 3: -A / (B * B) * U}[op]
    ex = rg.sum(axis=(0, 2), keepdims=True)
    g = ENG.backward(1, op, ug, a, b)
    assert_sum_close(g.reshape(-1), ex.reshape(-1).astype(np.float32), ex.reshape(-1), f"op {op}",
                     terms_abs=np.abs(rg).sum(axis=(0, 2)).reshape(-1))


def test_div_backward_scalar_rule():
    # t2 of shape (1): factor = -1 / (s*s), rg = (factor * t1) * ug (basics.mojo:168-180)
    rng = np.random.default_rng(18)
    a = rng.uniform(-1, 1, 64).astype(np.float32)
    s = np.array([1.7], np.float32)
    ug = rng.standard_normal(64).astype(np.float32)
    g = ENG.backward(1, 3, ug, a, s)
    ref = (-a.astype(np.float64) / (1.7 ** 2) * ug).sum()
    assert abs(g[0] - ref) <= 1e-5 * np.abs(a.astype(np.float64) / 1.7 ** 2 * ug).sum()
    g0 = ENG.backward(0, 3, ug, a, s)
    assert_bitexact(g0, np.float32(0) + ug / s[0], "div id0 scalar")


def test_unary_backward_matches_derivatives():
    rng = np.random.default_rng(19)
    x = rng.uniform(0.2, 3, 5000).astype(np.float32)
    ug = rng.standard_normal(5000).astype(np.float32)
    X, U = x.astype(np.float64), ug.astype(np.float64)
    sig = 1 / (1 + np.exp(-X))
    refs = {OPS["EXP"]: np.exp(X) * U, OPS["LOG"]: U / X, OPS["SIGMOID"]: sig * (1 - sig) * U,
            OPS["TANH"]: (1 - np.tanh(X) ** 2) * U, OPS["RELU"]: U}
    for op, ref in refs.items():
        g = ENG.backward(0, op, ug, x)
        # 1 - t*t cancels as t -> 1: TANH is bounded in absolute terms (ulp(1) * |ug| scale)
        slack = 4e-7 * np.abs(U) if op == OPS["TANH"] else 0.0
        assert (np.abs(g - ref) <= 1e-5 * np.abs(ref) + slack + 1e-30).all(), op


def test_pow_backward_derivatives():
    rng = np.random.default_rng(20)
    x = rng.uniform(0.1, 4, 3000).astype(np.float32)
    ug = rng.standard_normal(3000).astype(np.float32)
    a = np.array([1.7], np.float32)
    X, U, Af = x.astype(np.float64), ug.astype(np.float64), np.float64(a[0])
    g0 = ENG.backward(0, O.POW, ug, x, a)
    ref0 = Af * X ** (Af - 1) * U
    assert (np.abs(g0 - ref0) <= 1e-5 * np.abs(ref0) + 1e-30).all()
    g1 = ENG.backward(1, O.POW, ug, x, a)
    terms = X ** Af * np.log(X) * U
    assert abs(g1[0] - terms.sum()) <= 1e-5 * np.abs(terms).sum()


def test_max_backward_tie_rule_bruteforce():
    rng = np.random.default_rng(21)
    x = rng.integers(0, 4, (6, 5, 7)).astype(np.float32)  # many exact ties
    for ax in (0, 1, 2, None):
        ug_shape = (1,) if ax is None else tuple(1 if i == ax else d for i, d in enumerate(x.shape))
        ug = rng.standard_normal(ug_shape).astype(np.float32)
        g = ENG.backward(0, O.MAX, ug, x, axis=ax)
        m = x.max() if ax is None else x.max(axis=ax, keepdims=True)
        eq = x == m
        cnt = eq.sum() if ax is None else eq.sum(axis=ax, keepdims=True)
        f = (np.float32(1) / cnt.astype(np.float32)).astype(np.float32)
        ref = np.where(eq, (f * (ug[0] if ax is None else ug)).astype(np.float32), np.float32(0))
        assert_bitexact(g, np.float32(0) + ref, f"max axis {ax}")


def test_sum_backward_size1_axis_applies_mul_twice():
    # accumulate_op with res_shape == t1_shape applies func twice (tensorutils.mojo:380-393)
    x = np.ones((4, 1, 3), np.float32)
    ug = np.arange(12, dtype=np.float32).reshape(4, 1, 3) - 5
    assert_bitexact(ENG.backward(0, O.SUM, ug, x, axis=1), np.float32(0) + ug * ug, "sum size-1 axis")
    c = np.float32(1.0 / 1.0)
    assert_bitexact(ENG.backward(0, O.MEAN, ug, x, axis=1), np.float32(0) + (c * ug) * ug, "mean size-1 axis")


def test_mean_backward_all_uses_f32_of_f64_reciprocal():
    x = np.ones((3, 7), np.float32)
    ug = np.array([2.5], np.float32)
    g = ENG.backward(0, O.MEAN, ug, x)
    assert_bitexact(g, np.full((3, 7), np.float32(1.0 / 21.0) * np.float32(2.5), np.float32), "mean all")


# ---------------------------------------------------------------------------------------
# Adam.step (mantle/nn/optim.mojo:94-140)
# ---------------------------------------------------------------------------------------
def _adam64(p, g, m, v, it, lr, b1, b2, eps):
    m = b1 * m + (1 - b1) * g
    v = b2 * v + (1 - b2) * g * g
    mh = m / (1 - b1 ** it)
    vh = v / (1 - b2 ** it)
    return p - lr * mh / (np.sqrt(vh) + eps), m, v


def test_adam_matches_fp64_over_steps():
    rng = np.random.default_rng(5)
    n = 4096
    p = rng.standard_normal(n).astype(np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    P, M, V = (a.astype(np.float64) for a in (p, m, v))
    lr, b1, b2, eps = 0.01, 0.9, 0.999, 1e-8
    for it in range(1, 8):
        g = rng.standard_normal(n).astype(np.float32) * np.float32(0.1)
        p, m, v = O.adam_step(p, g, m, v, it, lr, b1, b2, eps)
        # fp64 on the same f32 hyper-parameters
        P, M, V = _adam64(P, g.astype(np.float64), M, V, it, float(np.float32(lr)), float(np.float32(b1)),
                          float(np.float32(b2)), float(np.float32(eps)))
        # m can cancel towards 0: the bound is relative to the gradient's scale there
        np.testing.assert_allclose(m, M, rtol=2e-6, atol=1e-7 * float(np.abs(g).max()))
        np.testing.assert_allclose(v, V, rtol=2e-6, atol=1e-12)
        # the update is lr-sized: its error stays a tiny fraction of lr
        assert np.abs(p.astype(np.float64) - P).max() <= 1e-6 * np.abs(P).max() + 1e-4 * lr


def test_adam_zero_gradient_leaves_state_unchanged():
    p = np.linspace(-3, 3, 1001).astype(np.float32)
    z = np.zeros_like(p)
    for it in (1, 2, 10):
        p2, m2, v2 = O.adam_step(p, z, z, z, it, 0.1)
        assert np.array_equal(p2, p) and not m2.any() and not v2.any()


def test_adam_first_step_moves_by_lr_times_sign():
    """From m = v = 0 the first step is p - lr * g / (|g| + eps) up to rounding."""
    g = np.array([0.5, -0.25, 3.0, -1e-3, 1e-6], np.float32)
    p = np.ones_like(g)
    z = np.zeros_like(g)
    lr, eps = 0.01, 1e-8
    p2, m2, v2 = O.adam_step(p, g, z, z, 1, lr, 0.9, 0.999, eps)
    exp = 1.0 - lr * g.astype(np.float64) / (np.abs(g.astype(np.float64)) + eps)
    np.testing.assert_allclose(p2, exp, rtol=1e-6)
    c1 = np.float32(np.float32(1.0) - np.float32(0.9))
    np.testing.assert_array_equal(m2, c1 * g)  # beta1 * 0 + (1 - beta1) * g, in f32


def test_adam_bias_correction_uses_square_and_multiply_power():
    """beta ** iter is Mojo's SIMD ** Int: 1 - powi(beta, iter) in f32, with powi pinned as
    square-and-multiply above; at iter = 3 the correction is 1 - beta * (beta * beta)."""
    b1 = np.float32(0.9)
    g = np.array([1.0], np.float32)
    z = np.zeros(1, np.float32)
    m3 = np.array([0.3], np.float32)
    p2, m2, _ = O.adam_step(np.zeros(1, np.float32), g, m3, np.ones(1, np.float32), 3, 1.0, 0.9, 0.999, 0.0)
    mj = np.float32(b1 * m3[0]) + np.float32(np.float32(1) - b1) * g[0]
    assert m2[0] == np.float32(mj)
    bc = np.float32(1) - np.float32(b1 * np.float32(b1 * b1))
    assert O.lib().or_powi(b1, 3) == np.float32(b1 * np.float32(b1 * b1))
    del p2, bc, z


# ---------------------------------------------------------------------------------------
# FMA, LEAKYRELU, CLIP (basics.mojo:759-817, mlops.mojo:128-186, 238-299)
# ---------------------------------------------------------------------------------------
def test_fma_is_one_rounding():
    rng = np.random.default_rng(40)
    a, b, c = (rng.standard_normal(100000).astype(np.float32) for _ in range(3))
    got = O.fma_fwd(a, b, c)
    # a*b is exact in fp64 (48 significant bits); one fp64 add then the f32 rounding agrees
    # with the exact single rounding except at an f32 tie after the fp64 rounding (~2^-29)
    ref = (a.astype(np.float64) * b + c).astype(np.float32)
    assert_bitexact(got, ref, "fma vs fp64")
    unfused = (a * b) + c
    assert (got != unfused).sum() > 100  # a two-rounding product-then-add would match this
    assert_bitexact(O.fma_fwd(a, b, np.zeros_like(c)), a * b, "fma(a, b, 0) = a*b")
    ug, g0 = rng.standard_normal(1000).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    assert_bitexact(O.fma_bwd_accum(0, g0, ug, a[:1000], b[:1000]), g0 + ug * b[:1000], "fma bwd 0")
    assert_bitexact(O.fma_bwd_accum(1, g0, ug, a[:1000], b[:1000]), g0 + ug * a[:1000], "fma bwd 1")
    assert_bitexact(O.fma_bwd_accum(2, g0, ug, a[:1000], b[:1000]), g0 + ug, "fma bwd 2")


def test_leakyrelu_identities_and_derivative():
    rng = np.random.default_rng(41)
    x = (rng.standard_normal(20000) * 4).astype(np.float32)
    assert_bitexact(O.leakyrelu_fwd(x, 1.0), x, "slope 1 is the identity")
    for slope in (0.1, 0.01, -0.5, 3.0):
        y = O.leakyrelu_fwd(x, slope)
        assert_bitexact(O.leakyrelu_fwd(x * 4, slope), y * 4, "positive homogeneity (x4 exact)")
        assert_bitexact(y[x > 0], x[x > 0], "identity on positives")
        # backward = d fwd / dx, from fp64 central differences away from the kink
        h = 1e-3
        sel = np.abs(x) > 1e-2
        xd = x[sel].astype(np.float64)
        yd = np.where(xd > 0, xd, xd * np.float64(np.float32(slope)))
        deriv = (np.where(xd + h > 0, xd + h, (xd + h) * np.float64(np.float32(slope)))
                 - np.where(xd - h > 0, xd - h, (xd - h) * np.float64(np.float32(slope)))) / (2 * h)
        assert np.allclose(y[sel], yd, rtol=1e-6)
        ug = np.ones(sel.sum(), np.float32)
        gb = O.leakyrelu_bwd_accum(np.zeros_like(ug), x[sel], ug, slope)
        np.testing.assert_allclose(gb, deriv, rtol=1e-6)


def test_clip_against_numpy_and_special_values():
    rng = np.random.default_rng(42)
    x = (rng.standard_normal(20000) * 3).astype(np.float32)
    for lo, hi in [(-1.1, 1.1), (-O.FLT_MAX, O.FLT_MAX), (0.0, 2.5), (-0.5, -0.5)]:
        lo32, hi32 = np.float32(lo), np.float32(hi)
        y = O.clip_fwd(x, lo, hi)
        assert_bitexact(y, np.clip(x, lo32, hi32), f"clip [{lo}, {hi}]")
        assert_bitexact(O.clip_fwd(y, lo, hi), y, "idempotent")
        ug = rng.standard_normal(x.size).astype(np.float32)
        inside = np.clip(x, lo32, hi32) == x
        assert_bitexact(O.clip_bwd_accum(np.zeros_like(x), x, ug, lo, hi), np.where(inside, ug, 0) + 0.0, "clip bwd")
    sp = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, O.FLT_MAX, -O.FLT_MAX], np.float32)
    y = O.clip_fwd(sp)  # absent attributes: min_finite / max_finite
    assert_bitexact(y[1:], np.array([O.FLT_MAX, -O.FLT_MAX, 0.0, -0.0, O.FLT_MAX, -O.FLT_MAX], np.float32), "default")
    assert y[0] == np.float32(O.FLT_MAX)  # minnum(NaN, hi) = hi
    g = O.clip_bwd_accum(np.zeros(7, np.float32), sp, np.ones(7, np.float32))
    assert_bitexact(g, np.array([0, 0, 0, 1, 1, 1, 1], np.float32), "default bwd: inf and NaN outside")


# ---------------------------------------------------------------------------------------
# tstd (tensorutils.mojo:724-741, 776-840)
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("nelts", [8, 32])
def test_tstd_against_fp64(nelts):
    O.set_nelts(nelts)
    rng = np.random.default_rng(43)
    for shape in [(5,), (100,), (2, 10), (37, 63), (7, 40, 3), (3, 4, 5), (1, 70), (70, 1), (4, 1, 9)]:
        x = (rng.standard_normal(shape) * 2 + 1).astype(np.float32)
        ref = np.array([x.astype(np.float64).std()])
        assert_sum_close(O.tstd(x), ref, ref, f"all {shape}")
        for ax in range(len(shape)):
            got = O.tstd(x, ax)
            ref = x.astype(np.float64).std(axis=ax, keepdims=True)
            np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7, err_msg=f"{shape} axis {ax}")


def test_tstd_lines_are_tmean_lines():
    """Each output is the spread of its own line: lines of distinct spreads, so reading any
    other line (the reference's `i % shape[k]` addressing) would fail here."""
    a = np.arange(1, 9, dtype=np.float32)
    x = np.stack([np.array([-s, s], np.float32) * 1 for s in a]).reshape(2, 4, 2)  # line (i, j) = +/- a
    got = O.tstd(x, 2).reshape(-1)
    np.testing.assert_array_equal(got, a)
    y = np.transpose(x, (2, 0, 1)).copy()  # the same lines along axis 0
    np.testing.assert_array_equal(O.tstd(y, 0).reshape(-1), a)


@pytest.mark.parametrize("shape,axis", [((64, 37), 0), ((37, 64), 1), ((5, 7, 33), 1), ((3, 1), 0), ((1000, 3), 0)])
@pytest.mark.parametrize("nthreads", [1, 3, 8])
def test_threaded_axis_reduce_is_identical(shape, axis, nthreads):
    """The CPU baseline's threaded axis reduce (outputs split over a pool, tensorutils.mojo:682)
    gives the serial restatement's bits: every output is computed the same way."""
    x = np.random.default_rng(13).standard_normal(shape).astype(np.float32)
    for op in (O.SUM, O.MEAN, O.MAX):
        assert_bitexact(O.reduce_axis_mt(op, x, axis, nthreads), O.forward_op(op, x, axis=axis), f"op {op}")


# ---------------------------------------------------------------------------------------
# row graphs: the summation order's effect, bounded by the fp64 magnitude comparator
# ---------------------------------------------------------------------------------------
ROW_ORDER_SHAPES = [(513, 17), (300, 24), (1000, 31), (40, 33), (777, 47), (1200, 64), (500, 32)]


def _row_graph_cases(rows, k):
    """(name, nodes, output, inputs, seed) of Softmax, LogSoftmax (activations.mojo:74-108) and
    CrossEntropyLoss (loss.mojo:45-61) over [rows, k], ties injected, soft targets."""
    from mantle_amd import synth
    x = synth.normal((rows, k), 0, 2, 1300)
    synth.inject_ties(x, 1, 1301)
    gout = synth.normal((rows, k), 0, 1, 1303)
    target = synth.uniform((rows, k), 0, 1, 1304)
    cn = np.array([np.float32(-1.0 / rows)], np.float32)
    return [("softmax", softmax_nodes("x", 1), "sm", {"x": x}, gout),
            ("logsoftmax", logsoftmax_nodes("x", 1), "lsm", {"x": x}, gout),
            ("cross_entropy", cross_entropy_nodes("x", "target"), "loss", {"x": x, "target": target, "cN": cn},
             np.array([0.7], np.float32))]


def _run_graph(eng, nodes, inputs, seed, g0, out):
    g = Graph(nodes, ["x"])
    v = g.forward(eng, inputs)
    return v[out], g.backward(eng, v, seed=seed, init={"x": g0})["x"]


@pytest.mark.parametrize("rows,k", ROW_ORDER_SHAPES, ids=[f"{r}x{c}" for r, c in ROW_ORDER_SHAPES])
def test_row_graph_summation_orders_meet_in_the_sum_class(rows, k):
    """The oracle's row graphs at nelts 1 (every row sum in element order, the order of the
    GPU's row engines up to 64 classes) and at nelts 32 (the reference's AVX-512 lane order):
    bit-identical below 32 classes, where both orders are the element order; from 32 classes
    every output and gradient element meets the fp64 comparator (assert_order_close: no farther
    from fp64 than the other order plus 2 ulp, or within 1e-5 of its first-order magnitude).
    A result whose row sums drop one term must fail the same comparator."""
    from mantle_amd import synth
    g0 = synth.normal((rows, k), 0, 1, 1302)
    f64 = Mag64Engine()
    for name, nodes, out, inputs, seed in _row_graph_cases(rows, k):
        O.set_nelts(1)
        o1 = _run_graph(ENG, nodes, inputs, seed, g0, out)
        O.set_nelts(32)
        o32 = _run_graph(ENG, nodes, inputs, seed, g0, out)
        ex = _run_graph(f64, nodes, inputs, seed, g0, out)
        for got, ref, e, what in zip(o1, o32, ex, ("forward", "backward")):
            if k < 32 and not (name == "cross_entropy" and what == "forward"):
                assert_bitexact(got, ref, f"{name} {what}: element order below 32 lanes")
            assert_order_close(got, ref, e, f"{name} {what}")
    # negative control: a Softmax whose row sums miss their last term is far outside the class
    x = _row_graph_cases(rows, k)[0][3]["x"]
    O.set_nelts(32)
    v = Graph(softmax_nodes("x", 1), ["x"]).forward(ENG, {"x": x})
    short = O.forward_op(O.DIV, v["e"], v["s"] - v["e"][:, -1:])
    with pytest.raises(AssertionError):
        assert_order_close(short, v["sm"], Graph(softmax_nodes("x", 1), ["x"]).forward(f64, {"x": x})["sm"],
                           "softmax with a dropped term")
