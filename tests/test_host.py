"""Host-side checks that need no GPU: the C-ABI library loads and exports every symbol the
header declares, argument validation rejects bad calls before any device work, and the
launch planning (dim collapsing, un-broadcast reduction chains) is right."""
import ctypes
import os
import re

import numpy as np
import pytest

from util import ROOT

import mantle_amd
from mantle_amd import _lib

HEADER = os.path.join(ROOT, "include", "mantle_hip.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(mh_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    names = header_functions()
    assert len(names) >= 30
    L = _lib.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes binding covers the whole header
    assert sorted(_lib.SIGNATURES) == names


def test_status_strings():
    L = _lib.lib()
    for code in range(-9, 1):
        assert L.mh_status_string(code)
    assert L.mh_status_string(-2) == b"shape mismatch"


S = _lib.make_shape


def test_noalloc_reduce_refuses_oversized_partials_on_the_host():
    """mh_reduce_fwd_noalloc checks its partials against the fixed 16 MiB scratch before
    anything else (no device needed): an all-element SUM of 2^34 elements needs 32 MiB."""
    L = _lib.lib()
    assert L.mh_reduce_fwd_noalloc(8, None, None, S((1 << 34,)), -1) == _lib.ERR_OVERFLOW
    assert b"no-allocation scratch" in L.mh_last_error()
    # within the scratch, the call goes on to the usual checks (null tensors here)
    assert L.mh_reduce_fwd_noalloc(8, None, None, S((8192, 8192)), 0) == _lib.ERR_NULL


def test_shape_errors_before_device_work():
    L = _lib.lib()
    # non-broadcastable (the reference only prints, tensorutils.mojo:116-122)
    assert L.mh_binary_fwd(0, None, S((3,)), None, S((4,)), None, S((3,))) == _lib.ERR_SHAPE
    assert b"broadcast" in L.mh_last_error()
    # result shape must be broadcast(a, b)
    assert L.mh_binary_fwd(0, None, S((2, 3)), None, S((3,)), None, S((3,))) == _lib.ERR_SHAPE
    # rank outside 1..8 and negative dims
    bad = _lib.mh_shape()
    bad.rank = 0
    assert L.mh_binary_fwd(0, None, bad, None, S((1,)), None, S((1,))) == _lib.ERR_RANK
    bad.rank = 9
    assert L.mh_binary_fwd(0, None, bad, None, S((1,)), None, S((1,))) == _lib.ERR_RANK
    assert L.mh_binary_fwd(0, None, S((2, -1)), None, S((2, -1)), None, S((2, -1))) == _lib.ERR_RANK
    # op ids outside the entry point
    assert L.mh_binary_fwd(4, None, S((1,)), None, S((1,)), None, S((1,))) == _lib.ERR_OP
    assert L.mh_unary_fwd(0, None, None, 4) == _lib.ERR_OP
    assert L.mh_reduce_fwd(0, None, None, S((2, 3)), -1) == _lib.ERR_OP
    # axis outside [-1, rank)
    assert L.mh_reduce_fwd(8, None, None, S((2, 3)), 2) == _lib.ERR_INVALID
    # tensor_id
    assert L.mh_binary_bwd_accum(0, 2, None, S((1,)), None, S((1,)), None, S((1,)), None, S((1,))) == _lib.ERR_INVALID
    # grad shape must be the operand's
    assert L.mh_binary_bwd_accum(0, 0, None, S((3,)), None, S((2, 3)), None, S((2, 3)), None, S((3,))) == _lib.ERR_SHAPE
    # the reference's non-numpy accumulate pair (test_tensorutils.mojo:409-414) is rejected
    assert L.mh_accumulate_grad(None, S((2, 1)), None, S((2, 3, 4))) == _lib.ERR_SHAPE
    # null tensors on non-empty work
    assert L.mh_binary_fwd(0, None, S((3,)), None, S((3,)), None, S((3,))) == _lib.ERR_NULL
    assert L.mh_unary_fwd(4, None, None, 5) == _lib.ERR_NULL
    # shapes cross the ABI by pointer: a null shape pointer is an error, not a crash
    assert L.mh_binary_fwd(0, None, None, None, S((3,)), None, S((3,))) == _lib.ERR_NULL
    assert b"null shape" in L.mh_last_error()
    assert L.mh_reduce_fwd(8, None, None, None, -1) == _lib.ERR_NULL
    assert L.mh_accumulate_grad(None, S((3,)), None, None) == _lib.ERR_NULL
    # empty work is a no-op
    assert L.mh_binary_fwd(0, None, S((0, 3)), None, S((0, 3)), None, S((1,))) == _lib.OK
    assert L.mh_unary_fwd(4, None, None, 0) == _lib.OK


def test_requires_init_or_reports_no_device():
    L = _lib.lib()
    n = ctypes.c_int(-1)
    assert L.mh_device_count(ctypes.byref(n)) == _lib.OK
    if n.value == 0:
        assert L.mh_init(0, 0) == _lib.ERR_NO_DEVICE
        p = ctypes.c_void_p(16)
        assert L.mh_unary_fwd(4, p, p, 4) == _lib.ERR_NOT_INIT
        assert L.mh_malloc(ctypes.byref(ctypes.c_void_p()), 16) == _lib.ERR_NOT_INIT
        with pytest.raises(mantle_amd.MantleHipError):
            mantle_amd.init(0)


def plan(sres, sa, sb):
    info = _lib.mh_plan_info()
    _lib.check(_lib.lib().mh_plan_binary(S(sres), S(sa), S(sb), ctypes.byref(info)))
    r = info.rank
    return info.kind, list(info.dims)[:r], list(info.stride_a)[:r], list(info.stride_b)[:r]


def test_plan_binary_collapses_dims():
    # config 1: Linear bias [32,32] + [1,32]
    assert plan((32, 32), (32, 32), (1, 32)) == (3, [32, 32], [32, 1], [0, 1])
    # config 3: NCHW bias: [256,32,28,28] + [1,32,1,1] -> [256, 32, 784]
    assert plan((256, 32, 28, 28), (256, 32, 28, 28), (1, 32, 1, 1)) == \
        (3, [256, 32, 784], [25088, 784, 1], [0, 1, 0])
    # config 5: [N,10] - [N,1]
    assert plan((1048576, 10), (1048576, 10), (1048576, 1)) == (3, [1048576, 10], [10, 1], [1, 0])
    # same shape collapses to one dim; graph scalars on either side
    assert plan((4, 5, 6), (4, 5, 6), (4, 5, 6)) == (0, [120], [1], [1])
    assert plan((4, 5, 6), (4, 5, 6), (1,)) == (1, [120], [1], [0])
    assert plan((4, 5, 6), (1,), (4, 5, 6)) == (2, [120], [0], [1])
    # the reference's broadcast fixture [2,3,4] + [5,2,1,4] (test_tensorutils.mojo:161-181)
    k, dims, sa, sb = plan((5, 2, 3, 4), (2, 3, 4), (5, 2, 1, 4))
    assert k == 3 and dims == [5, 2, 3, 4] and sa == [0, 12, 4, 1] and sb == [8, 4, 0, 1]


def unb(sg, srg):
    info = _lib.mh_reduce_plan_info()
    _lib.check(_lib.lib().mh_plan_unbroadcast(S(sg), S(srg), ctypes.byref(info)))
    return [(info.a[i], info.b[i], info.c[i]) for i in range(info.nsteps)]


def test_plan_unbroadcast_chains():
    assert unb((1, 32), (32, 32)) == [(1, 32, 32)]                       # config 1 bias grad
    assert unb((1, 32, 1, 1), (256, 32, 28, 28)) == [(8192, 784, 1), (1, 256, 32)]  # config 3
    assert unb((1048576, 1), (1048576, 10)) == [(1048576, 10, 1)]        # config 5 row sums
    assert unb((1,), (6, 7)) == [(1, 42, 1)]                              # everything
    assert unb((32,), (1, 32)) == []                                      # only unit dims differ
    assert unb((3, 1, 5, 1), (3, 4, 5, 6)) == [(60, 6, 1), (3, 4, 5)]     # K R K R
    with pytest.raises(_lib.MantleHipError):
        unb((2, 1), (2, 3, 4))


def test_python_mirror_broadcast_and_result_shapes():
    from mantle_amd.ops import broadcast_shapes, static_result_shape, OP
    rng = np.random.default_rng(3)
    for _ in range(300):
        r = int(rng.integers(1, 5))
        a = tuple(int(x) for x in rng.integers(1, 4, r))
        b = tuple(d if rng.random() < 0.5 else 1 for d in a)[int(rng.integers(0, r)):] or (1,)
        assert broadcast_shapes(a, b).dims == np.broadcast_shapes(a, b)
    assert static_result_shape(OP.SUM, (4, 5, 6), attributes={"axis": 1}).dims == (4, 1, 6)
    assert static_result_shape(OP.MAX, (4, 5, 6)).dims == (1,)
    assert static_result_shape(OP.POW, (4, 5), (1,)).dims == (4, 5)
    with pytest.raises(mantle_amd.MantleHipError):
        broadcast_shapes((3,), (4,))


# ---------------------------------------------------------------------------------------
# graph builder (host-only: mh_graph_*)
# ---------------------------------------------------------------------------------------
def test_graph_builder_shapes_and_trainable():
    import mantle_amd as m
    g = m.Graph()
    x = g.input((32, 32))
    b = g.param((1, 32), init=np.zeros(32, np.float32))
    y = g.op(m.OP.ADD, x, b)
    assert (y.shape.dims, y.trainable) == ((32, 32), True)  # trainable if any operand is
    z = g.op(m.OP.EXP, x)
    assert not z.trainable
    s0 = g.op(m.OP.SUM, y, attributes={"axis": 0})
    assert s0.shape.dims == (1, 32)
    sa = g.op(m.OP.MEAN, y)
    assert sa.shape.dims == (1,)
    p = g.op(m.OP.POW, y, 2.0)  # a float operand becomes a graph scalar
    assert p.shape.dims == (32, 32) and g.params[-1].shape.dims == (1,) and not g.params[-1].trainable
    f = g.op(m.OP.FMA, y, y, x)
    c = g.op(m.OP.CLIP, f, attributes={"min": -1.0})
    lr = g.op(m.OP.LEAKYRELU, c, attributes={"negative_slope": 0.1})
    assert lr.shape.dims == (32, 32)
    assert [s.name for s in g.symbols] == list(range(len(g.symbols)))
    assert g.trainable_parameters() == [b]


@pytest.mark.parametrize("build", [
    lambda m, g, x: g.op(m.OP.ADD, x, g.input((4,))),                   # not broadcastable
    lambda m, g, x: g.op(m.OP.POW, x, x),                               # exponent not shape (1)
    lambda m, g, x: g.op(m.OP.LEAKYRELU, x),                            # negative_slope missing
    lambda m, g, x: g.op(m.OP.FMA, x, x, g.input((4,))),                # FMA shapes differ
    lambda m, g, x: g.op(m.OP.SUM, x, attributes={"axis": 2}),          # axis out of range
    lambda m, g, x: g.op(7, x, x),                                      # DOT: not on this path
    lambda m, g, x: g.op(m.OP.EXP, x, x),                               # arity
    lambda m, g, x: g.param((2, 2), init=[1.0, 2.0]),                   # init size
    lambda m, g, x: g.op(m.OP.SUM, x, attributes={"dim": 0}),           # unknown attribute
])
def test_graph_builder_rejects(build):
    import mantle_amd as m
    g = m.Graph()
    x = g.input((5, 3))
    with pytest.raises(m.MantleHipError):
        build(m, g, x)


class _HostTensor:
    """A shape-only stand-in for mantle_amd.Tensor (no device memory): enough for the fused-row
    wrappers' checks, which run before anything reaches the library."""

    def __init__(self, *dims):
        self._s = mantle_amd.TensorShape(*dims)
        self.ptr = None

    def shape(self):
        return self._s

    def num_elements(self):
        return self._s.num_elements()

    def rank(self):
        return self._s.rank()


FUSED_ROW_CALLS = [
    ("softmax_forward", ("out", "x")),
    ("softmax_backward", ("grad_x", "x", "grad_out")),
    ("logsoftmax_forward", ("out", "x")),
    ("logsoftmax_backward", ("grad_x", "x", "grad_out")),
    ("cross_entropy_forward", ("loss", "x", "target")),
    ("cross_entropy_backward", ("grad_x", "x", "target", "ug")),
    ("softmax_log_mul_mean_forward", ("loss", "x", "target")),
    ("softmax_log_mul_mean_backward", ("grad_x", "x", "target", "ug")),
]


@pytest.mark.parametrize("fn,args", FUSED_ROW_CALLS, ids=[c[0] for c in FUSED_ROW_CALLS])
def test_fused_row_wrappers_check_shapes_before_any_launch(monkeypatch, fn, args):
    """The fused row entry points take bare pointers and (rows, classes) from x: every other
    tensor must be x's shape (or hold one element: a loss or its gradient), else the binding
    raises MH_ERR_SHAPE before the library is called."""
    calls = []
    monkeypatch.setattr(_lib, "call", lambda name, *a: calls.append((name, a[-2:])))
    f = getattr(mantle_amd.ops, fn)
    x = (37, 33)

    def make(bad=None, how=None):
        out = []
        for a in args:
            scalar = a in ("loss", "ug")
            dims = (1,) if scalar else x
            if a == bad:
                dims = (2,) if scalar else (how or (36, 33))
            out.append(_HostTensor(*dims))
        return out

    f(*make())
    assert calls and calls[-1][1] == (37, 33)
    for a in args:
        if a == "x":
            continue
        for how in ((36, 33), (37, 32), (37 * 33,)):
            with pytest.raises(_lib.MantleHipError) as e:
                f(*make(a, how))
            assert e.value.code == _lib.ERR_SHAPE and a in str(e.value)
    assert len(calls) == 1  # no mismatched call reached the library


@pytest.mark.parametrize("what", range(6))
def test_launch_grids_fit_one_dispatch(what):
    """Every element-streaming launch stays below the 2^32 work-items of one dispatch, up to
    tensors of 2^40 elements (no 64 GiB device run needed to see it), and covers the tensor in
    one pass wherever that fits (the kernels loop over the grid beyond)."""
    L = _lib.lib()
    info = _lib.mh_launch_info()
    per_thread = {_lib.LAUNCH_FILL_UNALIGNED: 1}.get(what, 4)
    for n in (1, 1000, 1 << 28, (1 << 33) - 4, 1 << 33, (1 << 33) + 8, (1 << 34) - 4, 1 << 34, (1 << 34) + 5,
              1 << 36, 1 << 40):
        assert L.mh_plan_launch(what, n, ctypes.byref(info)) == 0, L.mh_last_error()
        items = info.blocks * info.threads
        assert 1 <= info.blocks and items < (1 << 32), (what, n, info.blocks, info.threads)
        assert info.launches >= 1
        need = (n + per_thread - 1) // per_thread
        if what in (_lib.LAUNCH_FILL, _lib.LAUNCH_COPY, _lib.LAUNCH_SAME_SHAPE):
            # a thread per quad with no grid loop: at most 2^31 quads per launch, the launches
            # together covering the tensor
            nq = n // 4
            assert info.launches == max(1, -(-nq // (1 << 31))), (what, n, info.launches)
            assert items >= min(nq, 1 << 31) and items * info.launches >= nq, (what, n, items)
        elif need < (1 << 32) - info.threads:
            assert items >= need, (what, n, items, need)  # one pass covers the tensor
        if what == _lib.LAUNCH_ADAM:
            # k_adam_al has no stride loop: it takes only tensors whose quads and tail its grid covers
            fits = (n >> 2) + 1 <= ((1 << 32) - 1) // info.threads * info.threads
            assert info.kernel == (0 if fits else 1), (n, info.kernel)
            if info.kernel == 0:
                assert items >= (n >> 2) + 1
        elif what == _lib.LAUNCH_ADAM_UNALIGNED:
            assert info.kernel == 1
    assert L.mh_plan_launch(7, 10, ctypes.byref(info)) == _lib.ERR_INVALID


def test_row_engine_launches_split_rows_past_one_dispatch():
    """The row-fused one-shot kernels (64-row workgroups of one wavefront) stay below the 2^32
    work-items of one dispatch and cover every row, in consecutive launches whose row runs
    start at multiples of 64 rows (so each launch's operands stay 16-byte aligned), up to
    2^40 rows; zero rows make no launch."""
    L = _lib.lib()
    info = _lib.mh_launch_info()
    assert L.mh_plan_launch(_lib.LAUNCH_ROWS16, 0, ctypes.byref(info)) == 0
    assert info.launches == 0
    for rows in (1, 63, 64, 65, 1 << 20, (1 << 32) - 64, (1 << 32) - 1, 1 << 32, (1 << 32) + 1, 1 << 36, 1 << 40):
        assert L.mh_plan_launch(_lib.LAUNCH_ROWS16, rows, ctypes.byref(info)) == 0, L.mh_last_error()
        assert info.threads == 64 and 1 <= info.blocks and info.blocks * 64 < (1 << 32), (rows, info.blocks)
        nb = -(-rows // 64)
        assert info.launches == -(-nb // info.blocks), (rows, info.launches)
        assert info.blocks == min(nb, ((1 << 32) - 1) // 64), (rows, info.blocks)
        assert info.blocks * 64 * info.launches >= rows > info.blocks * 64 * (info.launches - 1), rows
    assert L.mh_plan_launch(0, -1, ctypes.byref(info)) == _lib.ERR_INVALID
