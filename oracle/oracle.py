"""ctypes view of the CPU restatement in oracle/liboracle.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()`` and by the
``cpu_baseline`` leg of ``bench.py``, always as the checker (or the timed CPU baseline),
never as the product path. The library is built by ``make -C oracle``.

Each wrapper mirrors one reference function; the C side cites the reference file:line.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# MANTLE_ORACLE_LIB: another build of the same source (the sanitizer build, oracle/_san/)
_LIB_PATH = os.environ.get("MANTLE_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")

# Mantle OP ids (mantle/autograd/ops/ops.mojo:57-83).
ADD, SUB, MUL, DIV, EXP, LOG, POW = 0, 1, 2, 3, 4, 5, 6
SUM, MEAN, MAX = 8, 9, 10
SIGMOID, RELU, TANH = 13, 14, 15
FMA, CLIP, LEAKYRELU = 19, 20, 28

FLT_MAX = float(np.finfo(np.float32).max)
MAX_RANK = 8


class Shape(ctypes.Structure):
    _fields_ = [("rank", ctypes.c_int32), ("dims", ctypes.c_int64 * MAX_RANK)]


def make_shape(dims) -> Shape:
    dims = tuple(int(d) for d in dims)
    s = Shape()
    s.rank = len(dims)
    for i, d in enumerate(dims[:MAX_RANK]):
        s.dims[i] = d
    return s


class OracleError(RuntimeError):
    pass


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise OracleError(f"{_LIB_PATH} is missing: run `make -C oracle`")
        L = ctypes.CDLL(_LIB_PATH)
        f32p = ctypes.POINTER(ctypes.c_float)
        shp = ctypes.POINTER(Shape)
        i64 = ctypes.c_int64
        for name, res, args in [
            ("or_set_nelts", None, [ctypes.c_int]),
            ("or_get_nelts", ctypes.c_int, []),
            ("or_exp", ctypes.c_float, [ctypes.c_float]),
            ("or_log", ctypes.c_float, [ctypes.c_float]),
            ("or_powi", ctypes.c_float, [ctypes.c_float, i64]),
            ("or_powf", ctypes.c_float, [ctypes.c_float, ctypes.c_float]),
            ("or_sigmoid", ctypes.c_float, [ctypes.c_float]),
            ("or_tanh", ctypes.c_float, [ctypes.c_float]),
            ("or_relu", ctypes.c_float, [ctypes.c_float]),
            ("or_fill", None, [f32p, i64, ctypes.c_float]),
            ("or_broadcast_shapes", ctypes.c_int, [shp, shp, shp]),
            ("or_broadcast_calculate_strides", None, [ctypes.c_int, shp, ctypes.POINTER(i64)]),
            ("or_get_real_index", i64, [ctypes.c_int, ctypes.POINTER(i64), shp, i64]),
            ("or_elwise_transform", ctypes.c_int, [ctypes.c_int, f32p, f32p, i64]),
            ("or_elwise_pow", None, [f32p, f32p, i64, i64]),
            ("or_elwise_op", ctypes.c_int, [ctypes.c_int, f32p, f32p, shp, f32p, shp]),
            ("or_accumulate_grad", ctypes.c_int, [f32p, shp, f32p, shp]),
            ("or_reduce_all", ctypes.c_float, [ctypes.c_int, f32p, i64]),
            ("or_reduce_axis", ctypes.c_int, [ctypes.c_int, f32p, f32p, shp, ctypes.c_int]),
            ("or_reduce_axis_mt", ctypes.c_int, [ctypes.c_int, f32p, f32p, shp, ctypes.c_int, ctypes.c_int]),
            ("or_forward_op", ctypes.c_int,
             [ctypes.c_int, f32p, f32p, shp, f32p, shp, ctypes.c_int]),
            ("or_backward_op", ctypes.c_int,
             [ctypes.c_int, ctypes.c_int, f32p, shp, f32p, shp, f32p, shp, ctypes.c_int, f32p]),
            ("or_adam_step", None, [f32p, f32p, f32p, f32p, i64, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                    ctypes.c_float, i64]),
            ("or_fma_fwd", None, [f32p, f32p, f32p, f32p, i64]),
            ("or_fma_bwd_accum", ctypes.c_int, [ctypes.c_int, f32p, f32p, f32p, f32p, i64]),
            ("or_leakyrelu_fwd", None, [f32p, f32p, i64, ctypes.c_float]),
            ("or_leakyrelu_bwd_accum", None, [f32p, f32p, f32p, i64, ctypes.c_float]),
            ("or_clip_fwd", None, [f32p, f32p, i64, ctypes.c_float, ctypes.c_float]),
            ("or_clip_bwd_accum", None, [f32p, f32p, f32p, i64, ctypes.c_float, ctypes.c_float]),
            ("or_tstd_all", ctypes.c_float, [f32p, i64]),
            ("or_tstd_axis", ctypes.c_int, [f32p, f32p, shp, ctypes.c_int]),
        ]:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _check(rc: int, what: str):
    if rc != 0:
        raise OracleError(f"{what} failed with code {rc}")


def set_nelts(n: int):
    lib().or_set_nelts(int(n))


def get_nelts() -> int:
    return lib().or_get_nelts()


# ---- scalar math, vectorised over numpy arrays by a python loop (small inputs only) ----
def exp_scalar(x: float) -> np.float32:
    return np.float32(lib().or_exp(float(np.float32(x))))


def log_scalar(x: float) -> np.float32:
    return np.float32(lib().or_log(float(np.float32(x))))


def powf_scalar(x: float, y: float) -> np.float32:
    return np.float32(lib().or_powf(float(np.float32(x)), float(np.float32(y))))


def broadcast_shapes(s1, s2):
    out = Shape()
    rc = lib().or_broadcast_shapes(make_shape(s1), make_shape(s2), out)
    if rc != 0:
        return None
    return tuple(out.dims[i] for i in range(out.rank))


def broadcast_calculate_strides(size: int, shape):
    st = (ctypes.c_int64 * MAX_RANK)()
    lib().or_broadcast_calculate_strides(size, make_shape(shape), st)
    return tuple(st[i] for i in range(size))


def get_real_index(strides, bshape, i: int) -> int:
    st = (ctypes.c_int64 * MAX_RANK)(*strides)
    return lib().or_get_real_index(len(bshape), st, make_shape(bshape), int(i))


def elwise_transform(op: int, x) -> np.ndarray:
    x = _f32(x)
    res = np.empty_like(x)
    _check(lib().or_elwise_transform(op, _ptr(res), _ptr(x), x.size), "elwise_transform")
    return res


def elwise_pow(x, n: int) -> np.ndarray:
    x = _f32(x)
    res = np.empty_like(x)
    lib().or_elwise_pow(_ptr(res), _ptr(x), x.size, int(n))
    return res


def elwise_op(op: int, a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    rs = broadcast_shapes(a.shape or (1,), b.shape or (1,))
    if rs is None:
        raise OracleError("shapes do not broadcast")
    res = np.zeros(rs, dtype=np.float32)
    _check(lib().or_elwise_op(op, _ptr(res), _ptr(a), make_shape(a.shape or (1,)),
                              _ptr(b), make_shape(b.shape or (1,))), "elwise_op")
    return res


def accumulate_grad(grad, rg) -> np.ndarray:
    """Returns grad + un-broadcast(rg); grad is copied, not modified."""
    g = _f32(grad).copy()
    rg = _f32(rg)
    rc = lib().or_accumulate_grad(_ptr(g), make_shape(g.shape or (1,)), _ptr(rg),
                                  make_shape(rg.shape or (1,)))
    _check(rc, "accumulate_grad")
    return g


def accumulate_grad_rc(grad_shape, rg) -> int:
    g = np.zeros(grad_shape, dtype=np.float32)
    rg = _f32(rg)
    return lib().or_accumulate_grad(_ptr(g), make_shape(grad_shape), _ptr(rg),
                                    make_shape(rg.shape))


def reduce_all(op: int, x) -> np.float32:
    x = _f32(x)
    return np.float32(lib().or_reduce_all(op, _ptr(x), x.size))


def reduce_axis_mt(op: int, x, axis: int, nthreads: int) -> np.ndarray:
    """SUM/MEAN/MAX along `axis` with the outputs spread over `nthreads` threads
    (tensorutils.mojo:682 parallelize); the result keeps the reduced axis as size 1."""
    x = _f32(x)
    res = np.zeros(reduced_shape(x.shape, axis), np.float32)
    _check(lib().or_reduce_axis_mt(op, _ptr(res), _ptr(x), make_shape(x.shape), int(axis), int(nthreads)),
           "reduce_axis_mt")
    return res


def reduced_shape(shape, axis):
    if axis is None or axis < 0:
        return (1,)
    s = list(shape)
    s[axis] = 1
    return tuple(s)


def forward_op(op: int, t1, t2=None, axis=None) -> np.ndarray:
    """forward_op (ops.mojo:243-311) on numpy inputs; returns the result tensor."""
    t1 = _f32(t1)
    s1 = t1.shape or (1,)
    ax = -1 if axis is None else int(axis)
    if op in (ADD, SUB, MUL, DIV):
        t2 = _f32(t2)
        rs = broadcast_shapes(s1, t2.shape or (1,))
        if rs is None:
            raise OracleError("shapes do not broadcast")
    elif op == POW:
        t2 = _f32(t2)
        rs = s1
    elif op in (SUM, MEAN, MAX):
        rs = reduced_shape(s1, ax)
    else:
        rs = s1
    res = np.zeros(rs, dtype=np.float32)
    if t2 is None:
        rc = lib().or_forward_op(op, _ptr(res), _ptr(t1), make_shape(s1), None, None, ax)
    else:
        rc = lib().or_forward_op(op, _ptr(res), _ptr(t1), make_shape(s1), _ptr(t2),
                                 make_shape(t2.shape or (1,)), ax)
    _check(rc, f"forward_op({op})")
    return res


def backward_op(tensor_id: int, op: int, ug, t1, t2=None, grad=None, axis=None) -> np.ndarray:
    """backward_op (ops.mojo:355-463): returns grad + (accumulated) op gradient.

    ``grad`` defaults to zeros of the operand's shape, as in the reference test harness
    (tests/testing_utils.mojo:119,137,141)."""
    ug, t1 = _f32(ug), _f32(t1)
    s1 = t1.shape or (1,)
    ax = -1 if axis is None else int(axis)
    if t2 is not None:
        t2 = _f32(t2)
        s2 = t2.shape or (1,)
        gshape = s1 if tensor_id == 0 else s2
    else:
        s2 = None
        gshape = s1
    g = np.zeros(gshape, dtype=np.float32) if grad is None else _f32(grad).copy()
    rc = lib().or_backward_op(
        tensor_id, op, _ptr(ug), make_shape(ug.shape or (1,)), _ptr(t1), make_shape(s1),
        _ptr(t2) if t2 is not None else None, make_shape(s2) if s2 is not None else None,
        ax, _ptr(g))
    _check(rc, f"backward_op({tensor_id}, {op})")
    return g


def forward_op_into(op: int, res: np.ndarray, t1: np.ndarray, t2: np.ndarray = None, axis: int = -1) -> None:
    """forward_op into a preallocated float32 result (as Model's arena slots are); contiguous
    float32 inputs only, no copies. For the timed CPU baseline."""
    rc = lib().or_forward_op(op, _ptr(res), _ptr(t1), make_shape(t1.shape or (1,)),
                             _ptr(t2) if t2 is not None else None,
                             make_shape(t2.shape or (1,)) if t2 is not None else None, int(axis))
    _check(rc, f"forward_op({op})")


def backward_op_into(tensor_id: int, op: int, grad: np.ndarray, ug: np.ndarray, t1: np.ndarray,
                     t2: np.ndarray = None, axis: int = -1) -> None:
    """backward_op accumulating into `grad` in place (ops.mojo:355-463); contiguous float32
    arrays only, no copies. For the timed CPU baseline."""
    rc = lib().or_backward_op(tensor_id, op, _ptr(ug), make_shape(ug.shape or (1,)), _ptr(t1),
                              make_shape(t1.shape or (1,)), _ptr(t2) if t2 is not None else None,
                              make_shape(t2.shape or (1,)) if t2 is not None else None, int(axis), _ptr(grad))
    _check(rc, f"backward_op({tensor_id}, {op})")


def backward_op_rc(tensor_id: int, op: int, ug, t1, t2=None, axis=None) -> int:
    """Return code only (for the shape-rejection tests)."""
    try:
        backward_op(tensor_id, op, ug, t1, t2, axis=axis)
        return 0
    except OracleError as e:
        return int(str(e).rsplit(" ", 1)[-1])


def adam_step(param, grad, m, v, iter_: int, lr=0.001, beta1=0.9, beta2=0.999, eps=1e-8):
    """Adam.step (mantle/nn/optim.mojo:94-140) on one parameter tensor at iteration iter_;
    returns new (param, m, v) arrays."""
    p, g, mm, vv = (_f32(a).copy() for a in (param, grad, m, v))
    lib().or_adam_step(_ptr(p), _ptr(g), _ptr(mm), _ptr(vv), p.size, float(lr), float(beta1), float(beta2),
                       float(eps), int(iter_))
    return p, mm, vv


def fma_fwd(t1, t2, t3) -> np.ndarray:
    """FMA.forward (basics.mojo:768-788)."""
    a, b, c = _f32(t1), _f32(t2), _f32(t3)
    r = np.zeros_like(a)
    lib().or_fma_fwd(_ptr(r), _ptr(a), _ptr(b), _ptr(c), a.size)
    return r


def fma_bwd_accum(tensor_id: int, grad, ug, t1, t2) -> np.ndarray:
    """FMA.backward (basics.mojo:790-817) accumulated into a copy of grad."""
    g, u, a, b = _f32(grad).copy(), _f32(ug), _f32(t1), _f32(t2)
    _check(lib().or_fma_bwd_accum(int(tensor_id), _ptr(g), _ptr(u), _ptr(a), _ptr(b), g.size), "or_fma_bwd_accum")
    return g


def leakyrelu_fwd(x, slope: float) -> np.ndarray:
    """LEAKYRELU.forward (mlops.mojo:134-156)."""
    x = _f32(x)
    r = np.zeros_like(x)
    lib().or_leakyrelu_fwd(_ptr(r), _ptr(x), x.size, float(slope))
    return r


def leakyrelu_bwd_accum(grad, x, ug, slope: float) -> np.ndarray:
    """LEAKYRELU.backward (mlops.mojo:158-186) accumulated into a copy of grad."""
    g, x, u = _f32(grad).copy(), _f32(x), _f32(ug)
    lib().or_leakyrelu_bwd_accum(_ptr(g), _ptr(x), _ptr(u), g.size, float(slope))
    return g


def clip_fwd(x, lo: float = -FLT_MAX, hi: float = FLT_MAX) -> np.ndarray:
    """CLIP.forward (mlops.mojo:243-266)."""
    x = _f32(x)
    r = np.zeros_like(x)
    lib().or_clip_fwd(_ptr(r), _ptr(x), x.size, float(lo), float(hi))
    return r


def clip_bwd_accum(grad, x, ug, lo: float = -FLT_MAX, hi: float = FLT_MAX) -> np.ndarray:
    """CLIP.backward (mlops.mojo:268-299) accumulated into a copy of grad."""
    g, x, u = _f32(grad).copy(), _f32(x), _f32(ug)
    lib().or_clip_bwd_accum(_ptr(g), _ptr(x), _ptr(u), g.size, float(lo), float(hi))
    return g


def tstd(x, axis=None) -> np.ndarray:
    """tstd (tensorutils.mojo:724-741 all elements, :776-840 one axis); returns the reduced
    tensor ((1,) for all elements)."""
    x = _f32(x)
    if axis is None or axis < 0:
        return np.array([lib().or_tstd_all(_ptr(x), x.size)], np.float32)
    r = np.zeros(reduced_shape(x.shape, axis), np.float32)
    _check(lib().or_tstd_axis(_ptr(r), _ptr(x), make_shape(x.shape), int(axis)), "or_tstd_axis")
    return r
