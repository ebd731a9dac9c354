"""ctypes binding of libmantle_hip.so (the C ABI declared in include/mantle_hip.h).

The library is loaded from this package directory; there is no fallback. If it is missing,
every call raises: build it with ``python -m mantle_amd.build``.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libmantle_hip.so")

MAX_RANK = 8

# include/mantle_hip.h enum mh_op (= Mantle OP ids, mantle/autograd/ops/ops.mojo:57-83)
ADD, SUB, MUL, DIV, EXP, LOG, POW = 0, 1, 2, 3, 4, 5, 6
SUM, MEAN, MAX = 8, 9, 10
SIGMOID, RELU, TANH = 13, 14, 15

# enum mh_status
OK = 0
ERR_INVALID, ERR_SHAPE, ERR_RANK, ERR_NULL, ERR_OP = -1, -2, -3, -4, -5
ERR_NOT_INIT, ERR_HIP, ERR_NO_DEVICE, ERR_OVERFLOW = -6, -7, -8, -9

INIT_ASYNC = 1


class mh_shape(ctypes.Structure):
    _fields_ = [("rank", ctypes.c_int32), ("dims", ctypes.c_int64 * MAX_RANK)]


class mh_plan_info(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("dims", ctypes.c_int64 * MAX_RANK), ("stride_a", ctypes.c_int64 * MAX_RANK),
                ("stride_b", ctypes.c_int64 * MAX_RANK)]


class mh_reduce_plan_info(ctypes.Structure):
    _fields_ = [("nsteps", ctypes.c_int32), ("a", ctypes.c_int64 * MAX_RANK),
                ("b", ctypes.c_int64 * MAX_RANK), ("c", ctypes.c_int64 * MAX_RANK)]


class mh_launch_info(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int32), ("threads", ctypes.c_int32), ("blocks", ctypes.c_int64),
                ("launches", ctypes.c_int64)]


(LAUNCH_FILL, LAUNCH_FILL_UNALIGNED, LAUNCH_COPY, LAUNCH_SAME_SHAPE, LAUNCH_ADAM, LAUNCH_ADAM_UNALIGNED,
 LAUNCH_ROWS16) = range(7)


class mh_attrs(ctypes.Structure):
    """AttributeVector entries of the ops on this path (mantle/autograd/attributes.mojo)."""
    _fields_ = [("flags", ctypes.c_int32), ("axis", ctypes.c_int32), ("negative_slope", ctypes.c_float),
                ("min_val", ctypes.c_float), ("max_val", ctypes.c_float)]


ATTR_AXIS, ATTR_NEGATIVE_SLOPE, ATTR_MIN, ATTR_MAX = 1, 2, 4, 8
SYM_INPUT, SYM_PARAM, SYM_NODE = 0, 1, 2
FROM_HOST, FROM_DEVICE = 0, 1
MODEL_FUSE_BIAS_RELU = 1
MODEL_FUSE_ROWS = 2
PASS_FORWARD, PASS_BACKWARD, PASS_STEP = 0, 1, 2


class MantleHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def make_shape(dims) -> mh_shape:
    dims = tuple(int(d) for d in dims)
    s = mh_shape()
    s.rank = len(dims)
    for i, d in enumerate(dims[:MAX_RANK]):
        s.dims[i] = d
    return s


_VP = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_S = ctypes.POINTER(mh_shape)  # shapes cross the ABI by pointer (ctypes passes an mh_shape byref)

# name -> argtypes (all return int unless listed in _RESTYPE)
SIGNATURES = {
    "mh_init": [_I, ctypes.c_uint64],
    "mh_shutdown": [],
    "mh_sync": [],
    "mh_last_error": [],
    "mh_status_string": [_I],
    "mh_device_count": [ctypes.POINTER(_I)],
    "mh_malloc": [ctypes.POINTER(_VP), ctypes.c_size_t],
    "mh_free": [_VP],
    "mh_memcpy_h2d": [_VP, _VP, ctypes.c_size_t],
    "mh_memcpy_d2h": [_VP, _VP, ctypes.c_size_t],
    "mh_memcpy_d2d": [_VP, _VP, ctypes.c_size_t],
    "mh_zero": [_VP, _I64],
    "mh_fill": [_VP, _F, _I64],
    "mh_binary_fwd": [_I, _VP, _S, _VP, _S, _VP, _S],
    "mh_unary_fwd": [_I, _VP, _VP, _I64],
    "mh_pow_fwd": [_VP, _VP, _I64, _VP],
    "mh_powi_fwd": [_VP, _VP, ctypes.c_int32, _I64],
    "mh_reduce_fwd": [_I, _VP, _VP, _S, ctypes.c_int32],
    "mh_reduce_fwd_noalloc": [_I, _VP, _VP, _S, ctypes.c_int32],
    "mh_binary_bwd_accum": [_I, _I, _VP, _S, _VP, _S, _VP, _S, _VP, _S],
    "mh_binary_bwd_accum2": [_I, _VP, _VP, _VP, _VP, _VP, _S],
    "mh_unary_bwd_accum": [_I, _VP, _VP, _VP, _I64],
    "mh_pow_bwd_accum": [_I, _VP, _VP, _VP, _VP, _I64],
    "mh_pow_bwd_accum2": [_VP, _VP, _VP, _VP, _VP, _I64],
    "mh_reduce_bwd_accum": [_I, _VP, _VP, _S, _VP, ctypes.c_int32],
    "mh_accumulate_grad": [_VP, _S, _VP, _S],
    "mh_bias_relu_fwd": [_VP, _VP, _VP, _S, _VP, _S],
    "mh_bias_relu_bwd_accum": [_VP, _VP, _VP, _VP, _VP, _S, _S],
    "mh_softmax_log_mul_mean_fwd": [_VP, _VP, _VP, _I64, _I64],
    "mh_softmax_log_mul_mean_bwd_accum": [_VP, _VP, _VP, _VP, _I64, _I64],
    "mh_softmax_fwd": [_VP, _VP, _I64, _I64],
    "mh_softmax_bwd_accum": [_VP, _VP, _VP, _I64, _I64],
    "mh_logsoftmax_fwd": [_VP, _VP, _I64, _I64],
    "mh_logsoftmax_bwd_accum": [_VP, _VP, _VP, _I64, _I64],
    "mh_cross_entropy_fwd": [_VP, _VP, _VP, _I64, _I64],
    "mh_cross_entropy_bwd_accum": [_VP, _VP, _VP, _VP, _I64, _I64],
    "mh_fma_fwd": [_VP, _VP, _VP, _VP, _I64],
    "mh_fma_bwd_accum": [_I, _VP, _VP, _VP, _VP, _I64],
    "mh_leakyrelu_fwd": [_VP, _VP, _I64, _F],
    "mh_leakyrelu_bwd_accum": [_VP, _VP, _VP, _I64, _F],
    "mh_clip_fwd": [_VP, _VP, _I64, _F, _F],
    "mh_clip_bwd_accum": [_VP, _VP, _VP, _I64, _F, _F],
    "mh_tstd": [_VP, _VP, _S, ctypes.c_int32],
    "mh_adam_step": [_VP, _VP, _VP, _VP, _I64, _F, _F, _F, _F, _I64],
    "mh_adam_step_multi": [_I64, ctypes.POINTER(_VP), ctypes.POINTER(_VP), ctypes.POINTER(_VP), ctypes.POINTER(_VP),
                           ctypes.POINTER(_I64), _F, _F, _F, _F, _I64],
    "mh_rand_uniform": [_VP, _I64, ctypes.c_uint64, _F, _F],
    "mh_rand_normal": [_VP, _I64, ctypes.c_uint64, _F, _F],
    "mh_event_create": [ctypes.POINTER(_VP)],
    "mh_event_destroy": [_VP],
    "mh_event_record": [_VP],
    "mh_event_elapsed_ms": [ctypes.POINTER(_F), _VP, _VP],
    "mh_graph_create": [ctypes.POINTER(_VP)],
    "mh_graph_destroy": [_VP],
    "mh_graph_input": [_VP, _S, _I, ctypes.POINTER(ctypes.c_int32)],
    "mh_graph_param": [_VP, _S, _I, _VP, _I64, ctypes.POINTER(ctypes.c_int32)],
    "mh_graph_scalar": [_VP, _F, ctypes.POINTER(ctypes.c_int32)],
    "mh_graph_op": [_VP, _I, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(mh_attrs), ctypes.POINTER(ctypes.c_int32)],
    "mh_graph_out": [_VP, ctypes.c_int32],
    "mh_graph_loss": [_VP, ctypes.c_int32],
    "mh_graph_symbol": [_VP, ctypes.c_int32, _S, ctypes.POINTER(_I), ctypes.POINTER(_I)],
    "mh_graph_counts": [_VP, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)],
    "mh_model_create": [_VP, ctypes.c_uint64, ctypes.POINTER(_VP)],
    "mh_model_destroy": [_VP],
    "mh_model_forward": [_VP, ctypes.c_int32, ctypes.POINTER(_VP), _I],
    "mh_model_inference": [_VP, ctypes.c_int32, ctypes.POINTER(_VP), _I],
    "mh_model_backward": [_VP, ctypes.c_int32, ctypes.POINTER(_VP), _I],
    "mh_model_tensor": [_VP, ctypes.c_int32, ctypes.POINTER(_VP)],
    "mh_model_grad": [_VP, ctypes.c_int32, ctypes.POINTER(_VP)],
    "mh_model_zero_grad": [_VP],
    "mh_model_capture": [_VP, _I],
    "mh_model_replay": [_VP, _I],
    "mh_model_param_span": [_VP, ctypes.POINTER(_VP), ctypes.POINTER(_VP), ctypes.POINTER(_I64)],
    "mh_model_info": [_VP, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.POINTER(ctypes.c_int32)],
    "mh_plan_binary": [_S, _S, _S, ctypes.POINTER(mh_plan_info)],
    "mh_plan_unbroadcast": [_S, _S, ctypes.POINTER(mh_reduce_plan_info)],
    "mh_plan_launch": [ctypes.c_int32, _I64, ctypes.POINTER(mh_launch_info)],
}
_RESTYPE = {"mh_last_error": ctypes.c_char_p, "mh_status_string": ctypes.c_char_p}

_lib = None


def lib():
    """The loaded library (raises if libmantle_hip.so has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m mantle_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        _lib = L
    return _lib


def last_error() -> str:
    return lib().mh_last_error().decode()


def check(rc: int, what: str = "") -> None:
    if rc != OK:
        raise MantleHipError(rc, f"{what}: {last_error()}" if what else last_error())


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)
