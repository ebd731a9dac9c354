"""Mantle's op layer for the elementwise / broadcast / reduction path, on the HIP library.

Mirrors the reference interface so that its callers read the same:
  * ``OP`` ids and ``forward_op`` / ``backward_op`` (mantle/autograd/ops/ops.mojo:52-101,
    243-311, 355-463);
  * the op structs ``ADD SUB MUL DIV EXP LOG POW SUM MEAN MAX SIGMOID RELU TANH FMA CLIP
    LEAKYRELU`` with ``result_shape`` and ``forward`` (mantle/autograd/ops/basics.mojo,
    mlops.mojo);
  * the tensorutils primitives ``fill``, ``elwise_transform``, ``elwise_pow``, ``elwise_op``,
    ``broadcast_shapes``, ``get_reduce_shape``, ``accumulate_grad``, ``tsum``, ``tmean``,
    ``tmax``, ``tstd`` (mantle/core/tensorutils.mojo).

Every call runs the gfx950 kernels of libmantle_hip.so on device-resident ``Tensor``s.
Errors the reference only prints (non-broadcastable shapes, unknown ops) raise
``MantleHipError`` here. Backward calls accumulate into ``grad`` as backward_op does.
"""
from __future__ import annotations

from typing import Optional

from . import _lib
from .tensor import Tensor, TensorShape, as_shape


class OP:
    """Operator ids (ops.mojo:57-83); only the ids this layer implements."""
    ADD, SUB, MUL, DIV, EXP, LOG, POW = 0, 1, 2, 3, 4, 5, 6
    SUM, MEAN, MAX = 8, 9, 10
    SIGMOID, RELU, TANH = 13, 14, 15
    FMA, CLIP, LEAKYRELU = 19, 20, 28

    NAMES = {0: "ADD", 1: "SUB", 2: "MUL", 3: "DIV", 4: "EXP", 5: "LOG", 6: "POW", 8: "SUM",
             9: "MEAN", 10: "MAX", 13: "SIGMOID", 14: "RELU", 15: "TANH", 19: "FMA", 20: "CLIP",
             28: "LEAKYRELU"}


BINARY = (OP.ADD, OP.SUB, OP.MUL, OP.DIV)
UNARY = (OP.EXP, OP.LOG, OP.SIGMOID, OP.RELU, OP.TANH)
REDUCE = (OP.SUM, OP.MEAN, OP.MAX)
ATTR_UNARY = (OP.LEAKYRELU, OP.CLIP)

FLT_MAX = 3.4028234663852886e38  # max_finite[f32]; CLIP's absent bounds are -/+ this


def _attr(attributes, name: str):
    if attributes is None or not isinstance(attributes, dict):
        return None
    return attributes.get(name)


def _axis(attributes) -> int:
    if attributes is None:
        return -1
    ax = attributes.get("axis") if isinstance(attributes, dict) else attributes
    return -1 if ax is None else int(ax)


# ---------------------------------------------------------------------------------------
# tensorutils
# ---------------------------------------------------------------------------------------
def broadcast_shapes(s1, s2) -> TensorShape:
    """broadcast_shapes, tensorutils.mojo:88-127 (raises on a mismatch)."""
    a, b = as_shape(s1).dims, as_shape(s2).dims
    big, small = (a, b) if len(a) > len(b) else (b, a)
    diff = len(big) - len(small)
    res = list(big)
    for i in range(len(big) - 1, diff - 1, -1):
        x, y = big[i], small[i - diff]
        if x == y:
            res[i] = x
        elif x == 1 or y == 1:
            res[i] = x * y
        else:
            raise _lib.MantleHipError(_lib.ERR_SHAPE, f"Shapes {a} and {b} cannot be broadcasted together.")
    return TensorShape(res)


def get_reduce_shape(t, axis: int) -> TensorShape:
    """get_reduce_shape, tensorutils.mojo:601-619."""
    d = list(as_shape(t).dims)
    d[axis] = 1
    return TensorShape(d)


def fill(t: Tensor, val: float) -> None:
    _lib.call("mh_fill", t.ptr, float(val), t.num_elements())


def elwise_transform(op: int, res: Tensor, t: Tensor) -> None:
    """elwise_transform, tensorutils.mojo:181-200, with op in EXP/LOG/SIGMOID/RELU/TANH."""
    _lib.call("mh_unary_fwd", int(op), res.ptr, t.ptr, t.num_elements())


def elwise_pow(res: Tensor, t: Tensor, n: int) -> None:
    """elwise_pow, tensorutils.mojo:226-239: res = t ** n for an integer n (square and
    multiply; 1 / result for negative n)."""
    n = int(n)
    if not -(1 << 31) <= n < (1 << 31):
        raise ValueError(f"elwise_pow: exponent {n} outside int32")
    _lib.call("mh_powi_fwd", res.ptr, t.ptr, n, t.num_elements())


def elwise_op(op: int, res: Tensor, t1: Tensor, t2: Tensor) -> None:
    """elwise_op dispatcher, tensorutils.mojo:242-357."""
    _lib.call("mh_binary_fwd", int(op), res.ptr, res.shape().c(), t1.ptr, t1.shape().c(), t2.ptr,
              t2.shape().c())


def accumulate_grad(grad: Tensor, res_grad: Tensor) -> None:
    """accumulate_grad, tensorutils.mojo:442-487 (same shape, scalar or un-broadcast)."""
    _lib.call("mh_accumulate_grad", grad.ptr, grad.shape().c(), res_grad.ptr, res_grad.shape().c())


def _reduce(op: int, t: Tensor, axis: int, res: Optional[Tensor]) -> Tensor:
    if res is None:
        res = Tensor(TensorShape(1) if axis < 0 else get_reduce_shape(t.shape(), axis))
    _lib.call("mh_reduce_fwd", int(op), res.ptr, t.ptr, t.shape().c(), int(axis))
    return res


def tsum(t: Tensor, axis: int = -1, res: Optional[Tensor] = None) -> Tensor:
    return _reduce(OP.SUM, t, axis, res)


def tmean(t: Tensor, axis: int = -1, res: Optional[Tensor] = None) -> Tensor:
    return _reduce(OP.MEAN, t, axis, res)


def tmax(t: Tensor, axis: int = -1, res: Optional[Tensor] = None) -> Tensor:
    return _reduce(OP.MAX, t, axis, res)


def tstd(t: Tensor, axis: int = -1, res: Optional[Tensor] = None) -> Tensor:
    """tstd, tensorutils.mojo:724-741 (all elements, shape (1)) and :776-840 (one axis):
    population standard deviation. Each output reads the line tmean reads."""
    if res is None:
        res = Tensor(TensorShape(1) if axis < 0 else get_reduce_shape(t.shape(), axis))
    _lib.call("mh_tstd", res.ptr, t.ptr, t.shape().c(), int(axis))
    return res


# ---------------------------------------------------------------------------------------
# op structs (result_shape + forward); backward goes through backward_op
# ---------------------------------------------------------------------------------------
class _Binary:
    op = -1

    @staticmethod
    def result_shape(t1_shape, t2_shape) -> TensorShape:
        return broadcast_shapes(t1_shape, t2_shape)

    @classmethod
    def forward(cls, res: Tensor, t1: Tensor, t2: Tensor) -> None:
        elwise_op(cls.op, res, t1, t2)


class ADD(_Binary):
    op = OP.ADD


class SUB(_Binary):
    op = OP.SUB


class MUL(_Binary):
    op = OP.MUL


class DIV(_Binary):
    op = OP.DIV


class _Unary:
    op = -1

    @staticmethod
    def result_shape(t1_shape) -> TensorShape:
        return as_shape(t1_shape)

    @classmethod
    def forward(cls, res: Tensor, t1: Tensor) -> None:
        elwise_transform(cls.op, res, t1)


class EXP(_Unary):
    op = OP.EXP


class LOG(_Unary):
    op = OP.LOG


class SIGMOID(_Unary):
    op = OP.SIGMOID


class RELU(_Unary):
    op = OP.RELU


class TANH(_Unary):
    op = OP.TANH


class POW:
    """POW with a shape-(1) graph-scalar exponent (basics.mojo:312-378)."""
    op = OP.POW

    @staticmethod
    def result_shape(t1_shape, t2_shape) -> TensorShape:
        return as_shape(t1_shape)

    @staticmethod
    def forward(res: Tensor, t1: Tensor, t2: Tensor) -> None:
        _lib.call("mh_pow_fwd", res.ptr, t1.ptr, t1.num_elements(), t2.ptr)


class _Reduce:
    op = -1

    @staticmethod
    def result_shape(t_shape, attributes=None) -> TensorShape:
        ax = _axis(attributes)
        return TensorShape(1) if ax < 0 else get_reduce_shape(t_shape, ax)

    @classmethod
    def forward(cls, res: Tensor, t: Tensor, attributes=None) -> None:
        _reduce(cls.op, t, _axis(attributes), res)


class SUM(_Reduce):
    op = OP.SUM


class MEAN(_Reduce):
    op = OP.MEAN


class MAX(_Reduce):
    op = OP.MAX


class FMA:
    """FMA, basics.mojo:758-817: fma(t1, t2, t3) over three equal shapes."""
    op = OP.FMA

    @staticmethod
    def result_shape(t1_shape, t2_shape, t3_shape) -> TensorShape:
        return as_shape(t1_shape)

    @staticmethod
    def forward(res: Tensor, t1: Tensor, t2: Tensor, t3: Tensor) -> None:
        if not (t1.shape() == t2.shape() == t3.shape() == res.shape()):
            raise _lib.MantleHipError(_lib.ERR_SHAPE, "FMA needs four equal shapes")
        _lib.call("mh_fma_fwd", res.ptr, t1.ptr, t2.ptr, t3.ptr, t1.num_elements())


class LEAKYRELU:
    """LEAKYRELU, mlops.mojo:128-186; attribute ``negative_slope`` (required)."""
    op = OP.LEAKYRELU

    @staticmethod
    def result_shape(t1_shape, attributes=None) -> TensorShape:
        return as_shape(t1_shape)

    @staticmethod
    def slope(attributes) -> float:
        v = _attr(attributes, "negative_slope")
        if v is None:
            raise _lib.MantleHipError(_lib.ERR_INVALID, "LEAKYRELU needs the negative_slope attribute")
        return float(v)

    @classmethod
    def forward(cls, res: Tensor, t1: Tensor, attributes=None) -> None:
        _lib.call("mh_leakyrelu_fwd", res.ptr, t1.ptr, t1.num_elements(), cls.slope(attributes))


class CLIP:
    """CLIP, mlops.mojo:236-299; attributes ``min`` / ``max`` (absent: min_finite /
    max_finite)."""
    op = OP.CLIP

    @staticmethod
    def result_shape(t1_shape, attributes=None) -> TensorShape:
        return as_shape(t1_shape)

    @staticmethod
    def bounds(attributes):
        lo, hi = _attr(attributes, "min"), _attr(attributes, "max")
        return (-FLT_MAX if lo is None else float(lo)), (FLT_MAX if hi is None else float(hi))

    @classmethod
    def forward(cls, res: Tensor, t1: Tensor, attributes=None) -> None:
        lo, hi = cls.bounds(attributes)
        _lib.call("mh_clip_fwd", res.ptr, t1.ptr, t1.num_elements(), lo, hi)


STRUCTS = {OP.ADD: ADD, OP.SUB: SUB, OP.MUL: MUL, OP.DIV: DIV, OP.EXP: EXP, OP.LOG: LOG,
           OP.POW: POW, OP.SUM: SUM, OP.MEAN: MEAN, OP.MAX: MAX, OP.SIGMOID: SIGMOID,
           OP.RELU: RELU, OP.TANH: TANH, OP.FMA: FMA, OP.LEAKYRELU: LEAKYRELU, OP.CLIP: CLIP}


def static_result_shape(op: int, *shapes, attributes=None) -> TensorShape:
    """static_result_shape, ops.mojo:104-218 (the subset of ops implemented here)."""
    s = STRUCTS.get(op)
    if s is None:
        raise _lib.MantleHipError(_lib.ERR_OP, f"Operator {op} not found.")
    if op in REDUCE or op in ATTR_UNARY:
        return s.result_shape(shapes[0], attributes)
    return s.result_shape(*shapes)


# ---------------------------------------------------------------------------------------
# dispatch
# ---------------------------------------------------------------------------------------
def forward_op(op: int, res: Tensor, t1: Tensor, t2: Optional[Tensor] = None, attributes=None,
               t3: Optional[Tensor] = None) -> None:
    """forward_op, ops.mojo:243-341: writes op(t1[, t2[, t3]]) into the preallocated res."""
    if op == OP.FMA:
        if t2 is None or t3 is None:
            raise _lib.MantleHipError(_lib.ERR_INVALID, "FMA needs three operands")
        FMA.forward(res, t1, t2, t3)
    elif op in ATTR_UNARY:
        STRUCTS[op].forward(res, t1, attributes)
    elif op in BINARY or op == OP.POW:
        if t2 is None:
            raise _lib.MantleHipError(_lib.ERR_INVALID, f"{OP.NAMES[op]} needs two operands")
        STRUCTS[op].forward(res, t1, t2)
    elif op in UNARY:
        STRUCTS[op].forward(res, t1)
    elif op in REDUCE:
        STRUCTS[op].forward(res, t1, attributes)
    else:
        raise _lib.MantleHipError(_lib.ERR_OP, f"Operator {op} not found.")


def backward_op(tensor_id: int, op: int, ug: Tensor, t1: Tensor, t2: Optional[Tensor] = None,
                grad: Optional[Tensor] = None, attributes=None, t3: Optional[Tensor] = None) -> None:
    """backward_op, ops.mojo:355-497: grad += the gradient of operand ``tensor_id``.

    Signature order follows the reference's binary form (ug, t1, t2, grad); for unary and
    reduce ops pass ``t2=None`` and ``grad`` by keyword or positionally; FMA's third operand
    goes in ``t3`` (its gradient does not read it)."""
    if grad is None:
        raise _lib.MantleHipError(_lib.ERR_NULL, "backward_op needs the grad tensor")
    if op == OP.FMA:
        if t2 is None or not (ug.shape() == t1.shape() == t2.shape() == grad.shape()):
            raise _lib.MantleHipError(_lib.ERR_SHAPE, "FMA backward needs equal shapes")
        _lib.call("mh_fma_bwd_accum", int(tensor_id), grad.ptr, ug.ptr, t1.ptr, t2.ptr, t1.num_elements())
    elif op in ATTR_UNARY:
        if ug.shape() != t1.shape() or grad.shape() != t1.shape():
            raise _lib.MantleHipError(_lib.ERR_SHAPE, "ug / grad shape differs from the operand shape")
        if op == OP.LEAKYRELU:
            _lib.call("mh_leakyrelu_bwd_accum", grad.ptr, t1.ptr, ug.ptr, t1.num_elements(),
                      LEAKYRELU.slope(attributes))
        else:
            lo, hi = CLIP.bounds(attributes)
            _lib.call("mh_clip_bwd_accum", grad.ptr, t1.ptr, ug.ptr, t1.num_elements(), lo, hi)
    elif op in BINARY:
        _lib.call("mh_binary_bwd_accum", int(op), int(tensor_id), grad.ptr, grad.shape().c(), ug.ptr,
                  ug.shape().c(), t1.ptr, t1.shape().c(), t2.ptr, t2.shape().c())
    elif op == OP.POW:
        if t2.num_elements() != 1 or t2.shape() != TensorShape(1):
            raise _lib.MantleHipError(_lib.ERR_SHAPE, "POW exponent must be a shape-(1) graph scalar")
        _lib.call("mh_pow_bwd_accum", int(tensor_id), grad.ptr, t1.ptr, t2.ptr, ug.ptr, t1.num_elements())
    elif op in UNARY:
        if ug.shape() != t1.shape():
            raise _lib.MantleHipError(_lib.ERR_SHAPE, "ug shape differs from the operand shape")
        _lib.call("mh_unary_bwd_accum", int(op), grad.ptr, t1.ptr, ug.ptr, t1.num_elements())
    elif op in REDUCE:
        ax = _axis(attributes)
        if ug.shape() != _Reduce.result_shape(t1.shape(), attributes):
            raise _lib.MantleHipError(_lib.ERR_SHAPE, "ug shape is not the reduced shape")
        _lib.call("mh_reduce_bwd_accum", int(op), grad.ptr, t1.ptr, t1.shape().c(), ug.ptr, ax)
    else:
        raise _lib.MantleHipError(_lib.ERR_OP, f"Operator {op} not found.")


def backward_op_both(op: int, ug: Tensor, t1: Tensor, t2: Tensor, grad1: Optional[Tensor],
                     grad2: Optional[Tensor]) -> None:
    """Both backward_op calls of a same-shape binary op in one fused pass. grad1 and grad2 may be
    the same tensor (an op over one symbol twice, x * x): both gradients then accumulate into it,
    operand 0's first, as the two calls of Model.backward do (model.mojo:233-270). For POW, t2 is
    the shape-(1) exponent: grad1 takes x's gradient and grad2 the exponent's, from one read of
    t1 and ug, with the bits of the two calls."""
    if op == OP.POW:
        if t2.shape() != TensorShape(1) or ug.shape() != t1.shape():
            raise _lib.MantleHipError(_lib.ERR_SHAPE, "POW exponent must be a shape-(1) graph scalar")
        _lib.call("mh_pow_bwd_accum2", grad1.ptr if grad1 is not None else None,
                  grad2.ptr if grad2 is not None else None, t1.ptr, t2.ptr, ug.ptr, t1.num_elements())
        return
    if t1.shape() != t2.shape() or ug.shape() != t1.shape():
        if grad1 is not None:
            backward_op(0, op, ug, t1, t2, grad1)
        if grad2 is not None:
            backward_op(1, op, ug, t1, t2, grad2)
        return
    _lib.call("mh_binary_bwd_accum2", int(op), grad1.ptr if grad1 is not None else None,
              grad2.ptr if grad2 is not None else None, ug.ptr, t1.ptr, t2.ptr, t1.shape().c())


# ---------------------------------------------------------------------------------------
# fused graph patterns (no single reference counterpart)
# ---------------------------------------------------------------------------------------
def bias_relu_forward(y: Tensor, r: Tensor, x: Tensor, bias: Tensor) -> None:
    """The graph ADD(x, bias) -> RELU in one pass: y = x + bias (broadcast), r = relu(y)."""
    _lib.call("mh_bias_relu_fwd", y.ptr, r.ptr, x.ptr, x.shape().c(), bias.ptr, bias.shape().c())


def bias_relu_backward(ug: Tensor, y: Tensor, bias_shape, grad_x: Optional[Tensor], grad_bias: Optional[Tensor],
                       grad_y: Optional[Tensor] = None) -> None:
    """Backward of ADD(x, bias) -> RELU from the grad ug of r: grad_y (if kept) += relu'(y) * ug,
    then grad_x += grad_y and grad_bias += its sum over the broadcast axes of bias_shape."""
    _lib.call("mh_bias_relu_bwd_accum", grad_y.ptr if grad_y is not None else None,
              grad_x.ptr if grad_x is not None else None, grad_bias.ptr if grad_bias is not None else None,
              y.ptr, ug.ptr, y.shape().c(), as_shape(bias_shape).c())


def softmax_log_mul_mean_forward(loss: Tensor, x: Tensor, target: Tensor) -> None:
    """The graph MAX -> SUB -> EXP -> SUM -> DIV -> LOG -> MUL(target) -> MEAN over the rows of
    x [rows, classes] in one pass (Softmax, mantle/nn/activations.mojo:74-87, then LOG, MUL,
    MEAN): loss[0] = mean(log(softmax(x)) * target)."""
    rows, classes = _row_operands(x, same=(("target", target),), scalar=(("loss", loss),))
    _lib.call("mh_softmax_log_mul_mean_fwd", loss.ptr, x.ptr, target.ptr, rows, classes)


def softmax_log_mul_mean_backward(grad_x: Tensor, x: Tensor, target: Tensor, ug: Tensor) -> None:
    """Backward of the same graph from the loss grad ug (shape (1)): grad_x += d loss / dx."""
    rows, classes = _row_operands(x, same=(("grad_x", grad_x), ("target", target)), scalar=(("ug", ug),))
    _lib.call("mh_softmax_log_mul_mean_bwd_accum", grad_x.ptr, x.ptr, target.ptr, ug.ptr, rows, classes)


def _rows_classes(t: Tensor):
    k = t.shape()[t.rank() - 1] if t.rank() else 1
    return (t.num_elements() // k if k else 0), k


def _row_operands(x: Tensor, same=(), scalar=()):
    """(rows, classes) of x over its last axis, after checking every tensor the fused row
    kernels read or write beside x: those in `same` must have x's shape and those in `scalar`
    one element. The C entry points take bare pointers and sizes, so a smaller tensor would
    reach the kernel as an out-of-bounds access; the check runs before any launch."""
    xs = x.shape()
    for name, t in same:
        if t is None or t.shape() != xs:
            got = None if t is None else t.shape()
            raise _lib.MantleHipError(_lib.ERR_SHAPE, f"{name} shape {got} differs from x shape {xs}")
    for name, t in scalar:
        if t is None or t.num_elements() != 1:
            got = None if t is None else t.num_elements()
            raise _lib.MantleHipError(_lib.ERR_SHAPE, f"{name} must hold one element (holds {got})")
    return _rows_classes(x)


def softmax_forward(out: Tensor, x: Tensor) -> None:
    """Softmax over the last axis (activations.mojo:74-87), one fused pass."""
    r, k = _row_operands(x, same=(("out", out),))
    _lib.call("mh_softmax_fwd", out.ptr, x.ptr, r, k)


def softmax_backward(grad_x: Tensor, x: Tensor, grad_out: Tensor) -> None:
    """grad_x += the five Softmax backward nodes' contribution from grad_out."""
    r, k = _row_operands(x, same=(("grad_x", grad_x), ("grad_out", grad_out)))
    _lib.call("mh_softmax_bwd_accum", grad_x.ptr, x.ptr, grad_out.ptr, r, k)


def logsoftmax_forward(out: Tensor, x: Tensor) -> None:
    """LogSoftmax over the last axis (activations.mojo:94-108), one fused pass."""
    r, k = _row_operands(x, same=(("out", out),))
    _lib.call("mh_logsoftmax_fwd", out.ptr, x.ptr, r, k)


def logsoftmax_backward(grad_x: Tensor, x: Tensor, grad_out: Tensor) -> None:
    """grad_x += the six LogSoftmax backward nodes' contribution from grad_out."""
    r, k = _row_operands(x, same=(("grad_x", grad_x), ("grad_out", grad_out)))
    _lib.call("mh_logsoftmax_bwd_accum", grad_x.ptr, x.ptr, grad_out.ptr, r, k)


def cross_entropy_forward(loss: Tensor, x: Tensor, target: Tensor) -> None:
    """CrossEntropyLoss (loss.mojo:45-61) of x [rows, classes] against target, one fused pass."""
    r, k = _row_operands(x, same=(("target", target),), scalar=(("loss", loss),))
    _lib.call("mh_cross_entropy_fwd", loss.ptr, x.ptr, target.ptr, r, k)


def cross_entropy_backward(grad_x: Tensor, x: Tensor, target: Tensor, ug: Tensor) -> None:
    """grad_x += d loss / dx of CrossEntropyLoss from the loss grad ug (one element)."""
    r, k = _row_operands(x, same=(("grad_x", grad_x), ("target", target)), scalar=(("ug", ug),))
    _lib.call("mh_cross_entropy_bwd_accum", grad_x.ptr, x.ptr, target.ptr, ug.ptr, r, k)
