"""mantle_amd: Mantle's elementwise / broadcast / reduction op layer on MI355X (gfx950).

The compute path is libmantle_hip.so (hand-written HIP kernels behind the C ABI in
include/mantle_hip.h); this package is its Python host side: a device-resident Tensor and
a mirror of Mantle's op structs and forward_op / backward_op. Nothing here falls back to
the CPU: if the library is missing or the device is absent, calls raise.
"""
from ._lib import MantleHipError, lib  # noqa: F401
from .tensor import Tensor, TensorShape, init, sync  # noqa: F401
from .optim import Adam  # noqa: F401
from .graph import Graph, Symbol  # noqa: F401
from .model import Collection, Model, Parameters  # noqa: F401
from .checkpoint import (  # noqa: F401
    CheckpointError, CheckpointInfo, load_checkpoint, load_checkpoint_with_optim, save_checkpoint,
    save_checkpoint_with_optim,
)
from .ops import (  # noqa: F401
    OP, ADD, SUB, MUL, DIV, EXP, LOG, POW, SUM, MEAN, MAX, SIGMOID, RELU, TANH, FMA, CLIP, LEAKYRELU,
    forward_op, backward_op, backward_op_both, broadcast_shapes, get_reduce_shape, fill,
    elwise_transform, elwise_pow, elwise_op, accumulate_grad, tsum, tmean, tmax, tstd, static_result_shape,
    bias_relu_forward, bias_relu_backward, softmax_log_mul_mean_forward, softmax_log_mul_mean_backward,
    softmax_forward, softmax_backward, logsoftmax_forward, logsoftmax_backward, cross_entropy_forward,
    cross_entropy_backward,
)

__all__ = [
    "Adam", "Collection", "Graph", "Model", "Parameters", "Symbol", "MantleHipError", "Tensor", "TensorShape", "init", "sync", "OP", "forward_op", "backward_op",
    "backward_op_both", "broadcast_shapes", "get_reduce_shape", "fill", "elwise_transform",
    "elwise_pow", "elwise_op", "accumulate_grad", "tsum", "tmean", "tmax", "tstd", "static_result_shape", "bias_relu_forward",
    "bias_relu_backward", "softmax_log_mul_mean_forward", "softmax_log_mul_mean_backward", "softmax_forward",
    "softmax_backward", "logsoftmax_forward", "logsoftmax_backward", "cross_entropy_forward",
    "cross_entropy_backward", "CheckpointError", "CheckpointInfo", "save_checkpoint", "save_checkpoint_with_optim",
    "load_checkpoint", "load_checkpoint_with_optim",
]
