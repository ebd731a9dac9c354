"""Model executor: a mirror of mantle/nn/model.mojo:55-340 and its Parameters / Collections
(mantle/nn/parameters.mojo, mantle/autograd/collection.mojo:24-224) on the native model of
libmantle_hip.so (mh_model_*).

Every symbol's tensor lives in one device arena and every trainable symbol's gradient in a
second; ``parameters.tensors[sym]`` / ``parameters.grads[sym]`` are aliasing ``Tensor`` views
of those slots (Collection.__getitem__ returns share()). ``forward`` copies the inputs in,
in graph input order, and runs every node on the device; ``backward`` seeds the loss
gradient with 1.0 (or takes the last node's upper gradient) and accumulates into every
trainable gradient in reverse node order.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional

import numpy as np

from . import _lib
from .graph import Graph, Symbol
from .tensor import Tensor, ensure_init


class Collection:
    """One of the model's arenas (tensors or grads), keyed by symbol."""

    def __init__(self, model: "Model", grads: bool):
        self._m, self._grads = model, grads

    def _slot(self, sym: Symbol) -> int:
        p = ctypes.c_void_p()
        _lib.call("mh_model_grad" if self._grads else "mh_model_tensor", self._m._h, sym.name, ctypes.byref(p))
        return p.value

    def __contains__(self, sym: Symbol) -> bool:
        return (not self._grads) or sym.trainable

    def __getitem__(self, sym: Symbol) -> Tensor:
        return Tensor(sym.shape, _ptr=self._slot(sym), _owner=self._m)

    def __setitem__(self, sym: Symbol, value) -> None:
        """Collection.__setitem__ (collection.mojo:202-209): copies into the slot."""
        dst = self._slot(sym)
        n = sym.shape.num_elements()
        if isinstance(value, Tensor):
            if value.num_elements() != n:
                raise _lib.MantleHipError(_lib.ERR_SHAPE, f"{value.num_elements()} elements for a slot of {n}")
            _lib.call("mh_memcpy_d2d", dst, value.ptr, n * 4)
        else:
            a = np.ascontiguousarray(value, dtype=np.float32)
            if a.size != n:
                raise _lib.MantleHipError(_lib.ERR_SHAPE, f"{a.size} elements for a slot of {n}")
            _lib.call("mh_memcpy_h2d", dst, a.ctypes.data, n * 4)

    def set_zero(self) -> None:
        """Collection.set_zero (collection.mojo:221-224)."""
        if self._grads:
            _lib.call("mh_model_zero_grad", self._m._h)
        else:
            for s in self._m.graph.symbols:
                self[s].zero()


class Parameters:
    """mantle/nn/parameters.mojo: the tensors and grads collections of a model."""

    def __init__(self, model: "Model"):
        self.tensors = Collection(model, grads=False)
        self.grads = Collection(model, grads=True)
        self.graph = model.graph
        self._m = model

    def param_span(self):
        """(params, grads, n): the device spans holding every trainable parameter and its
        gradient, in the same layout; None without trainable parameters."""
        p, g, n = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int64()
        _lib.call("mh_model_param_span", self._m._h, ctypes.byref(p), ctypes.byref(g), ctypes.byref(n))
        return (p.value, g.value, n.value) if n.value else None


class Model:
    def __init__(self, g: Graph, inference_only: bool = False, fuse_bias_relu: bool = False,
                 fuse_rows: bool = False):
        """fuse_bias_relu: ADD(bias) -> RELU pairs run fused (every slot still written).
        fuse_rows: Softmax / LogSoftmax / CrossEntropyLoss node groups run as one row kernel
        each way (their intermediate slots are not written; gradients assume zero_grad)."""
        ensure_init()
        self.graph = g
        h = ctypes.c_void_p()
        flags = (_lib.MODEL_FUSE_BIAS_RELU if fuse_bias_relu else 0) | (_lib.MODEL_FUSE_ROWS if fuse_rows else 0)
        _lib.call("mh_model_create", g.handle, flags, ctypes.byref(h))
        self._h = h.value
        self.parameters = Parameters(self)
        self.inference_only = inference_only

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.lib().mh_model_destroy(h)
            except Exception:
                pass
            self._h = None

    @staticmethod
    def _table(tensors, symbols: List[Symbol]):
        """(ctypes pointer table, location, keep-alive) of host arrays or device Tensors."""
        if len(tensors) == 0:
            return None, _lib.FROM_HOST, ()
        on_dev = [isinstance(t, Tensor) for t in tensors]
        if any(on_dev) and not all(on_dev):
            raise _lib.MantleHipError(_lib.ERR_INVALID, "pass all inputs as device Tensors or all as host arrays")
        keep = list(tensors) if all(on_dev) else [np.ascontiguousarray(t, dtype=np.float32) for t in tensors]
        for t, s in zip(keep, symbols):
            n = t.num_elements() if isinstance(t, Tensor) else t.size
            if n != s.shape.num_elements():
                raise _lib.MantleHipError(_lib.ERR_SHAPE, f"{n} elements for {s}")
        ptrs = [t.ptr if isinstance(t, Tensor) else t.ctypes.data for t in keep]
        tab = (ctypes.c_void_p * len(ptrs))(*ptrs)
        return tab, (_lib.FROM_DEVICE if all(on_dev) else _lib.FROM_HOST), keep

    def forward(self, *t_inputs) -> Tensor:
        """Model.forward (model.mojo:80-96): runs every node; returns the loss slot."""
        if self.graph.loss_out is None:
            raise _lib.MantleHipError(_lib.ERR_INVALID, "no loss defined: model.forward() is unavailable")
        self._run("mh_model_forward", t_inputs)
        return self.parameters.tensors[self.graph.loss_out]

    def inference(self, *t_inputs) -> List[Tensor]:
        """Model.inference (model.mojo:98-111): runs up to the last output node; returns copies
        of the graph outputs."""
        self._run("mh_model_inference", t_inputs)
        return [self.parameters.tensors[s].copy() for s in self.graph.outputs]

    def _run(self, fn: str, t_inputs) -> None:
        if len(t_inputs) != len(self.graph.inputs):
            raise _lib.MantleHipError(_lib.ERR_INVALID,
                                      f"{len(t_inputs)} inputs given, the graph has {len(self.graph.inputs)}")
        tab, where, keep = self._table(t_inputs, self.graph.inputs)
        _lib.call(fn, self._h, len(t_inputs), tab, where)
        del keep

    def backward(self, *upper_grads) -> None:
        """Model.backward (model.mojo:173-330)."""
        if upper_grads:
            last = self.graph.nodes[-1][3] if self.graph.nodes else None
            tab, where, keep = self._table(upper_grads[:1], [last])
            _lib.call("mh_model_backward", self._h, len(upper_grads), tab, where)
            del keep
        else:
            _lib.call("mh_model_backward", self._h, 0, None, _lib.FROM_HOST)

    # ---- HIP-graph replay of the passes ----
    _PASSES = {"forward": _lib.PASS_FORWARD, "backward": _lib.PASS_BACKWARD, "step": _lib.PASS_STEP}

    def capture(self, pass_: str) -> None:
        """Records the forward pass (every node), the backward pass (loss seed + every node in
        reverse) or a whole step (zero_grad, forward, backward) as a HIP graph; the pass runs
        once eagerly first."""
        _lib.call("mh_model_capture", self._h, self._PASSES[pass_])

    def replay(self, pass_: str) -> Optional[Tensor]:
        """Launches the captured pass; write inputs into parameters.tensors first. The forward
        pass returns the loss slot."""
        _lib.call("mh_model_replay", self._h, self._PASSES[pass_])
        if pass_ in ("forward", "step") and self.graph.loss_out is not None:
            return self.parameters.tensors[self.graph.loss_out]
        return None

    def info(self) -> dict:
        n, tb, gb, fp = ctypes.c_int32(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
        _lib.call("mh_model_info", self._h, ctypes.byref(n), ctypes.byref(tb), ctypes.byref(gb), ctypes.byref(fp))
        return {"n_inference_nodes": n.value, "tensor_bytes": tb.value, "grad_bytes": gb.value,
                "fused_groups": fp.value}
