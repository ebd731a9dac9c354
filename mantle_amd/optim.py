"""Adam over device-resident parameters: a mirror of mantle/nn/optim.mojo:51-149.

``Adam(params, lr, beta1, beta2, epsilon)`` takes a model's ``Parameters`` (its graph's
trainable parameters, get_trainable_parameters, optim.mojo:27-44) or (param, grad) ``Tensor``
pairs, and keeps
the momentum and rms tensors, zero-initialised, beside them. ``step()`` increments ``iter``
and updates every parameter with one ``mh_adam_step_multi`` launch per 80 tensors;
``zero_grad()`` zeroes the gradients (``Collection.set_zero``, collection.mojo:221-224).
"""
from __future__ import annotations

import ctypes
from typing import List, Sequence, Tuple

from . import _lib
from .tensor import Tensor


class SymbolTensors(list):
    """Adam's momentum / rms tensors, one per parameter in order; indexable by position or, for
    an Adam built from a model's parameters, by the parameter's Symbol (as the reference's
    ``optim.momentum_grads[sym]`` collections are)."""

    def __init__(self, tensors, symbols=None):
        super().__init__(tensors)
        self.symbols = list(symbols) if symbols is not None else None

    def __getitem__(self, key):
        if self.symbols is not None and hasattr(key, "name") and hasattr(key, "shape"):
            return super().__getitem__(self.symbols.index(key))
        return super().__getitem__(key)


class Adam:
    def __init__(self, params, lr: float = 0.001, beta1: float = 0.9, beta2: float = 0.999,
                 epsilon: float = 1e-8):
        """``params``: a model's ``Parameters`` (its graph's trainable parameters, as
        ``Adam[g](model.parameters, ...)`` takes them), or (param, grad) Tensor pairs."""
        self._collection = None
        self._span = None  # (params, grads, n) of a model's contiguous trainable span
        self.symbols = None  # the trainable parameters' symbols, for a model's parameters
        if hasattr(params, "tensors") and hasattr(params, "grads") and hasattr(params, "graph"):
            self._collection = params
            span = params.param_span()
            if span is not None:
                self._span = span
            self.symbols = params.graph.trainable_parameters()
            params = [(params.tensors[s], params.grads[s]) for s in self.symbols]
        self.params: List[Tuple[Tensor, Tensor]] = list(params)
        for p, g in self.params:
            if p.shape() != g.shape():
                raise _lib.MantleHipError(_lib.ERR_SHAPE, "a parameter and its gradient differ in shape")
        self.lr, self.beta1, self.beta2, self.epsilon = float(lr), float(beta1), float(beta2), float(epsilon)
        self.iter = 0
        # allocate_rms_and_momentum (optim.mojo:142-149): zero-initialised, one per parameter;
        # over a model's span, two span-sized buffers whose slices are the per-parameter tensors
        if self._span is not None:
            _, _, n = self._span
            self._m_span, self._v_span = Tensor(n), Tensor(n)
            offs = [p.ptr - self._span[0] for p, _ in self.params]
            mom = [Tensor(p.shape(), _ptr=self._m_span.ptr + o, _owner=self._m_span)
                   for (p, _), o in zip(self.params, offs)]
            rms = [Tensor(p.shape(), _ptr=self._v_span.ptr + o, _owner=self._v_span)
                   for (p, _), o in zip(self.params, offs)]
        else:
            mom = [Tensor(p.shape()) for p, _ in self.params]
            rms = [Tensor(p.shape()) for p, _ in self.params]
        self.momentum_grads = SymbolTensors(mom, self.symbols)
        self.rms_grads = SymbolTensors(rms, self.symbols)

    def zero_grad(self) -> None:
        """Adam.zero_grad (optim.mojo:90-92): parameters.grads.set_zero()."""
        if self._collection is not None:
            self._collection.grads.set_zero()
            return
        for _, g in self.params:
            g.zero()

    def step(self) -> None:
        self.iter += 1
        if self._span is not None:  # every parameter of the model in one launch
            p, g, n = self._span
            _lib.call("mh_adam_step", p, g, self._m_span.ptr, self._v_span.ptr, n, self.lr, self.beta1, self.beta2,
                      self.epsilon, self.iter)
            return
        n = len(self.params)
        if n == 0:
            return
        VP = ctypes.c_void_p * n
        ps = VP(*[p.ptr for p, _ in self.params])
        gs = VP(*[g.ptr for _, g in self.params])
        ms = VP(*[t.ptr for t in self.momentum_grads])
        vs = VP(*[t.ptr for t in self.rms_grads])
        sizes = (ctypes.c_int64 * n)(*[p.num_elements() for p, _ in self.params])
        _lib.call("mh_adam_step_multi", n, ps, gs, ms, vs, sizes, self.lr, self.beta1, self.beta2, self.epsilon,
                  self.iter)
