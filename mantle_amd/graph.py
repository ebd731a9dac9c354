"""Graph builder: a mirror of mantle/autograd/graph.mojo:33-217 on the native graph of
libmantle_hip.so (mh_graph_*).

``Graph`` records inputs, parameters and op nodes in creation order (a topological order);
``op`` computes the result shape as static_result_shape does and marks the result trainable
when any operand is. Symbols are numbered in creation order, like ``Symbol.name``. The
graph is host-only: building one needs no device.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence, Union

import numpy as np

from . import _lib
from .tensor import TensorShape, as_shape


class Symbol:
    """Symbol (mantle/autograd/symbol.mojo:21-45): id, shape and trainable flag."""

    __slots__ = ("name", "shape", "trainable")

    def __init__(self, name: int, shape: TensorShape, trainable: bool):
        self.name, self.shape, self.trainable = int(name), shape, bool(trainable)

    def __eq__(self, other) -> bool:
        return isinstance(other, Symbol) and other.name == self.name

    def __hash__(self) -> int:
        return hash(self.name)

    def __repr__(self) -> str:
        return f"Symbol(s{self.name}, {self.shape}, trainable={self.trainable})"


def make_attrs(attributes: Optional[Dict]) -> Optional[_lib.mh_attrs]:
    """AttributeVector -> mh_attrs: keys "axis", "negative_slope", "min", "max"."""
    if not attributes:
        return None
    a = _lib.mh_attrs()
    for k, v in attributes.items():
        if v is None:
            continue
        if k == "axis":
            a.flags |= _lib.ATTR_AXIS
            a.axis = int(v)
        elif k == "negative_slope":
            a.flags |= _lib.ATTR_NEGATIVE_SLOPE
            a.negative_slope = float(v)
        elif k == "min":
            a.flags |= _lib.ATTR_MIN
            a.min_val = float(v)
        elif k == "max":
            a.flags |= _lib.ATTR_MAX
            a.max_val = float(v)
        else:
            raise _lib.MantleHipError(_lib.ERR_INVALID, f"attribute {k!r} is not used by the ops of this path")
    return a


class Graph:
    def __init__(self):
        h = ctypes.c_void_p()
        _lib.call("mh_graph_create", ctypes.byref(h))
        self._h = h.value
        self.inputs: List[Symbol] = []
        self.params: List[Symbol] = []
        self.outputs: List[Symbol] = []
        self.loss_out: Optional[Symbol] = None
        self.nodes: List[tuple] = []  # (op, operands, attributes, result)
        self.symbols: List[Symbol] = []

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.lib().mh_graph_destroy(h)
            except Exception:
                pass
            self._h = None

    @property
    def handle(self) -> int:
        return self._h

    @property
    def symbol_count(self) -> int:
        return len(self.symbols)

    def _new(self, sid: int) -> Symbol:
        shp = _lib.mh_shape()
        tr = ctypes.c_int()
        _lib.call("mh_graph_symbol", self._h, sid, ctypes.byref(shp), ctypes.byref(tr), None)
        s = Symbol(sid, TensorShape(*[shp.dims[i] for i in range(shp.rank)]), bool(tr.value))
        assert sid == len(self.symbols)
        self.symbols.append(s)
        return s

    # graph.mojo:85-102
    def input(self, shape, trainable: bool = False) -> Symbol:
        sid = ctypes.c_int32()
        _lib.call("mh_graph_input", self._h, as_shape(shape).c(), int(trainable), ctypes.byref(sid))
        s = self._new(sid.value)
        self.inputs.append(s)
        return s

    def param(self, shape, init=None, trainable: bool = True) -> Symbol:
        """A parameter: zero-initialised, or holding ``init`` (array-like of the shape's size)."""
        shape = as_shape(shape)
        sid = ctypes.c_int32()
        if init is None:
            _lib.call("mh_graph_param", self._h, shape.c(), int(trainable), None, 0, ctypes.byref(sid))
        else:
            d = np.ascontiguousarray(init, dtype=np.float32).reshape(-1)
            _lib.call("mh_graph_param", self._h, shape.c(), int(trainable), d.ctypes.data, d.size, ctypes.byref(sid))
        s = self._new(sid.value)
        self.params.append(s)
        return s

    def scalar(self, value: float) -> Symbol:
        sid = ctypes.c_int32()
        _lib.call("mh_graph_scalar", self._h, float(value), ctypes.byref(sid))
        s = self._new(sid.value)
        self.params.append(s)
        return s

    def constant(self, shape, data) -> Symbol:
        return self.param(shape, init=data, trainable=False)

    def out(self, symbol: Symbol) -> None:
        _lib.call("mh_graph_out", self._h, symbol.name)
        self.outputs.append(symbol)

    def loss(self, symbol: Symbol) -> None:
        _lib.call("mh_graph_loss", self._h, symbol.name)
        self.loss_out = symbol

    # graph.mojo:110-157: operands are symbols, or floats that become graph scalars
    def op(self, op: int, *operands: Union[Symbol, float], attributes: Optional[Dict] = None) -> Symbol:
        syms = [o if isinstance(o, Symbol) else self.scalar(float(o)) for o in operands]
        arr = (ctypes.c_int32 * max(len(syms), 1))(*[s.name for s in syms])
        at = make_attrs(attributes)
        sid = ctypes.c_int32()
        _lib.call("mh_graph_op", self._h, int(op), len(syms), arr, ctypes.byref(at) if at is not None else None,
                  ctypes.byref(sid))
        s = self._new(sid.value)
        self.nodes.append((int(op), syms, dict(attributes or {}), s))
        return s

    def trainable_parameters(self) -> List[Symbol]:
        """get_trainable_parameters (optim.mojo:27-44)."""
        return [p for p in self.params if p.trainable]
