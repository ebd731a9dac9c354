"""Device-resident Tensor[f32] and TensorShape, mirroring mantle/core/tensor.mojo.

The reference keeps tensors in host memory (``Tensor`` allocates with ``alloc`` and zero-fills,
tensor.mojo:250-302). Here the storage is HBM on the initialised gfx950 device
(``mh_malloc`` + a zero-fill kernel); host copies are explicit (``from_numpy`` /
``to_numpy``), so chains of ops never cross PCIe.
"""
from __future__ import annotations

import ctypes
from typing import Iterable, Optional, Tuple, Union

import numpy as np

from . import _lib

MAX_RANK = _lib.MAX_RANK

_initialized = False


def init(device: int = 0, asynchronous: bool = False) -> None:
    """Initialise the library on `device` (idempotent)."""
    global _initialized
    _lib.call("mh_init", int(device), _lib.INIT_ASYNC if asynchronous else 0)
    _initialized = True


def ensure_init() -> None:
    if not _initialized:
        init(0)


def sync() -> None:
    _lib.call("mh_sync")


class TensorShape:
    """Row-major shape of rank 1..8 (tensor.mojo:28-229)."""

    __slots__ = ("_dims",)

    def __init__(self, *dims: Union[int, Iterable[int]]):
        if len(dims) == 1 and not isinstance(dims[0], (int, np.integer)):
            dims = tuple(dims[0])
        d = tuple(int(x) for x in dims)
        if not 1 <= len(d) <= MAX_RANK:
            raise ValueError(f"rank {len(d)} outside 1..{MAX_RANK}")
        self._dims = d

    def rank(self) -> int:
        return len(self._dims)

    def num_elements(self) -> int:
        n = 1
        for x in self._dims:
            n *= x
        return n

    def strides(self) -> Tuple[int, ...]:  # tensor.mojo:143-155
        st, s = [], 1
        for x in reversed(self._dims):
            st.append(s)
            s *= x
        return tuple(reversed(st))

    @property
    def dims(self) -> Tuple[int, ...]:
        return self._dims

    def __getitem__(self, i: int) -> int:
        return self._dims[i]

    def __len__(self) -> int:
        return len(self._dims)

    def __eq__(self, other) -> bool:
        if isinstance(other, TensorShape):
            return self._dims == other._dims
        if isinstance(other, tuple):
            return self._dims == other
        return NotImplemented

    def __hash__(self):
        return hash(self._dims)

    def __repr__(self) -> str:
        return "TensorShape(" + ", ".join(str(x) for x in self._dims) + ")"

    def c(self) -> _lib.mh_shape:
        return _lib.make_shape(self._dims)


def as_shape(s) -> TensorShape:
    return s if isinstance(s, TensorShape) else TensorShape(s)


class Tensor:
    """fp32 tensor in device memory. ``share()`` aliases, ``copy()`` deep-copies
    (tensor.mojo:345-393)."""

    __slots__ = ("_shape", "_ptr", "_owner", "__weakref__")

    def __init__(self, *shape, _ptr: Optional[int] = None, _owner=None):
        ensure_init()
        self._shape = as_shape(shape[0]) if len(shape) == 1 and not isinstance(shape[0], (int, np.integer)) \
            else TensorShape(*shape)
        if _ptr is not None:
            self._ptr, self._owner = _ptr, _owner
            return
        p = ctypes.c_void_p()
        n = self._shape.num_elements()
        _lib.call("mh_malloc", ctypes.byref(p), max(n, 1) * 4)
        self._ptr, self._owner = p.value, None
        _lib.call("mh_zero", self._ptr, n)  # zero-initialised, tensor.mojo:266, 284

    def __del__(self):
        if getattr(self, "_owner", 1) is None and getattr(self, "_ptr", None):
            try:
                _lib.lib().mh_free(self._ptr)
            except Exception:
                pass
            self._ptr = None

    # ---- properties ----
    def shape(self) -> TensorShape:
        return self._shape

    def num_elements(self) -> int:
        return self._shape.num_elements()

    def rank(self) -> int:
        return self._shape.rank()

    def dim(self, i: int) -> int:
        return self._shape[i]

    @property
    def ptr(self) -> int:
        return self._ptr

    # ---- host transfer ----
    @staticmethod
    def from_numpy(a) -> "Tensor":
        a = np.ascontiguousarray(a, dtype=np.float32)
        t = Tensor(TensorShape(a.shape if a.ndim else (1,)))
        if a.size:
            _lib.call("mh_memcpy_h2d", t._ptr, a.ctypes.data, a.size * 4)
        return t

    def to_numpy(self) -> np.ndarray:
        out = np.empty(self._shape.dims, dtype=np.float32)
        if out.size:
            _lib.call("mh_memcpy_d2h", out.ctypes.data, self._ptr, out.size * 4)
        return out

    # ---- tensor.mojo API ----
    def copy(self) -> "Tensor":
        t = Tensor(self._shape)
        _lib.call("mh_memcpy_d2d", t._ptr, self._ptr, self.num_elements() * 4)
        return t

    def share(self) -> "Tensor":
        return Tensor(self._shape, _ptr=self._ptr, _owner=self)

    def zero(self) -> None:
        _lib.call("mh_zero", self._ptr, self.num_elements())

    def __getitem__(self, i: int) -> float:
        v = np.empty(1, dtype=np.float32)
        _lib.call("mh_memcpy_d2h", v.ctypes.data, self._ptr + 4 * int(i), 4)
        return float(v[0])

    def __setitem__(self, i: int, val: float) -> None:
        v = np.array([val], dtype=np.float32)
        _lib.call("mh_memcpy_h2d", self._ptr + 4 * int(i), v.ctypes.data, 4)

    def __repr__(self) -> str:
        return f"Tensor({self._shape})"
