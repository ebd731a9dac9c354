"""Checkpoints of device-resident models in the reference's native binary format: a mirror of
mantle/serialize/checkpoint.mojo:196-419 (save_checkpoint, save_checkpoint_with_optim,
load_checkpoint, load_checkpoint_with_optim, CheckpointInfo).

File layout (checkpoint.mojo:25-38, 81-108; every integer little-endian):

    u32 magic 0x42534C54, u32 version 1, u32 iter, u32 model tensors, u32 optimizer entries
    per entry: u32 symbol id, u8 kind (0 tensor, 1 momentum, 2 rms), u32 rank,
               rank x u32 dims, then the fp32 elements

Model tensors are written in the order the reference's Model allocates them (inputs,
parameters, node outputs; model.mojo:332-372), then every momentum entry, then every rms
entry, each in trainable-parameter order. A load matches entries to slots by symbol id and
skips ids the model does not have, as the reference does. The tensors live in device arenas,
so a save downloads each slot and a load uploads into it (mh_memcpy_d2h / mh_memcpy_h2d).

Where the reference would read or write out of bounds, this raises CheckpointError: an
entry whose element count differs from its slot's, and a file that ends inside an entry.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass
from typing import List, Sequence, Tuple

import numpy as np

from . import _lib
from .tensor import Tensor

CHECKPOINT_MAGIC = 0x42534C54
CHECKPOINT_VERSION = 1
OPTIM_KIND_NONE = 0
OPTIM_KIND_MOMENTUM = 1
OPTIM_KIND_RMS = 2


class CheckpointError(ValueError):
    """A file that is not a readable checkpoint for the given model."""


@dataclass
class CheckpointInfo:
    """checkpoint.mojo:169-194: the stored optimizer step count, and whether the file holds
    Adam momentum / rms entries."""

    iter: int
    has_optim_state: bool


def _model_entries(parameters) -> List[Tuple[int, Tensor]]:
    """(symbol id, slot) of every model tensor in allocation order."""
    g = parameters.graph
    syms = list(g.inputs) + list(g.params) + [node[3] for node in g.nodes]
    return [(s.name, parameters.tensors[s]) for s in syms]


def _optim_entries(optim, kind: int) -> List[Tuple[int, Tensor]]:
    syms = getattr(optim, "symbols", None)
    if syms is None:
        raise CheckpointError("optimizer state has no symbol ids: build Adam from a model's parameters")
    tensors = optim.momentum_grads if kind == OPTIM_KIND_MOMENTUM else optim.rms_grads
    return [(s.name, t) for s, t in zip(syms, tensors)]


def _write_entry(f, symbol_id: int, kind: int, t: Tensor) -> None:
    """checkpoint.mojo:81-108: the header, then the slot's elements downloaded and written as
    they are (little-endian fp32, no second host copy)."""
    dims = t.shape().dims
    f.write(struct.pack("<IBI", symbol_id, kind, len(dims)) + struct.pack(f"<{len(dims)}I", *dims))
    a = np.ascontiguousarray(t.to_numpy(), dtype="<f4").reshape(-1)
    if a.size:
        f.write(memoryview(a).cast("B"))


def _write(path: str, iter: int, model: Sequence[Tuple[int, Tensor]],
           optim: Sequence[Tuple[int, int, Tensor]]) -> None:
    with open(path, "wb") as f:
        f.write(struct.pack("<5I", CHECKPOINT_MAGIC, CHECKPOINT_VERSION, int(iter), len(model), len(optim)))
        for sid, t in model:
            _write_entry(f, sid, OPTIM_KIND_NONE, t)
        for sid, kind, t in optim:
            _write_entry(f, sid, kind, t)


def save_checkpoint(path: str, parameters, iter: int = 0) -> None:
    """save_checkpoint (checkpoint.mojo:196-230): every model tensor, no optimizer state."""
    _write(path, iter, _model_entries(parameters), [])


def save_checkpoint_with_optim(path: str, parameters, optim, iter: int = 0) -> None:
    """save_checkpoint_with_optim (checkpoint.mojo:233-290), with ``optim`` an Adam built from
    the model's parameters: its momentum and rms tensors follow the model tensors."""
    opt = [(sid, OPTIM_KIND_MOMENTUM, t) for sid, t in _optim_entries(optim, OPTIM_KIND_MOMENTUM)]
    opt += [(sid, OPTIM_KIND_RMS, t) for sid, t in _optim_entries(optim, OPTIM_KIND_RMS)]
    _write(path, iter, _model_entries(parameters), opt)


class _Reader:
    def __init__(self, data: bytes, path: str):
        self.data, self.off, self.path = data, 0, path

    def take(self, n: int) -> bytes:
        if self.off + n > len(self.data):
            raise CheckpointError(f"Truncated checkpoint file: {self.path}")
        b = self.data[self.off:self.off + n]
        self.off += n
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def entry(self) -> Tuple[int, int, Tuple[int, ...], bytes]:
        """checkpoint.mojo:111-134 and the entry's element bytes."""
        sid = self.u32()
        kind = self.take(1)[0]
        rank = self.u32()
        dims = tuple(self.u32() for _ in range(rank))
        n = 1
        for d in dims:
            n *= d
        return sid, kind, dims, self.take(4 * n)


def _header(r: _Reader) -> Tuple[int, int, int]:
    if r.u32() != CHECKPOINT_MAGIC:
        raise CheckpointError(f"Not a mantle checkpoint file (bad magic): {r.path}")
    version = r.u32()
    if version != CHECKPOINT_VERSION:
        raise CheckpointError(f"Unsupported checkpoint version: {version}")
    return r.u32(), r.u32(), r.u32()  # iter, tensors, optimizer entries


def _read(path: str, parameters, optim) -> CheckpointInfo:
    """checkpoint.mojo:137-166, 313-343, 371-419: every entry is matched to the slot of its
    symbol id (skipped when the model has none; optimizer entries are skipped without
    ``optim``). The whole file is parsed and checked before any slot is written."""
    with open(path, "rb") as f:
        r = _Reader(f.read(), path)
    it, ntensors, noptim = _header(r)
    model = dict(_model_entries(parameters))
    mom = dict(_optim_entries(optim, OPTIM_KIND_MOMENTUM)) if optim is not None else {}
    rms = dict(_optim_entries(optim, OPTIM_KIND_RMS)) if optim is not None else {}
    writes = []
    for i in range(ntensors + noptim):
        sid, kind, _, raw = r.entry()
        slots = model if i < ntensors else (mom if kind == OPTIM_KIND_MOMENTUM else rms)
        t = slots.get(sid)
        if t is None:
            continue
        if len(raw) != 4 * t.num_elements():
            raise CheckpointError(f"checkpoint entry for symbol {sid} holds {len(raw) // 4} elements, "
                                  f"its slot {t.num_elements()}")
        writes.append((t, raw))
    for t, raw in writes:
        a = np.frombuffer(raw, dtype="<f4")
        if a.size:
            _lib.call("mh_memcpy_h2d", t.ptr, a.ctypes.data, a.size * 4)
    return CheckpointInfo(it, noptim > 0)


def load_checkpoint(path: str, parameters) -> CheckpointInfo:
    """load_checkpoint (checkpoint.mojo:293-343): model tensors only; optimizer entries are
    skipped."""
    return _read(path, parameters, None)


def load_checkpoint_with_optim(path: str, parameters, optim) -> CheckpointInfo:
    """load_checkpoint_with_optim (checkpoint.mojo:346-419): model tensors and, when the file
    has them, Adam's momentum and rms (kind 1 is momentum, any other kind rms, as in the
    reference). The caller sets ``optim.iter`` from the returned info."""
    return _read(path, parameters, optim)
