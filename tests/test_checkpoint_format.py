"""The checkpoint file format on the host (no GPU): a save of stand-in slots produces the byte
layout of mantle/serialize/checkpoint.mojo (magic "TLSB", version 1, iter, counts, then per
entry id, kind byte, rank, dims and the little-endian fp32 elements), in the reference's entry
order; and a load rejects a bad magic, a wrong version, a file that ends inside an entry and
an entry whose size differs from its slot's, before it writes any slot."""
from __future__ import annotations

import numpy as np
import pytest

from mantle_amd import checkpoint as ck
from mantle_amd.graph import Symbol
from mantle_amd.tensor import TensorShape


class _Slot:
    """A host stand-in for a device slot: shape(), num_elements(), to_numpy(); ptr is not a
    device address, so a load that reached the upload would fail."""

    def __init__(self, data):
        self.data = np.asarray(data, np.float32)
        self.ptr = 0

    def shape(self):
        return TensorShape(*self.data.shape)

    def num_elements(self):
        return self.data.size

    def to_numpy(self):
        return self.data.copy()


class _Graph:
    def __init__(self, inputs, params, outs):
        self.inputs, self.params = inputs, params
        self.nodes = [(0, [], {}, s) for s in outs]

    def trainable_parameters(self):
        return [p for p in self.params if p.trainable]


class _Params:
    def __init__(self, graph, slots):
        self.graph, self.tensors = graph, slots


class _Adam:
    def __init__(self, symbols, mom, rms):
        self.symbols, self.momentum_grads, self.rms_grads = symbols, mom, rms


def _model():
    x = Symbol(0, TensorShape(2, 3), False)
    w = Symbol(1, TensorShape(1, 3), True)
    y = Symbol(2, TensorShape(2, 3), True)
    slots = {x: _Slot([[1, 2, 3], [4, 5, 6]]), w: _Slot([[0.5, -0.25, 2.0]]), y: _Slot(np.full((2, 3), -0.0))}
    return _Params(_Graph([x], [w], [y]), slots), w


def _u32(v):
    return int(v).to_bytes(4, "little")


def _entry(sid, kind, dims, values):
    b = _u32(sid) + bytes([kind]) + _u32(len(dims)) + b"".join(_u32(d) for d in dims)
    return b + np.asarray(values, "<f4").tobytes()


def test_save_writes_the_reference_layout(tmp_path):
    params, w = _model()
    path = str(tmp_path / "plain.bin")
    ck.save_checkpoint(path, params, iter=7)
    want = b"TLSB" + _u32(1) + _u32(7) + _u32(3) + _u32(0)
    want += _entry(0, 0, (2, 3), [1, 2, 3, 4, 5, 6])
    want += _entry(1, 0, (1, 3), [0.5, -0.25, 2.0])
    want += _entry(2, 0, (2, 3), [-0.0] * 6)
    assert open(path, "rb").read() == want


def test_save_with_optim_appends_momentum_then_rms(tmp_path):
    params, w = _model()
    adam = _Adam([w], [_Slot([[1e-3, 2e-3, 3e-3]])], [_Slot([[4e-6, 5e-6, 6e-6]])])
    path = str(tmp_path / "optim.bin")
    ck.save_checkpoint_with_optim(path, params, adam, iter=1)
    data = open(path, "rb").read()
    assert data[:20] == b"TLSB" + _u32(1) + _u32(1) + _u32(3) + _u32(2)
    tail = _entry(1, 1, (1, 3), [1e-3, 2e-3, 3e-3]) + _entry(1, 2, (1, 3), [4e-6, 5e-6, 6e-6])
    assert data.endswith(tail)


def test_save_with_optim_needs_symbols(tmp_path):
    params, _ = _model()
    with pytest.raises(ck.CheckpointError):
        ck.save_checkpoint_with_optim(str(tmp_path / "x.bin"), params, _Adam(None, [], []))


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b"XXXX" + b[4:], "bad magic"),
    (lambda b: b[:4] + _u32(2) + b[8:], "Unsupported checkpoint version: 2"),
    (lambda b: b[:-1], "Truncated"),
    (lambda b: b[:20] + _entry(0, 0, (5,), [1, 2, 3, 4, 5]) + b[20 + len(_entry(0, 0, (2, 3), [0] * 6)):],
     "holds 5 elements, its slot 6"),
])
def test_load_rejects_before_writing(tmp_path, mutate, msg):
    params, _ = _model()
    path = str(tmp_path / "ok.bin")
    ck.save_checkpoint(path, params)
    bad = str(tmp_path / "bad.bin")
    open(bad, "wb").write(mutate(open(path, "rb").read()))
    with pytest.raises(ck.CheckpointError, match=msg):
        ck.load_checkpoint(bad, params)


def test_load_skips_unknown_symbols_and_optimizer_entries(tmp_path):
    """Entries for ids the model lacks, and optimizer entries under load_checkpoint, are
    skipped (nothing to write, so the stand-in slots are never uploaded to)."""
    params, _ = _model()
    path = str(tmp_path / "other.bin")
    data = b"TLSB" + _u32(1) + _u32(3) + _u32(1) + _u32(1)
    data += _entry(99, 0, (4,), [1, 2, 3, 4]) + _entry(1, 1, (1, 3), [0, 0, 0])
    open(path, "wb").write(data)
    info = ck.load_checkpoint(path, params)
    assert info == ck.CheckpointInfo(3, True)


def test_adam_state_indexable_by_symbol():
    """Adam's momentum / rms lists answer to a parameter's Symbol as the reference's
    collections do (optim.momentum_grads[param_sym]), and to positions as before."""
    from mantle_amd.optim import SymbolTensors
    a, b = Symbol(3, TensorShape(2), True), Symbol(5, TensorShape(4), True)
    ta, tb = _Slot([1, 2]), _Slot([3, 4, 5, 6])
    st = SymbolTensors([ta, tb], [a, b])
    assert st[b] is tb and st[a] is ta and st[0] is ta and st[-1] is tb and len(st) == 2
    with pytest.raises(ValueError):
        st[Symbol(9, TensorShape(1), True)]
    plain = SymbolTensors([ta])  # built from (param, grad) pairs: positions only
    assert plain[0] is ta
