"""Checkpoints of a device-resident model (mantle/serialize/checkpoint.mojo, exercised as
tests/mojo/test_checkpoint.mojo does): a regression graph trains one Adam step, is saved with
and without its optimizer state, and is loaded into a fresh model; every tensor slot and Adam
state tensor comes back with the same bits, and training resumed from the file follows the
original run bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

from mantle_amd import synth
from util import GpuEngine

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def m():
    return GpuEngine().m


def _graph(m):
    """y = SUM(x * w, axis 1) + b, loss = MEAN((y - t)^2), w [1, 3] and b [1, 1] trainable."""
    g = m.Graph()
    x, t = g.input((4, 3)), g.input((4, 1))
    w = g.param((1, 3), init=[0.3, -0.2, 0.5])
    b = g.param((1, 1), init=[0.1])
    s = g.op(m.OP.SUM, g.op(m.OP.MUL, x, w), attributes={"axis": 1})
    y = g.op(m.OP.ADD, s, b)
    d = g.op(m.OP.SUB, y, t)
    loss = g.op(m.OP.MEAN, g.op(m.OP.MUL, d, d))
    g.out(y)
    g.loss(loss)
    return g


def _inputs():
    return (np.arange(12, dtype=np.float32).reshape(4, 3) * np.float32(0.1),
            np.arange(4, dtype=np.float32).reshape(4, 1))


def _bits(t):
    return t.to_numpy().view(np.uint32)


def _train_step(model, opt, x, y):
    model.forward(x, y)
    opt.zero_grad()
    model.backward()
    opt.step()


def test_save_load_plain(m, tmp_path):
    g = _graph(m)
    model = m.Model(g)
    model.forward(*_inputs())
    path = str(tmp_path / "plain.bin")
    m.save_checkpoint(path, model.parameters)
    model2 = m.Model(_graph(m))
    info = m.load_checkpoint(path, model2.parameters)
    assert info == m.CheckpointInfo(0, False)
    for s in g.symbols:  # inputs, parameters and node outputs
        assert (_bits(model2.parameters.tensors[s]) == _bits(model.parameters.tensors[s])).all(), s


def test_save_load_with_optim_and_resume(m, tmp_path):
    g = _graph(m)
    model = m.Model(g)
    opt = m.Adam(model.parameters, lr=0.01)
    x, y = _inputs()
    _train_step(model, opt, x, y)
    path = str(tmp_path / "optim.bin")
    m.save_checkpoint_with_optim(path, model.parameters, opt, iter=opt.iter)

    g2 = _graph(m)
    model2 = m.Model(g2)
    opt2 = m.Adam(model2.parameters, lr=0.01)
    info = m.load_checkpoint_with_optim(path, model2.parameters, opt2)
    assert info == m.CheckpointInfo(1, True)
    for s, s2 in zip(g.trainable_parameters(), g2.trainable_parameters()):
        assert (_bits(model2.parameters.tensors[s2]) == _bits(model.parameters.tensors[s])).all()
        assert (_bits(opt2.momentum_grads[s2]) == _bits(opt.momentum_grads[s])).all()
        assert (_bits(opt2.rms_grads[s2]) == _bits(opt.rms_grads[s])).all()
        assert np.any(opt2.rms_grads[s2].to_numpy() != 0)

    # a plain load of the same file restores the model and ignores the optimizer entries
    model3 = m.Model(_graph(m))
    assert m.load_checkpoint(path, model3.parameters) == m.CheckpointInfo(1, True)

    # resume: the next steps of the loaded run match the original run's bits
    opt2.iter = info.iter
    for k in range(2):
        xs = synth.normal((4, 3), 0, 1, 1300 + k)
        _train_step(model, opt, xs, y)
        _train_step(model2, opt2, xs, y)
    for s, s2 in zip(g.trainable_parameters(), g2.trainable_parameters()):
        assert (_bits(model2.parameters.tensors[s2]) == _bits(model.parameters.tensors[s])).all()
