"""Library lifecycle on the GPU: mh_shutdown frees the library's scratch, staging and arrival
counters and destroys its stream; calls before the next mh_init fail with an error (no
crash); after mh_init the library starts clean, and ops that use scratch and counters give
the same bits as before (the one-launch bias gradient, a fused loss's in-kernel sum, a
split all-element reduction, a broadcast MUL backward through scratch)."""
from __future__ import annotations

import numpy as np
import pytest

from mantle_amd import synth
from util import GpuEngine

pytestmark = pytest.mark.gpu


def test_shutdown_then_init_again():
    eng = GpuEngine()
    m = eng.m
    tx = eng.T(synth.normal((8, 32, 28, 28), 0, 1, 1200))
    tb = eng.T(synth.normal((1, 32, 1, 1), 0, 0.1, 1201))
    tu = eng.T(synth.normal((8, 32, 28, 28), 0, 1, 1202))
    tl = eng.T(synth.normal((4099, 10), 0, 2, 1203))
    tt = eng.T(synth.uniform((4099, 10), 0, 1, 1204))
    tbig = eng.T(synth.normal((3, 700001), 0, 1, 1205))
    tw = eng.T(synth.uniform((3, 1), 0.5, 2, 1206))

    def run():
        gb = m.Tensor(tb.shape())
        m.backward_op(1, m.OP.ADD, tu, tx, tb, gb)  # bias gradient: planes and tickets
        loss = m.Tensor(m.TensorShape(1))
        m.cross_entropy_forward(loss, tl, tt)  # in-kernel loss sum: tickets
        s = m.Tensor(m.TensorShape(1))
        m.forward_op(m.OP.SUM, s, tbig)  # split partials in scratch
        gw = m.Tensor(tw.shape())
        m.backward_op(1, m.OP.MUL, tbig, tbig, tw, gw)  # broadcast MUL backward: scratch
        return [t.to_numpy() for t in (gb, loss, s, gw)]

    first = run()
    m._lib.call("mh_shutdown")
    with pytest.raises(m.MantleHipError):
        m._lib.call("mh_sync")
    m.init(0)
    second = run()
    for a, b in zip(first, second):
        assert (np.asarray(a).view(np.uint32) == np.asarray(b).view(np.uint32)).all()
    third = run()  # counters left at zero by the second run
    for a, b in zip(first, third):
        assert (np.asarray(a).view(np.uint32) == np.asarray(b).view(np.uint32)).all()
