"""Tensors of more than 2^31 elements (8.6 GB each, device memory only): the 64-bit index
paths of the same-shape, broadcast and reduction engines. Inputs come from the device
generator; each check downloads slices past index 2^31 (and at the start) and recomputes
them with numpy from the downloaded inputs, in the same single fp32 operations."""
from __future__ import annotations

import numpy as np
import pytest

from util import GpuEngine

pytestmark = pytest.mark.gpu

BIG = (1 << 31) + 7


@pytest.fixture(scope="module")
def m():
    print("\n[gpu] init device 0", flush=True)
    return GpuEngine().m


def _rand(m, shape, seed, lo=-1.0, hi=1.0):
    t = m.Tensor(m.TensorShape(*shape))
    m._lib.call("mh_rand_uniform", t.ptr, t.num_elements(), seed, lo, hi)
    return t


def _slice(m, t, start, count):
    """Elements [start, start + count) of t, downloaded through a view."""
    v = m.Tensor(m.TensorShape(count), _ptr=t.ptr + 4 * start, _owner=t)
    return v.to_numpy()


def test_same_shape_past_2_31(m):
    n = BIG
    print(f"[big] same shape, n = {n}", flush=True)
    a, b = _rand(m, (n,), 11), _rand(m, (n,), 12, 0.5, 2.0)
    out = m.Tensor(m.TensorShape(n))
    m.forward_op(m.OP.MUL, out, a, b)
    for start in (0, (1 << 31) - 5, n - 70):
        cnt = min(70, n - start)
        want = _slice(m, a, start, cnt) * _slice(m, b, start, cnt)
        assert (_slice(m, out, start, cnt).view(np.uint32) == want.view(np.uint32)).all(), start
    del a, b, out


def test_broadcasts_past_2_31(m):
    # columns: [R, 4096] + [1, 4096]
    R = (1 << 31) // 4096 + 1
    print(f"[big] column broadcast [{R}, 4096]", flush=True)
    x, bias = _rand(m, (R, 4096), 21), _rand(m, (1, 4096), 22)
    out = m.Tensor(m.TensorShape(R, 4096))
    m.forward_op(m.OP.ADD, out, x, bias)
    bv = bias.to_numpy().reshape(-1)
    for r in (0, R - 1):
        want = _slice(m, x, r * 4096, 4096) + bv
        assert (_slice(m, out, r * 4096, 4096).view(np.uint32) == want.view(np.uint32)).all(), r
    del x, bias, out
    # rows: [R2, 10] - [R2, 1], the per-row operands of a row max
    R2 = (1 << 31) // 10 + 1
    print(f"[big] row broadcast [{R2}, 10]", flush=True)
    y, mx = _rand(m, (R2, 10), 31), _rand(m, (R2, 1), 32)
    out = m.Tensor(m.TensorShape(R2, 10))
    m.forward_op(m.OP.SUB, out, y, mx)
    for r0 in (0, R2 - 8):
        ys = _slice(m, y, r0 * 10, 80).reshape(8, 10)
        want = ys - _slice(m, mx, r0, 8).reshape(8, 1)
        assert (_slice(m, out, r0 * 10, 80).view(np.uint32) == want.reshape(-1).view(np.uint32)).all(), r0
    del out, mx
    # reductions of the same [R2, 10]: row sums (element order) and maxima, and the maximum of
    # all elements planted past 2^31
    print("[big] reductions", flush=True)
    s = m.Tensor(m.TensorShape(R2, 1))
    m.forward_op(m.OP.SUM, s, y, attributes={"axis": 1})
    mxr = m.Tensor(m.TensorShape(R2, 1))
    m.forward_op(m.OP.MAX, mxr, y, attributes={"axis": 1})
    ys = _slice(m, y, (R2 - 8) * 10, 80).reshape(8, 10)
    want_s = np.add.accumulate(ys, axis=1, dtype=np.float32)[:, -1]
    assert (_slice(m, s, R2 - 8, 8).view(np.uint32) == want_s.view(np.uint32)).all()
    assert (_slice(m, mxr, R2 - 8, 8) == ys.max(axis=1)).all()
    n = R2 * 10
    planted = np.array([7.0], np.float32)
    m._lib.call("mh_memcpy_h2d", y.ptr + 4 * (n - 3), planted.ctypes.data, 4)
    tot = m.Tensor(m.TensorShape(1))
    m.forward_op(m.OP.MAX, tot, y)
    assert tot.to_numpy()[0] == np.float32(7.0)
    # the un-broadcast of SUB's operand 1 with ug = 1: every row's gradient is -10 exactly
    ug = m.Tensor(m.TensorShape(R2, 10))
    m._lib.call("mh_fill", ug.ptr, 1.0, n)
    g = m.Tensor(m.TensorShape(R2, 1))
    m.backward_op(1, m.OP.SUB, ug, y, mxr, g)
    for r0 in (0, R2 - 8):
        assert (_slice(m, g, r0, 8) == np.float32(-10.0)).all(), r0


def test_axis0_reduce_past_the_wide_column_grid(m):
    """Axis-0 SUM and MAX of [4, C] with C / 4 = 16 777 217 column quads: 65 537 blocks of 256,
    past the 65 535 the wide column layout can put on grid y, so the reduction takes the other
    column launch. Column slices at the start, middle and end are checked against the four
    downloaded rows: MAX bit-exact, SUM within the rtol class of the fp64 sum (4 terms)."""
    from util import assert_sum_close
    C = 67_108_868
    print(f"[big] axis-0 reduce of [4, {C}]", flush=True)
    x = _rand(m, (4, C), 41)
    s = m.Tensor(m.TensorShape(1, C))
    mx = m.Tensor(m.TensorShape(1, C))
    m.forward_op(m.OP.SUM, s, x, attributes={"axis": 0})
    m.forward_op(m.OP.MAX, mx, x, attributes={"axis": 0})
    for start in (0, C // 2 + 1, C - 70):
        rows = np.stack([_slice(m, x, r * C + start, 70) for r in range(4)])
        want_max = rows.max(axis=0)
        assert (_slice(m, mx, start, 70).view(np.uint32) == want_max.view(np.uint32)).all(), start
        seq = ((rows[0] + rows[1]) + rows[2]) + rows[3]
        r64 = rows.astype(np.float64)
        assert_sum_close(_slice(m, s, start, 70), seq, r64.sum(axis=0), f"column sums at {start}",
                         terms_abs=np.abs(r64).sum(axis=0))
