"""mh_reduce_fwd_noalloc (the no-allocation form of mh_reduce_fwd, for callers that cannot
allocate device memory) against mh_reduce_fwd through the C ABI: the same kernels, so the same
bits, on two calls in a row with the second smaller, for SUM / MEAN / MAX over axis 0, the last
axis and all elements. The library is shut down and initialised again first, so it holds no
scratch buffer; the no-allocation calls then run, and the device's free memory does not drop
across them. A small call before them has the runtime load the kernels' code object. As a
positive control, mh_reduce_fwd over axis 0 of [8192, 8192] right after them must allocate
its 8 MiB of partials, and the same probe must see that drop."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from mantle_amd import synth
from util import TEST_ASYNC, GpuEngine

pytestmark = pytest.mark.gpu

HIP = "/opt/rocm/lib/libamdhip64.so"


def _free_bytes():
    hip = ctypes.CDLL(HIP)
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


@pytest.mark.parametrize("axis_kind", ["axis0", "last", "all"])
def test_noalloc_matches_reduce_fwd(axis_kind):
    print(f"\n[noalloc] {axis_kind}", flush=True)
    eng = GpuEngine()
    m = eng.m
    L = m.lib()
    big = m.Tensor(m.TensorShape(8192, 8192))
    m._lib.call("mh_rand_normal", big.ptr, big.num_elements(), 77, 0.0, 1.0)
    small_np = synth.normal((777, 300), 0, 1, 78)
    small = eng.T(small_np)
    cases = [(big, (8192, 8192)), (small, (777, 300))]  # the second call is smaller
    axis = {"axis0": 0, "last": 1, "all": -1}[axis_kind]
    outs = {}
    for op in (8, 9, 10):  # SUM, MEAN, MAX
        for k, (t, shape) in enumerate(cases):
            rshape = (1,) if axis < 0 else tuple(1 if i == axis else d for i, d in enumerate(shape))
            r = m.Tensor(m.TensorShape(*rshape))
            outs[(op, k)] = r
    warm = m.Tensor(m.TensorShape(1))
    # an empty library: earlier calls in this process may have grown its scratch, which
    # mh_shutdown frees (device tensors stay valid across it)
    m._lib.call("mh_shutdown")
    m.init(0, asynchronous=TEST_ASYNC)
    # one small call first: the HIP runtime loads a module's code object on the first launch of
    # one of its kernels, which takes device memory once per process (not the entry point's)
    m._lib.check(L.mh_reduce_fwd_noalloc(8, warm.ptr, small.ptr, m.TensorShape(777 * 300).c(), -1), "warm-up")
    f1 = _free_bytes()  # result tensors allocated above, outside the measured span
    for op in (8, 9, 10):
        for k, (t, shape) in enumerate(cases):
            m._lib.check(L.mh_reduce_fwd_noalloc(op, outs[(op, k)].ptr, t.ptr, m.TensorShape(*shape).c(), axis),
                         f"noalloc op {op} call {k}")
    f2 = _free_bytes()
    assert f1 - f2 < (1 << 20), f"free memory dropped by {f1 - f2} bytes across the no-allocation calls"
    # positive control: the allocating form grows the (empty) library scratch by its partials
    col = m.Tensor(m.TensorShape(1, 8192))
    f3 = _free_bytes()
    m._lib.check(L.mh_reduce_fwd(8, col.ptr, big.ptr, m.TensorShape(8192, 8192).c(), 0), "reduce_fwd axis 0")
    f4 = _free_bytes()
    assert f3 - f4 >= (4 << 20), f"mh_reduce_fwd's partials were not seen: free memory dropped by {f3 - f4} bytes"
    for op in (8, 9, 10):
        for k, (t, shape) in enumerate(cases):
            got = outs[(op, k)].to_numpy()
            ref = m.Tensor(outs[(op, k)].shape())
            m._lib.check(L.mh_reduce_fwd(op, ref.ptr, t.ptr, m.TensorShape(*shape).c(), axis), "reduce_fwd")
            assert (got.view(np.uint32) == ref.to_numpy().view(np.uint32)).all(), (axis_kind, op, k)


def test_noalloc_rejects_partials_beyond_its_scratch():
    eng = GpuEngine()
    m = eng.m
    L = m.lib()
    x = m.Tensor(m.TensorShape(4))
    res = m.Tensor(m.TensorShape(1))
    # an all-element reduction of 2^34 elements would need 32 MiB of chunk partials: refused on
    # the host before any device work (x is never read)
    rc = L.mh_reduce_fwd_noalloc(8, res.ptr, x.ptr, m.TensorShape(1 << 34).c(), -1)
    assert rc == m._lib.ERR_OVERFLOW
    assert b"no-allocation scratch" in L.mh_last_error()
