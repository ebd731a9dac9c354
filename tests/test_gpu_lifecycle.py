"""Library lifecycle on the GPU: mh_shutdown frees the library's scratch, staging and arrival
counters and destroys its stream; calls before the next mh_init fail with an error (no
crash); after mh_init the library starts clean, and ops that use scratch and counters give
the same bits as before (the one-launch bias gradient, a fused loss's in-kernel sum, a
split all-element reduction, a broadcast MUL backward through scratch)."""
from __future__ import annotations

import numpy as np
import pytest

from mantle_amd import synth
from util import TEST_ASYNC, GpuEngine

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
    m.init(0, asynchronous=TEST_ASYNC)
    second = run()
    for a, b in zip(first, second):
        assert (np.asarray(a).view(np.uint32) == np.asarray(b).view(np.uint32)).all()
    third = run()  # counters left at zero by the second run
    for a, b in zip(first, third):
        assert (np.asarray(a).view(np.uint32) == np.asarray(b).view(np.uint32)).all()


def _sequence(m, L):
    """init, a device-generated [8192, 4096] input, an axis-0 SUM (library scratch), a config-3
    shaped bias gradient (arrival counters), a download, frees and shutdown, stopping at the
    first call that fails. Returns (name of the failing call or None, its code, its message,
    the downloaded sums)."""
    import ctypes
    allocated = []
    sums = np.zeros(4096, np.float32)
    fail = (None, 0, "")

    def call(name, *args):
        rc = getattr(L, name)(*args)
        if rc != 0:
            raise _Stop(name, rc, L.mh_last_error().decode())

    try:
        call("mh_init", 0, 0)
        ptrs = {}
        for key, n in (("x", 8192 * 4096), ("res", 4096), ("ug", 8 * 32 * 28 * 28), ("gb", 32)):
            p = ctypes.c_void_p()
            call("mh_malloc", ctypes.byref(p), n * 4)
            allocated.append(p.value)
            ptrs[key] = p.value
        call("mh_rand_uniform", ptrs["x"], 8192 * 4096, 5, ctypes.c_float(-1.0), ctypes.c_float(1.0))
        call("mh_rand_normal", ptrs["ug"], 8 * 32 * 28 * 28, 6, ctypes.c_float(0.0), ctypes.c_float(1.0))
        call("mh_zero", ptrs["gb"], 32)
        sx = m.TensorShape(8192, 4096).c()
        call("mh_reduce_fwd", 8, ptrs["res"], ptrs["x"], ctypes.byref(sx), 0)
        s_ug, s_b = m.TensorShape(8, 32, 28, 28).c(), m.TensorShape(1, 32, 1, 1).c()
        call("mh_binary_bwd_accum", 0, 1, ptrs["gb"], ctypes.byref(s_b), ptrs["ug"], ctypes.byref(s_ug),
             ptrs["ug"], ctypes.byref(s_ug), ptrs["gb"], ctypes.byref(s_b))
        call("mh_memcpy_d2h", sums.ctypes.data, ptrs["res"], 4096 * 4)
    except _Stop as e:
        fail = e.args
    for p in allocated:  # a failed free is retried: each injected failure happens once
        if L.mh_free(p) != 0:
            assert L.mh_free(p) == 0
    if L.mh_shutdown() != 0:
        assert L.mh_shutdown() == 0, L.mh_last_error().decode()
    return fail + (sums,)


class _Stop(Exception):
    pass


def test_injected_hip_failures_return_cleanly():
    """MANTLE_HIP_FAIL_AT=k makes the k-th HIP runtime call after mh_init fail without being
    made. For every k up to the length of a whole sequence of library calls, exactly the call
    that reaches it returns MH_ERR_HIP with a message naming the injection (no crash, no
    fault); the frees and mh_shutdown afterwards succeed (retried once where the injection hit
    them), the device memory in use returns to its level before the loop, and a clean run
    after all of them gives the same bits as the first."""
    import ctypes
    import os
    hip = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so")

    def free_bytes():
        free, total = ctypes.c_size_t(), ctypes.c_size_t()
        assert hip.hipDeviceSynchronize() == 0
        assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
        return free.value

    eng = GpuEngine()
    m = eng.m
    L = m.lib()
    m._lib.call("mh_shutdown")
    free0 = free_bytes()
    hit = []
    try:
        os.environ["MANTLE_HIP_FAIL_AT"] = "0"
        name, code, msg, clean = _sequence(m, L)
        assert name is None, (name, code, msg)
        for k in range(1, 200):
            os.environ["MANTLE_HIP_FAIL_AT"] = str(k)
            print(f"[fail-at] k={k}", flush=True)
            name, code, msg, _ = _sequence(m, L)
            if name is None:
                break
            assert code == -7 and "injected failure" in msg, (k, name, code, msg)
            hit.append(name)
        else:
            raise AssertionError("the sequence never ran clean")
        os.environ["MANTLE_HIP_FAIL_AT"] = "0"
        name, code, msg, again = _sequence(m, L)
        assert name is None
    finally:
        os.environ.pop("MANTLE_HIP_FAIL_AT", None)
        m.init(0, asynchronous=TEST_ASYNC)
    assert (again.view(np.uint32) == clean.view(np.uint32)).all()
    # the injection reached the init, the allocations, the growth of scratch and counters and
    # the end-of-call checks
    assert {"mh_init", "mh_malloc", "mh_reduce_fwd", "mh_binary_bwd_accum"} <= set(hit), sorted(set(hit))
    drift = free0 - free_bytes()
    print(f"[fail-at] {len(hit)} injected failures, free-memory drift {drift} bytes", flush=True)
    assert drift < (8 << 20), drift


def test_graph_replay_survives_buffer_growth_and_refuses_after_shutdown():
    """A captured pass keeps using the library buffers it was captured with: an op that grows
    scratch between capture and replay (an axis-0 SUM of [8192, 8192], 4 MiB of partials) leaves
    every replay bit-identical to the eager passes. After mh_shutdown and mh_init the replay is
    refused with an error (its buffers are gone) until the pass is captured again."""
    from util import config5_nodes, native_graph
    eng = GpuEngine()
    m = eng.m
    rows = 4099
    onehot = np.zeros((rows, 10), np.float32)
    onehot[np.arange(rows), synth.integers((rows,), 0, 10, 1600)] = 1
    values = {"logits": synth.normal((rows, 10), 0, 2, 1601), "onehot": onehot}
    models = []
    for _ in range(2):
        g, syms, inputs = native_graph(m, config5_nodes(), values, ["logits"])
        g.loss(syms["loss"])
        models.append((syms, inputs, m.Model(g)))
    (syms_a, inputs, eager), (syms_b, _, graphed) = models
    big = m.Tensor(m.TensorShape(8192, 8192))
    colsum = m.Tensor(m.TensorShape(1, 8192))

    def grow():
        m.forward_op(m.OP.SUM, colsum, big, attributes={"axis": 0})

    def check(it):
        lx = synth.normal((rows, 10), 0, 2, 1610 + it)
        eager.parameters.grads.set_zero()
        la = eager.forward(lx, onehot).to_numpy()
        eager.backward()
        graphed.parameters.tensors[syms_b["logits"]] = lx
        graphed.parameters.grads.set_zero()
        lb = graphed.replay("forward").to_numpy()
        graphed.replay("backward")
        assert (lb.view(np.uint32) == la.view(np.uint32)).all(), it
        ga = eager.parameters.grads[syms_a["logits"]].to_numpy()
        gb = graphed.parameters.grads[syms_b["logits"]].to_numpy()
        assert (ga.view(np.uint32) == gb.view(np.uint32)).all(), it

    graphed.parameters.tensors[syms_b["onehot"]] = onehot  # inputs are not part of a captured pass
    graphed.capture("forward")
    grow()  # scratch grows past what the forward graph was captured with
    graphed.capture("backward")
    check(0)
    grow()
    check(1)
    m._lib.call("mh_shutdown")
    m.init(0, asynchronous=TEST_ASYNC)
    with pytest.raises(m.MantleHipError):
        graphed.replay("forward")
    graphed.capture("forward")
    graphed.capture("backward")
    check(2)


def test_async_mode_gives_the_same_bits():
    """MH_INIT_ASYNC (no stream synchronisation at the end of each call, as bench.py runs):
    op-by-op calls that grow scratch and take tickets, a native Model training step and the
    fused rows give the bits of the synchronous mode. Every host boundary (copies to and from
    the host, frees, scratch growth) synchronises by itself, so nothing else may be needed."""
    eng = GpuEngine()
    m = eng.m
    x = synth.normal((8, 32, 28, 28), 0, 1, 1300)
    b = synth.normal((1, 32, 1, 1), 0, 0.1, 1301)
    u = synth.normal((8, 32, 28, 28), 0, 1, 1302)
    logits = synth.normal((4099, 10), 0, 2, 1303)
    onehot = np.zeros((4099, 10), np.float32)
    onehot[np.arange(4099), synth.integers((4099,), 0, 10, 1304)] = 1.0
    big = synth.normal((3, 700001), 0, 1, 1305)

    def run():
        tx, tb, tu, tbig = eng.T(x), eng.T(b), eng.T(u), eng.T(big)
        gb = m.Tensor(tb.shape())
        m.backward_op(1, m.OP.ADD, tu, tx, tb, gb)
        s = m.Tensor(m.TensorShape(3))
        m.forward_op(m.OP.SUM, s, tbig, attributes={"axis": 1})
        loss = m.Tensor(m.TensorShape(1))
        m.softmax_log_mul_mean_forward(loss, eng.T(logits), eng.T(onehot))
        g = m.Graph()
        sl = g.input((4099, 10), trainable=True)
        st = g.input((4099, 10))
        mx = g.op(m.OP.MAX, sl, attributes={"axis": 1})
        e = g.op(m.OP.EXP, g.op(m.OP.SUB, sl, mx))
        sm = g.op(m.OP.DIV, e, g.op(m.OP.SUM, e, attributes={"axis": 1}))
        lo = g.op(m.OP.MEAN, g.op(m.OP.MUL, g.op(m.OP.LOG, sm), st))
        g.loss(lo)
        g.out(lo)
        model = m.Model(g)
        ml = model.forward(logits, onehot).to_numpy()
        model.backward()
        gl = model.parameters.grads[sl].to_numpy()
        return [v.to_numpy() if hasattr(v, "to_numpy") else v for v in (gb, s, loss, ml, gl)]

    sync_out = run()
    try:
        m.init(0, asynchronous=True)
        async_out = run()
    finally:
        m.init(0, asynchronous=TEST_ASYNC)
    for k, (a, c) in enumerate(zip(sync_out, async_out)):
        assert (np.asarray(a).view(np.uint32) == np.asarray(c).view(np.uint32)).all(), k


def test_trace_ranges_leave_results_unchanged():
    """MANTLE_HIP_TRACE=1 at mh_init opens a roctx range around every entry point that queues
    GPU work (nested for the executor's nodes). Without a profiler attached the ranges cost a
    call each; the results keep their bits, and turning the variable off again (at the next
    mh_init) closes nothing that was not opened."""
    import os
    eng = GpuEngine()
    m = eng.m
    a = synth.normal((1000, 37), 0, 1, 1400)
    b = synth.uniform((1000, 1), 0.5, 2, 1401)
    u = synth.normal((1000, 37), 0, 1, 1402)

    def run():
        ta, tb, tu = eng.T(a), eng.T(b), eng.T(u)
        r = m.Tensor(ta.shape())
        m.forward_op(m.OP.DIV, r, ta, tb)
        gb = m.Tensor(tb.shape())
        m.backward_op(1, m.OP.DIV, tu, ta, tb, gb)
        s = m.Tensor(m.TensorShape(1000, 1))
        m.forward_op(m.OP.MAX, s, ta, attributes={"axis": 1})
        return [t.to_numpy() for t in (r, gb, s)]

    plain = run()
    try:
        os.environ["MANTLE_HIP_TRACE"] = "1"
        m.init(0, asynchronous=TEST_ASYNC)
        traced = run()
    finally:
        os.environ.pop("MANTLE_HIP_TRACE", None)
        m.init(0, asynchronous=TEST_ASYNC)
    again = run()
    for x, y, z in zip(plain, traced, again):
        assert (x.view(np.uint32) == y.view(np.uint32)).all()
        assert (x.view(np.uint32) == z.view(np.uint32)).all()


def _device_free_bytes():
    import ctypes
    hip = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipDeviceSynchronize() == 0
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_scratch_grows_geometrically_under_a_live_graph():
    """While a captured graph exists, library scratch that grows is retired, not freed (the graph
    may still read it), until the last graph is released. Growth then at least doubles the
    buffer, so eager calls whose partials creep upward (axis-0 SUMs of [B, 8192] for B = 512 ...
    4096: 1 ... 8 MiB of partials in 0.5 MiB steps) retire buffers that together stay below the
    live one: the device's free memory drops by at most twice the largest growth in all, and
    releasing the graph gives the retired buffers back. Every sum stays right."""
    from util import config5_nodes, native_graph
    eng = GpuEngine()
    m = eng.m
    L = m.lib()
    m._lib.call("mh_shutdown")
    m.init(0, asynchronous=TEST_ASYNC)
    rows = 1025
    onehot = np.zeros((rows, 10), np.float32)
    onehot[np.arange(rows), synth.integers((rows,), 0, 10, 1620)] = 1
    values = {"logits": synth.normal((rows, 10), 0, 2, 1621), "onehot": onehot}
    g, syms, inputs = native_graph(m, config5_nodes(), values, ["logits"])
    g.loss(syms["loss"])
    model = m.Model(g)
    model.parameters.tensors[syms["onehot"]] = onehot
    model.parameters.tensors[syms["logits"]] = values["logits"]
    model.capture("forward")
    big_np = synth.normal((4096, 8192), 0, 1, 1622)
    big = eng.T(big_np)
    col = m.Tensor(m.TensorShape(1, 8192))
    free0 = _device_free_bytes()
    prev, drops = free0, []
    for b in range(512, 4097, 256):
        m._lib.check(L.mh_reduce_fwd(8, col.ptr, big.ptr, m.TensorShape(b, 8192).c(), 0), f"axis-0 SUM of [{b}, 8192]")
        f = _device_free_bytes()
        if prev - f > 0:
            drops.append(prev - f)
        prev = min(prev, f)
        if b in (512, 2048, 4096):
            ref = big_np[:b].astype(np.float64)
            np.testing.assert_allclose(col.to_numpy()[0], ref.sum(axis=0), rtol=1e-5,
                                       atol=1e-5 * float(np.abs(ref).sum(axis=0).max()))
    total = free0 - prev
    print(f"\n[growth] {len(drops)} growths {[d >> 20 for d in drops]} MiB, {total >> 20} MiB held", flush=True)
    assert len(drops) >= 2, drops
    assert total <= 2 * max(drops) + (2 << 20), (drops, total)
    lb = model.replay("forward").to_numpy()  # the graph still reads the buffers it was captured with
    la = model.forward(values["logits"], onehot).to_numpy()
    assert (lb.view(np.uint32) == la.view(np.uint32)).all()
    del model
    import gc
    gc.collect()
    back = _device_free_bytes() - prev
    assert back >= total - max(drops) - (2 << 20), (back, total, drops)
