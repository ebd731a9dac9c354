"""Benchmark: Mantle's elementwise / broadcast / reduction op layer on one MI355X.

The headline line is config 2 of BASELINE.json. A step is one forward + backward pass of
every config-2 op over 2^28-element fp32 tensors already resident in HBM:
  ADD/SUB/MUL/DIV   fwd (a ~ U(-1,1), b ~ U(0.5,2)) and the backward of both operands,
  EXP (x ~ U(-10,10)), LOG (x ~ U(1e-3,10)), TANH/SIGMOID/RELU (x ~ N(0,3))  fwd and bwd,
  POW (base ~ U(0.1,4), one seeded scalar exponent ~ U(0.5,3))  fwd, and the backward of x and of
      the exponent (one pass: both operands trainable, as the binary ops' backward).
Throughput is algorithmic bytes per step / step time (each input read once, each output
written once, each accumulated gradient read and written). Per-op times come from HIP events
recorded on the library's stream around each call.

The other configs are measured after the headline step and reported under "workloads"
(per op: ms, GB/s of algorithmic bytes, fraction of 8 TB/s):
  c3  NCHW bias + RELU, [256,32,28,28] + [1,32,1,1]: fused and op-by-op, fwd and bwd;
  c4  SUM/MEAN/MAX over axis 0, axis 1 and all of [8192,8192] (ties injected in half the
      lines) and over the last axis of [64,512,1024], fwd and bwd;
  c5  classifier head on logits [1048576,10]: MAX -> SUB -> EXP -> SUM -> DIV -> LOG ->
      MUL(onehot) -> MEAN, forward and backward op by op (the drop-in path), and the same graph
      row-fused (one kernel each way, caches flushed before each);
  adam  Adam.step (mantle/nn/optim.mojo:94-140) on one 2^28-element parameter and on 400
        tensors through the multi-tensor entry point, 28 B/elem;
  adj   FMA / LEAKYRELU / CLIP forward and backward over 2^28 elements, and tstd over
        [8192, 8192] (axis 0, axis 1, all);
  rows  row-fused CrossEntropyLoss ([2^20, 10], [32768, 1000]), Softmax and LogSoftmax
        ([32768, 1000]), forward and backward;
  graph a training step (zero_grad, forward, backward) through the native Model, eager against
        HIP-graph replay, for config 1's graph (with a MEAN loss) and config 5's chain;
  copy  the library's copy kernel over 1 GiB and over one config-3 and one config-5 tensor,
        and an all-element SUM (a read-only pass) over one config-3 tensor, one config-5
        tensor and the config-5 head's 84 MB: the practical streaming rates at those sizes.
Workload ops (c3, c4, c5 op by op and fused, rows) get two figures:
  ms            streamed: R launches back to back on the stream over S buffer sets (S copies
                of the op's tensors, S chosen so that the other sets' traffic between two
                uses of one set is at least twice the 256 MB Infinity Cache, so every launch
                reads cold operands), after a cache flush long enough for the host to queue
                all R launches behind it; ms = elapsed / R. This is the op's rate inside a
                step, where launches follow each other;
  ms_isolated   one launch on set 0 between two events, the caches flushed before it (a 1 GiB
                read sweep outside the events): it adds the event and dispatch latency of a
                lone launch, which the copy workload's `isolated_floor_ms` (a one-element
                fill timed this way) shows.
`frac` uses ms, `frac_isolated` ms_isolated. The model / chain / adam / adj / graph timings
are single bracketed launches or passes as described at each.

`roofline.traffic` is filled from profiles/traffic.json when that summary of the rocprofv3
FETCH_SIZE / WRITE_SIZE runs is present (see `--pmc-summary`), else null.

Prints one JSON line. `--gpus N` with N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import csv
import ctypes
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "elementwise/broadcast/reduce fwd+bwd: achieved HBM GB/s and % of MI355X peak"
PEAK_GBS = 8000.0
SEED = 42
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic.json")

BINARY = ["ADD", "SUB", "MUL", "DIV"]
UNARY = ["EXP", "LOG", "TANH", "SIGMOID", "RELU"]
OP_ID = {"ADD": 0, "SUB": 1, "MUL": 2, "DIV": 3, "EXP": 4, "LOG": 5, "POW": 6, "SUM": 8, "MEAN": 9, "MAX": 10,
         "SIGMOID": 13, "RELU": 14, "TANH": 15}
BWD2_BYTES = {"ADD": 20, "SUB": 20, "MUL": 28, "DIV": 28}  # ug (+a, b), both grads read+written


def step_plan():
    """Config 2: [(label, algorithmic bytes per element)] in execution order."""
    plan = []
    for op in BINARY:
        plan += [(f"{op}.fwd", 12), (f"{op}.bwd", BWD2_BYTES[op])]
    for op in UNARY:
        plan += [(f"{op}.fwd", 8), (f"{op}.bwd", 16)]
    # POW backward of both operands in one pass: x and ug read, grad_x read and written (the
    # exponent's gradient is a scalar)
    plan += [("POW.fwd", 8), ("POW.bwd", 16)]
    return plan


def chk(L, rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: [{rc}] {L.mh_last_error().decode()}")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Dev:
    """Device buffers (raw mh_malloc pointers), events and the cache flush of one run."""

    def __init__(self, L):
        self.L, self.ptrs, self.evs = L, {}, []
        self._flush = None

    def alloc(self, name, n):
        p = ctypes.c_void_p()
        chk(self.L, self.L.mh_malloc(ctypes.byref(p), max(int(n), 1) * 4), f"mh_malloc({name})")
        self.ptrs[name] = p.value
        return p.value

    def upload(self, name, arr):
        arr = np.ascontiguousarray(arr, np.float32)
        p = self.alloc(name, arr.size)
        chk(self.L, self.L.mh_memcpy_h2d(p, arr.ctypes.data, arr.size * 4), f"h2d {name}")
        return p

    def zeros(self, name, n):
        p = self.alloc(name, n)
        chk(self.L, self.L.mh_zero(p, n), f"zero {name}")
        return p

    def event(self):
        e = ctypes.c_void_p()
        chk(self.L, self.L.mh_event_create(ctypes.byref(e)), "event")
        self.evs.append(e.value)
        return e.value

    def flush(self):
        """Reads 1 GiB (a SUM over a buffer 4x the 256 MB Infinity Cache) so that no operand
        of the next op is cached. A read sweep leaves clean lines: a write sweep would leave
        dirty ones whose write-back the next op would pay for."""
        from mantle_amd._lib import make_shape
        if self._flush is None:
            self._flush = self.zeros("_flush", 1 << 28)
            self._flush_out = self.zeros("_flush_out", 1)
            self._flush_shape = make_shape((1 << 28,))
        chk(self.L, self.L.mh_reduce_fwd(8, self._flush_out, self._flush, self._flush_shape, -1), "flush")

    def free(self):
        for p in self.ptrs.values():
            self.L.mh_free(p)
        for e in self.evs:
            self.L.mh_event_destroy(e)
        self.ptrs, self.evs, self._flush = {}, [], None


def time_ops(d, ops, reps, flush=True, setup=None):
    """ops: [(label, fn, bytes)]. Each op timed alone between two events; with `flush`,
    the caches are flushed before it. `setup()` runs (untimed) before every repetition.
    Returns {label: median ms} and the summed medians."""
    L = d.L
    evs = [(d.event(), d.event()) for _ in ops]
    times = {label: [] for label, _, _ in ops}
    ms = ctypes.c_float()
    for _ in range(reps + 1):  # the first repetition is a warm-up
        if setup:
            setup()
            d.flush()  # the first op does not pay for the write-back of the setup's stores
        for (label, fn, _), (e0, e1) in zip(ops, evs):
            if flush:
                d.flush()
            chk(L, L.mh_event_record(e0), "record")
            chk(L, fn(), label)
            chk(L, L.mh_event_record(e1), "record")
        chk(L, L.mh_sync(), "sync")
        for (label, _, _), (e0, e1) in zip(ops, evs):
            chk(L, L.mh_event_elapsed_ms(ctypes.byref(ms), e0, e1), "elapsed")
            times[label].append(ms.value)
    return {k: statistics.median(v[1:]) for k, v in times.items()}


MALL_BYTES = 256 << 20  # MI355X Infinity Cache


def replicate(d, names, min_bytes_per_op):
    """Buffer sets for streamed timing: set 0 is d.ptrs, sets 1.. hold device copies of the
    named buffers (other names shared). The count makes the traffic of the other sets'
    launches between two uses of one set at least twice the Infinity Cache for the lightest
    op, so that every launch reads operands evicted from every cache."""
    L = d.L
    count = max(2, 1 + -(-2 * MALL_BYTES // int(min_bytes_per_op)))
    sizes = {name: n for name, n in names}
    sets = [dict(d.ptrs)]
    for s in range(1, count):
        P = dict(d.ptrs)
        for name, n in sizes.items():
            q = d.alloc(f"{name}#{s}", n)
            chk(L, L.mh_memcpy_d2d(q, d.ptrs[name], 4 * n), f"copy {name}")
            P[name] = q
        sets.append(P)
    chk(L, L.mh_sync(), "sync")
    return sets


def time_ops_streamed(d, ops, sets, reps, min_launches=24):
    """ops: [(label, fn(P), bytes)]. Per op: R launches back to back on the stream, launch i
    on buffer set i % len(sets), between two events after a flush of the caches; the figure
    is elapsed / R, the median over `reps` such regions (after one warm-up region). The
    flush runs long enough for the host to queue all R launches behind it (it is repeated
    when queueing took longer in the warm-up), so the GPU never waits for the host: this is
    the op's rate inside a step, where launches follow each other on the stream, without
    the event and dispatch latency of a single bracketed launch."""
    L = d.L
    S = len(sets)
    R = S * max(1, -(-min_launches // S))
    e0, e1 = d.event(), d.event()
    ms = ctypes.c_float()
    out = {}
    t0 = time.perf_counter()
    d.flush()
    chk(L, L.mh_sync(), "sync")
    flush_s = time.perf_counter() - t0
    for label, fn, _ in ops:
        nflush, vals = 1, []
        for rep in range(reps + 1):
            for _ in range(nflush):
                d.flush()
            chk(L, L.mh_event_record(e0), "record")
            th = time.perf_counter()
            for i in range(R):
                chk(L, fn(sets[i % S]), label)
            host_s = time.perf_counter() - th
            chk(L, L.mh_event_record(e1), "record")
            chk(L, L.mh_sync(), "sync")
            chk(L, L.mh_event_elapsed_ms(ctypes.byref(ms), e0, e1), "elapsed")
            if rep == 0:
                nflush = 1 + int(1.5 * host_s / max(flush_s, 1e-6))
            else:
                vals.append(ms.value / R)
        out[label] = statistics.median(vals)
    return out


def isolated_floor(d, reps):
    """The isolated method's floor: a one-element fill timed like an op (flush, then one
    launch between two events)."""
    L = d.L
    buf = d.zeros("_floor", 1)
    med = time_ops(d, [("floor", lambda: L.mh_fill(buf, 0.0, 1), 4)], reps)
    return round(med["floor"], 4)


def op_report(ops, med, iso=None, hbm=None):
    """Per op: ms, GB/s and frac of its algorithmic bytes; with `iso`, the isolated figures.
    With `hbm` ({label: bytes}): ops that move fewer bytes than the algorithmic count (a sparse
    accumulation that stores only the quads it changes) report GB/s and frac over the bytes
    they move, which cannot pass the peak, and the algorithmic rate beside them as
    GB/s_effective / frac_effective."""
    out = {}
    for label, _, nbytes in ops:
        t = med[label]
        moved = hbm[label] if hbm and label in hbm else nbytes
        gbs = moved / (t * 1e-3) / 1e9
        out[label] = {"ms": round(t, 4), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        if iso is not None:
            ti = iso[label]
            out[label]["ms_isolated"] = round(ti, 4)
            out[label]["frac_isolated"] = round(moved / (ti * 1e-3) / 1e9 / PEAK_GBS, 4)
        if moved != nbytes:
            eg = nbytes / (t * 1e-3) / 1e9
            out[label].update({"algorithmic_bytes": nbytes, "hbm_bytes": moved, "GB/s_effective": round(eg, 1),
                               "frac_effective": round(eg / PEAK_GBS, 4)})
    return out


def total_report(ops, med, iso=None, hbm=None):
    """Sum over ops of op_report's bytes (moved bytes for sparse ops) and times."""
    tot_b = sum(hbm[label] if hbm and label in hbm else b for label, _, b in ops)
    tot_t = sum(med[label] for label, _, _ in ops)
    gbs = tot_b / (tot_t * 1e-3) / 1e9
    out = {"bytes": tot_b, "ms": round(tot_t, 4), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
    if iso is not None:
        ti = sum(iso[label] for label, _, _ in ops)
        out["ms_isolated"] = round(ti, 4)
        out["frac_isolated"] = round(tot_b / (ti * 1e-3) / 1e9 / PEAK_GBS, 4)
    return out


def time_both(d, ops, sets, reps, flush=True, setup=None):
    """Streamed figures over `sets` and isolated ones on set 0 (ops take the set's pointers)."""
    streamed = time_ops_streamed(d, ops, sets, reps)
    iso = time_ops(d, [(label, (lambda fn=fn: fn(sets[0])), b) for label, fn, b in ops], reps, flush=flush,
                   setup=setup)
    return streamed, iso


# ---------------------------------------------------------------------------------------
# config 2 (headline)
# ---------------------------------------------------------------------------------------
def setup_c2(d, n):
    L = d.L
    gens = [("a", "u", -1, 1), ("b", "u", 0.5, 2), ("ug", "n", 0, 1), ("x_exp", "u", -10, 10),
            ("x_log", "u", 1e-3, 10), ("x_act", "n", 0, 3), ("x_pow", "u", 0.1, 4)]
    for i, (name, kind, p, q) in enumerate(gens):
        ptr = d.alloc(name, n)
        fn = L.mh_rand_uniform if kind == "u" else L.mh_rand_normal
        chk(L, fn(ptr, n, SEED * 1000 + i, p, q), f"rand {name}")
    for name in ("res", "ga", "gb", "gx"):
        d.zeros(name, n)
    expo = np.array([np.float32(0.5 + 2.5 * np.random.default_rng(SEED).random())], np.float32)
    d.upload("exp", expo)
    d.zeros("gexp", 1)
    chk(L, L.mh_sync(), "sync")
    return float(expo[0])


def make_c2_calls(d, n):
    from mantle_amd._lib import make_shape
    L, p = d.L, d.ptrs
    s = make_shape((n,))
    x_of = {"EXP": "x_exp", "LOG": "x_log", "TANH": "x_act", "SIGMOID": "x_act", "RELU": "x_act"}
    calls = []
    for op in BINARY:
        o = OP_ID[op]
        calls.append((f"{op}.fwd", lambda o=o: L.mh_binary_fwd(o, p["res"], s, p["a"], s, p["b"], s)))
        calls.append((f"{op}.bwd", lambda o=o: L.mh_binary_bwd_accum2(o, p["ga"], p["gb"], p["ug"], p["a"], p["b"], s)))
    for op in UNARY:
        o, x = OP_ID[op], p[x_of[op]]
        calls.append((f"{op}.fwd", lambda o=o, x=x: L.mh_unary_fwd(o, p["res"], x, n)))
        calls.append((f"{op}.bwd", lambda o=o, x=x: L.mh_unary_bwd_accum(o, p["gx"], x, p["ug"], n)))
    calls.append(("POW.fwd", lambda: L.mh_pow_fwd(p["res"], p["x_pow"], n, p["exp"])))
    calls.append(("POW.bwd", lambda: L.mh_pow_bwd_accum2(p["gx"], p["gexp"], p["x_pow"], p["exp"], p["ug"], n)))
    return calls


def run_c2(L, n, steps, warmup):
    """The headline step: every config-2 op back to back, events between the ops."""
    d = Dev(L)
    expo = setup_c2(d, n)
    calls = make_c2_calls(d, n)
    plan = dict(step_plan())
    evs = [d.event() for _ in range(len(calls) + 1)]

    def run_step(timed):
        if timed:
            chk(L, L.mh_event_record(evs[0]), "record")
        for i, (label, fn) in enumerate(calls):
            chk(L, fn(), label)
            if timed:
                chk(L, L.mh_event_record(evs[i + 1]), "record")

    for _ in range(warmup):
        run_step(False)
    chk(L, L.mh_sync(), "sync")
    log(f"c2 warmup done ({warmup} steps)")
    op_ms = {label: 0.0 for label, _ in calls}
    ms = ctypes.c_float()
    t0 = time.perf_counter()
    step_ms_sum = 0.0
    for _ in range(steps):
        run_step(True)
        chk(L, L.mh_sync(), "sync")
        for i, (label, _) in enumerate(calls):
            chk(L, L.mh_event_elapsed_ms(ctypes.byref(ms), evs[i], evs[i + 1]), "elapsed")
            op_ms[label] += ms.value
        chk(L, L.mh_event_elapsed_ms(ctypes.byref(ms), evs[0], evs[-1]), "elapsed")
        step_ms_sum += ms.value
    wall = time.perf_counter() - t0
    d.free()
    avg = {k: v / steps for k, v in op_ms.items()}
    return {"ms_per_step": step_ms_sum / steps, "op_ms": avg, "wall": wall, "expo": expo,
            "bytes_per_step": sum(plan.values()) * n, "plan": plan}


# ---------------------------------------------------------------------------------------
# config 3: NCHW bias + RELU
# ---------------------------------------------------------------------------------------
def run_c3(L, reps):
    from mantle_amd import synth
    from mantle_amd._lib import make_shape
    shape, bshape = (256, 32, 28, 28), (1, 32, 1, 1)
    n, nb = int(np.prod(shape)), 32
    d = Dev(L)
    d.upload("x", synth.normal(shape, 0, 1, 11))
    d.upload("bias", synth.normal(bshape, 0, 0.1, 12))
    d.upload("ug", synth.normal(shape, 0, 1, 13))
    for k in ("y", "r", "gy", "gx"):
        d.zeros(k, n)
    d.zeros("gb", nb)
    sx, sb = make_shape(shape), make_shape(bshape)
    chk(L, L.mh_sync(), "sync")
    B = 4 * n
    fused = [("bias_relu.fwd", lambda P: L.mh_bias_relu_fwd(P["y"], P["r"], P["x"], sx, P["bias"], sb), 3 * B + 128),
             ("bias_relu.bwd", lambda P: L.mh_bias_relu_bwd_accum(None, P["gx"], P["gb"], P["y"], P["ug"], sx, sb),
              4 * B + 256)]
    opbyop = [("ADD.fwd", lambda P: L.mh_binary_fwd(0, P["y"], sx, P["x"], sx, P["bias"], sb), 2 * B + 128),
              ("RELU.fwd", lambda P: L.mh_unary_fwd(14, P["r"], P["y"], n), 2 * B),
              ("RELU.bwd", lambda P: L.mh_unary_bwd_accum(14, P["gy"], P["y"], P["ug"], n), 4 * B),
              ("ADD.bwd_x", lambda P: L.mh_binary_bwd_accum(0, 0, P["gx"], sx, P["gy"], sx, P["x"], sx, P["bias"], sb),
               3 * B),
              ("ADD.bwd_bias", lambda P: L.mh_binary_bwd_accum(0, 1, P["gb"], sb, P["gy"], sx, P["x"], sx, P["bias"],
                                                               sb), B + 256)]
    for label, fn, _ in fused + opbyop:  # real intermediates in the copied sets
        chk(L, fn(d.ptrs), label)
    sets = replicate(d, [(k, n) for k in ("x", "ug", "y", "r", "gy", "gx")] + [("bias", nb), ("gb", nb)], B + 256)
    mf, mfi = time_both(d, fused, sets, reps)
    mo, moi = time_both(d, opbyop, sets, reps)
    d.free()
    return {"shape": [list(shape), list(bshape)], "elements": n, "buffer_sets": len(sets),
            "fused": op_report(fused, mf, mfi), "fused_total": total_report(fused, mf, mfi),
            "op_by_op": op_report(opbyop, mo, moi), "op_by_op_total": total_report(opbyop, mo, moi)}


# ---------------------------------------------------------------------------------------
# config 4: axis reductions
# ---------------------------------------------------------------------------------------
def run_c4(L, reps):
    from mantle_amd import synth
    from mantle_amd._lib import make_shape
    d = Dev(L)
    ops, bufs, hbm = [], [], {}
    cases = [("8192x8192", (8192, 8192), 0, "n"), ("8192x8192", (8192, 8192), 1, "n"),
             ("8192x8192", (8192, 8192), -1, "n"), ("64x512x1024", (64, 512, 1024), 2, "u")]
    for tag, shape, axis, dist in cases:
        n = int(np.prod(shape))
        x = synth.normal(shape, 0, 1, 40) if dist == "n" else synth.uniform(shape, -1, 1, 41)
        if axis >= 0:
            synth.inject_ties(x, axis, 42)
        else:
            x.reshape(-1)[n // 2] = x.max()
        name = f"x_{tag}_{axis}"
        d.upload(name, x)
        del x
        red = (1,) if axis < 0 else tuple(1 if i == axis else s for i, s in enumerate(shape))
        m = int(np.prod(red))
        d.upload(f"ug_{name}", synth.normal(red, 0, 1, 43))
        d.zeros(f"res_{name}", m)
        d.zeros(f"g_{name}", n)
        bufs += [(name, n), (f"g_{name}", n), (f"ug_{name}", m), (f"res_{name}", m)]
        s = make_shape(shape)
        ax = "all" if axis < 0 else f"ax{axis}"
        for op in ("SUM", "MEAN", "MAX"):
            o = OP_ID[op]
            ops.append((f"{tag}.{ax}.{op}.fwd",
                        lambda P, o=o, name=name, s=s, axis=axis: L.mh_reduce_fwd(o, P[f"res_{name}"], P[name], s, axis),
                        4 * n + 4 * m))
        # MAX backward reads x and grad once each and stores only the grad quads that hold a
        # line maximum (at most m of them). Where the line maxima are a pass of their own
        # (axis 0, all), the routing pass reads x again only in the splits whose partials say
        # they hold several maxima of a line (rare); the split partials themselves (under 7 %
        # of the bytes at these shapes) are not counted
        hbm[f"{tag}.{ax}.MAX.bwd"] = 8 * n + 4 * m + 16 * m
        for op in ("SUM", "MEAN", "MAX"):
            o = OP_ID[op]
            nb = (12 * n + 8 * m) if op == "MAX" else (8 * n + 4 * m)
            ops.append((f"{tag}.{ax}.{op}.bwd",
                        lambda P, o=o, name=name, s=s, axis=axis: L.mh_reduce_bwd_accum(o, P[f"g_{name}"], P[name], s,
                                                                                        P[f"ug_{name}"], axis), nb))
    chk(L, L.mh_sync(), "sync")
    sets = replicate(d, bufs, min(b for _, _, b in ops))
    med, iso = time_both(d, ops, sets, reps)
    d.free()
    fwd = [o for o in ops if o[0].endswith(".fwd")]
    bwd = [o for o in ops if o[0].endswith(".bwd")]
    return {"buffer_sets": len(sets), "ops": op_report(ops, med, iso, hbm), "fwd_total": total_report(fwd, med, iso),
            "bwd_total": total_report(bwd, med, iso, hbm)}


# ---------------------------------------------------------------------------------------
# config 5: classifier head, op by op
# ---------------------------------------------------------------------------------------
def run_c5(L, reps, rows=1 << 20, classes=10):
    from mantle_amd import synth
    from mantle_amd._lib import make_shape
    d = Dev(L)
    p = d.ptrs
    E, N = rows * classes, rows
    logits = synth.normal((rows, classes), 0, 2, 31)
    cls = synth.integers((rows,), 0, classes, 32)
    onehot = np.zeros((rows, classes), np.float32)
    onehot[np.arange(rows), cls] = 1.0
    d.upload("logits", logits)
    d.upload("onehot", onehot)
    for k in ("xm", "e", "sm", "lp", "t"):
        d.zeros(k, E)
    for k in ("max", "s"):
        d.zeros(k, N)
    d.zeros("loss", 1)
    grads_full = ("g_logits", "g_xm", "g_e", "g_sm", "g_lp", "g_t")
    grads_row = ("g_max", "g_s")
    for k in grads_full:
        d.zeros(k, E)
    for k in grads_row:
        d.zeros(k, N)
    d.zeros("g_loss", 1)
    SE, SN, S1 = make_shape((rows, classes)), make_shape((rows, 1)), make_shape((1,))
    F, R = 4 * E, 4 * N
    fwd = [
        ("MAX.fwd", lambda P: L.mh_reduce_fwd(10, P["max"], P["logits"], SE, 1), F + R),
        ("SUB.fwd", lambda P: L.mh_binary_fwd(1, P["xm"], SE, P["logits"], SE, P["max"], SN), 2 * F + R),
        ("EXP.fwd", lambda P: L.mh_unary_fwd(4, P["e"], P["xm"], E), 2 * F),
        ("SUM.fwd", lambda P: L.mh_reduce_fwd(8, P["s"], P["e"], SE, 1), F + R),
        ("DIV.fwd", lambda P: L.mh_binary_fwd(3, P["sm"], SE, P["e"], SE, P["s"], SN), 2 * F + R),
        ("LOG.fwd", lambda P: L.mh_unary_fwd(5, P["lp"], P["sm"], E), 2 * F),
        ("MUL.fwd", lambda P: L.mh_binary_fwd(2, P["t"], SE, P["lp"], SE, P["onehot"], SE), 3 * F),
        ("MEAN.fwd", lambda P: L.mh_reduce_fwd(9, P["loss"], P["t"], SE, -1), F + 4),
    ]
    bwd = [
        ("MEAN.bwd", lambda P: L.mh_reduce_bwd_accum(9, P["g_t"], P["t"], SE, P["g_loss"], -1), 2 * F + 4),
        ("MUL.bwd0", lambda P: L.mh_binary_bwd_accum(2, 0, P["g_lp"], SE, P["g_t"], SE, P["lp"], SE, P["onehot"], SE),
         4 * F),
        ("LOG.bwd", lambda P: L.mh_unary_bwd_accum(5, P["g_sm"], P["sm"], P["g_lp"], E), 4 * F),
        ("DIV.bwd0", lambda P: L.mh_binary_bwd_accum(3, 0, P["g_e"], SE, P["g_sm"], SE, P["e"], SE, P["s"], SN),
         3 * F + R),
        ("DIV.bwd1", lambda P: L.mh_binary_bwd_accum(3, 1, P["g_s"], SN, P["g_sm"], SE, P["e"], SE, P["s"], SN),
         2 * F + 3 * R),
        ("SUM.bwd", lambda P: L.mh_reduce_bwd_accum(8, P["g_e"], P["e"], SE, P["g_s"], 1), 2 * F + R),
        ("EXP.bwd", lambda P: L.mh_unary_bwd_accum(4, P["g_xm"], P["xm"], P["g_e"], E), 4 * F),
        ("SUB.bwd0", lambda P: L.mh_binary_bwd_accum(1, 0, P["g_logits"], SE, P["g_xm"], SE, P["logits"], SE,
                                                   P["max"], SN), 3 * F),
        ("SUB.bwd1", lambda P: L.mh_binary_bwd_accum(1, 1, P["g_max"], SN, P["g_xm"], SE, P["logits"], SE,
                                                   P["max"], SN), F + 2 * R),
        ("MAX.bwd", lambda P: L.mh_reduce_bwd_accum(10, P["g_logits"], P["logits"], SE, P["g_max"], 1), 3 * F + 2 * R),
    ]

    def zero_grads():  # optim.zero_grad + the loss-grad seed (model.mojo:178-180)
        for k in grads_full:
            chk(L, L.mh_zero(p[k], E), "zero")
        for k in grads_row:
            chk(L, L.mh_zero(p[k], N), "zero")
        chk(L, L.mh_fill(p["g_loss"], 1.0, 1), "seed")

    zero_grads()
    for label, fn, _ in fwd + bwd:  # real intermediates (and the loss-grad seed) in the copied sets
        chk(L, fn(p), label)
    chk(L, L.mh_sync(), "sync")
    sets = replicate(d, [(k, E) for k in ("logits", "onehot", "xm", "e", "sm", "lp", "t") + grads_full] +
                     [(k, N) for k in ("max", "s") + grads_row] + [("loss", 1), ("g_loss", 1)], F + 4)
    med, iso = time_both(d, fwd + bwd, sets, reps, flush=False, setup=zero_grads)
    # the whole chain between two events (includes host launch gaps), caches flushed first
    e0, e1 = d.event(), d.event()
    ms = ctypes.c_float()
    chain = []
    for _ in range(reps + 1):
        zero_grads()
        d.flush()
        chk(L, L.mh_event_record(e0), "record")
        for label, fn, _ in fwd + bwd:
            chk(L, fn(p), label)
        chk(L, L.mh_event_record(e1), "record")
        chk(L, L.mh_sync(), "sync")
        chk(L, L.mh_event_elapsed_ms(ctypes.byref(ms), e0, e1), "elapsed")
        chain.append(ms.value)
    chain_ms = statistics.median(chain[1:])
    # the same graph row-fused: 8 B/elem forward (logits, onehot), 16 B/elem backward
    fused = [("fused.fwd", lambda P: L.mh_softmax_log_mul_mean_fwd(P["loss"], P["logits"], P["onehot"], rows, classes),
              2 * F + 4),
             ("fused.bwd", lambda P: L.mh_softmax_log_mul_mean_bwd_accum(P["g_logits"], P["logits"], P["onehot"],
                                                                       P["g_loss"], rows, classes), 4 * F + 4)]
    mf, mfi = time_both(d, fused, sets, reps)
    # the same graph through the native executor: Model.forward (inputs copied into the
    # arena from device memory, then the 8 nodes) and Model.backward (loss seed + 10 calls)
    import mantle_amd as mm
    g = mm.Graph()
    s_lg, s_oh = g.input((rows, classes), trainable=True), g.input((rows, classes))
    s_mx = g.op(mm.OP.MAX, s_lg, attributes={"axis": 1})
    s_e = g.op(mm.OP.EXP, g.op(mm.OP.SUB, s_lg, s_mx))
    s_sm = g.op(mm.OP.DIV, s_e, g.op(mm.OP.SUM, s_e, attributes={"axis": 1}))
    g.loss(g.op(mm.OP.MEAN, g.op(mm.OP.MUL, g.op(mm.OP.LOG, s_sm), s_oh)))
    model = mm.Model(g)
    tab = (ctypes.c_void_p * 2)(p["logits"], p["onehot"])
    fwd_bytes = sum(b for _, _, b in fwd) + 2 * 2 * F  # + the two input copies
    bwd_bytes = sum(b for _, _, b in bwd)
    model_ops = [("model.forward", lambda: L.mh_model_forward(model._h, 2, tab, 1), fwd_bytes),
                 ("model.backward", lambda: L.mh_model_backward(model._h, 0, None, 0), bwd_bytes)]
    mmed = time_ops(d, model_ops, reps, setup=lambda: chk(L, L.mh_model_zero_grad(model._h), "zero_grad"))
    # the same graph with its head run as the row-fused kernels (MH_MODEL_FUSE_ROWS)
    fmodel = mm.Model(g, fuse_rows=True)
    # bytes the fused model moves: the two input copies (read + write, 4F) and the row kernel's
    # x and target (2F) forward; x, target and grad_x read and written (4F) backward
    fused_model_ops = [("model_fused.forward", lambda: L.mh_model_forward(fmodel._h, 2, tab, 1), 6 * F + 4),
                       ("model_fused.backward", lambda: L.mh_model_backward(fmodel._h, 0, None, 0), 4 * F + 4)]
    fmed = time_ops(d, fused_model_ops, reps, setup=lambda: chk(L, L.mh_model_zero_grad(fmodel._h), "zero_grad"))
    del model, fmodel, g
    d.free()
    return {"shape": [rows, classes], "elements": E,
            "model": op_report(model_ops, mmed), "model_total": total_report(model_ops, mmed),
            "model_fused_rows": op_report(fused_model_ops, fmed),
            "model_fused_rows_total": total_report(fused_model_ops, fmed),
            "fused": op_report(fused, mf, mfi), "fused_total": total_report(fused, mf, mfi),
            "buffer_sets": len(sets),
            "fwd": op_report(fwd, med, iso), "bwd": op_report(bwd, med, iso),
            "fwd_total": total_report(fwd, med, iso), "bwd_total": total_report(bwd, med, iso),
            "chain_ms": round(chain_ms, 4), "chain_rows_per_s": round(rows / (chain_ms * 1e-3), 1),
            "fused_min_bytes": 24 * E}


def run_adam(L, reps):
    """Adam.step on one 2^28-element parameter (28 B/elem) and on 400 tensors of 1..2^18
    elements (about 2^26 in all) through the multi-tensor entry point."""
    d = Dev(L)
    n = 1 << 28
    for k in ("p", "g", "m", "v"):
        d.zeros(k, n)
    chk(L, L.mh_rand_normal(d.ptrs["p"], n, 7, 0.0, 1.0), "rand")
    chk(L, L.mh_rand_normal(d.ptrs["g"], n, 8, 0.0, 0.1), "rand")
    p = d.ptrs
    sizes = [int(x) for x in np.random.default_rng(SEED).integers(1, 1 << 18, size=400)]
    slot = [(n + 63) & ~63 for n in sizes]  # arena slots on 256-byte boundaries, as mh_malloc places tensors
    tot = sum(sizes)
    for k in ("P", "G", "M", "V"):
        d.zeros(k, sum(slot))
    chk(L, L.mh_rand_normal(d.ptrs["G"], sum(slot), 9, 0.0, 0.1), "rand")
    off = np.concatenate([[0], np.cumsum(slot)[:-1]])
    VP = ctypes.c_void_p * len(sizes)
    tabs = {k: VP(*[p[k] + 4 * int(o) for o in off]) for k in ("P", "G", "M", "V")}
    csz = (ctypes.c_int64 * len(sizes))(*sizes)
    it = [0]

    def single():
        it[0] += 1
        return L.mh_adam_step(p["p"], p["g"], p["m"], p["v"], n, 1e-3, 0.9, 0.999, 1e-8, it[0])

    def multi():
        return L.mh_adam_step_multi(len(sizes), tabs["P"], tabs["G"], tabs["M"], tabs["V"], csz, 1e-3, 0.9, 0.999,
                                    1e-8, 1)
    chk(L, L.mh_sync(), "sync")
    ops = [("adam.single_2^28", single, 28 * n), ("adam.multi_400", multi, 28 * tot)]
    med = time_ops(d, ops, reps, flush=False)
    d.free()
    return {"elements_single": n, "elements_multi": tot, "tensors_multi": len(sizes), **op_report(ops, med)}


def run_adj(L, reps):
    """FMA, LEAKYRELU and CLIP forward / backward over 2^28 elements, and tstd over
    [8192, 8192] (axis 0, axis 1, all elements; x read once for both fp64 moments, 4 B/elem
    algorithmic)."""
    from mantle_amd._lib import make_shape
    d = Dev(L)
    n = 1 << 28
    for k in ("a", "b", "c", "r", "g"):
        d.zeros(k, n)
    p = d.ptrs
    chk(L, L.mh_rand_normal(p["a"], n, 11, 0.0, 3.0), "rand")
    chk(L, L.mh_rand_normal(p["b"], n, 12, 0.0, 1.0), "rand")
    chk(L, L.mh_rand_normal(p["c"], n, 13, 0.0, 1.0), "rand")
    ops = [("FMA.fwd", lambda: L.mh_fma_fwd(p["r"], p["a"], p["b"], p["c"], n), 16 * n),
           ("FMA.bwd0", lambda: L.mh_fma_bwd_accum(0, p["g"], p["c"], p["a"], p["b"], n), 16 * n),
           ("FMA.bwd2", lambda: L.mh_fma_bwd_accum(2, p["g"], p["c"], p["a"], p["b"], n), 12 * n),
           ("LEAKYRELU.fwd", lambda: L.mh_leakyrelu_fwd(p["r"], p["a"], n, 0.1), 8 * n),
           ("LEAKYRELU.bwd", lambda: L.mh_leakyrelu_bwd_accum(p["g"], p["a"], p["b"], n, 0.1), 16 * n),
           ("CLIP.fwd", lambda: L.mh_clip_fwd(p["r"], p["a"], n, -1.1, 1.1), 8 * n),
           ("CLIP.bwd", lambda: L.mh_clip_bwd_accum(p["g"], p["a"], p["b"], n, -1.1, 1.1), 16 * n)]
    chk(L, L.mh_sync(), "sync")
    med = time_ops(d, ops, reps)  # one launch each after a flush: 1 GiB operands, 0.3-0.7 ms ops
    out = {"elements": n, **op_report(ops, med)}
    # tstd over [8192, 8192] (40-50 us): streamed over cold buffer sets like config 4's
    # reductions of the same shape, with the isolated figure beside it
    m = 8192 * 8192
    s = make_shape((8192, 8192))
    d.zeros("tx", m)
    d.zeros("tr", 8192)
    chk(L, L.mh_rand_normal(d.ptrs["tx"], m, 14, 0.0, 3.0), "rand")
    tops = []
    for axis, nout in ((0, 8192), (1, 8192), (-1, 1)):
        ax = "all" if axis < 0 else f"ax{axis}"
        tops.append((f"tstd.8192x8192.{ax}", lambda P, axis=axis: L.mh_tstd(P["tr"], P["tx"], s, axis), 4 * m + 4 * nout))
    chk(L, L.mh_sync(), "sync")
    sets = replicate(d, [("tx", m), ("tr", 8192)], min(b for _, _, b in tops))
    tmed, tiso = time_both(d, tops, sets, reps)
    out.update(op_report(tops, tmed, tiso))
    d.free()
    return out


def run_rows(L, reps):
    """Row-fused graphs: CrossEntropyLoss, Softmax and LogSoftmax over [2^20, 10] and
    [32768, 1000]. Bytes: loss forward 8 B/elem (x, target), loss backward
    16 (x, target, grad_x read and written), Softmax / LogSoftmax forward 8 (x, out) and
    backward 16 (x, grad_out, grad_x read and written)."""
    d = Dev(L)
    p = d.ptrs
    ops, bufs = [], []
    for rows, k in ((1 << 20, 10), (32768, 1000)):
        n = rows * k
        tag = f"{rows}x{k}"
        for nm in ("x", "t", "o", "g"):
            d.zeros(f"{nm}{tag}", n)
        d.zeros(f"loss{tag}", 1)
        d.zeros(f"ug{tag}", 1)
        bufs += [(f"{nm}{tag}", n) for nm in ("x", "t", "o", "g")] + [(f"loss{tag}", 1), (f"ug{tag}", 1)]
        chk(L, L.mh_rand_normal(p[f"x{tag}"], n, 21, 0.0, 2.0), "rand")
        chk(L, L.mh_rand_uniform(p[f"t{tag}"], n, 22, 0.0, 1.0), "rand")
        chk(L, L.mh_fill(p[f"ug{tag}"], 1.0, 1), "fill")
        ops += [(f"cross_entropy.fwd.{tag}", lambda P, tag=tag, r=rows, k=k: L.mh_cross_entropy_fwd(
                    P[f"loss{tag}"], P[f"x{tag}"], P[f"t{tag}"], r, k), 8 * n + 4),
                (f"cross_entropy.bwd.{tag}", lambda P, tag=tag, r=rows, k=k: L.mh_cross_entropy_bwd_accum(
                    P[f"g{tag}"], P[f"x{tag}"], P[f"t{tag}"], P[f"ug{tag}"], r, k), 16 * n + 4)]
        for nm, f, b in (("softmax", L.mh_softmax_fwd, L.mh_softmax_bwd_accum),
                         ("logsoftmax", L.mh_logsoftmax_fwd, L.mh_logsoftmax_bwd_accum)):
            ops += [(f"{nm}.fwd.{tag}", lambda P, tag=tag, r=rows, k=k, f=f: f(P[f"o{tag}"], P[f"x{tag}"], r, k), 8 * n),
                    (f"{nm}.bwd.{tag}", lambda P, tag=tag, r=rows, k=k, b=b: b(P[f"g{tag}"], P[f"x{tag}"], P[f"t{tag}"],
                                                                          r, k), 16 * n)]
    chk(L, L.mh_sync(), "sync")
    for label, fn, _ in ops:  # real outputs and gradients in the copied sets
        chk(L, fn(d.ptrs), label)
    sets = replicate(d, bufs, min(b for _, _, b in ops))
    med, iso = time_both(d, ops, sets, reps)
    d.free()
    return {"buffer_sets": len(sets), **op_report(ops, med, iso)}


def run_graph(L, reps, steps=200):
    """One training step (zero_grad, forward, backward) of a model through the native executor,
    eager against the replay of the step captured as one HIP graph (MH_PASS_STEP): config 1's
    ADD(bias) -> RELU graph with a MEAN loss (the launch-bound case), a deep chain of 24
    MUL -> ADD -> RELU layers over [32, 32] and config 5's head chain. Wall time per step on the
    host (inputs copied from device buffers into their slots every step), one synchronisation per
    `steps` steps."""
    import time
    import mantle_amd as mm
    from mantle_amd import synth
    out = {}

    def c1():
        g = mm.Graph()
        x = g.input((32, 32), trainable=True)
        b = g.param((1, 32), init=synth.normal((1, 32), 0, 0.1, 51))
        g.loss(g.op(mm.OP.MEAN, g.op(mm.OP.RELU, g.op(mm.OP.ADD, x, b))))
        return g, [synth.normal((32, 32), 0, 1, 52)]

    def c5():
        rows = 1 << 20
        g = mm.Graph()
        lg, oh = g.input((rows, 10), trainable=True), g.input((rows, 10))
        mx = g.op(mm.OP.MAX, lg, attributes={"axis": 1})
        e = g.op(mm.OP.EXP, g.op(mm.OP.SUB, lg, mx))
        sm = g.op(mm.OP.DIV, e, g.op(mm.OP.SUM, e, attributes={"axis": 1}))
        g.loss(g.op(mm.OP.MEAN, g.op(mm.OP.MUL, g.op(mm.OP.LOG, sm), oh)))
        onehot = np.zeros((rows, 10), np.float32)
        onehot[np.arange(rows), synth.integers((rows,), 0, 10, 54)] = 1
        return g, [synth.normal((rows, 10), 0, 2, 53), onehot]

    def deep():  # a deep chain of small tensors: 24 layers of MUL(w) -> ADD(b) -> RELU over [32, 32]
        g = mm.Graph()
        x = g.input((32, 32), trainable=True)
        h = x
        for i in range(24):
            w = g.param((1, 32), init=synth.normal((1, 32), 1, 0.1, 60 + 2 * i))
            b = g.param((1, 32), init=synth.normal((1, 32), 0, 0.1, 61 + 2 * i))
            h = g.op(mm.OP.RELU, g.op(mm.OP.ADD, g.op(mm.OP.MUL, h, w), b))
        g.loss(g.op(mm.OP.MEAN, h))
        return g, [synth.normal((32, 32), 0, 1, 59)]

    for name, make, n in (("c1", c1, steps), ("deep", deep, steps), ("c5", c5, max(steps // 10, 10))):
        g, inputs = make()
        res = {}
        for mode in ("eager", "graph"):
            model = mm.Model(g)
            srcs = [mm.Tensor.from_numpy(v) for v in inputs]  # the step's inputs, already on the device
            tab = (ctypes.c_void_p * len(srcs))(*[t.ptr for t in srcs])
            slots = [(model.parameters.tensors[sym].ptr, t.ptr, t.num_elements() * 4) for sym, t in zip(g.inputs, srcs)]
            h = model._h
            if mode == "graph":
                for dst, src, nb in slots:
                    chk(L, L.mh_memcpy_d2d(dst, src, nb), "copy")
                model.capture("step")

                def step():  # inputs into their slots, then one graph: zero_grad, forward, backward
                    for dst, src, nb in slots:
                        chk(L, L.mh_memcpy_d2d(dst, src, nb), "copy")
                    chk(L, L.mh_model_replay(h, 2), "replay step")
            else:
                def step():  # Model.forward copies the inputs in, then every node; Model.backward
                    chk(L, L.mh_model_zero_grad(h), "zero_grad")
                    chk(L, L.mh_model_forward(h, len(srcs), tab, 1), "fwd")
                    chk(L, L.mh_model_backward(h, 0, None, 0), "bwd")
            for _ in range(3):
                step()
            chk(L, L.mh_sync(), "sync")
            t0 = time.perf_counter()
            for _ in range(n):
                step()
            chk(L, L.mh_sync(), "sync")
            res[mode] = round((time.perf_counter() - t0) / n * 1e6, 2)
            del model, srcs
        out[name] = {"us_per_step": res, "speedup": round(res["eager"] / res["graph"], 2)}
    return out


def run_copy(L, reps):
    """Practical streaming ceilings: the library's copy kernel over 1 GiB (the headline's size)
    and over one tensor of config 3 and of config 5; and, for kernels that only read, the
    library's all-element SUM (one read pass plus a one-block combine) over one config-3 tensor,
    one config-5 tensor and the config-5 head's two tensors (84 MB, what its fused forward
    reads). The small sizes are streamed and isolated like their ops; plus the isolated method's
    floor. Every source holds normal random data, as the ops' operands do (a copy of zeros
    streams about 3 % faster)."""
    from mantle_amd._lib import make_shape
    d = Dev(L)
    n = 1 << 28
    src, dst = d.zeros("src", n), d.zeros("dst", n)
    chk(L, L.mh_rand_normal(src, n, 41, 0.0, 1.0), "rand")
    ops = [("copy_1GiB", lambda: L.mh_memcpy_d2d(dst, src, 4 * n), 8 * n)]
    med = time_ops(d, ops, reps, flush=False)
    out = op_report(ops, med)
    for tag, m in (("copy_c3_tensor", 6422528), ("copy_c5_tensor", 10485760)):
        chk(L, L.mh_rand_normal(d.zeros(f"s_{tag}", m), m, 42, 0.0, 1.0), "rand")
        d.zeros(f"d_{tag}", m)
        small = [(tag, lambda P, tag=tag, m=m: L.mh_memcpy_d2d(P[f"d_{tag}"], P[f"s_{tag}"], 4 * m), 8 * m)]
        sets = replicate(d, [(f"s_{tag}", m), (f"d_{tag}", m)], 8 * m)
        sm, si = time_both(d, small, sets, reps)
        out.update(op_report(small, sm, si))
    for tag, m in (("read_c3_tensor", 6422528), ("read_c5_tensor", 10485760), ("read_c5_head", 2 * 10485760)):
        chk(L, L.mh_rand_normal(d.zeros(f"r_{tag}", m), m, 43, 0.0, 1.0), "rand")
        d.zeros(f"o_{tag}", 1)
        shp = make_shape((m,))
        rd = [(tag, lambda P, tag=tag, shp=shp: L.mh_reduce_fwd(8, P[f"o_{tag}"], P[f"r_{tag}"], shp, -1), 4 * m + 4)]
        sets = replicate(d, [(f"r_{tag}", m), (f"o_{tag}", 1)], 4 * m)
        sm, si = time_both(d, rd, sets, reps)
        out.update(op_report(rd, sm, si))
    out["isolated_floor_ms"] = isolated_floor(d, reps)
    d.free()
    return out


# ---------------------------------------------------------------------------------------
# CPU baseline
# ---------------------------------------------------------------------------------------
def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cores_available() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def _median_pass(fn, reps: int):
    """Median wall time of `reps` calls of fn after one untimed warm-up call."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _cpu_c2(n_sample: int, reps: int, expo: float):
    """Config 2's op sequence on n_sample elements per tensor, one thread (the reference's
    elementwise paths are single-threaded)."""
    from oracle import oracle as O
    from mantle_amd import synth
    a = synth.uniform((n_sample,), -1, 1, 1)
    b = synth.uniform((n_sample,), 0.5, 2, 2)
    ug = synth.normal((n_sample,), 0, 1, 3)
    xs = {"EXP": synth.uniform((n_sample,), -10, 10, 4), "LOG": synth.uniform((n_sample,), 1e-3, 10, 5)}
    xs["TANH"] = xs["SIGMOID"] = xs["RELU"] = synth.normal((n_sample,), 0, 3, 6)
    xp = synth.uniform((n_sample,), 0.1, 4, 7)
    e = np.array([expo], np.float32)
    res = np.zeros(n_sample, np.float32)
    ga, gb = np.zeros(n_sample, np.float32), np.zeros(n_sample, np.float32)
    ge = np.zeros(1, np.float32)

    def one_pass():
        for op in BINARY:
            o = OP_ID[op]
            O.forward_op_into(o, res, a, b)
            O.backward_op_into(0, o, ga, ug, a, b)
            O.backward_op_into(1, o, gb, ug, a, b)
        for op in UNARY:
            O.forward_op_into(OP_ID[op], res, xs[op])
            O.backward_op_into(0, OP_ID[op], ga, ug, xs[op])
        O.forward_op_into(6, res, xp, e)
        O.backward_op_into(0, 6, ga, ug, xp, e)
        O.backward_op_into(1, 6, ge, ug, xp, e)

    t = _median_pass(one_pass, reps)
    nbytes = sum(bb for _, bb in step_plan()) * n_sample
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "ms_per_pass": round(t * 1e3, 2),
            "sample": f"config-2 op sequence (fwd, both backward operands, POW's exponent gradient) on "
                      f"{n_sample} elements per tensor (1/{(1 << 28) // n_sample} of the workload), median of "
                      f"{reps} passes after 1 warm-up; single-threaded C restatement (oracle/, -O3), results "
                      f"and gradients in preallocated arrays"}


def _cpu_c3(reps: int):
    """Config 3 op by op at full size ([256,32,28,28] + [1,32,1,1]), one thread."""
    from oracle import oracle as O
    from mantle_amd import synth
    shape, bshape = (256, 32, 28, 28), (1, 32, 1, 1)
    n = int(np.prod(shape))
    x, bias, ug = synth.normal(shape, 0, 1, 11), synth.normal(bshape, 0, 0.1, 12), synth.normal(shape, 0, 1, 13)
    y, r = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    gy, gx, gb = np.zeros(shape, np.float32), np.zeros(shape, np.float32), np.zeros(bshape, np.float32)

    def one_pass():
        O.forward_op_into(0, y, x, bias)
        O.forward_op_into(14, r, y)
        O.backward_op_into(0, 14, gy, ug, y)
        O.backward_op_into(0, 0, gx, gy, x, bias)
        O.backward_op_into(1, 0, gb, gy, x, bias)

    t = _median_pass(one_pass, reps)
    B = 4 * n
    nbytes = (2 * B + 128) + 2 * B + 4 * B + 3 * B + (B + 256)  # the GPU op-by-op accounting
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "ms_per_pass": round(t * 1e3, 2),
            "sample": f"config 3 op by op at full size (ADD, RELU forward; RELU, ADD x and bias backward), "
                      f"median of {reps} after 1 warm-up; single-threaded like the reference's elementwise, "
                      f"broadcast and accumulate_grad paths"}


def _cpu_c4(reps: int, threads: int, rows: int = 1024):
    """Config 4's reductions on a [rows, 8192] sample of the [8192, 8192] workload: axis
    forwards over a pool of `threads` (the reference's parallelize over outputs,
    tensorutils.mojo:682), all-element forwards and every backward on one thread."""
    from oracle import oracle as O
    from mantle_amd import synth
    shape = (rows, 8192)
    n = rows * 8192
    x = synth.normal(shape, 0, 1, 40)
    out = {}
    for axis in (0, 1, -1):
        red = (1,) if axis < 0 else tuple(1 if i == axis else d for i, d in enumerate(shape))
        m = int(np.prod(red))
        ug = synth.normal(red, 0, 1, 43)
        g = np.zeros(shape, np.float32)
        res = np.zeros(red, np.float32)
        ax = "all" if axis < 0 else f"ax{axis}"
        for op, name in ((8, "SUM"), (9, "MEAN"), (10, "MAX")):
            if axis >= 0:
                tf = _median_pass(lambda op=op, axis=axis: O.reduce_axis_mt(op, x, axis, threads), reps)
                fc = threads
            else:
                tf = _median_pass(lambda op=op: O.forward_op_into(op, res, x, None, -1), reps)
                fc = 1
            tb = _median_pass(lambda op=op, axis=axis, ug=ug: O.backward_op_into(0, op, g, ug, x, None, axis), reps)
            fb, bb = 4 * n + 4 * m, (12 * n + 8 * m) if name == "MAX" else (8 * n + 4 * m)
            out[f"{ax}.{name}.fwd"] = {"GB/s": round(fb / tf / 1e9, 3), "ms": round(tf * 1e3, 2), "cores": fc}
            out[f"{ax}.{name}.bwd"] = {"GB/s": round(bb / tb / 1e9, 3), "ms": round(tb * 1e3, 2), "cores": 1}
    fwd = [v for k, v in out.items() if k.endswith(".fwd")]
    tot_b = sum(v["GB/s"] * v["ms"] for v in out.values())  # GB/s * ms = MB
    tot_ms = sum(v["ms"] for v in out.values())
    return {"value": round(tot_b / tot_ms, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "fwd_GB/s": round(sum(v["GB/s"] * v["ms"] for v in fwd) / sum(v["ms"] for v in fwd), 3),
            "ops": out,
            "sample": f"SUM/MEAN/MAX over axis 0, axis 1 and all of a [{rows}, 8192] sample ({rows / 8192:.3g} of "
                      f"the [8192, 8192] workload), forward and backward, median of {reps} after 1 warm-up each; "
                      f"axis forwards on {threads} threads (outputs split as the reference's parallelize), "
                      f"all-element forwards and backwards single-threaded as in the reference"}


def _cpu_c5(reps: int, threads: int, rows: int = 1 << 17, classes: int = 10):
    """Config 5's chain op by op on `rows` rows: the two axis-1 reductions on `threads` threads,
    the rest single-threaded, as in the reference."""
    from oracle import oracle as O
    from mantle_amd import synth
    E, N = rows * classes, rows
    lg = synth.normal((rows, classes), 0, 2, 31)
    oh = np.zeros((rows, classes), np.float32)
    oh[np.arange(rows), synth.integers((rows,), 0, classes, 32)] = 1.0
    full = lambda: np.zeros((rows, classes), np.float32)  # noqa: E731
    xm, e, sm, lp, t = full(), full(), full(), full(), full()
    g = {k: full() for k in ("logits", "xm", "e", "sm", "lp", "t")}
    gmax, gs = np.zeros((rows, 1), np.float32), np.zeros((rows, 1), np.float32)
    gl = np.ones(1, np.float32)
    loss = np.zeros(1, np.float32)
    st = {}

    def one_pass():
        mx = O.reduce_axis_mt(10, lg, 1, threads)
        O.forward_op_into(1, xm, lg, mx)
        O.forward_op_into(4, e, xm)
        s = O.reduce_axis_mt(8, e, 1, threads)
        O.forward_op_into(3, sm, e, s)
        O.forward_op_into(5, lp, sm)
        O.forward_op_into(2, t, lp, oh)
        O.forward_op_into(9, loss, t, None, -1)
        O.backward_op_into(0, 9, g["t"], gl, t, None, -1)
        O.backward_op_into(0, 2, g["lp"], g["t"], lp, oh)
        O.backward_op_into(0, 5, g["sm"], g["lp"], sm)
        O.backward_op_into(0, 3, g["e"], g["sm"], e, s)
        O.backward_op_into(1, 3, gs, g["sm"], e, s)
        O.backward_op_into(0, 8, g["e"], gs, e, None, 1)
        O.backward_op_into(0, 4, g["xm"], g["e"], xm)
        O.backward_op_into(0, 1, g["logits"], g["xm"], lg, mx)
        O.backward_op_into(1, 1, gmax, g["xm"], lg, mx)
        O.backward_op_into(0, 10, g["logits"], gmax, lg, None, 1)
        st["ok"] = True

    t_pass = _median_pass(one_pass, reps)
    F, R = 4 * E, 4 * N
    fwd_b = (F + R) + (2 * F + R) + 2 * F + (F + R) + (2 * F + R) + 2 * F + 3 * F + (F + 4)
    bwd_b = (2 * F + 4) + 4 * F + 4 * F + (3 * F + R) + (2 * F + 3 * R) + (2 * F + R) + 4 * F + 3 * F + (F + 2 * R) + \
        (3 * F + 2 * R)
    return {"value": round((fwd_b + bwd_b) / t_pass / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_pass": round(t_pass * 1e3, 2), "rows_per_s": round(rows / t_pass, 1),
            "sample": f"config-5 chain op by op (8 forward, 10 backward calls) on [{rows}, {classes}] "
                      f"(1/{(1 << 20) // rows} of the rows), median of {reps} after 1 warm-up; the two axis-1 "
                      f"reduction forwards on {threads} threads, every other call single-threaded, as in "
                      f"the reference; the GPU op-by-op byte accounting"}


def cpu_baseline(n_sample: int, reps: int, expo: float):
    """The CPU restatement (oracle/) timed on the host's cores, beside the GPU figures: config 2
    (the headline metric: `value`), and configs 3-5 under `configs`, each a bounded sample with
    the GPU workload's byte accounting and the reference's threading (one thread except the axis
    reductions, which run on the cores available to the job)."""
    threads = _cores_available()
    out = _cpu_c2(n_sample, reps, expo)
    out.update({"host_cpu": _cpu_model(), "host_cores_available": threads})
    out["configs"] = {"c3": _cpu_c3(reps), "c4": _cpu_c4(reps, threads), "c5": _cpu_c5(reps, threads)}
    return out


def _fracs(d, strip=""):
    return {k.replace(strip, ""): v["frac"] for k, v in d.items() if isinstance(v, dict) and "frac" in v}


def _lowest(fr):
    k = min(fr, key=fr.get)
    return [k, fr[k]]


def summary(out):
    """A compact digest of every config, written as the JSON line's last key so that a reader
    who keeps only the end of the line still sees all of them: each op family's streamed
    fraction of peak, the lowest family and the total per config, the copy ceiling at that
    tensor size, and the CPU baseline figure (GB/s, same byte accounting)."""
    s = {}
    cpu = out.get("cpu_baseline") or {}
    cpu_cfg = cpu.get("configs", {})
    if out.get("ops"):
        fr = _fracs(out["ops"])
        s["c2"] = {"step": out["config"]["frac_of_peak"], "lowest": _lowest(fr), "highest": [max(fr, key=fr.get),
                   max(fr.values())], "cpu_GB/s": cpu.get("value")}
    w = out.get("workloads", {})
    copy = w.get("copy", {})
    if "c3" in w:
        c3 = w["c3"]
        fr = _fracs(c3["op_by_op"])
        s["c3"] = {"op_by_op": fr, "op_by_op_total": c3["op_by_op_total"]["frac"],
                   "fused": _fracs(c3["fused"]), "fused_total": c3["fused_total"]["frac"],
                   "lowest": _lowest({**fr, **_fracs(c3["fused"])}),
                   "copy_ceiling": copy.get("copy_c3_tensor", {}).get("frac"),
                   "cpu_GB/s": cpu_cfg.get("c3", {}).get("value")}
    if "c4" in w:
        c4 = w["c4"]
        fr = {k.replace("8192x8192.", "").replace("64x512x1024.", "3d."): v for k, v in _fracs(c4["ops"]).items()}
        s["c4"] = {"ops": fr, "fwd_total": c4["fwd_total"]["frac"], "bwd_total": c4["bwd_total"]["frac"],
                   "lowest": _lowest(fr), "cpu_GB/s": cpu_cfg.get("c4", {}).get("value")}
    if "c5" in w:
        c5 = w["c5"]
        fr = {**_fracs(c5["fwd"]), **_fracs(c5["bwd"])}
        s["c5"] = {"op_by_op": fr, "fwd_total": c5["fwd_total"]["frac"], "bwd_total": c5["bwd_total"]["frac"],
                   "fused": _fracs(c5["fused"]), "fused_total": c5["fused_total"]["frac"],
                   "model_total": c5.get("model_total", {}).get("frac"),
                   "lowest": _lowest(fr), "copy_ceiling": copy.get("copy_c5_tensor", {}).get("frac"),
                   "cpu_GB/s": cpu_cfg.get("c5", {}).get("value")}
    extra = {}
    for name in ("adam", "adj", "rows"):
        if name in w:
            extra.update({(k if k.startswith(name) else f"{name}.{k}"): v for k, v in _fracs(w[name]).items()})
    if extra:
        s["next_rows"] = extra
    return s


# ---------------------------------------------------------------------------------------
# rocprofv3 summaries
# ---------------------------------------------------------------------------------------
def _read_pmc_csv(path, counter):
    """{kernel name: {grid size: [counter value per dispatch]}} from a rocprofv3 --pmc
    counter_collection.csv."""
    out = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            out.setdefault(row["Kernel_Name"], {}).setdefault(int(row["Grid_Size"]), []).append(
                float(row["Counter_Value"]))
    return out


def pmc_summary(fetch_csv, write_csv, copy_bytes=8 << 28):
    """Writes profiles/traffic.json: HBM bytes per dispatch of each kernel, from FETCH_SIZE
    and WRITE_SIZE (KiB per dispatch), each scaled by the factor that makes the library's
    copy kernel (k_copy over `copy_bytes / 2` read and as many written) count exactly its
    bytes. Per kernel, dispatches are grouped by grid size (median per group); `hbm_bytes`
    is the largest launch, which for the config-2 kernels is the 2^28-element one."""
    fetch, write = _read_pmc_csv(fetch_csv, "FETCH_SIZE"), _read_pmc_csv(write_csv, "WRITE_SIZE")
    copy_k = [k for k in fetch if "k_copy" in k]
    if not copy_k:
        raise SystemExit("no k_copy dispatch in the FETCH_SIZE run: run the 'copy' workload under rocprofv3")
    half = copy_bytes / 2
    cf, cw = fetch[copy_k[0]], write[copy_k[0]]
    f_scale = half / (statistics.median(cf[max(cf)]) * 1024)
    w_scale = half / (statistics.median(cw[max(cw)]) * 1024)
    kernels = {}
    for k in sorted(set(fetch) | set(write)):
        grids = sorted(set(fetch.get(k, {})) | set(write.get(k, {})))
        by_grid = {}
        for g in grids:
            fv = statistics.median(fetch[k][g]) * 1024 * f_scale if g in fetch.get(k, {}) else None
            wv = statistics.median(write[k][g]) * 1024 * w_scale if g in write.get(k, {}) else None
            by_grid[str(g)] = {"fetch_bytes": None if fv is None else round(fv),
                               "write_bytes": None if wv is None else round(wv),
                               "hbm_bytes": round((fv or 0) + (wv or 0))}
        top = by_grid[str(grids[-1])]
        kernels[k] = {"largest_grid": grids[-1], "fetch_bytes": top["fetch_bytes"], "write_bytes": top["write_bytes"],
                      "hbm_bytes": top["hbm_bytes"], "by_grid": by_grid}
    summary = {"fetch_scale": f_scale, "write_scale": w_scale, "copy_kernel": copy_k[0], "kernels": kernels}
    os.makedirs(os.path.dirname(TRAFFIC_JSON), exist_ok=True)
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(summary, f, indent=0, sort_keys=True)
    return summary


# label of a config-2 op -> prefix of its kernel's name (the 2^28-element launch)
C2_KERNEL = {"ADD.bwd": "void mh::k_bwd2_same4<0, false>", "SUB.bwd": "void mh::k_bwd2_same4<1, false>",
             "MUL.bwd": "void mh::k_bwd2_same4<2, false>", "DIV.bwd": "void mh::k_bwd2_same4<3, false>",
             "ADD.fwd": "void mh::k_same4<mh::FBin<0>,", "SUB.fwd": "void mh::k_same4<mh::FBin<1>,",
             "MUL.fwd": "void mh::k_same4<mh::FBin<2>,", "DIV.fwd": "void mh::k_same4<mh::FBin<3>,",
             "EXP.fwd": "void mh::k_same4<mh::FUn<4>,", "LOG.fwd": "void mh::k_same4<mh::FUn<5>,",
             "SIGMOID.fwd": "void mh::k_same4<mh::FUn<13>,", "RELU.fwd": "void mh::k_same4<mh::FUn<14>,",
             "TANH.fwd": "void mh::k_same4<mh::FUn<15>,", "EXP.bwd": "void mh::k_same4<mh::FUnBwd<4>,",
             "LOG.bwd": "void mh::k_same4<mh::FUnBwd<5>,", "SIGMOID.bwd": "void mh::k_same4<mh::FUnBwd<13>,",
             "RELU.bwd": "void mh::k_same4<mh::FUnBwd<14>,", "TANH.bwd": "void mh::k_same4<mh::FUnBwd<15>,",
             "POW.fwd": "void mh::k_same4<mh::FPowi,", "POW.bwd": "void mh::k_pow_grad_quads<true>("}


# workload kernels for the traffic table: (op, kernel-name prefix, launch grid in threads,
# algorithmic bytes of the kernel, note)
_N3, _N4, _N5 = 6422528, 1 << 26, 10485760
WL_KERNELS = [
    ("c3 bias_relu.fwd (fused)", "mh::k_bias_relu_fwd_planes", 1605632, 12 * _N3 + 128, ""),
    ("c3 ADD.fwd", "void mh::k_planebc4<mh::FBin<0>, 2, false, 8>", 1605632, 8 * _N3 + 128, ""),
    ("c3 bias_relu.bwd (fused), stream", "void mh::k_bias_relu_bwd_flat<false, true, true, true>", 1605632, 16 * _N3,
     "grad_x read and written; a wave's plane partials into the slot table"),
    ("c3 bias_relu.bwd (fused), combine", "mh::k_bias_partials_comb8", 8192, 4 * 8 * (_N3 // 784) + 256,
     "the slot table (8 slots per plane) read, 32 bias values updated"),
    ("c3 ADD.bwd_bias", "void mh::k_unb_planes<false>", 131072, 4 * _N3 + 256, "one launch, arrival tickets"),
    ("c4 [8192,8192] axis 0 MAX.fwd", "void mh::k_cols<mh::RMax, mh::LdPlain<mh::RMax>, true, true>", 262144,
     4 * _N4, "first of two launches (split partials)"),
    ("c4 [8192,8192] axis 0 MAX.bwd, route", "void mh::k_max_route_cols<true>", 262144, 4 * _N4,
     "grad read; x read again only in splits holding several maxima of a column; stores only quads "
     "holding a maximum"),
    ("c4 [8192,8192] axis 0 SUM.bwd", "void mh::k_colbc4<mh::FScaleBcast<false>, 1, true, -1>", 16777216, 8 * _N4, ""),
    ("c4 [8192,8192] axis 1 MAX.bwd", "void mh::k_max_bwd_rowreg<4, 8>", 2097152, 12 * _N4,
     "one pass; stores only quads holding a line maximum"),
    ("c4 [8192,8192] all MAX.bwd, route", "mh::k_max_route_rows", 8388608, 4 * _N4,
     "grad read; x read again only in the chunk holding the maximum; stores only quads holding it"),
    ("c4 [64,512,1024] axis 2 MAX.bwd", "void mh::k_max_bwd_rowreg<1, 4>", 2097152, 12 * (1 << 25),
     "one pass; stores only quads holding a line maximum"),
    ("c5 SUB.fwd [N,10] - [N,1]", "void mh::k_rowbc4<mh::FBin<1>, 2, false, 8>", 2621440, 8 * _N5 + 4 * (_N5 // 10), ""),
    ("c5 DIV.bwd0", "void mh::k_rowbc4<mh::FBinRg<3, 0, false>, 2, true, 8>", 2621440, 12 * _N5 + 4 * (_N5 // 10), ""),
    ("c5 DIV.bwd1 (un-broadcast into [N,1])", "void mh::k_rows_binrg<3, 1, false, 16, true>", 1048576,
     8 * _N5 + 12 * (_N5 // 10), "the rg terms computed in the loader, added into the gradient in row order"),
    ("c5 MAX.bwd (rows of 10)", "void mh::k_max_bwd_rows<16>", 1048576, 12 * _N5 + 8 * (_N5 // 10),
     "stores only quads holding a row maximum (most quads, at 10 classes)"),
    ("c5 fused head forward", "void mh::k_rowo_fwd<0, 10>", 1048576, 8 * _N5,
     "logits and targets read once; 64 KB of block partials written for k_loss_comb<0>"),
    ("c5 fused head backward", "void mh::k_rowo_bwd<0, 10>", 1048576, 16 * _N5, ""),
    ("CrossEntropy [32768,1000] backward", "void mh::k_roww_bwd<1, true, 16>", 2097152, 16 * 32768000, ""),
]


# (workload, group, op label, kernel-name prefix) of single-shape workload kernels whose
# rocprofv3 duration the stats summary sets beside the bench's figures
WL_STATS = [("c3", "op_by_op", "ADD.bwd_bias", "void mh::k_unb_planes<false>"),
            ("c3", "fused", "bias_relu.fwd", "mh::k_bias_relu_fwd_planes"),
            ("c3", "op_by_op", "ADD.fwd", "void mh::k_planebc4<mh::FBin<0>, 2, false, 8>"),
            ("c3", "fused", "bias_relu.bwd", ("void mh::k_bias_relu_bwd_flat<false, true, true, true>",
                                              "mh::k_bias_partials_comb8")),
            ("c4", "ops", "8192x8192.ax1.MAX.bwd", "void mh::k_max_bwd_rowreg<4, 8>"),
            ("c5", "fused", "fused.fwd", ("void mh::k_rowo_fwd<0, 10>", "void mh::k_loss_comb<0>")),
            ("c5", "fused", "fused.bwd", "void mh::k_rowo_bwd<0, 10>"),
            ("c5", "fwd", "SUB.fwd", "void mh::k_rowbc4<mh::FBin<1>, 2, false, 8>"),
            ("c5", "fwd", "DIV.fwd", "void mh::k_rowbc4<mh::FBin<3>, 2, false, 8>"),
            ("c5", "bwd", "DIV.bwd1", "void mh::k_rows_binrg<3, 1, false, 16, true>")]


def stats_summary(stats_csv, command, bench_json=None):
    """Writes profiles/bench_kernel_stats.md from a rocprofv3 --kernel-trace --stats
    kernel_stats.csv (durations in microseconds), with the command that made it."""
    rows = list(csv.DictReader(open(stats_csv, newline="")))
    lines = ["# rocprofv3 kernel statistics: bench.py (config 2 headline step + configs 3, 4, 5 and the copy reference)",
             "", "Command (run from the repository root on one MI355X):", "", "```", command, "```", "",
             "Durations in microseconds, as rocprofv3 `--stats` reports them (`*_kernel_stats.csv`). Counts include the",
             "bench's warm-up launches, the Infinity Cache flush before each small op (`k_rows_block<RSum, LdPlain>` over",
             "a 1 GiB buffer and its combine passes), gradient zeroing (`k_fill`) and input generation (`k_rand`).", "",
             "| Kernel | Calls | Avg us | Min us | Max us | % time |", "|---|---:|---:|---:|---:|---:|"]
    for r in rows:
        name = r["Name"].replace("|", "\\|")
        if len(name) > 120:
            name = name[:117] + "..."
        lines.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                     f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    if bench_json:
        rf = json.load(open(bench_json))["roofline"]
        lines += ["", "## Dominant config-2 kernel", "",
                  f"In the bench run of the same tree, `bench.py` (HIP events on the library stream) timed `{rf['kernel']}` "
                  f"at {rf['avg_launch_ms'] * 1e3:.1f} us per launch: {rf['achieved']} GB/s of algorithmic bytes "
                  f"({rf['bytes_per_launch']} B per launch), {rf['frac']:.3f} of 8 TB/s."]
        prefix = C2_KERNEL.get(rf["kernel"])
        match = [r for r in rows if prefix and r["Name"].startswith(prefix)]
        if match:
            avg = float(match[0]["AverageNs"]) / 1e3
            ev = rf["avg_launch_ms"] * 1e3
            lines.append(f"rocprofv3 averages `{match[0]['Name'].split('(')[0]}` at {avg:.1f} us over its "
                         f"{match[0]['Calls']} launches (the table above), {abs(avg - ev) / ev * 100:.1f} % from the "
                         f"event timing.")
        wl = json.load(open(bench_json)).get("workloads", {})
        rows_cmp = []
        for w, group, label, prefixes in WL_STATS:  # an op of two launches sums their averages
            rec = wl.get(w, {}).get(group, {}).get(label)
            prefixes = prefixes if isinstance(prefixes, tuple) else (prefixes,)
            matches = [[r for r in rows if r["Name"].startswith(pf)] for pf in prefixes]
            if rec and all(len(m) == 1 for m in matches):
                avg = sum(float(m[0]["AverageNs"]) for m in matches) / 1e3
                names = " + ".join(f"`{pf.replace('void ', '')}`" for pf in prefixes)
                rows_cmp.append(f"| {w} {label} | {names} | {avg:.2f} | {rec['ms'] * 1e3:.2f} | "
                                f"{rec['ms_isolated'] * 1e3:.2f} |")
        if rows_cmp:
            lines += ["", "## Workload kernels: rocprofv3 against the bench's two timings", "",
                      "A kernel of one launch shape in the bench: rocprofv3's average duration, the bench's streamed "
                      "figure (launches back to back over rotating cold buffers, elapsed / launches) and its isolated "
                      "one (a single launch between two events after a cache flush).", "",
                      "| Op | Kernel | rocprofv3 avg us | streamed us | isolated us |", "|---|---|---:|---:|---:|",
                      *rows_cmp]
    os.makedirs(os.path.dirname(TRAFFIC_JSON), exist_ok=True)
    with open(os.path.join(os.path.dirname(TRAFFIC_JSON), "bench_kernel_stats.md"), "w") as f:
        f.write("\n".join(lines) + "\n")


def traffic_summary_md(commands):
    """Writes profiles/traffic.md from profiles/traffic.json: the config-2 kernels' HBM bytes
    against their algorithmic bytes."""
    t = json.load(open(TRAFFIC_JSON))
    alg = dict(step_plan())
    lines = ["# HBM traffic per dispatch (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
             "Commands (run from the repository root on one MI355X; one counter per run):", "", "```", *commands, "```", "",
             f"Calibration: the library's copy kernel `k_copy` over a 1 GiB buffer (reads 1 GiB, writes 1 GiB) counts "
             f"FETCH_SIZE = {1 / t['fetch_scale']:.4f} x and WRITE_SIZE = {1 / t['write_scale']:.4f} x its bytes, so "
             f"FETCH_SIZE is scaled by {t['fetch_scale']:.4f} and WRITE_SIZE by {t['write_scale']:.4f}. Values are medians "
             "over the dispatches of each kernel's largest launch (for config 2, the 2^28-element one); "
             "`profiles/traffic.json` holds every kernel and launch size, and `bench.py` reads it for `roofline.traffic`.",
             "", "Config-2 kernels (2^28 fp32 elements per tensor):", "",
             "| Op | Kernel | Fetch GB | Write GB | HBM GB | Algorithmic GB |", "|---|---|---:|---:|---:|---:|"]
    for label, key in C2_KERNEL.items():
        hits = [(k, v) for k, v in t["kernels"].items() if k.startswith(key)]
        if len(hits) != 1:
            continue
        k, v = hits[0]
        short = k.split("(")[0].replace("void ", "")
        lines.append(f"| {label} | `{short}` | {(v['fetch_bytes'] or 0) / 1e9:.3f} | {(v['write_bytes'] or 0) / 1e9:.3f} | "
                     f"{v['hbm_bytes'] / 1e9:.3f} | {alg[label] * 2 ** 28 / 1e9:.3f} |")
    lines += ["", "Workload kernels (the launch of the named shape; algorithmic bytes of that kernel: inputs read "
              "once, outputs written once, accumulators read and written):", "",
              "| Workload op | Kernel | Fetch GB | Write GB | HBM GB | Algorithmic GB | Note |",
              "|---|---|---:|---:|---:|---:|---|"]
    for label, key, grid, nbytes, note in WL_KERNELS:
        hits = [v for k, v in t["kernels"].items() if k.startswith(key) and str(grid) in v["by_grid"]]
        if len(hits) != 1:
            continue
        v = hits[0]["by_grid"][str(grid)]
        short = key.replace("void ", "")
        lines.append(f"| {label} | `{short}` | {(v['fetch_bytes'] or 0) / 1e9:.4f} | {(v['write_bytes'] or 0) / 1e9:.4f} | "
                     f"{v['hbm_bytes'] / 1e9:.4f} | {nbytes / 1e9:.4f} | {note} |")
    with open(os.path.join(os.path.dirname(TRAFFIC_JSON), "traffic.md"), "w") as f:
        f.write("\n".join(lines) + "\n")


VALU_KERNELS = [  # (label, kernel-name prefix, elements per dispatch)
    ("c5 fused head forward [2^20, 10]", "void mh::k_rowo_fwd<0, 10>", _N5),
    ("c5 fused head backward [2^20, 10]", "void mh::k_rowo_bwd<0, 10>", _N5),
    ("c2 POW backward, x and exponent gradients (2^28)", "void mh::k_pow_grad_quads<true>(", 1 << 28),
    ("c2 TANH backward (2^28)", "void mh::k_same4<mh::FUnBwd<15>, 2, true>", 1 << 28),
    ("c2 MUL backward, both operands (2^28)", "void mh::k_bwd2_same4<2, false>", 1 << 28),
    ("c2 ADD forward (2^28)", "void mh::k_same4<mh::FBin<0>, 2, false>", 1 << 28),
]


def trace_summary(marker_csv, kernel_csv, command, out_md):
    """Writes `out_md`: each roctx range of a MANTLE_HIP_TRACE=1 run (rocprofv3 --marker-trace
    --kernel-trace) in call order with the kernels that ran inside it. A kernel belongs to the
    innermost range whose host interval contains its execution (the library synchronises at the
    end of each call unless initialised asynchronous, as the traced program here is not)."""
    import csv
    with open(marker_csv) as f:
        ranges = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Function"]) for r in csv.DictReader(f)]
    with open(kernel_csv) as f:
        kernels = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]) for r in csv.DictReader(f)]
    ranges.sort()
    inside = {i: [] for i in range(len(ranges))}
    for ks, ke, kn in kernels:
        best = None
        for i, (rs, re_, _) in enumerate(ranges):
            if rs <= ks and ke <= re_ and (best is None or re_ - rs < ranges[best][1] - ranges[best][0]):
                best = i
        if best is not None:
            inside[best].append((kn, (ke - ks) / 1e3))
    lines = ["# roctx ranges of a traced run (MANTLE_HIP_TRACE=1)", "",
             "Commands (run from the repository root on one MI355X):", "", "```", *command, "```", "",
             "Each entry point that queues GPU work opens a range named after itself (and its op); the "
             "kernels that ran inside it follow, with their durations in microseconds.", "",
             "| # | Range | Host us | Kernels (us) |", "|---:|---|---:|---|"]
    for i, (rs, re_, name) in enumerate(ranges):
        ks = ", ".join(f"`{n.split('(')[0]}` {d:.1f}" for n, d in inside[i]) or "—"
        lines.append(f"| {i + 1} | `{name}` | {(re_ - rs) / 1e3:.1f} | {ks} |")
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")


def valu_summary(csv_paths, command):
    """Writes profiles/valu_per_element.md from rocprofv3 --pmc SQ_INSTS_VALU SQ_WAVES runs:
    wave-level VALU instructions per element (SQ_INSTS_VALU * 64 / elements) of the kernels in
    VALU_KERNELS (median over each kernel's dispatches of the named size)."""
    vals = {}
    for path in csv_paths:
        for r in csv.DictReader(open(path, newline="")):
            vals.setdefault((r["Kernel_Name"], r["Counter_Name"]), []).append(float(r["Counter_Value"]))
    lines = ["# VALU instructions per element (rocprofv3 SQ_INSTS_VALU)", "",
             "Commands (run from the repository root on one MI355X):", "", "```", *command, "```", "",
             "SQ_INSTS_VALU counts wave-level vector ALU instructions, summed over the device; one covers 64 lanes, "
             "so VALU per element = SQ_INSTS_VALU x 64 / elements. At 256 CUs issuing one wave-level VALU "
             "instruction per cycle each at 2.4 GHz (614 G/s), the last column is the time that instruction count "
             "alone would take.", "",
             "| Kernel (workload) | Kernel | SQ_INSTS_VALU | SQ_WAVES | VALU / element | VALU time at 614 G/s (us) |",
             "|---|---|---:|---:|---:|---:|"]
    for label, prefix, n in VALU_KERNELS:
        keys = [k for k in vals if k[0].startswith(prefix) and k[1] == "SQ_INSTS_VALU"]
        if len(keys) != 1:
            continue
        v = statistics.median(vals[keys[0]])
        w = statistics.median(vals.get((keys[0][0], "SQ_WAVES"), [0]))
        lines.append(f"| {label} | `{prefix.replace('void ', '')}` | {v:.0f} | {w:.0f} | {v * 64 / n:.1f} | "
                     f"{v / 614e9 * 1e6:.2f} |")
    with open(os.path.join(os.path.dirname(TRAFFIC_JSON), "valu_per_element.md"), "w") as f:
        f.write("\n".join(lines) + "\n")


def traffic_for(label):
    if not os.path.exists(TRAFFIC_JSON):
        return None
    with open(TRAFFIC_JSON) as f:
        kernels = json.load(f)["kernels"]
    key = C2_KERNEL.get(label)
    hits = [v for k, v in kernels.items() if key and k.startswith(key)]
    return round(hits[0]["hbm_bytes"]) if len(hits) == 1 else None


# ---------------------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--log2n", type=int, default=28)
    ap.add_argument("--workloads", default="c3,c4,c5,adam,adj,rows,graph,copy",
                    help="extra workloads after the headline step (comma list of c3,c4,c5,adam,adj,rows,graph,"
                         "copy; 'none')")
    ap.add_argument("--reps", type=int, default=10, help="repetitions per op of the extra workloads")
    ap.add_argument("--cpu-log2n", type=int, default=23)
    ap.add_argument("--cpu-reps", type=int, default=5, help="timed passes of each CPU baseline (after 1 warm-up)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="write profiles/traffic.json and traffic.md from two rocprofv3 --pmc runs and exit")
    ap.add_argument("--stats-summary", metavar="KERNEL_STATS_CSV",
                    help="write profiles/bench_kernel_stats.md from a rocprofv3 --stats run and exit")
    ap.add_argument("--command", default="", help="the rocprofv3 command(s) a summary records (';'-separated)")
    ap.add_argument("--bench-json", default=None, help="a bench JSON line of the same tree (for --stats-summary)")
    ap.add_argument("--trace-summary", nargs=2, metavar=("MARKER_CSV", "KERNEL_CSV"),
                    help="write profiles/trace_ranges_smoke.md from a MANTLE_HIP_TRACE=1 rocprofv3 "
                         "--marker-trace --kernel-trace run and exit")
    ap.add_argument("--valu-summary", nargs="+", metavar="PMC_CSV",
                    help="write profiles/valu_per_element.md from rocprofv3 --pmc SQ_INSTS_VALU SQ_WAVES runs and exit")
    args = ap.parse_args()
    if args.trace_summary:
        out = os.path.join(os.path.dirname(TRAFFIC_JSON), "trace_ranges_smoke.md")
        trace_summary(args.trace_summary[0], args.trace_summary[1],
                      [c.strip() for c in args.command.split(";") if c.strip()] +
                      [f"python bench.py --trace-summary {args.trace_summary[0]} {args.trace_summary[1]}"], out)
        return
    if args.valu_summary:
        valu_summary(args.valu_summary, [c.strip() for c in args.command.split(";") if c.strip()] +
                     [f"python bench.py --valu-summary {' '.join(args.valu_summary)}"])
        return
    if args.pmc_summary:
        s = pmc_summary(*args.pmc_summary)
        traffic_summary_md([c.strip() for c in args.command.split(";") if c.strip()] +
                           [f"python bench.py --pmc-summary {args.pmc_summary[0]} {args.pmc_summary[1]}"])
        print(json.dumps({"fetch_scale": s["fetch_scale"], "write_scale": s["write_scale"]}))
        return
    if args.stats_summary:
        stats_summary(args.stats_summary, args.command, args.bench_json)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py: this build runs the op layer on one GPU; --gpus {args.gpus} "
              f"(WORLD_SIZE={world}) is not supported: every op family would shard by contiguous slices "
              f"with exchanges of at most 32 KB, and only one GPU's share is built and measured.",
              file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    from mantle_amd._lib import lib
    L = lib()
    n = 1 << args.log2n
    log(f"init, n = 2^{args.log2n}")
    from mantle_amd import init as mh_init_py
    mh_init_py(0, asynchronous=True)  # MH_INIT_ASYNC: no host sync per call (and mantle_amd knows it)
    r = run_c2(L, n, args.steps, args.warmup) if args.steps > 0 else None
    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seeded: device SplitMix64 for config 2, numpy SFC64 for configs 3-5)"}
    if r is not None:
        K = args.steps
        value = r["bytes_per_step"] / (r["ms_per_step"] * 1e-3) / 1e9
        plan = r["plan"]
        ops = {}
        for label, avg in r["op_ms"].items():
            gbs = plan[label] * n / (avg * 1e-3) / 1e9
            ops[label] = {"ms": round(avg, 4), "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}
        dom = max(r["op_ms"], key=r["op_ms"].get)
        dom_ms = r["op_ms"][dom]
        dom_bytes = plan[dom] * n
        achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
        out.update({
            "value": round(value, 1), "unit": "GB/s", "ms_per_step": round(r["ms_per_step"], 4),
            "config": {"workload": "config2: fp32 2^28-element elementwise fwd+bwd "
                                   "(ADD/SUB/MUL/DIV/EXP/LOG/TANH/SIGMOID/RELU/POW)",
                       "elements": n, "bytes_per_step": r["bytes_per_step"], "pow_exponent": r["expo"],
                       "frac_of_peak": round(value / PEAK_GBS, 4), "elements_per_s": round(n / (r["ms_per_step"] * 1e-3)),
                       "wall_s": round(r["wall"], 3)},
            "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS,
                         "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic_for(dom),
                         "bytes_per_launch": dom_bytes, "avg_launch_ms": round(dom_ms, 4)},
            "ops": ops})
        log(f"c2: {value:.1f} GB/s, {r['ms_per_step']:.3f} ms/step")
    wl = [w for w in args.workloads.split(",") if w and w != "none"]
    runners = {"c3": lambda: run_c3(L, args.reps), "c4": lambda: run_c4(L, args.reps),
               "c5": lambda: run_c5(L, args.reps), "adam": lambda: run_adam(L, args.reps),
               "adj": lambda: run_adj(L, args.reps), "rows": lambda: run_rows(L, args.reps),
               "graph": lambda: run_graph(L, args.reps),
               "copy": lambda: run_copy(L, args.reps)}
    if wl:
        out["workloads"] = {}
    for w in wl:
        log(f"workload {w}")
        out["workloads"][w] = runners[w]()
    if rank == 0 and not args.no_cpu_baseline and r is not None:
        log("cpu baseline")
        out["cpu_baseline"] = cpu_baseline(1 << args.cpu_log2n, args.cpu_reps, r["expo"])
    elif rank == 0:
        out["cpu_baseline"] = None
    if rank == 0:
        out["summary"] = summary(out)  # last: the end of the line holds every config
        print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
