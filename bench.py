"""Benchmark: Mantle's elementwise op layer on one MI355X.

A step is one forward + backward pass of every config-2 op over 2^28-element fp32 tensors
already resident in HBM:
  ADD/SUB/MUL/DIV   fwd (a ~ U(-1,1), b ~ U(0.5,2)) and the backward of both operands,
  EXP (x ~ U(-10,10)), LOG (x ~ U(1e-3,10)), TANH/SIGMOID/RELU (x ~ N(0,3))  fwd and bwd,
  POW (base ~ U(0.1,4), one seeded scalar exponent ~ U(0.5,3))  fwd, bwd of x, bwd of the exponent.
Throughput is algorithmic bytes per step / step time (inputs read once, outputs written once,
accumulated gradients read and written). Per-op times come from HIP events recorded on the
library's stream between the ops of each timed step.

Prints one JSON line. `--gpus N` with N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "elementwise/broadcast/reduce fwd+bwd: achieved HBM GB/s and % of MI355X peak"
PEAK_GBS = 8000.0
SEED = 42

# (name, algorithmic bytes per element)
BINARY = ["ADD", "SUB", "MUL", "DIV"]
UNARY = ["EXP", "LOG", "TANH", "SIGMOID", "RELU"]
OP_ID = {"ADD": 0, "SUB": 1, "MUL": 2, "DIV": 3, "EXP": 4, "LOG": 5, "POW": 6, "SIGMOID": 13,
         "RELU": 14, "TANH": 15}
BWD2_BYTES = {"ADD": 20, "SUB": 20, "MUL": 28, "DIV": 28}  # ug (+a, b), both grads read+written


def step_plan():
    """[(label, bytes per element)] in execution order."""
    plan = []
    for op in BINARY:
        plan += [(f"{op}.fwd", 12), (f"{op}.bwd", BWD2_BYTES[op])]
    for op in UNARY:
        plan += [(f"{op}.fwd", 8), (f"{op}.bwd", 16)]
    plan += [("POW.fwd", 8), ("POW.bwd_x", 16), ("POW.bwd_exp", 8)]
    return plan


class Dev:
    """Owns the device tensors of the workload (raw mh_malloc pointers)."""

    def __init__(self, L, n):
        self.L, self.n, self.ptrs = L, n, {}

    def alloc(self, name, n=None):
        p = ctypes.c_void_p()
        n = self.n if n is None else n
        rc = self.L.mh_malloc(ctypes.byref(p), n * 4)
        if rc:
            raise RuntimeError(f"mh_malloc({name}): {self.L.mh_last_error().decode()}")
        self.ptrs[name] = p.value
        return p.value

    def free(self):
        for p in self.ptrs.values():
            self.L.mh_free(p)


def chk(L, rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: [{rc}] {L.mh_last_error().decode()}")


def setup_gpu(L, n):
    d = Dev(L, n)
    P = d.alloc
    gens = [("a", "u", -1, 1), ("b", "u", 0.5, 2), ("ug", "n", 0, 1), ("x_exp", "u", -10, 10),
            ("x_log", "u", 1e-3, 10), ("x_act", "n", 0, 3), ("x_pow", "u", 0.1, 4)]
    for i, (name, kind, p, q) in enumerate(gens):
        ptr = P(name)
        fn = L.mh_rand_uniform if kind == "u" else L.mh_rand_normal
        chk(L, fn(ptr, n, SEED * 1000 + i, p, q), f"rand {name}")
    for name in ("res", "ga", "gb", "gx"):
        chk(L, L.mh_zero(P(name), n), f"zero {name}")
    e = P("exp", 1)
    ge = P("gexp", 1)
    expo = np.array([np.float32(0.5 + 2.5 * np.random.default_rng(SEED).random())], np.float32)
    chk(L, L.mh_memcpy_h2d(e, expo.ctypes.data, 4), "exponent")
    chk(L, L.mh_zero(ge, 1), "zero gexp")
    chk(L, L.mh_sync(), "sync")
    return d, float(expo[0])


def make_step(L, d, n):
    from mantle_amd._lib import make_shape
    s = make_shape((n,))
    p = d.ptrs
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
    calls.append(("POW.bwd_x", lambda: L.mh_pow_bwd_accum(0, p["gx"], p["x_pow"], p["exp"], p["ug"], n)))
    calls.append(("POW.bwd_exp", lambda: L.mh_pow_bwd_accum(1, p["gexp"], p["x_pow"], p["exp"], p["ug"], n)))
    return calls


def cpu_baseline(n_sample: int, reps: int, expo: float):
    """The CPU restatement (oracle/, single thread, like the reference's elementwise paths)
    on the same op sequence over a bounded sample; GB/s with the same byte accounting."""
    from oracle import oracle as O
    from mantle_amd import synth
    a = synth.uniform((n_sample,), -1, 1, 1)
    b = synth.uniform((n_sample,), 0.5, 2, 2)
    ug = synth.normal((n_sample,), 0, 1, 3)
    xs = {"EXP": synth.uniform((n_sample,), -10, 10, 4), "LOG": synth.uniform((n_sample,), 1e-3, 10, 5)}
    xs["TANH"] = xs["SIGMOID"] = xs["RELU"] = synth.normal((n_sample,), 0, 3, 6)
    xp = synth.uniform((n_sample,), 0.1, 4, 7)
    e = np.array([expo], np.float32)
    ga = np.zeros(n_sample, np.float32)
    best = None
    for _ in range(reps):
        t0 = time.perf_counter()
        for op in BINARY:
            o = OP_ID[op]
            O.forward_op(o, a, b)
            ga = O.backward_op(0, o, ug, a, b, grad=ga)
            ga = O.backward_op(1, o, ug, a, b, grad=ga)
        for op in UNARY:
            O.forward_op(OP_ID[op], xs[op])
            ga = O.backward_op(0, OP_ID[op], ug, xs[op], grad=ga)
        O.forward_op(6, xp, e)
        ga = O.backward_op(0, 6, ug, xp, e, grad=ga)
        O.backward_op(1, 6, ug, xp, e)
        dt = time.perf_counter() - t0
        best = dt if best is None else min(best, dt)
    bytes_per_elem = sum(b for _, b in step_plan())
    return {"value": round(bytes_per_elem * n_sample / best / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"same op sequence on {n_sample} elements per tensor (1/{(1 << 28) // n_sample} of the "
                      f"workload), best of {reps}, {best:.2f} s per pass; single-threaded C restatement "
                      f"(oracle/mantle_oracle.c, -O3)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--log2n", type=int, default=28)
    ap.add_argument("--cpu-log2n", type=int, default=24)
    ap.add_argument("--cpu-reps", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print(f"bench.py: this build runs the op layer on one GPU; --gpus {args.gpus} "
              f"(WORLD_SIZE={world}) is not supported. Multi-GPU sharding is described in DESIGN.md.",
              file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))

    from mantle_amd._lib import lib
    L = lib()
    n = 1 << args.log2n
    print(f"[bench] init, n = 2^{args.log2n}", file=sys.stderr, flush=True)
    chk(L, L.mh_init(0, 1), "mh_init")  # MH_INIT_ASYNC: no host sync per call
    d, expo = setup_gpu(L, n)
    calls = make_step(L, d, n)
    plan = dict(step_plan())
    evs = []
    for _ in range(len(calls) + 1):
        e = ctypes.c_void_p()
        chk(L, L.mh_event_create(ctypes.byref(e)), "event")
        evs.append(e.value)

    def run_step(timed):
        if timed:
            chk(L, L.mh_event_record(evs[0]), "record")
        for i, (label, fn) in enumerate(calls):
            chk(L, fn(), label)
            if timed:
                chk(L, L.mh_event_record(evs[i + 1]), "record")

    for _ in range(args.warmup):
        run_step(False)
    chk(L, L.mh_sync(), "sync")
    print(f"[bench] warmup done ({args.warmup} steps)", file=sys.stderr, flush=True)

    op_ms = {label: 0.0 for label, _ in calls}
    ms = ctypes.c_float()
    t0 = time.perf_counter()
    step_ms_sum = 0.0
    for _ in range(args.steps):
        run_step(True)
        chk(L, L.mh_sync(), "sync")
        for i, (label, _) in enumerate(calls):
            chk(L, L.mh_event_elapsed_ms(ctypes.byref(ms), evs[i], evs[i + 1]), "elapsed")
            op_ms[label] += ms.value
        chk(L, L.mh_event_elapsed_ms(ctypes.byref(ms), evs[0], evs[-1]), "elapsed")
        step_ms_sum += ms.value
    wall = time.perf_counter() - t0
    K = args.steps
    ms_per_step = step_ms_sum / K
    bytes_per_step = sum(plan.values()) * n
    value = bytes_per_step / (ms_per_step * 1e-3) / 1e9
    ops = {}
    for label, tot in op_ms.items():
        avg = tot / K
        ops[label] = {"ms": round(avg, 4), "GB/s": round(plan[label] * n / (avg * 1e-3) / 1e9, 1),
                      "frac": round(plan[label] * n / (avg * 1e-3) / 1e9 / PEAK_GBS, 4)}
    dom = max(op_ms, key=op_ms.get)
    dom_avg_ms = op_ms[dom] / K
    dom_bytes = plan[dom] * n
    achieved = dom_bytes / (dom_avg_ms * 1e-3) / 1e9
    roof = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4), "traffic": None, "bytes_per_launch": dom_bytes,
            "avg_launch_ms": round(dom_avg_ms, 4)}
    out = {"metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": K,
           "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seeded device SplitMix64: U/N as in config 2)",
           "config": {"workload": "config2: fp32 2^28-element elementwise fwd+bwd "
                                  "(ADD/SUB/MUL/DIV/EXP/LOG/TANH/SIGMOID/RELU/POW)",
                      "elements": n, "bytes_per_step": bytes_per_step, "pow_exponent": expo,
                      "frac_of_peak": round(value / PEAK_GBS, 4), "wall_s": round(wall, 3)},
           "roofline": roof, "ops": ops}
    d.free()
    for e in evs:
        L.mh_event_destroy(e)
    if rank == 0 and not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(1 << args.cpu_log2n, args.cpu_reps, expo)
    elif rank == 0:
        out["cpu_baseline"] = None
    if rank == 0:
        print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
