"""Writes tests/golden/config_goldens.json: the oracle's outputs of the five BASELINE.json
configurations at full size (tests/golden/config_workloads.py), as
  bit outputs   SHA-256 of the full float32 array, plus a seeded slice of its values (bits);
  sum outputs   a seeded slice (every value for short outputs: config 3's 32-value bias
                gradient in full) of the oracle's values, their fp64 sums and the fp64 sums
                of the terms' magnitudes.
Run from the repository root (builds nothing; needs oracle/liboracle.so and about 12 GB of
memory, about two minutes on one core of the GPU box's host, where the committed fixture was
written; no GPU is used):  python tests/golden/make_config_goldens.py [--out PATH]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.dirname(HERE), os.path.dirname(os.path.dirname(HERE)), HERE]

import config_workloads as W  # noqa: E402
from util import OracleEngine  # noqa: E402


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


def entry(key, out, kind, exact, terms_abs):
    out = np.asarray(out, np.float32)
    idx = W.slice_idx(out.size, key)
    flat = out.reshape(-1)
    e = {"kind": kind, "shape": list(out.shape), "idx": idx.tolist(),
         "bits": flat[idx].view(np.uint32).tolist()}
    if kind == "bit":
        e["sha256"] = sha256(out)
    else:
        e["exact"] = np.asarray(exact, np.float64).reshape(-1)[idx].tolist()
        e["terms_abs"] = np.asarray(terms_abs, np.float64).reshape(-1)[idx].tolist()
    return e


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=os.path.join(HERE, "config_goldens.json"))
    args = ap.parse_args()
    eng = OracleEngine()
    fixture, cache = {}, {}
    for config, part in W.workloads():
        wkey = config if part is None else f"{config}.{part}"
        t0 = time.time()
        fixture[wkey] = {}
        for name, out, kind, exact, terms_abs in W.run(eng, config, part, cache):
            fixture[wkey][name] = entry(f"{wkey}.{name}", out, kind, exact, terms_abs)
            print(f"  {wkey}.{name} ({time.time() - t0:.1f} s)", flush=True)
            del out
        print(f"{wkey}: {len(fixture[wkey])} outputs, {time.time() - t0:.1f} s", flush=True)
        if config == "c2" and part == "pow":
            cache.clear()
    os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
    with open(args.out, "w") as f:
        json.dump(fixture, f, separators=(",", ":"))


if __name__ == "__main__":
    main()
