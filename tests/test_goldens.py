"""The committed golden fixture of the BASELINE.json configurations (no GPU): every workload and
output present, config 1 recomputed by the oracle here matching its hashes and values, and
every sum entry's oracle value within the sum class of its fp64 value."""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

from util import OracleEngine

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import config_workloads as W  # noqa: E402

GOLDEN = os.path.join(HERE, "golden", "config_goldens.json")


def _load():
    with open(GOLDEN) as f:
        return json.load(f)


def test_fixture_covers_every_workload():
    fx = _load()
    want = {c if p is None else f"{c}.{p}" for c, p in W.workloads()}
    assert set(fx) == want
    for wkey, outs in fx.items():
        assert outs, wkey
        for name, e in outs.items():
            n = int(np.prod(e["shape"]))
            assert len(e["idx"]) == len(e["bits"]) == min(n, W.SLICE), (wkey, name)
            assert e["kind"] in ("bit", "sum")
            if e["kind"] == "bit":
                assert len(e["sha256"]) == 64
            else:
                assert len(e["exact"]) == len(e["terms_abs"]) == len(e["idx"])
    # config 3's bias gradient is committed whole (32 channels)
    assert fx["c3"]["grad_bias"]["shape"] == [1, 32, 1, 1] and len(fx["c3"]["grad_bias"]["idx"]) == 32


def test_config1_recomputed_by_the_oracle():
    fx = _load()["c1"]
    for name, out, kind, exact, terms_abs in W.config1(OracleEngine()):
        e = fx[name]
        out = np.asarray(out, np.float32)
        flat = out.reshape(-1)
        idx = np.asarray(e["idx"])
        assert flat[idx].view(np.uint32).tolist() == e["bits"], name
        if kind == "bit":
            assert hashlib.sha256(np.ascontiguousarray(out).tobytes()).hexdigest() == e["sha256"], name
        else:
            np.testing.assert_allclose(np.asarray(exact).reshape(-1)[idx], e["exact"], rtol=0, atol=0)


def test_sum_entries_are_in_the_sum_class():
    """The oracle's fp32 sums sit within 1e-5 of the sum of their terms' magnitudes from the
    fp64 value (measured: at most 5e-7); relative to the value itself a sum with
    cancellation can be further off, which is why the comparator has that clause."""
    for wkey, outs in _load().items():
        for name, e in outs.items():
            if e["kind"] != "sum":
                continue
            ref = np.asarray(e["bits"], np.uint32).view(np.float32).astype(np.float64)
            err = np.abs(ref - np.asarray(e["exact"]))
            assert (err <= 1e-5 * np.asarray(e["terms_abs"])).all(), f"{wkey}.{name}: oracle sum off its fp64 value"
