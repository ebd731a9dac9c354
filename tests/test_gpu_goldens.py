"""The HIP path against the committed golden fixture of the five BASELINE.json configurations
at full size (tests/golden/config_goldens.json, written from the oracle by
tests/golden/make_config_goldens.py): bit outputs by SHA-256 of the whole array (on a
mismatch the seeded slice names the first differing value), sums in the rtol class on their
seeded slice against the fp64 values."""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import pytest

from util import GpuEngine, assert_sum_close

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import config_workloads as W  # noqa: E402

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(HERE, "golden", "config_goldens.json")
_CACHE: dict = {}


@pytest.fixture(scope="module")
def gpu():
    print("\n[gpu] init device 0", flush=True)
    return GpuEngine()


def _fixture():
    if "fixture" not in _CACHE:
        with open(GOLDEN) as f:
            _CACHE["fixture"] = json.load(f)
    return _CACHE["fixture"]


def _check(key, got, e):
    got = np.asarray(got, np.float32)
    assert list(got.shape) == e["shape"], f"{key}: shape {got.shape} vs {e['shape']}"
    flat = got.reshape(-1)
    idx = np.asarray(e["idx"], np.int64)
    ref = np.asarray(e["bits"], np.uint32).view(np.float32)
    if e["kind"] == "bit":
        h = hashlib.sha256(np.ascontiguousarray(got).tobytes()).hexdigest()
        if h != e["sha256"]:
            diff = np.flatnonzero(flat[idx].view(np.uint32) != ref.view(np.uint32))
            where = (f"slice index {int(idx[diff[0]])}: {flat[idx[diff[0]]]!r} vs {ref[diff[0]]!r}" if diff.size
                     else "the seeded slice agrees")
            raise AssertionError(f"{key}: SHA-256 differs from the golden ({where})")
    else:
        assert_sum_close(flat[idx], ref, np.asarray(e["exact"]), key, terms_abs=np.asarray(e["terms_abs"]))


@pytest.mark.parametrize("config,part", W.workloads(),
                         ids=[c if p is None else f"{c}.{p}" for c, p in W.workloads()])
def test_config_golden(gpu, config, part):
    wkey = config if part is None else f"{config}.{part}"
    want = _fixture()[wkey]
    seen = []
    for name, out, _kind, _exact, _terms in W.run(gpu, config, part, _CACHE):
        print(f"[golden] {wkey}.{name}", flush=True)
        _check(f"{wkey}.{name}", out, want[name])
        seen.append(name)
        del out
    assert sorted(seen) == sorted(want), f"{wkey}: outputs {sorted(seen)} vs golden {sorted(want)}"
    if config == "c2" and part == "pow":
        _CACHE.pop("c2", None)
