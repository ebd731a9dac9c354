"""Seeded synthetic inputs for the benchmark configurations and the tests.

Each tensor is drawn from its own stream: numpy's SFC64 generator seeded with
SeedSequence((seed, tensor_id)), so a tensor's bytes do not depend on which other tensors were
drawn (and 2^28-element tensors take about a second each). ``normal(mean, std)`` takes
the standard deviation, as Mantle's ``rand_normal(mean, std)`` does
(mantle/core/rand_utils.mojo:48-63).
"""
from __future__ import annotations

import numpy as np

SEED = 42  # mantle/__init__.mojo:23


def rng(tensor_id: int, seed: int = SEED) -> np.random.Generator:
    return np.random.Generator(np.random.SFC64(np.random.SeedSequence([int(seed), int(tensor_id)])))


def uniform(shape, lo: float, hi: float, tensor_id: int, seed: int = SEED) -> np.ndarray:
    g = rng(tensor_id, seed)
    u = g.random(size=shape, dtype=np.float32)
    u *= np.float32(hi - lo)
    u += np.float32(lo)
    return u


def normal(shape, mean: float, std: float, tensor_id: int, seed: int = SEED) -> np.ndarray:
    g = rng(tensor_id, seed)
    z = g.standard_normal(size=shape, dtype=np.float32)
    if std != 1.0:
        z *= np.float32(std)
    if mean != 0.0:
        z += np.float32(mean)
    return z


def integers(shape, lo: int, hi: int, tensor_id: int, seed: int = SEED) -> np.ndarray:
    return rng(tensor_id, seed).integers(lo, hi, size=shape)


def inject_ties(x: np.ndarray, axis: int, tensor_id: int, seed: int = SEED) -> np.ndarray:
    """Copies each even-indexed reduction line's maximum to a second position on that line
    (exact ties for MAX backward). Works in place on a contiguous array and returns it."""
    g = rng(tensor_id, seed)
    xm = np.moveaxis(x, axis, -1)  # view
    d = xm.shape[-1]
    lines = xm.reshape(-1, d) if xm.flags.c_contiguous else None
    if lines is None:
        flat = xm.reshape(-1, d).copy()
    else:
        flat = lines
    if d < 2:
        return x
    idx = np.arange(0, flat.shape[0], 2)
    amax = flat[idx].argmax(axis=1)
    other = (amax + 1 + g.integers(0, d - 1, size=idx.size)) % d
    flat[idx, other] = flat[idx, amax]
    if lines is None:
        xm[...] = flat.reshape(xm.shape)
    return x
