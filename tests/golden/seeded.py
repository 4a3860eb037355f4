"""Deterministic test values that do not depend on any library's random stream.

The golden fixtures in this folder were written by running the reference's own modules on
these values; the tests regenerate the same values to feed the oracle and the HIP path.
Every value is a pure function of (seed, element index) through the splitmix64 mixer
(Steele, Lea and Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014), so
neither numpy's nor torch's generator versions can change them.  Each fixture also stores a
SHA-256 of the values it was made from, which the tests check before comparing outputs.
"""

from __future__ import annotations

import hashlib
import zlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _splitmix64(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = x + _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, shape, low: float = -1.0, high: float = 1.0) -> np.ndarray:
    """float32 values on a 2**-24 grid of [low, high), element i from splitmix64(seed, i)."""

    n = int(np.prod(shape, dtype=np.int64))
    with np.errstate(over="ignore"):
        base = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * _GOLDEN
        z = _splitmix64(np.arange(n, dtype=np.uint64) + base)
    u = (z >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    return (low + (high - low) * u).astype(np.float32).reshape(shape)


def integers(seed: int, shape, low: int, high: int) -> np.ndarray:
    """int64 values in [low, high) (high - low < 2**24), element i from splitmix64(seed, i)."""

    n = int(np.prod(shape, dtype=np.int64))
    with np.errstate(over="ignore"):
        base = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) * _GOLDEN
        z = _splitmix64(np.arange(n, dtype=np.uint64) + base)
    span = high - low
    return (low + ((z >> np.uint64(40)) % np.uint64(span)).astype(np.int64)).reshape(shape)


def _is_gain(name: str) -> bool:
    return name.endswith(("norm.weight", "ln_attn.weight", "ln_mlp.weight"))


def state_values(shapes: dict[str, tuple[int, ...]], seed: int) -> dict[str, np.ndarray]:
    """A perturbed parameter set for a module with the given parameter names and shapes.

    Norm gains are 1 + U(-0.1, 0.1), biases U(-0.05, 0.05), matrices and tables
    U(-a, a) with a = sqrt(3) / sqrt(fan_in) for matrices (unit-variance products) and
    a = 0.2 for embedding tables.  Each tensor's stream is keyed by its name, so the values
    do not depend on the order the names are listed in."""

    out = {}
    for name, shape in shapes.items():
        key = seed * 1_000_003 + zlib.crc32(name.encode())
        if _is_gain(name):
            out[name] = 1.0 + uniform(key, shape, -0.1, 0.1)
        elif name.endswith(".bias"):
            out[name] = uniform(key, shape, -0.05, 0.05)
        elif len(shape) == 2 and not name.endswith(("fields.weight", "code.weight", "rank.weight")):
            a = float(np.sqrt(3.0 / shape[1]))
            out[name] = uniform(key, shape, -a, a)
        elif len(shape) == 3:  # Conv1d [out, in, kernel]
            a = float(np.sqrt(3.0 / (shape[1] * shape[2])))
            out[name] = uniform(key, shape, -a, a)
        else:
            out[name] = uniform(key, shape, -0.2, 0.2)
        out[name] = out[name].astype(np.float32)
    return out


def digest(arrays: dict[str, np.ndarray]) -> str:
    """SHA-256 over the arrays' names, shapes, dtypes and bytes, in name order."""

    h = hashlib.sha256()
    for name in sorted(arrays):
        a = np.ascontiguousarray(arrays[name])
        h.update(name.encode())
        h.update(str(a.shape).encode())
        h.update(str(a.dtype).encode())
        h.update(a.tobytes())
    return h.hexdigest()
