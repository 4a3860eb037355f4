"""Shapes and inputs of the golden cases, shared by make_golden.py and the tests.

Nothing here imports the reference: the inputs are pure functions of fixed seeds
(``seeded.py``), so the tests can rebuild them on any machine.
"""

from __future__ import annotations

import numpy as np

try:
    from . import seeded
except ImportError:  # run as a script from this folder
    import seeded

# cfg1's trunk shape (8 layers, d_model 256, 8 query / 2 KV heads, head_dim 32, MLP 4x).
TRUNK = {"d_model": 256, "n_layers": 8, "n_heads": 8, "n_kv_heads": 2, "d_ff": 1024, "seed": 11}

# One token per game; gathered rows; game 3 restarts at length 0 over a stale prefix.
STEP1 = {"name": "step1", "seed": 21, "capacity": 24, "max_len": 64, "games": 16, "T": 1}
# A padded run of 4 tokens with 1-4 real ones; rows near the pool's end clamp their
# padding onto the reserved last slot.
CHUNK = {"name": "chunk", "seed": 31, "capacity": 24, "max_len": 64, "games": 16, "T": 4}

# The reference actor's default embedder (PiquetModelConfig(): d_model 256, card width 32,
# hidden 64, 2 grid blocks, kernel 3) with its trunk's PLE (16 layers x 64) and
# alternating value embeddings (8 layers x 64).
PIQUET = {"seed": 41, "tokens": 12, "ple_width": 1024, "value_width": 512}


def _permutation(seed: int, n: int) -> np.ndarray:
    return np.argsort(seeded.uniform(seed, (n,), 0.0, 1.0), kind="stable").astype(np.int64)


def trunk_inputs(case: dict) -> dict[str, np.ndarray]:
    """x [B, T, d] (pre-conditioning embedding sums), positions [B], rows [B], readout [B],
    counts [B] (real tokens per row; the rest repeat the last real one)."""

    seed, B, T, max_len = case["seed"], case["games"], case["T"], case["max_len"]
    rows = _permutation(seed + 1, case["capacity"])[:B]
    if T == 1:
        counts = np.ones(B, dtype=np.int64)
        positions = seeded.integers(seed + 2, (B,), 1, max_len - 4)
        positions[3] = 0  # a fresh game in a reused slot
        positions[5] = max_len - 2  # the last slot before the reserved one
    else:
        counts = seeded.integers(seed + 3, (B,), 1, T + 1)
        positions = seeded.integers(seed + 2, (B,), 0, max_len - T - 1)
        positions[2], counts[2] = max_len - 3, 2  # padding clamps twice onto the last slot
        positions[6], counts[6] = max_len - 2, 1  # padding clamps three times
        positions[9], counts[9] = max_len - 4, 3  # padding lands once on the last slot
        positions[12], counts[12] = 0, 4  # a fresh game's first chunk
    x = seeded.uniform(seed + 4, (B, T, TRUNK["d_model"]), -1.0, 1.0)
    for b in range(B):
        x[b, counts[b]:] = x[b, counts[b] - 1]
    return {"x": x, "positions": positions.astype(np.int64), "rows": rows, "readout": counts - 1,
            "counts": counts.astype(np.int64)}


def pool_contents(case: dict) -> tuple[np.ndarray, np.ndarray]:
    """The pool before the step: finite values in every slot of every row (stale games'
    leftovers included), [layers, capacity, kv_heads, max_len, head_dim] float32 holding
    bf16-representable values."""

    head_dim = TRUNK["d_model"] // TRUNK["n_heads"]
    shape = (TRUNK["n_layers"], case["capacity"], TRUNK["n_kv_heads"], case["max_len"], head_dim)
    k = seeded.uniform(case["seed"] + 5, shape, -1.7, 1.7)
    v = seeded.uniform(case["seed"] + 6, shape, -1.7, 1.7)
    return _round_bf16(k), _round_bf16(v)


def _round_bf16(a: np.ndarray) -> np.ndarray:
    bits = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return rounded.astype(np.uint32).view(np.float32)


def write_positions(case: dict, positions: np.ndarray) -> np.ndarray:
    """[B, T]: min(positions[b] + t, max_len - 1) (trunk.py:419-420)."""

    return np.minimum(positions[:, None] + np.arange(case["T"])[None, :], case["max_len"] - 1)


def defined_writes(case: dict, positions: np.ndarray) -> np.ndarray:
    """[B, T] bool: the slot token t of game b writes is written by no other token of
    the step, so its final content is defined (clamped padding writes the reserved slot
    several times, in an order the reference leaves to index_put)."""

    wp = write_positions(case, positions)
    out = np.ones(wp.shape, dtype=bool)
    for b in range(wp.shape[0]):
        values, counts = np.unique(wp[b], return_counts=True)
        for value, count in zip(values, counts):
            if count > 1:
                out[b, wp[b] == value] = False
    return out


def piquet_tokens(field_vocab: tuple[int, ...]) -> np.ndarray:
    """[n, 64] int64: 32 field values inside each field's vocabulary, then 32 card codes
    in [0, 12)."""

    n = PIQUET["tokens"]
    out = np.zeros((n, 64), dtype=np.int64)
    for f, vocab in enumerate(field_vocab):
        out[:, f] = seeded.integers(PIQUET["seed"] * 100 + f, (n,), 0, vocab)
    out[:, 32:] = seeded.integers(PIQUET["seed"] * 100 + 99, (n, 32), 0, 12)
    return out
