"""ORACLE -- test infrastructure only.

CPU restatement of the reference's policy sampling, cardgym/rl/ppo.py:75-94:
  * ``masked_probabilities`` (ppo.py:75-82): softmax over the legal entries of each row,
    exactly zero on the illegal ones, in numpy float32.
  * ``sample_rows`` (ppo.py:85-94): the count of a row's float32 running sums below its
    float64 uniform, clamped to the last legal index, replaced by it when illegal.
  * ``pairwise_sum_f32``: the order in which numpy 2.2 sums a contiguous float32 row
    (numpy/_core/src/umath/loops_utils.h.src, pairwise sum: blocks of at most 128 with
    eight running sums, halves split at multiples of 8) -- the order the device
    normaliser reproduces.  Pinned against numpy itself in tests/test_oracle.py.
Only ``tests/`` may import this module.
"""

from __future__ import annotations

import numpy as np


def masked_probabilities(logits: np.ndarray, mask: np.ndarray) -> np.ndarray:
    legal_logits = np.where(mask, logits, -np.inf)
    shifted = legal_logits - legal_logits.max(axis=-1, keepdims=True)
    weights = np.exp(shifted)
    weights[~mask] = 0.0
    return weights / weights.sum(axis=-1, keepdims=True)


def sample_rows(probabilities: np.ndarray, mask: np.ndarray, uniforms: np.ndarray) -> np.ndarray:
    rows, width = probabilities.shape
    below = (np.cumsum(probabilities, axis=1) < uniforms[:, None]).sum(axis=1)
    # Last legal index of each row (width - 1 when a row has none, as argmax of all-False).
    reversed_first = np.argmax(mask[:, ::-1], axis=1)
    last_legal = width - 1 - reversed_first
    picked = np.minimum(below, last_legal)
    illegal = ~mask[np.arange(rows), picked]
    picked[illegal] = last_legal[illegal]
    return picked


def pairwise_sum_f32(row: np.ndarray) -> np.float32:
    """numpy's float32 pairwise summation order, written out with float32 scalars."""

    row = np.asarray(row, dtype=np.float32)
    n = row.shape[0]
    if n < 8:
        total = np.float32(0.0)
        for v in row:
            total = np.float32(total + v)
        return total
    if n <= 128:
        r = [np.float32(v) for v in row[:8]]
        i = 8
        while i < n - (n % 8):
            for j in range(8):
                r[j] = np.float32(r[j] + row[i + j])
            i += 8
        total = np.float32(np.float32(np.float32(r[0] + r[1]) + np.float32(r[2] + r[3]))
                           + np.float32(np.float32(r[4] + r[5]) + np.float32(r[6] + r[7])))
        while i < n:
            total = np.float32(total + row[i])
            i += 1
        return total
    half = n // 2
    half -= half % 8
    return np.float32(pairwise_sum_f32(row[:half]) + pairwise_sum_f32(row[half:]))
