"""The persistent decode-attention kernel (cg_decode_attention_ordered with the order of
cg_decode_attention_order): the kernel the ordered entry points launch for decode runs on
a 16-bit pool whose span reaches 1024 keys.  Checked against the oracle's grouped attention
(cardgym/nn/trunk.py:225-256 restated) in float64 and with the reference's rounding, at the
bf16 bar (2e-2), and against the split kernel (cg_decode_attention without an order) on the
same inputs.

Cases: one to four tokens per row (G * T <= 16 queries per unit), head_dim 32 and 64,
fp32 queries and queries already in the cache type, gathered rows, more units than the
grid has waves (several units per wave, dealt in snake order), rows outside the pool and
rows without a visible key (zero output, as the split kernel writes), and a span cap.
The order itself must be a permutation of the units sorted by descending 64-key tiles.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from card_playing_gym_amd.nn.decode import attention_into, attention_order
from oracle.reference_path import RefConfig, RefTrunk

pytestmark = pytest.mark.gpu

TOL = 2e-2


def oracle(q, k_cache, v_cache, rows, key_lengths, span, heads, kv_heads, literal):
    """Grouped attention of the reference on the gathered rows (gathered on the device, then
    brought to the host: the pools here are hundreds of MB)."""

    D = q.shape[-1]
    trunk = RefTrunk({}, RefConfig(d_model=heads * D, n_layers=1, n_heads=heads, n_kv_heads=kv_heads, d_ff=8))
    width = int(min(span, int(key_lengths.max()) + q.shape[2]))
    index = rows.to(k_cache.device)
    k = k_cache[index, :, :width].cpu()
    v = v_cache[index, :, :width].cpu()
    if literal:
        return trunk.grouped_attention(q.to(k.dtype), k, v, key_lengths).float()
    return trunk.grouped_attention(q.double(), k.double(), v.double(), key_lengths).float()


def expected_tiles(rows, key_lengths, T, span, capacity, kv_heads):
    rows, kl = rows.numpy(), key_lengths.numpy()
    kend = np.minimum(kl + T - 1, span)
    kend = np.where((rows >= 0) & (rows < capacity) & (kend > 0), kend, 0)
    tiles = np.minimum(255, (kend + 63) // 64)
    return np.repeat(tiles, kv_heads)  # unit u = b * kv_heads + h


def run(device, q, k_cache, v_cache, rows, key_lengths, span, ordered):
    B, heads, T, D = q.shape
    out = torch.empty(q.shape, dtype=k_cache.dtype, device=device)
    order = None
    if ordered:
        order = attention_order(k_cache, rows, key_lengths, B, heads, T, span)
        assert order is not None
    attention_into(out, q, k_cache, v_cache, rows, key_lengths, span, 1.0 / math.sqrt(D), order)
    return out, order


CASES = [
    # (dtype, D, heads, kv_heads, T, B, q_in_cache_type)
    (torch.bfloat16, 32, 8, 2, 1, 9, False),
    (torch.bfloat16, 32, 8, 2, 1, 2601, False),   # 5202 units: more than the grid's waves
    (torch.bfloat16, 32, 8, 2, 1, 2600, True),
    (torch.bfloat16, 32, 8, 2, 4, 700, False),    # 16 queries per unit
    (torch.bfloat16, 32, 4, 4, 2, 500, False),    # G = 1
    (torch.float16, 32, 8, 2, 3, 600, True),
    (torch.bfloat16, 64, 4, 1, 1, 2500, False),
    (torch.float16, 64, 16, 1, 1, 300, False),    # G = 16
    (torch.bfloat16, 64, 8, 2, 2, 900, True),
]


def pools(device, capacity, kv_heads, max_len, D, dtype, seed):
    gen = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(capacity, kv_heads, max_len, D, generator=gen, device=device).to(dtype)
    v = torch.randn(capacity, kv_heads, max_len, D, generator=gen, device=device).to(dtype)
    return k, v


@pytest.mark.parametrize("dtype,D,heads,kv_heads,T,B,q_cache", CASES)
def test_ordered_decode_attention_matches_oracle(device, dtype, D, heads, kv_heads, T, B, q_cache):
    gen = torch.Generator().manual_seed(B + 13 * T + D)
    capacity, max_len = B + 7, 1100
    k_cache, v_cache = pools(device, capacity, kv_heads, max_len, D, dtype, B + T)
    rows = torch.randperm(capacity, generator=gen)[:B]
    # Mostly short rows with a few long ones (restarted games beside old ones).
    positions = torch.randint(0, 200, (B,), generator=gen)
    long = torch.randperm(B, generator=gen)[: max(2, B // 20)]
    positions[long] = torch.randint(200, max_len - T, (long.numel(),), generator=gen)
    positions[0] = 0
    positions[1] = max_len - T - 1
    key_lengths = positions + 1
    span = max_len if B % 2 else 1030  # a cap below some rows' lengths
    q = torch.randn(B, heads, T, D, generator=gen)
    if q_cache:
        q = q.to(dtype)
    print(f"case {dtype} D{D} H{heads}/{kv_heads} T{T} B{B} q {q.dtype}", flush=True)
    dev = lambda t: t.to(device)  # noqa: E731
    got, order = run(device, dev(q), k_cache, v_cache, dev(rows), dev(key_lengths), span, True)
    split, _ = run(device, dev(q), k_cache, v_cache, dev(rows), dev(key_lengths), span, False)
    torch.cuda.synchronize()
    got, split = got.float().cpu(), split.float().cpu()
    exact = oracle(q, k_cache, v_cache, rows, key_lengths, span, heads, kv_heads, literal=False)
    assert (got - exact).abs().max().item() <= TOL
    literal = oracle(q, k_cache, v_cache, rows, key_lengths, span, heads, kv_heads, literal=True)
    assert (got - literal).abs().max().item() <= TOL
    assert (got - split).abs().max().item() <= TOL
    # The order: a permutation of the units, longest first.
    o = order.cpu().numpy()
    assert sorted(o.tolist()) == list(range(B * kv_heads))
    tiles = expected_tiles(rows, key_lengths, T, span, capacity, kv_heads)[o]
    assert (np.diff(tiles) <= 0).all()


def test_rows_without_keys_and_outside_the_pool(device):
    """Rows outside the pool and rows with no visible key give zero output, like the split
    kernel; the other rows are unaffected."""

    gen = torch.Generator().manual_seed(3)
    dtype, D, heads, kv_heads, T, B = torch.bfloat16, 32, 8, 2, 1, 40
    capacity, max_len = 50, 1024
    k_cache, v_cache = pools(device, capacity, kv_heads, max_len, D, dtype, 4)
    rows = torch.randperm(capacity, generator=gen)[:B]
    key_lengths = torch.randint(1, max_len, (B,), generator=gen)
    rows[3] = capacity + 5  # outside the pool
    rows[7] = -1
    key_lengths[11] = 0  # no visible key
    q = torch.randn(B, heads, T, D, generator=gen)
    dev = lambda t: t.to(device)  # noqa: E731
    got, _ = run(device, dev(q), k_cache, v_cache, dev(rows), dev(key_lengths), max_len, True)
    split, _ = run(device, dev(q), k_cache, v_cache, dev(rows), dev(key_lengths), max_len, False)
    torch.cuda.synchronize()
    got, split = got.float().cpu(), split.float().cpu()
    for b in (3, 7, 11):
        assert (got[b] == 0).all() and (split[b] == 0).all()
    keep = [b for b in range(B) if b not in (3, 7, 11)]
    want = oracle(q[keep], k_cache, v_cache, rows[keep], key_lengths[keep], max_len, heads, kv_heads, literal=False)
    assert (got[keep] - want).abs().max().item() <= TOL


def test_order_not_used_where_it_does_not_apply(device):
    """fp32 pools, more than 16 queries per unit and spans below 1024 keys keep the split
    kernel: no order."""

    k32 = torch.zeros(4, 2, 1024, 32, device=device)
    lengths = torch.ones(4, dtype=torch.int64, device=device)
    assert attention_order(k32, None, lengths, 4, 8, 1, 1024) is None
    kb = k32.to(torch.bfloat16)
    assert attention_order(kb, None, lengths, 4, 8, 5, 1024) is None  # 4 heads x 5 tokens
    assert attention_order(kb, None, lengths, 4, 8, 1, 1000) is None  # span below 1024
    assert attention_order(kb, None, lengths, 4, 8, 4, 1024) is not None
