"""cg_decode_attention against the oracle's grouped attention (cardgym/nn/trunk.py:225-256
restated) on the same cache contents.

fp32 caches: max |err| <= 1e-5 against the float64 evaluation.  bf16 / fp16 caches: the
kernel rounds q and the probabilities to the cache type as the reference does
(trunk.py:222, 255) but keeps scores and sums in fp32, so it is compared with the
reference's rounding path at the bf16 bar (2e-2) and with float64 at the same bar.
"""

from __future__ import annotations

import math

import pytest
import torch

from card_playing_gym_amd.nn.decode import decode_attention, supported
from oracle.reference_path import RefConfig, RefTrunk

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-2}


def oracle(q, k_cache, v_cache, rows, key_lengths, span, heads, kv_heads, literal):
    """Gather + grouped attention of the reference; float64 unless ``literal``."""

    D = q.shape[-1]
    trunk = RefTrunk({}, RefConfig(d_model=heads * D, n_layers=1, n_heads=heads, n_kv_heads=kv_heads, d_ff=8))
    k = k_cache[rows, :, :span]
    v = v_cache[rows, :, :span]
    if literal:
        return trunk.grouped_attention(q.to(k.dtype), k, v, key_lengths).float()
    return trunk.grouped_attention(q.double(), k.double(), v.double(), key_lengths).float()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,heads,kv_heads", [(32, 8, 2), (64, 4, 1), (24, 10, 2), (16, 4, 2), (8, 4, 4)])
@pytest.mark.parametrize("T", [1, 3, 5])
def test_decode_attention_matches_oracle(device, dtype, D, heads, kv_heads, T):
    gen = torch.Generator().manual_seed(D * 100 + T)
    capacity, max_len, B = 13, 150, 9
    k_cache = torch.randn(capacity, kv_heads, max_len, D, generator=gen).to(dtype)
    v_cache = torch.randn(capacity, kv_heads, max_len, D, generator=gen).to(dtype)
    rows = torch.randperm(capacity, generator=gen)[:B]
    positions = torch.randint(0, max_len - T, (B,), generator=gen)
    positions[0] = 0  # a row with one visible key for its first query
    positions[1] = max_len - T - 1  # a row reaching the end of the pool
    key_lengths = positions + 1
    span = int(positions.max()) + T
    q = torch.randn(B, heads, T, D, generator=gen)
    assert supported(D, span, heads * T)
    out = decode_attention(q.to(device), k_cache.to(device), v_cache.to(device), rows.to(device),
                           key_lengths.to(device), span, 1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == q.shape
    got = out.float().cpu()
    exact = oracle(q, k_cache, v_cache, rows, key_lengths, span, heads, kv_heads, literal=False)
    err = (got - exact).abs().max().item()
    assert err <= TOL[dtype], f"vs float64: {err}"
    if dtype != torch.float32:
        literal = oracle(q, k_cache, v_cache, rows, key_lengths, span, heads, kv_heads, literal=True)
        assert (got - literal).abs().max().item() <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("T,prefix", [(16, 0), (40, 0), (40, 30), (150, 0), (64, 200)])
def test_multi_token_rows(device, dtype, D, T, prefix):
    """Prefill-sized rows: 4 query heads per KV head x T tokens, so several 64-query groups
    per (row, head), dealt over the launch's second dimension; spans of at most 64 keys
    (prefill of a short chunk) take one wave per (row, head)."""

    gen = torch.Generator().manual_seed(T * 7 + prefix + D)
    heads, kv_heads = 8, 2
    capacity, max_len, B = 11, 320, 7
    k_cache = torch.randn(capacity, kv_heads, max_len, D, generator=gen).to(dtype)
    v_cache = torch.randn(capacity, kv_heads, max_len, D, generator=gen).to(dtype)
    rows = torch.randperm(capacity, generator=gen)[:B]
    positions = torch.full((B,), prefix) if prefix == 0 else torch.randint(0, prefix + 1, (B,), generator=gen)
    key_lengths = positions + 1
    span = int(positions.max()) + T
    q = torch.randn(B, heads, T, D, generator=gen)
    out = decode_attention(q.to(device), k_cache.to(device), v_cache.to(device), rows.to(device),
                           key_lengths.to(device), span, 1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    got = out.float().cpu()
    exact = oracle(q, k_cache, v_cache, rows, key_lengths, span, heads, kv_heads, literal=False)
    assert (got - exact).abs().max().item() <= TOL[dtype]
    literal = oracle(q, k_cache, v_cache, rows, key_lengths, span, heads, kv_heads, literal=True)
    assert (got - literal).abs().max().item() <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_span_caps_the_visible_keys(device, dtype):
    """A span shorter than a row's length truncates its keys, as reading k[:, :, :span] does."""

    gen = torch.Generator().manual_seed(9)
    k_cache = torch.randn(4, 2, 300, 32, generator=gen).to(dtype)
    v_cache = torch.randn(4, 2, 300, 32, generator=gen).to(dtype)
    rows = torch.tensor([2, 0, 3])
    key_lengths = torch.tensor([290, 17, 200])
    q = torch.randn(3, 8, 1, 32, generator=gen)
    span = 150
    out = decode_attention(q.to(device), k_cache.to(device), v_cache.to(device), rows.to(device),
                           key_lengths.to(device), span, 32 ** -0.5).float().cpu()
    want = oracle(q, k_cache, v_cache, rows, key_lengths, span, 8, 2, literal=False)
    assert (out - want).abs().max().item() <= TOL[dtype]


def test_long_rows_and_many_sequences(device):
    """Rows up to 2048 keys (the continuous workload's cap) across 300 sequences, bf16."""

    gen = torch.Generator().manual_seed(10)
    B, L = 300, 2048
    k_cache = torch.randn(B, 2, L, 32, generator=gen).to(torch.bfloat16)
    v_cache = torch.randn(B, 2, L, 32, generator=gen).to(torch.bfloat16)
    rows = torch.randperm(B, generator=gen)
    positions = torch.randint(0, L - 1, (B,), generator=gen)
    q = torch.randn(B, 8, 1, 32, generator=gen)
    out = decode_attention(q.to(device), k_cache.to(device), v_cache.to(device), rows.to(device),
                           (positions + 1).to(device), L, 32 ** -0.5).float().cpu()
    sample = torch.tensor([0, 1, 77, 150, 299])
    want = oracle(q[sample], k_cache, v_cache, rows[sample], positions[sample] + 1, L, 8, 2, literal=False)
    assert (out[sample] - want).abs().max().item() <= 2e-2


def test_empty_inputs_are_no_ops(device):
    k = torch.zeros(2, 2, 8, 32, device=device)
    out = decode_attention(torch.zeros(0, 8, 1, 32, device=device), k, k, torch.zeros(0, dtype=torch.int64, device=device),
                           torch.zeros(0, dtype=torch.int64, device=device), 8, 1.0)
    assert out.shape == (0, 8, 1, 32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("D,heads,kv_heads", [(32, 8, 2), (64, 4, 1), (16, 4, 2)])
def test_packed_decode_attention_matches_oracle(device, dtype, D, heads, kv_heads):
    """cg_decode_attention_packed: chunks of 1-16 tokens packed back to back (no padding),
    each token t of a chunk seeing its row's prefix plus its chunk up to itself; against the
    oracle's grouped attention on each chunk padded to 16 with its own key lengths."""

    from card_playing_gym_amd.nn.decode import attention_packed_into

    gen = torch.Generator().manual_seed(D * 7 + heads)
    capacity, max_len, B = 40, 300, 33
    k_cache = torch.randn(capacity, kv_heads, max_len, D, generator=gen).to(dtype)
    v_cache = torch.randn(capacity, kv_heads, max_len, D, generator=gen).to(dtype)
    rows = torch.randperm(capacity, generator=gen)[:B]
    counts = torch.randint(1, 17, (B,), generator=gen)
    positions = torch.randint(0, max_len - 17, (B,), generator=gen)
    positions[0], counts[0] = 0, 16  # a fresh game's first chunk: its own keys only
    positions[1], counts[1] = max_len - 17, 16  # the pool's end
    seq_start = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(counts, 0)])
    n = int(seq_start[-1])
    q = torch.randn(n, heads, D, generator=gen)
    out = torch.empty(n, heads, D, dtype=dtype, device=device)
    span = int((positions + counts).max())
    attention_packed_into(out, q.to(device), k_cache.to(device), v_cache.to(device), rows.to(device),
                          positions.to(device), seq_start.to(device), span, 1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    got = out.float().cpu()
    # The oracle: each chunk as a padded run of 16 queries (repeat-last), key_lengths = positions + 1.
    padded = torch.zeros(B, heads, 16, D)
    for b in range(B):
        chunk = q[seq_start[b] : seq_start[b + 1]].transpose(0, 1)  # [heads, c, D]
        padded[b, :, : counts[b]] = chunk
        padded[b, :, counts[b] :] = chunk[:, -1:]
    exact = oracle(padded, k_cache, v_cache, rows, positions + 1, span, heads, kv_heads, literal=False)
    want = torch.cat([exact[b, :, : counts[b]].transpose(0, 1) for b in range(B)])
    err = (got - want).abs().max().item()
    assert err <= TOL[dtype], f"vs float64: {err}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,heads,kv_heads", [(32, 8, 2), (64, 4, 1), (16, 4, 2)])
def test_packed_order_is_a_work_sort_and_keeps_results(device, dtype, D, heads, kv_heads):
    """cg_decode_attention_packed_order / _ordered: the order is a permutation of the
    (row, KV head) units with non-increasing work (64-key tiles of the last token's keys,
    capped at the span, x 16-query tiles; a row outside the pool counts 0), and dealing the
    units in it leaves every output bit as the unordered launch writes it."""

    from card_playing_gym_amd.nn.decode import attention_packed_into, attention_packed_order

    gen = torch.Generator().manual_seed(D * 11 + heads)
    capacity, max_len, B = 70, 600, 61
    k_cache = torch.randn(capacity, kv_heads, max_len, D, generator=gen).to(dtype)
    v_cache = torch.randn(capacity, kv_heads, max_len, D, generator=gen).to(dtype)
    rows = torch.randperm(capacity, generator=gen)[:B]
    counts = torch.randint(1, 17, (B,), generator=gen)
    positions = torch.randint(0, max_len - 17, (B,), generator=gen)
    positions[:4] = torch.tensor([0, 63, 64, max_len - 17])  # tile boundaries and the pool's end
    seq_start = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(counts, 0)])
    n = int(seq_start[-1])
    span = 500  # below the longest rows: the cap shows in the work
    q = torch.randn(n, heads, D, generator=gen).to(device)
    args = (k_cache.to(device), v_cache.to(device), rows.to(device), positions.to(device), seq_start.to(device))

    order = attention_packed_order(args[0], args[2], args[3], args[4], n, heads, span).cpu()
    assert sorted(order.tolist()) == list(range(B * kv_heads))
    g = heads // kv_heads
    kend = torch.clamp(positions + counts, max=span)  # keys of the chunk's last token
    work = (kend + 63) // 64 * ((g * counts + 15) // 16)
    unit_work = work.repeat_interleave(kv_heads)
    seq = unit_work[order.long()]
    assert bool((seq[:-1] >= seq[1:]).all()), seq.tolist()

    plain = torch.empty(n, heads, D, dtype=dtype, device=device)
    ordered = torch.empty_like(plain)
    attention_packed_into(plain, q, *args, span, 1.0 / math.sqrt(D))
    attention_packed_into(ordered, q, *args, span, 1.0 / math.sqrt(D), order.to(device))
    torch.cuda.synchronize()
    assert torch.equal(plain.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       ordered.view(torch.int16 if dtype != torch.float32 else torch.int32))


@pytest.mark.parametrize("B, distinct", [(3000, 1), (3000, 3), (20000, 5)])
def test_packed_order_with_shared_work_and_many_units(device, B, distinct):
    """The unit sort when most units share a few work values (games of one length: whole
    waves fall into one bucket) and, at 20000 rows x 2 KV heads, more units than the sort
    keeps in LDS between its passes: still a permutation with non-increasing work."""

    from card_playing_gym_amd.nn.decode import attention_packed_order

    gen = torch.Generator().manual_seed(B + distinct)
    capacity, max_len, kv_heads, heads, D = 64, 256, 2, 8, 32
    k_cache = torch.zeros(capacity, kv_heads, max_len, D, dtype=torch.bfloat16, device=device)
    rows = torch.randint(0, capacity, (B,), generator=gen)
    rows[::97] = capacity  # outside the pool: work 0
    levels = torch.tensor([7, 70, 200, 130, 1])[:distinct]
    positions = levels[torch.randint(0, distinct, (B,), generator=gen)]
    counts = torch.full((B,), 4, dtype=torch.int64)
    seq_start = torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(counts, 0)])
    n, span = int(seq_start[-1]), max_len
    order = attention_packed_order(k_cache, rows.to(device), positions.to(device), seq_start.to(device), n, heads,
                                   span).cpu()
    assert torch.equal(order.sort().values, torch.arange(B * kv_heads, dtype=order.dtype))
    kend = torch.clamp(positions + counts, max=span)
    work = (kend + 63) // 64 * ((heads // kv_heads * counts + 15) // 16)
    work[rows >= capacity] = 0
    seq = work.repeat_interleave(kv_heads)[order.long()]
    assert bool((seq[:-1] >= seq[1:]).all())
