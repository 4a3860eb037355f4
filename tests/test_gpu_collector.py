"""Collector-shaped waves, the step's status words, the fused append's conversion and fp16
pools, on the HIP path against the oracle (cardgym/nn/trunk.py, kv_cache.py restated).

* Collector waves, as the reference's continuous collector builds them
  (cardgym/rl/continuous.py:114-115, 216-217, 326-338): rows rounded up to a multiple of 64,
  every padding row on one shared scratch row past every game, at position 0 with token 0,
  ``span`` rounded up to a multiple of 32, real chunks padded by repeating their last token.
  Many writers of one slot in one wave (all padding rows write the same K / V), and
  attention over a row that the same wave appends to.
* Status words (``cg_ragged.status``): a row outside the pool, a negative position, a
  readout offset outside its sequence are reported without a host read-back, where the
  reference's indexing raises; negative readout offsets count from the end, as torch
  indexing does (trunk.py:429).
* The fused append (the QKV epilogue of the layer kernel): the bits it stores in a 16-bit
  pool are ``Tensor.to`` of the fp32 values the same step stores in an fp32 pool (nearest
  even; NaN -> 0x7fc0 in bf16).
* fp16 pools (``kv_dtype = "fp16"`` of the reference's configs) with fp32 projections and
  under bf16 autocast (the reference's own pairing), through ``forward_ragged`` (rows,
  resets), ``forward_packed`` and prefill; fp16 autocast itself is refused.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from card_playing_gym_amd.nn.trunk import compute_dtype_code
from card_playing_gym_amd.synthetic import Driver, Workload, build_model, trunk_config
from tests.helpers import autocast, cache_pair, max_err, run_native, run_oracle, twins
from tests.test_gpu_reset import garbage_pools
from tests.test_gpu_trunk import BF16_TOL, FP32_TOL, check_step

pytestmark = pytest.mark.gpu

ROW_BUCKET, SPAN_BUCKET = 64, 32


def round_up(value: int, multiple: int) -> int:
    return -(-value // multiple) * multiple


def collector_wave(rng, slots: int, scratch: int, max_len: int, count: int, run: int, vocab: int = 512):
    """Host arrays of one collector wave over ``count`` distinct slots."""

    rows = round_up(count, ROW_BUCKET)
    tokens = np.zeros((rows, run, 1), dtype=np.int64)
    cache_rows = np.full(rows, scratch, dtype=np.int64)
    positions = np.zeros(rows, dtype=np.int64)
    offsets = np.zeros(rows, dtype=np.int64)
    real_rows = rng.permutation(slots)[:count]
    lengths = rng.integers(1, run + 1, size=count)
    for i in range(count):
        block = rng.integers(0, vocab, size=int(lengths[i]))
        tokens[i, : block.size, 0] = block
        tokens[i, block.size :, 0] = block[-1]
        cache_rows[i] = real_rows[i]
        positions[i] = rng.integers(0, max_len - run)
        offsets[i] = block.size - 1
    span = round_up(int(positions.max()) + run, SPAN_BUCKET)
    return tokens, positions, offsets, cache_rows, span


@pytest.mark.parametrize("run", [1, 3])
@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_collector_wave_matches_oracle(device, precision, run):
    config = trunk_config(4)
    model, ref = twins(config, precision, device)
    dtype = torch.bfloat16 if precision == "bf16" else torch.float32
    tol = BF16_TOL if precision == "bf16" else FP32_TOL
    slots, max_len = 150, 96
    scratch = slots  # the reserved row past every game's slots
    native, oracle = cache_pair(config, slots + 1, max_len, dtype, device)
    garbage_pools(native, oracle, seed=5)
    rng = np.random.default_rng(10 + run)
    up = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    for wave, count in enumerate([100, 37, 128]):
        tokens, positions, offsets, cache_rows, span = collector_wave(rng, slots, scratch, max_len, count, run)
        print(f"{precision} run {run} wave {wave}: {count} games in {tokens.shape[0]} rows, span {span}", flush=True)
        before = [t.clone() for t in native.k + native.v]
        with torch.no_grad(), autocast(device, precision):
            hidden = model.forward_ragged(up(tokens), up(positions), native, up(offsets), span=span, rows=up(cache_rows))
            logits, values = model.heads(hidden)
        native.check()
        with torch.no_grad():
            r_hidden = ref.forward_ragged(torch.from_numpy(tokens), torch.from_numpy(positions), oracle,
                                          torch.from_numpy(offsets), span=span, rows=torch.from_numpy(cache_rows))
            r_logits, r_values = ref.heads(r_hidden)
        errs = (max_err(hidden[:count], r_hidden[:count]), max_err(logits[:count], r_logits[:count]),
                max_err(values[:count], r_values[:count]))
        print(f"  real games: {errs}", flush=True)
        assert max(errs) <= tol, errs
        for out in (hidden, logits, values):
            assert torch.isfinite(out[count:]).all(), "a padding row's output is not finite"
        # Real rows change only on their run [position, position + run), the scratch row only
        # on [0, run), no other slot of the pool.
        expected = torch.zeros(slots + 1, max_len, dtype=torch.bool)
        for i in range(count):
            expected[int(cache_rows[i]), int(positions[i]) : int(positions[i]) + run] = True
        if count < tokens.shape[0]:
            expected[scratch, :run] = True
        layers = config.n_layers
        for index, (now, want) in enumerate(zip(native.k + native.v, oracle.k + oracle.v)):
            what = f"{'kv'[index // layers]} layer {index % layers}"
            changed = (now != before[index]).any(dim=-1).any(dim=1).cpu()
            assert not (changed & ~expected).any(), f"{what}: a slot outside the wave's writes changed"
            written = expected[:, None, :, None].expand_as(want)
            diff = (now.cpu()[written].float() - want[written].float()).abs().max().item()
            assert diff <= (tol if dtype == torch.float32 else 0.1), (what, diff)


def test_step_status_words(device):
    config = trunk_config(2)
    model, _ = twins(config, "bf16", device)
    capacity, max_len, B, T = 32, 40, 8, 2
    cache = model.new_cache(capacity, max_len, torch.bfloat16)
    gen = torch.Generator().manual_seed(3)
    tokens = torch.randint(0, 512, (B, T, 1), generator=gen).to(device)
    positions = torch.randint(0, 30, (B,), generator=gen).to(device)
    rows = torch.randperm(capacity, generator=gen)[:B].to(device)
    last = torch.full((B,), T - 1, dtype=torch.int64, device=device)

    def step(rows=rows, positions=positions, offsets=last):
        with torch.no_grad(), autocast(device, "bf16"):
            return model.forward_ragged(tokens, positions, cache, offsets, rows=rows)

    want = step()
    cache.check()
    assert cache.step_errors() == []
    bad = rows.clone()
    bad[0] = capacity + 3
    step(rows=bad)
    with pytest.raises(IndexError, match="cache row outside"):
        cache.check()
    assert cache.step_errors() == []  # check() cleared the words
    bad[0] = -1  # torch indexing would wrap it; refused here
    step(rows=bad)
    assert cache.step_errors() == ["cache row outside [0, capacity)"]
    negative = positions.clone()
    negative[1] = -2
    step(positions=negative)
    with pytest.raises(IndexError, match="negative cache position"):
        cache.check()
    # Readout offsets: -1 is the last token (torch indexing), T is outside its sequence.
    offsets = torch.full((B,), -1, dtype=torch.int64, device=device)
    got = step(offsets=offsets)
    assert torch.equal(got, want) and cache.step_errors() == []
    offsets[3] = T
    got = step(offsets=offsets)
    assert torch.equal(got[3], torch.zeros_like(got[3]))
    assert torch.equal(got[:3], want[:3]) and torch.equal(got[4:], want[4:])
    assert cache.step_errors() == ["readout offset outside its sequence"]
    # A token id outside the embedding table (F.embedding would raise): a zero input row.
    bad_tokens = tokens.clone()
    bad_tokens[2, 0, 0] = 512 + 7
    with torch.no_grad(), autocast(device, "bf16"):
        model.forward_ragged(bad_tokens, positions, cache, last, rows=rows)
    assert cache.step_errors() == ["token id outside the embedding table"]


@pytest.mark.parametrize("mode", ["padded", "packed", "prefill"])
@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_token_step_matches_row_step(device, precision, mode):
    """The step from token ids (embedding and input norm inside the step,
    cg_trunk_forward_tokens) against the step from conditioned rows (embedding norm as
    its own launch, then cg_trunk_forward): fp32 bit-equal (the same kernels), bf16
    within the bf16 bar (the first layer kernel sums each row's squares in its own order)."""

    config = trunk_config(4)
    model, _ = twins(config, precision, device)
    dtype = torch.bfloat16 if precision == "bf16" else torch.float32
    capacity, max_len, B, T = 48, 64, 40, 3
    caches = [model.new_cache(capacity, max_len, dtype) for _ in range(2)]
    gen = torch.Generator().manual_seed(31)
    tokens = torch.randint(0, 512, (B, T, 1), generator=gen).to(device)
    positions = torch.randint(0, max_len - T, (B,), generator=gen).to(device)
    rows = torch.randperm(capacity, generator=gen)[:B].to(device)
    readout = torch.randint(0, T, (B,), generator=gen).to(device)
    seq_start = torch.arange(B + 1, device=device) * T
    trunk = model.trunk
    out = []
    with torch.no_grad(), autocast(device, precision):
        for fold, cache in zip((True, False), caches):
            if fold:
                if mode == "padded":
                    h = model.forward_ragged(tokens, positions, cache, readout, rows=rows)
                elif mode == "packed":
                    h = model.forward_packed(tokens.reshape(B * T, 1), seq_start, positions, cache, readout, rows)
                else:
                    h = model.forward_prefill(tokens, cache, rows)
            else:
                x, _, _ = model.prepare(tokens)
                if mode == "padded":
                    h = trunk.forward_ragged(x, None, None, cache, positions, readout, rows=rows)
                elif mode == "packed":
                    h = trunk.forward_packed(x.reshape(B * T, -1), None, None, cache, positions, seq_start, readout, rows)
                else:
                    h = trunk.forward_prefill(x, None, None, cache, rows)
            out.append(h)
    torch.cuda.synchronize()
    if precision == "fp32":
        assert torch.equal(out[0], out[1])
        assert all(torch.equal(a, b) for a, b in zip(caches[0].k + caches[0].v, caches[1].k + caches[1].v))
    else:
        assert max_err(out[0], out[1]) <= BF16_TOL
    for cache in caches:
        cache.check()


@pytest.mark.parametrize("precision", ["bf16", "fp32"])
def test_packed_step_without_tokens(device, precision):
    """Packed sequences that all carry zero tokens: nothing is written, every readout is
    outside its (empty) chunk, so every hidden row is zero and the readout status word is set
    (the reference's indexing of the empty packed rows would raise)."""

    config = trunk_config(2)
    model, _ = twins(config, precision, device)
    dtype = torch.bfloat16 if precision == "bf16" else torch.float32
    cache = model.new_cache(16, 32, dtype)
    before = [k.clone() for k in cache.k + cache.v]
    B = 5
    x = torch.empty((0, config.d_model), device=device)
    seq_start = torch.zeros(B + 1, dtype=torch.int64, device=device)
    positions = torch.arange(B, dtype=torch.int64, device=device)
    readout = torch.zeros(B, dtype=torch.int64, device=device)
    with torch.no_grad(), autocast(device, precision):
        hidden = model.trunk.forward_packed(x, None, None, cache, positions, seq_start, readout)
    torch.cuda.synchronize()
    assert hidden.shape == (B, config.d_model) and torch.equal(hidden, torch.zeros_like(hidden))
    assert all(torch.equal(a, b) for a, b in zip(before, cache.k + cache.v))
    assert cache.step_errors() == ["readout offset outside its sequence"]


def test_unaligned_table_takes_the_separate_embedding_launch(device):
    """An embedding table the first layer launch cannot read as float4 runs (not 16-byte
    aligned) is normed by its own launch first (cg_trunk_forward_tokens falls back instead of
    refusing): the same step as from the aligned table, at the bf16 bar, and the status word
    of a bad id still set."""

    config = trunk_config(2)
    model, _ = twins(config, "bf16", device)
    capacity, max_len, B = 48, 64, 40
    gen = torch.Generator().manual_seed(37)
    ids = torch.randint(0, 512, (B, 1), generator=gen).to(device)
    positions = torch.randint(0, max_len - 1, (B,), generator=gen).to(device)
    rows = torch.randperm(capacity, generator=gen)[:B].to(device)
    readout = torch.zeros(B, dtype=torch.int64, device=device)
    table = model.embedding.weight.detach()
    spare = torch.empty(table.numel() + 1, device=device, dtype=torch.float32)
    shifted = spare[1:].view_as(table)
    shifted.copy_(table)
    assert shifted.data_ptr() % 16 != 0
    caches = [model.new_cache(capacity, max_len, torch.bfloat16) for _ in range(2)]
    out = []
    with torch.no_grad(), autocast(device, "bf16"):
        for t, cache in zip((table, shifted), caches):
            out.append(model.trunk.forward_ragged_tokens(ids, t, cache, positions, readout, rows=rows))
        bad = ids.clone()
        bad[5, 0] = -3
        model.trunk.forward_ragged_tokens(bad, shifted, caches[1], positions, readout, rows=rows)
    torch.cuda.synchronize()
    assert max_err(out[0], out[1]) <= BF16_TOL
    caches[0].check()
    assert caches[1].step_errors() == ["token id outside the embedding table"]


@pytest.mark.parametrize("mode", ["decode", "padded", "packed"])
@pytest.mark.parametrize("pool", [torch.bfloat16, torch.float16])
def test_fused_append_converts_like_tensor_to(device, pool, mode):
    config = trunk_config(2)
    model = build_model(config, seed=21, device=device)
    capacity, max_len, B = 64, 48, 40
    T = 1 if mode == "decode" else 3
    low = model.new_cache(capacity, max_len, pool)
    wide = model.new_cache(capacity, max_len, torch.float32)
    gen = torch.Generator().manual_seed(22)
    x = (4 * torch.randn(B, T, config.d_model, generator=gen)).to(device)
    x[5] = float("nan")  # one game's tokens: its K / V come out NaN
    positions = torch.randint(0, max_len - T, (B,), generator=gen).to(device)
    rows = torch.randperm(capacity, generator=gen)[:B].to(device)
    readout = torch.full((B,), T - 1, dtype=torch.int64, device=device)
    trunk = model.trunk
    with torch.no_grad(), autocast(device, "bf16"):
        for cache in (low, wide):
            if mode == "packed":
                seq_start = torch.arange(B + 1, device=device) * T
                trunk.forward_packed(x.reshape(B * T, -1), None, None, cache, positions, seq_start, readout, rows)
            else:
                trunk.forward_ragged(x, None, None, cache, positions, readout, rows=rows)
    torch.cuda.synchronize()
    written = torch.zeros(capacity, max_len, dtype=torch.bool)
    for b in range(B):
        written[int(rows[b]), int(positions[b]) : int(positions[b]) + T] = True
    mask = written[:, None, :, None].expand(capacity, config.n_kv_heads, max_len, config.head_dim).to(device)
    for got_pool, wide_pool in ((low.k[0], wide.k[0]), (low.v[0], wide.v[0])):
        got = got_pool[mask]
        want = wide_pool[mask].to(pool)
        nan = torch.isnan(want.float())
        assert nan.any() and torch.equal(torch.isnan(got.float()), nan)
        assert torch.equal(got[~nan].view(torch.int16), want[~nan].view(torch.int16))
        if pool == torch.bfloat16:
            assert bool((got[nan].view(torch.int16) == 0x7FC0).all()), "NaN is not the canonical 0x7fc0"


FP16_WORKLOADS = {
    # (mode, end probability): slot reuse over stale rows with gathered rows; packed chunks.
    "rows_reset": Workload("fp16-rows", 4, 64, torch.float16, "fp32", "continuous", 0, 0, max_len_cap=48,
                           end_probability=0.25),
    "packed": Workload("fp16-chunks", 4, 48, torch.float16, "fp32", "chunks", 0, 40, max_chunk=6),
}


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
@pytest.mark.parametrize("name", sorted(FP16_WORKLOADS))
def test_fp16_pool_matches_oracle(device, name, precision):
    """fp16 K / V storage with fp32 projections, and under bf16 autocast (the reference's
    own configs pair ``precision = "bf16"`` with ``kv_dtype = "fp16"``, e.g.
    configs/piquet/base.toml:12-16): the reference rounds q, the scores and P to the pool's
    type (trunk.py:222, 245, 255); bar 2e-2 on hidden states, logits and values; cache slots
    as check_step compares them."""

    workload = FP16_WORKLOADS[name]
    config = workload.trunk_config()
    model, ref = twins(config, precision, device)
    max_len = workload.max_len(4)
    driver = Driver(workload, seed=2, max_len=max_len)
    native, oracle = cache_pair(config, workload.games, max_len, torch.float16, device)
    garbage_pools(native, oracle, seed=8)
    packed, rows = workload.mode == "chunks", workload.mode == "continuous"
    for step in range(4):
        plan = driver.step()
        errs = check_step(model, ref, native, oracle, plan, device, precision, packed, rows, BF16_TOL)
        print(f"{name} {precision} step {step}: {errs}", flush=True)
    native.check()


def test_fp16_pool_prefill_matches_oracle(device):
    config = trunk_config(4)
    model, ref = twins(config, "fp32", device)
    games, capacity, T = 24, 40, 20
    native, oracle = cache_pair(config, capacity, 32, torch.float16, device)
    garbage_pools(native, oracle, seed=9)
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, 512, size=(games, T, 1))
    rows = rng.permutation(capacity)[:games]
    with torch.no_grad():
        hidden = model.forward_prefill(torch.from_numpy(tokens).to(device), native, torch.from_numpy(rows).to(device))
        r_hidden = ref.forward_prefill(torch.from_numpy(tokens), oracle, torch.from_numpy(rows))
    assert max_err(hidden, r_hidden) <= BF16_TOL
    for layer in range(config.n_layers):
        got = native.k[layer][torch.from_numpy(rows).to(device), :, :T].cpu().float()
        want = oracle.k[layer][torch.from_numpy(rows), :, :T].float()
        assert (got - want).abs().max().item() <= 0.1


def test_fp16_autocast_is_refused(device):
    with torch.autocast("cuda", dtype=torch.float16):
        with pytest.raises(RuntimeError, match="fp16 autocast"):
            compute_dtype_code(device)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        assert compute_dtype_code(device) == 1
    assert compute_dtype_code(device) == 0
