"""Decode waves as HIP graphs, two ways, checked against the same waves run eagerly (no
compile, no graph) on a twin pool:

* ``WaveGraphs`` (card_playing_gym_amd/rl/wave_graphs.py): eager first wave per shape,
  capture without a second append, pinned staging reused per shape, least-recently-used
  shapes released;
* the reference's caller pattern (tests/caller.py: ``torch.compile(dynamic=True,
  fullgraph=True)`` of the wave body over the ``cardgym_hip`` ops, side-stream warm-up,
  capture, replay), which the reference's collectors run unchanged over this model.

Bar: bit-equal outputs and pools -- every path launches the same kernels on the same
inputs.  Also: the compiled body appends to the pool in place (functionalisation makes no
copy of it), replays follow weight updates (``load_state_dict``), and
``torch.library.opcheck`` passes on each op.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from card_playing_gym_amd.nn import ops
from card_playing_gym_amd.rl.wave_graphs import DecodeGraphs, WaveGraphs
from card_playing_gym_amd.synthetic import build_model, trunk_config
from tests.caller import CapturedWave, compiled, random_wave, to_device, wave_body

pytestmark = pytest.mark.gpu


def setup(device, layers: int, capacity: int, max_len: int, seed: int = 3):
    config = trunk_config(layers)
    model = build_model(config, seed=seed, device=device)
    cache = model.new_cache(capacity, max_len, torch.bfloat16)
    twin = model.new_cache(capacity, max_len, torch.bfloat16)
    gen = torch.Generator(device=device).manual_seed(seed + 1)
    for layer in range(layers):
        cache.k[layer].normal_(generator=gen)
        cache.v[layer].normal_(generator=gen)
        twin.k[layer].copy_(cache.k[layer])
        twin.v[layer].copy_(cache.v[layer])
    return model, cache, twin


def eager_wave(model, cache, tokens, positions, offsets, cache_rows, span):
    tokens, positions, offsets, cache_rows = to_device(cache.device, tokens, positions, offsets, cache_rows)
    with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
        hidden = model.forward_ragged(tokens, positions, cache, offsets, span=span, rows=cache_rows)
        logits, values = model.heads(hidden)
    return torch.cat([logits, values], dim=-1)


def pools_equal(a, b) -> bool:
    return all(torch.equal(x, y) for x, y in zip(a.k + a.v, b.k + b.v))


def test_wave_graphs_match_eager(device):
    capacity, max_len = 96, 128
    model, cache, twin = setup(device, 4, capacity, max_len)
    assert DecodeGraphs is WaveGraphs
    graphs = WaveGraphs(model, cache, precision="bf16", values=True, max_graphs=2)
    rng = np.random.default_rng(7)
    # (rows, run): repeats replay; a third shape releases the least recently used one.
    shapes = [(64, 1), (64, 1), (32, 3), (64, 1), (32, 3), (17, 2), (17, 2), (64, 1), (32, 3)]
    held = []
    with torch.no_grad():
        for index, (rows, run) in enumerate(shapes):
            wave = random_wave(rng, capacity, rows, run, 100)
            print(f"wave {index}: rows {rows} run {run}", flush=True)
            got = graphs.run(*wave, span=max_len).clone()
            want = eager_wave(model, twin, *wave, max_len)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"wave {index}"
            assert pools_equal(cache, twin), f"wave {index}"
            held.append(sorted(k[:2] for k in graphs._shapes))
        assert held[5] == [(17, 2), (32, 3)] and held[7] == [(17, 2), (64, 1)]
        assert len(graphs) == 2
        assert graphs.columns == {"policy": slice(0, 512), "values": slice(512, 514)}
        # New weights in place (as a trainer update lands): the captured graphs follow.
        fresh = build_model(trunk_config(4), seed=11, device=device)
        model.load_state_dict(fresh.state_dict())
        for rows, run in [(64, 1), (32, 3)]:
            wave = random_wave(rng, capacity, rows, run, 100)
            got = graphs.run(*wave, span=max_len).clone()
            want = eager_wave(model, twin, *wave, max_len)
            torch.cuda.synchronize()
            assert torch.equal(got, want)
            assert pools_equal(cache, twin)
        graphs.clear()
        assert len(graphs) == 0


def test_reference_caller_pattern(device):
    """Compiled body, side-stream warm-up, capture, replays with new inputs, replay after
    ``load_state_dict``: bit-equal to eager waves."""

    capacity, max_len = 96, 128
    model, cache, twin = setup(device, 4, capacity, max_len, seed=4)
    body = compiled(wave_body(model, cache, torch.bfloat16))
    rng = np.random.default_rng(8)
    rows, run = 48, 2
    with torch.no_grad():
        first = random_wave(rng, capacity, rows, run, 100)
        print("capture", flush=True)
        captured = CapturedWave(body, *to_device(device, *first), max_len)
        eager_wave(model, twin, *first, max_len)  # the warm-up's append
        for index in range(4):
            if index == 3:
                fresh = build_model(trunk_config(4), seed=12, device=device)
                model.load_state_dict(fresh.state_dict())
            wave = first if index == 0 else random_wave(rng, capacity, rows, run, 100)
            print(f"replay {index}", flush=True)
            got = captured.replay(*to_device(device, *wave)).clone()
            want = eager_wave(model, twin, *wave, max_len)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"replay {index}"
            assert pools_equal(cache, twin), f"replay {index}"


def test_wave_compiles_as_one_graph_and_appends_in_place(device):
    """``fullgraph=True``: no graph break anywhere in the wave (a ctypes call would be
    one).  The compiled call's extra memory stays far below the pool's size: the K / V
    append is not turned into a copy of the pool."""

    capacity, max_len = 256, 512
    model, cache, twin = setup(device, 4, capacity, max_len, seed=5)
    pool_bytes = sum(t.numel() * t.element_size() for t in cache.k + cache.v)
    body = compiled(wave_body(model, cache, torch.bfloat16))
    rng = np.random.default_rng(9)
    with torch.no_grad():
        for index, (rows, run) in enumerate([(128, 1), (96, 2), (128, 1)]):
            wave = random_wave(rng, capacity, rows, run, 400)
            inputs = to_device(device, *wave)
            print(f"compiled call {index}: rows {rows} run {run}", flush=True)
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats(device)
            base = torch.cuda.memory_allocated(device)
            out = body(*inputs, max_len)
            torch.cuda.synchronize()
            extra = torch.cuda.max_memory_allocated(device) - base
            want = eager_wave(model, twin, *wave, max_len)
            torch.cuda.synchronize()
            assert torch.equal(out, want), f"call {index}"
            assert pools_equal(cache, twin), f"call {index}"
            if index > 0:  # the first call compiles
                assert extra < pool_bytes // 8, (extra, pool_bytes)


def test_opcheck(device):
    """torch.library.opcheck: schema (declared mutations only), fake tensors, autograd
    registration and AOT dispatch of the trunk step, the heads and the embedding ops."""

    capacity, max_len = 16, 32
    model, cache, _ = setup(device, 2, capacity, max_len, seed=13)
    rows = 8
    x = torch.randn(rows, 256, device=device)
    positions = torch.randint(0, 20, (rows,), device=device)
    readout = torch.zeros(rows, dtype=torch.int64, device=device)
    cache_rows = torch.randperm(capacity, device=device)[:rows]
    k_pools, v_pools = cache.pools()
    with torch.no_grad():
        torch.library.opcheck(
            torch.ops.cardgym_hip.trunk_step.default,
            (x, None, None, k_pools, v_pools, cache.status, positions, None, cache_rows, readout, model.trunk.op_key, 1,
             rows, 1, max_len),
        )
        hidden = torch.randn(rows, 256, device=device)
        for compute in (0, 1):
            torch.library.opcheck(torch.ops.cardgym_hip.synthetic_heads.default, (hidden, model.op_key, compute, 512, 2))
        ids = torch.randint(0, 512, (rows,), device=device)
        trunk = model.trunk
        torch.library.opcheck(torch.ops.cardgym_hip.embed_rmsnorm.default,
                              (model.embedding.weight.detach(), ids, trunk.input_norm.weight.detach(), 1e-5))
        torch.library.opcheck(torch.ops.cardgym_hip.rmsnorm.default, (x, trunk.input_norm.weight.detach(), 1e-5))
    assert ops.lookup(model.trunk.op_key) is model.trunk
