"""The reference's rollout caller on the custom ops: ``DecodeGraphs``
(card_playing_gym_amd/rl/graphs.py, the interface of cardgym/rl/graphs.py:63-151) compiles
the wave body with ``torch.compile(dynamic=True)``, warms it up on a side stream, captures
it into a HIP graph and replays it.  Checked against the same waves run eagerly (no
compile, no graph) on a twin pool.

Bar: bit-equal outputs and pools -- the compiled, captured and eager paths launch the same
kernels on the same inputs.  Also: the body compiles as one graph (``fullgraph=True``), the
compiled body appends to the pool in place (functionalisation makes no copy of it), replays
follow in-place weight updates, and ``torch.library.opcheck`` passes on each op.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from card_playing_gym_amd.nn import ops
from card_playing_gym_amd.rl.graphs import DecodeGraphs, graphs_enabled
from card_playing_gym_amd.synthetic import build_model, trunk_config

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


def random_wave(rng, capacity: int, rows: int, run: int, max_pos: int):
    cache_rows = rng.permutation(capacity)[:rows]
    positions = rng.integers(0, max_pos, size=rows)
    tokens = rng.integers(0, 512, size=(rows, run, 1))
    offsets = rng.integers(0, run, size=rows)
    return tokens, positions, offsets, cache_rows


def eager_wave(model, cache, tokens, positions, offsets, cache_rows, span):
    dev = cache.device
    up = lambda a: torch.from_numpy(np.asarray(a, dtype=np.int64)).to(dev)  # noqa: E731
    with torch.autocast("cuda", dtype=torch.bfloat16, cache_enabled=False):
        hidden = model.forward_ragged(up(tokens), up(positions), cache, up(offsets), span=span, rows=up(cache_rows))
        logits, values = model.heads(hidden)
    return torch.cat([logits, values], dim=-1)


def pools_equal(a, b) -> bool:
    return all(torch.equal(x, y) for x, y in zip(a.k + a.v, b.k + b.v))


def test_decode_graphs_match_eager(device):
    capacity, max_len = 96, 128
    model, cache, twin = setup(device, 4, capacity, max_len)
    assert graphs_enabled(model, device)
    graphs = DecodeGraphs(model, cache, precision="bf16", values=True)
    rng = np.random.default_rng(7)
    shapes = [(64, 1), (64, 1), (32, 3), (64, 1), (32, 3), (17, 2), (17, 2)]
    with torch.no_grad():
        for index, (rows, run) in enumerate(shapes):
            wave = random_wave(rng, capacity, rows, run, 100)
            print(f"wave {index}: rows {rows} run {run}", flush=True)
            got = graphs.run(*wave, span=max_len).clone()
            want = eager_wave(model, twin, *wave, max_len)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"wave {index}"
            assert pools_equal(cache, twin), f"wave {index}"
        assert len(graphs) == 3
        assert graphs.columns == {"policy": slice(0, 512), "values": slice(512, 514)}
        # New weights in place (as a trainer update lands): the captured graphs follow.
        fresh = build_model(trunk_config(4), seed=11, device=device)
        model.load_state_dict(fresh.state_dict())
        wave = random_wave(rng, capacity, 64, 1, 100)
        got = graphs.run(*wave, span=max_len).clone()
        want = eager_wave(model, twin, *wave, max_len)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert pools_equal(cache, twin)
        assert len(graphs) == 3


def test_wave_compiles_as_one_graph_and_appends_in_place(device):
    """``fullgraph=True``: no graph break anywhere in the wave (a ctypes call would be
    one).  The compiled call's extra memory stays far below the pool's size: the K / V
    append is not turned into a copy of the pool."""

    capacity, max_len = 256, 512
    model, cache, twin = setup(device, 4, capacity, max_len, seed=5)
    pool_bytes = sum(t.numel() * t.element_size() for t in cache.k + cache.v)
    graphs = DecodeGraphs(model, cache, precision="bf16", values=True)
    body = torch.compile(graphs._outputs, dynamic=True, fullgraph=True)
    rng = np.random.default_rng(9)
    with torch.no_grad():
        for index, (rows, run) in enumerate([(128, 1), (96, 2), (128, 1)]):
            tokens, positions, offsets, cache_rows = random_wave(rng, capacity, rows, run, 400)
            packed = np.concatenate([a.reshape(-1) for a in (tokens, positions, offsets, cache_rows)]).astype(np.int64)
            inputs = torch.from_numpy(packed).to(device)
            print(f"compiled call {index}: rows {rows} run {run}", flush=True)
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats(device)
            base = torch.cuda.memory_allocated(device)
            out = torch.cat(body(inputs, rows, run, 1, max_len), dim=-1)
            torch.cuda.synchronize()
            extra = torch.cuda.max_memory_allocated(device) - base
            want = eager_wave(model, twin, tokens, positions, offsets, cache_rows, max_len)
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
            (x, None, None, k_pools, v_pools, positions, None, cache_rows, readout, model.trunk.op_key, 1, rows, 1,
             max_len),
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
