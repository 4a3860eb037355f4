"""cg_trunk_forward_static (the step on the library's static workspace, no allocation)
against cg_trunk_forward with a caller-allocated workspace, through the C-ABI.

Both run the same kernels, so the bar is bit-for-bit: the readout hidden states and every
slot of the KV pool after the step.  Two calls in a row, the second with a smaller step
(the static workspace keeps the first call's contents), in fp32 and bf16; a step larger
than the static workspace is refused with IndexError (CG_ERR_RANGE) before any launch.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from card_playing_gym_amd import _native as nat
from card_playing_gym_amd.nn.kv_cache import stream_handle
from card_playing_gym_amd.synthetic import build_model, trunk_config
from tests.helpers import autocast

pytestmark = pytest.mark.gpu


def _pool(model, capacity, max_len, dtype, seed):
    cache = model.new_cache(capacity, max_len, dtype)
    gen = torch.Generator(device=cache.device).manual_seed(seed)
    for layer in range(cache.n_layers):
        cache.k[layer].normal_(generator=gen)
        cache.v[layer].normal_(generator=gen)
    return cache


def _step(model, cache, tokens, positions, rows, seq_start, readout, static: bool):
    """One step through the C-ABI; returns the readout hidden states."""

    device = tokens.device
    trunk = model.trunk
    with torch.no_grad():
        x, _, _ = model.prepare(tokens[:, None])
    x = x.reshape(-1, trunk.config.d_model).contiguous()
    native = trunk.native(device)
    n_seqs = positions.numel()
    hidden = torch.full((n_seqs, trunk.config.d_model), float("nan"), device=device)
    step = nat.Ragged(n_seqs, x.shape[0], 0, 0, seq_start.data_ptr(), positions.data_ptr(), rows.data_ptr(),
                      readout.data_ptr())
    stream = stream_handle(device)
    if static:
        nat.call("cg_trunk_forward_static", native.handle, cache.layer_array(), x.data_ptr(), None, None,
                 ctypes.byref(step), hidden.data_ptr(), stream)
    else:
        size = nat.lib().cg_trunk_workspace_size(native.handle, x.shape[0], n_seqs)
        workspace = torch.empty(size, dtype=torch.uint8, device=device)
        nat.call("cg_trunk_forward", native.handle, cache.layer_array(), x.data_ptr(), None, None,
                 ctypes.byref(step), hidden.data_ptr(), workspace.data_ptr(), size, stream)
    torch.cuda.synchronize()
    return hidden


def _plan(rng, games, capacity, max_len, max_chunk, device):
    counts = rng.integers(1, max_chunk + 1, size=games)
    seq_start = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    positions = rng.integers(0, max_len - max_chunk - 1, size=games).astype(np.int64)
    rows = rng.permutation(capacity)[:games].astype(np.int64)
    tokens = rng.integers(0, 512, size=int(seq_start[-1])).astype(np.int64)
    to = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    return to(tokens), to(positions), to(rows), to(seq_start), to(counts - 1)


@pytest.mark.parametrize("precision,kv_dtype", [("bf16", torch.bfloat16), ("fp32", torch.float32)])
def test_static_workspace_matches_allocated_workspace(device, precision, kv_dtype):
    config = trunk_config(4)
    model = build_model(config, seed=2, device=device)
    capacity, max_len = 1200, 96
    rng = np.random.default_rng(5)
    for call, (games, chunk) in enumerate([(1100, 6), (300, 3)]):  # the second call is smaller
        plan = _plan(rng, games, capacity, max_len, chunk, device)
        print(f"{precision} call {call}: {games} games, {int(plan[3][-1])} tokens", flush=True)
        pools = [_pool(model, capacity, max_len, kv_dtype, seed=10 + call) for _ in range(2)]
        with autocast(device, precision):
            want = _step(model, pools[0], *plan, static=False)
            got = _step(model, pools[1], *plan, static=True)
        assert not torch.isnan(want).any()
        assert torch.equal(got, want), f"call {call}: max diff {(got - want).abs().max().item()}"
        for layer in range(config.n_layers):
            assert torch.equal(pools[0].k[layer], pools[1].k[layer]) and torch.equal(pools[0].v[layer],
                                                                                     pools[1].v[layer])


def test_static_workspace_refuses_a_step_too_large(device):
    config = trunk_config(2)
    model = build_model(config, seed=2, device=device)
    native = model.trunk.native(device)
    tokens = 200_000
    need = nat.lib().cg_trunk_workspace_size(native.handle, tokens, tokens)
    assert need > nat.CG_TRUNK_STATIC_WORKSPACE
    cache = model.new_cache(4, 8, torch.float32)
    dummy = torch.zeros(4, dtype=torch.int64, device=device)
    step = nat.Ragged(tokens, tokens, 1, 0, None, dummy.data_ptr(), None, None)
    with pytest.raises(IndexError, match="static workspace"):
        nat.call("cg_trunk_forward_static", native.handle, cache.layer_array(), dummy.data_ptr(), None, None,
                 ctypes.byref(step), dummy.data_ptr(), stream_handle(device))
