"""Shared setup for the parity tests: the native model, its oracle twin and step drivers."""

from __future__ import annotations

import contextlib

import numpy as np
import torch

from card_playing_gym_amd.nn.kv_cache import KVCache
from card_playing_gym_amd.nn.trunk import Trunk, TrunkConfig
from card_playing_gym_amd.synthetic import StepPlan, build_model
from oracle.reference_path import RefCache, RefSynthetic, ref_config_of


def twins(config, precision: str, device, seed: int = 0):
    """Native model on ``device`` and the oracle over the same (CPU copy of the) weights."""

    model = build_model(config, seed=seed, device=device)
    state = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    return model, RefSynthetic(state, ref_config_of(config), precision)


def autocast(device, precision: str):
    if precision == "bf16":
        return torch.autocast(device.type, dtype=torch.bfloat16)
    return contextlib.nullcontext()


def cache_pair(config, capacity: int, max_len: int, dtype, device):
    native = KVCache(n_layers=config.n_layers, kv_heads=config.n_kv_heads, head_dim=config.head_dim,
                     capacity=capacity, max_len=max_len, device=device, dtype=dtype)
    ref = RefCache(config.n_layers, config.n_kv_heads, config.head_dim, capacity, max_len, dtype)
    return native, ref


def fill_prefixes(native: KVCache, ref: RefCache, lengths: np.ndarray, rows: np.ndarray, seed: int = 0) -> None:
    """Random K/V (N(0,1)) in the first lengths[i] positions of rows[i], identical in both."""

    gen = torch.Generator().manual_seed(seed)
    for layer in range(ref.n_layers):
        k = torch.randn(ref.k[layer].shape, generator=gen).to(ref.dtype)
        v = torch.randn(ref.v[layer].shape, generator=gen).to(ref.dtype)
        mask = torch.zeros(ref.capacity, ref.max_len, dtype=torch.bool)
        for length, row in zip(lengths, rows):
            mask[int(row), : int(length)] = True
        keep = mask[:, None, :, None]
        k = torch.where(keep, k, torch.zeros((), dtype=ref.dtype))
        v = torch.where(keep, v, torch.zeros((), dtype=ref.dtype))
        ref.k[layer].copy_(k)
        ref.v[layer].copy_(v)
        native.k[layer].copy_(k.to(native.device))
        native.v[layer].copy_(v.to(native.device))


def run_native(model, cache: KVCache, plan: StepPlan, device, precision: str, packed: bool, rows: bool):
    """One native step: (hidden [B, d], logits, values) on the device."""

    with torch.no_grad(), autocast(device, precision):
        tokens = torch.from_numpy(plan.tokens).to(device)
        positions = torch.from_numpy(plan.positions).to(device)
        readout = torch.from_numpy(plan.readout).to(device)
        rows_d = torch.from_numpy(plan.rows).to(device) if rows else None
        if packed:
            hidden = model.forward_packed(tokens[:, None], torch.from_numpy(plan.seq_start).to(device), positions,
                                          cache, readout, rows_d)
        else:
            T = plan.T
            hidden = model.forward_ragged(tokens.view(-1, T, 1), positions, cache, readout, rows=rows_d)
        logits, values = model.heads(hidden)
    return hidden, logits, values


def run_oracle(ref: RefSynthetic, cache: RefCache, plan: StepPlan, rows: bool):
    """The same step through the oracle, with chunks padded to the longest (repeat-last),
    as the reference's collectors pad them (cardgym/rl/continuous.py:324-338)."""

    counts = np.diff(plan.seq_start)
    B, run = counts.size, int(counts.max())
    tokens = np.zeros((B, run, 1), dtype=np.int64)
    for b in range(B):
        chunk = plan.tokens[plan.seq_start[b] : plan.seq_start[b + 1]]
        tokens[b, : chunk.size, 0] = chunk
        tokens[b, chunk.size :, 0] = chunk[-1]
    with torch.no_grad():
        hidden = ref.forward_ragged(
            torch.from_numpy(tokens), torch.from_numpy(plan.positions), cache, torch.from_numpy(plan.readout),
            rows=torch.from_numpy(plan.rows) if rows else None,
        )
        logits, values = ref.heads(hidden)
    return hidden.float(), logits, values


def max_err(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.detach().float().cpu() - b.detach().float().cpu()).abs().max().item()


def random_trunk(config: TrunkConfig, seed: int = 0, scale: float = 0.05) -> dict[str, torch.Tensor]:
    """A trunk state dict with every parameter perturbed (so zero-initialised PLE / VE
    tables and biases carry signal), like the reference's ``randomize`` fixture."""

    with torch.random.fork_rng(devices=[]):
        torch.manual_seed(seed)
        trunk = Trunk(config)
        gen = torch.Generator().manual_seed(seed + 1)
        with torch.no_grad():
            for p in trunk.parameters():
                p.add_(scale * torch.randn(p.shape, generator=gen))
    return {f"trunk.{k}": v.detach().clone() for k, v in trunk.state_dict().items()}
