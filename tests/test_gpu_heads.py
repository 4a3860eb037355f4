"""Fused policy / value heads (cg_heads_forward) against the oracle's bf16 heads.

The heads are bf16 autocast Linear layers (cardgym/nn/model.py:12-17 evaluated as
cardgym/rl/graphs.py:88-104): both sides round operands to bf16, accumulate in fp32 and
round every Linear and GELU output to bf16, so they differ only where a different fp32
summation order moves a result across a bf16 rounding boundary: at most 2 bf16 ulps
(2 x 2^-8 relative) on logits; values also see such flips of single mid activations.
"""

from __future__ import annotations

import ctypes
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from card_playing_gym_amd import _native as nat
from card_playing_gym_amd.nn.kv_cache import stream_handle
from card_playing_gym_amd.synthetic import SyntheticModel, build_model, trunk_config
from oracle.reference_path import RefSynthetic, RefTrunk, ref_config_of
from tests.helpers import autocast

pytestmark = pytest.mark.gpu

ULP2 = 2.0 ** -7  # two bf16 ulps, relative


def rel_err(got: torch.Tensor, want: torch.Tensor, floor: float) -> float:
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    return ((got - want).abs() / (want.abs() + floor)).max().item()


def oracle_heads(model: SyntheticModel, hidden: torch.Tensor):
    state = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    return RefSynthetic(state, ref_config_of(model.trunk_config), "bf16").heads(hidden.detach().cpu())


@pytest.mark.parametrize("rows", [1, 17, 4096])
def test_synthetic_heads_match_the_oracle(device, rows):
    model = build_model(trunk_config(2), seed=3, device=device)
    gen = torch.Generator().manual_seed(rows)
    hidden = torch.randn(rows, 256, generator=gen).to(device)
    with torch.no_grad(), autocast(device, "bf16"):
        logits, values = model.heads(hidden)
    want_logits, want_values = oracle_heads(model, hidden)
    assert logits.shape == (rows, 512) and values.shape == (rows, 2)
    assert rel_err(logits, want_logits, 1e-3) <= ULP2
    assert rel_err(values, want_values, 1e-2) <= 4 * ULP2


def test_heads_follow_in_place_weight_updates(device):
    model = build_model(trunk_config(1), seed=4, device=device)
    hidden = torch.randn(64, 256, generator=torch.Generator().manual_seed(1)).to(device)
    with torch.no_grad(), autocast(device, "bf16"):
        before, _ = model.heads(hidden)
        model.policy_head.bias.add_(1.0)  # an optimiser-style in-place edit
        model.value_head[2].weight.mul_(-1.0)
        after, values = model.heads(hidden)
    want_logits, want_values = oracle_heads(model, hidden)
    assert (after - before).mean().item() == pytest.approx(1.0, abs=0.02)
    assert rel_err(after, want_logits, 1e-3) <= ULP2
    assert rel_err(values, want_values, 1e-2) <= 4 * ULP2


@pytest.mark.parametrize("d, n_policy, d_mid, n_value, rows", [
    (64, 48, 96, 1, 33), (128, 1024, 256, 16, 50), (256, 272, 16, 3, 16), (16, 16, 16, 2, 5),
])
def test_heads_shapes_through_the_c_abi(device, d, n_policy, d_mid, n_value, rows):
    """Every shape class the kernel takes: ragged last row block, partial policy chunk,
    narrow and wide value MLPs, the n_value limit."""

    gen = torch.Generator().manual_seed(d + n_policy + d_mid)
    t = lambda *shape, s=0.05: (s * torch.randn(*shape, generator=gen)).float()
    wp, bp, w1, b1, w2, b2 = t(n_policy, d), t(n_policy), t(d_mid, d), t(d_mid), t(n_value, d_mid, s=0.2), t(n_value)
    hidden = t(rows, d, s=1.0)
    dev = [x.to(device).contiguous() for x in (wp, bp, w1, b1, w2, b2, hidden)]
    config = nat.HeadsConfig(d, n_policy, d_mid, n_value)
    handle = ctypes.c_void_p()
    nat.call("cg_heads_create", ctypes.byref(config), *(x.data_ptr() for x in dev[:6]), ctypes.byref(handle))
    try:
        logits = torch.full((rows, n_policy), float("nan"), device=device)
        values = torch.full((rows, n_value), float("nan"), device=device)
        nat.call("cg_heads_forward", handle, dev[6].data_ptr(), rows, logits.data_ptr(), values.data_ptr(),
                 stream_handle(device))
        torch.cuda.synchronize()
    finally:
        nat.lib().cg_heads_destroy(handle)
    lin = lambda x, w, b: RefTrunk.lin(SimpleNamespace(bf16=True), x, w, b)  # the oracle's bf16 Linear
    want_logits = lin(hidden, wp, bp).float()
    want_values = lin(F.gelu(lin(hidden, w1, b1)), w2, b2).float()
    assert torch.isfinite(logits).all() and torch.isfinite(values).all()
    assert rel_err(logits, want_logits, 1e-3) <= ULP2
    assert rel_err(values, want_values, 1e-2) <= 4 * ULP2
