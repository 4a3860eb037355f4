"""The fused layer kernel's GELU against torch's own GELU on the device, for every one of
the 65536 bf16 bit patterns.

Under autocast the MLP's first Linear returns bf16 (cardgym/nn/trunk.py:135) and nn.GELU
maps that bf16 tensor to bf16 (x * 0.5 * (1 + erf(x / sqrt 2)) in fp32, then rounded).  The
kernel rounds the Linear's fp32 accumulators to bf16 the same way and evaluates GELU with
the erf of Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), so after the bf16 rounding it
differs from torch only where torch's fp32 value lies within that error of a rounding
boundary.  Bar: the same NaN positions, at most one bf16 ulp anywhere, and at most 16 of the
65280 finite patterns off by that ulp (an fp32 emulation of both formulas finds 3).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from card_playing_gym_amd import _native as nat
from card_playing_gym_amd.nn.kv_cache import stream_handle

pytestmark = pytest.mark.gpu


def test_kernel_gelu_is_torch_gelu_on_every_bf16(device):
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16).to(device)
    x = bits.view(torch.bfloat16)
    y = torch.empty_like(x)
    nat.call("cg_gelu_bf16", x.data_ptr(), y.data_ptr(), x.numel(), stream_handle(device))
    want = F.gelu(x)
    torch.cuda.synchronize()
    got_f, want_f = y.float(), want.float()
    nan_got, nan_want = torch.isnan(got_f), torch.isnan(want_f)
    assert torch.equal(nan_got, nan_want), "NaN positions differ"
    inf = torch.isinf(want_f)
    assert torch.equal(got_f[inf], want_f[inf])
    ok = ~nan_got & ~inf
    diff = (got_f[ok] - want_f[ok]).abs()
    off = diff > 0
    # One bf16 ulp of torch's value (its spacing at that magnitude; subnormal spacing floor).
    ulp = torch.clamp(want_f[ok].abs() * 2.0**-7, min=2.0**-133)
    worst = (diff / ulp).max().item()
    print(f"GELU: {int(off.sum())} of {int(ok.sum())} patterns differ, worst {worst:.3f} ulp")
    assert worst <= 1.0 + 1e-6
    assert int(off.sum()) <= 16
    infs = torch.tensor([float("inf"), float("-inf")], dtype=torch.bfloat16, device=device)
    out = torch.empty_like(infs.repeat(2))
    nat.call("cg_gelu_bf16", infs.repeat(2).data_ptr(), out.data_ptr(), 4, stream_handle(device))
    torch.cuda.synchronize()
    assert out[0].item() == float("inf") and torch.isnan(out[1].float()).item()


def test_gelu_refuses_bad_arguments(device):
    x = torch.zeros(6, dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        nat.call("cg_gelu_bf16", x.data_ptr(), x.data_ptr(), 6, stream_handle(device))  # not a multiple of 4
    with pytest.raises(ValueError):
        nat.call("cg_gelu_bf16", None, None, 4, stream_handle(device))
