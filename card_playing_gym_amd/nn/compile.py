"""``torch.compile`` of the decode wave on the GPU (API of cardgym.nn.compile).

Same switches as cardgym/nn/compile.py:20-44: compiled with dynamic shapes on a GPU device
unless ``CARDGYM_COMPILE=0``, the function itself elsewhere.  Every HIP launch of the wave
is a custom op (card_playing_gym_amd/nn/ops.py), so Inductor only fuses the small torch
glue between them (casts, reshapes, the output concatenation).
"""

from __future__ import annotations

import os

import torch


def compile_enabled(device: torch.device) -> bool:
    return device.type == "cuda" and os.environ.get("CARDGYM_COMPILE", "1") != "0"


def compiled(fn, device: torch.device):
    """``fn`` under ``torch.compile(dynamic=True)`` on the GPU (unless disabled)."""

    if not compile_enabled(device):
        return fn
    from torch._dynamo import config as dynamo_config
    from torch._inductor import config as inductor_config

    # One compile per wave shape family; keep the compile in this process (no worker pool
    # left resident beside a rollout worker), and room for the shapes a collection meets.
    inductor_config.compile_threads = 1
    dynamo_config.cache_size_limit = max(dynamo_config.cache_size_limit, 64)
    return torch.compile(fn, dynamic=True)
