"""Policy sampling on the device: ``masked_probabilities`` and ``sample_rows`` of
cardgym/rl/ppo.py:75-94 over ROCm tensors, so a wave's logits need not be copied to the
host to pick its actions (cardgym/rl/selfplay.py:532-567 does that in numpy).

Same signatures and meaning as the reference functions, on tensors instead of arrays:
``masked_probabilities(logits [rows, width] float32, mask [rows, width] bool)`` and
``sample_rows(probabilities, mask, uniforms [rows] float64) -> int64 [rows]``.  The
sampling is the reference's bit for bit given the same probabilities and uniforms; the
probabilities follow numpy's float32 order except for the exp itself (an ulp at most).
"""

from __future__ import annotations

import torch

from .. import _native as nat
from ..nn.kv_cache import require_device, stream_handle


def _rows(t: torch.Tensor, name: str, dtype: torch.dtype) -> torch.Tensor:
    if t.dim() != 2:
        raise ValueError(f"{name} must be [rows, width]")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, not {t.dtype}")
    if t.stride(1) != 1:
        t = t.contiguous()
    return t


def masked_probabilities(logits: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
    """Softmax over legal entries only; illegal entries get exactly zero."""

    require_device(logits)
    logits = _rows(logits, "logits", torch.float32)
    mask = _rows(mask, "mask", torch.bool)
    if mask.shape != logits.shape or mask.device != logits.device:
        raise ValueError("mask must match logits in shape and device")
    rows, width = logits.shape
    probs = torch.empty((rows, width), device=logits.device, dtype=torch.float32)
    nat.call(
        "cg_masked_probabilities", logits.data_ptr(), logits.stride(0), mask.data_ptr(), mask.stride(0), rows, width,
        probs.data_ptr(), probs.stride(0), stream_handle(logits.device),
    )
    return probs


def sample_rows(probabilities: torch.Tensor, mask: torch.Tensor, uniforms: torch.Tensor) -> torch.Tensor:
    """Inverse-CDF sample one legal index per row; robust to rounding at the tail."""

    require_device(probabilities)
    probabilities = _rows(probabilities, "probabilities", torch.float32)
    mask = _rows(mask, "mask", torch.bool)
    rows, width = probabilities.shape
    if mask.shape != probabilities.shape or mask.device != probabilities.device:
        raise ValueError("mask must match probabilities in shape and device")
    if uniforms.shape != (rows,) or uniforms.dtype != torch.float64 or uniforms.device != probabilities.device:
        raise ValueError("uniforms must be float64 [rows] on the same device")
    uniforms = uniforms.contiguous()
    sampled = torch.empty(rows, device=probabilities.device, dtype=torch.int64)
    nat.call(
        "cg_sample_rows", probabilities.data_ptr(), probabilities.stride(0), mask.data_ptr(), mask.stride(0),
        uniforms.data_ptr(), rows, width, sampled.data_ptr(), stream_handle(probabilities.device),
    )
    return sampled
