"""Token embedder in front of the shared trunk (API of cardgym.nn.model.SequenceModel).

``SequenceModel`` keeps the reference's entry points (cardgym/nn/model.py:20-106):
``embed`` (the game's hook), ``prepare``, ``forward_hidden``, ``forward_prefill``,
``forward_ragged`` and ``new_cache``, plus ``forward_packed`` for variable-length chunks
without padding.  Everything after ``embed`` runs on the HIP kernels.
"""

from __future__ import annotations

import torch
from torch import nn

from .kv_cache import KVCache
from .trunk import Trunk, TrunkConfig, init_weights


def value_mlp(d_model: int, outputs: int) -> nn.Sequential:
    """Hidden -> GELU MLP -> per-seat outputs (cardgym/nn/model.py:12-17)."""

    head = nn.Sequential(nn.Linear(d_model, d_model), nn.GELU(), nn.Linear(d_model, outputs))
    head.apply(init_weights)
    return head


class SequenceModel(nn.Module):
    """Subclasses implement :meth:`embed` (raw embedding sum [B, T, d] plus the packed
    per-layer and value-embedding lookups, or None) and add their own heads."""

    def __init__(self, trunk_config: TrunkConfig) -> None:
        super().__init__()
        self.trunk = Trunk(trunk_config)

    @property
    def trunk_config(self) -> TrunkConfig:
        return self.trunk.config

    @property
    def device(self) -> torch.device:
        return next(self.parameters()).device

    def packs(self, device: torch.device) -> bool:
        """Whether this model runs packed rows (cardgym.nn.packing) on ``device`` (model.py:50-58):
        the trunk's HIP path takes per-row sequence bounds on the GPU, forward and backward, so
        the trainer's microbatches may be packed there; elsewhere padded batches run as they are."""

        return device.type == "cuda" and torch.version.hip is not None

    def enable_metal_trunk(self, max_length: int | None = None) -> None:
        """The reference routes MPS bf16 trunks through fused Metal kernels (model.py:108-115);
        the HIP trunk is always fused, so there is nothing to enable and ``trunk.metal`` stays None."""

    def embed(self, tokens: torch.Tensor):
        raise NotImplementedError

    def prepare(self, tokens: torch.Tensor):
        """Embed and condition: the trunk's (x, ple, values) inputs."""

        return self.trunk.condition(*self.embed(tokens))

    def forward_hidden(self, tokens: torch.Tensor, bounds: torch.Tensor | None = None) -> torch.Tensor:
        """Full causal forward; final-norm hidden states [B, T, d]."""

        return self.trunk(*self.prepare(tokens), bounds)

    def forward_prefill(self, tokens: torch.Tensor, cache: KVCache, rows: torch.Tensor | None) -> torch.Tensor:
        """Encode fresh prefixes [B, T, W] into cache rows; last hidden [B, d]."""

        return self.trunk.forward_prefill(*self.prepare(tokens), cache, rows)

    def forward_ragged(
        self,
        tokens: torch.Tensor,
        positions: torch.Tensor,
        cache: KVCache,
        readout_offsets: torch.Tensor,
        span: int | None = None,
        rows: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Append a padded run per cache row 0..B-1 (or ``rows``); hidden at each readout [B, d]."""

        return self.trunk.forward_ragged(*self.prepare(tokens), cache, positions, readout_offsets, span, rows)

    def forward_packed(
        self,
        tokens: torch.Tensor,
        seq_start: torch.Tensor,
        positions: torch.Tensor,
        cache: KVCache,
        readout_offsets: torch.Tensor | None,
        rows: torch.Tensor | None = None,
        span: int | None = None,
    ) -> torch.Tensor:
        """Append packed chunks [N, W] (sequence b owns tokens seq_start[b]..seq_start[b+1]-1)."""

        x, ple, values = self.prepare(tokens.unsqueeze(0))
        return self.trunk.forward_packed(
            x[0], None if ple is None else ple[0], None if values is None else values[0],
            cache, positions, seq_start, readout_offsets, rows, span,
        )

    def new_cache(self, capacity: int, max_len: int, dtype: torch.dtype = torch.float32) -> KVCache:
        config = self.trunk_config
        return KVCache(
            n_layers=config.n_layers,
            kv_heads=config.n_kv_heads,
            head_dim=config.head_dim,
            capacity=capacity,
            max_len=max_len,
            device=self.device,
            dtype=dtype,
        )
