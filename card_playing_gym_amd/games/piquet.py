"""Piquet's token embedder on the HIP path (API of cardgym.games.piquet.model).

``PiquetEmbedding`` keeps the reference's module tree and parameter names
(cardgym/games/piquet/model.py:114-341: ``fields``, ``ple_fields``, ``value_fields``,
``grid.code``, ``grid.rank``, ``grid.blocks.{i}.{norm, along_rank, across_suits, out}``,
``grid.norm``, ``grid.summary``), so a PiquetActor state dict's ``embedding.*`` entries load
unchanged, and returns what the reference's forward returns under bf16 autocast: the
trunk input sum, the per-layer and value lookups (bf16), keeping the per-card features
for the card heads (``kept``, fp32).  The whole forward is two launches of
``cg_piquet_embed`` (csrc/piquet.hip); there is no CPU path and no other precision: it
runs on a ROCm device under ``torch.autocast("cuda", dtype=torch.bfloat16)``, the
precision the reference's CUDA rollouts use, and raises otherwise.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch
from torch import nn

from .. import _native as nat
from ..nn import ops
from ..nn.derived import DerivedCopies, HandleCache, after_load_hook
from ..nn.kv_cache import require_device, stream_handle
from ..nn.trunk import TrunkConfig

# The token layout of cardgym/games/piquet/tokens.py:108-152 and the card numbering of
# cards.py:11-14, 26-35 (card = suit * 8 + rank).
NUM_SUITS, NUM_RANKS = 4, 8
NUM_CARDS = NUM_SUITS * NUM_RANKS
NUM_FIELDS = 32
CARD_START = NUM_FIELDS
CARD_VOCAB = 12
_HEADS, _TRICKS, _TALON = 3, 12, 8  # engine.py:50-56
_TOTAL_VOCAB = 120 + 21
_LEAD_VOCAB = 2 * (60 + 14) + 1
FIELD_VOCAB = (
    8, 1 + _HEADS, 3, 2, NUM_CARDS + 1, 9, 9, 4, 4, 9, 76, 9, 3, 4, 64, 5, 3,
    _TRICKS + 1, 3, 5, _TRICKS + 1, _TRICKS + 1, 100, 100, _TOTAL_VOCAB, _TOTAL_VOCAB,
    6, 2, _TALON + 1, 16, 4, _LEAD_VOCAB,
)
FIELD_OFFSETS = tuple(sum(FIELD_VOCAB[:i]) for i in range(NUM_FIELDS))
CARD_RANKS = tuple(card & 7 for card in range(NUM_CARDS))


@dataclass(frozen=True)
class PiquetModelConfig:
    """The [model] section's embedder and trunk fields (model.py:79-112, same defaults)."""

    d_model: int = 256
    n_layers: int = 16
    n_heads: int = 8
    n_kv_heads: int = 2
    d_ff: int = 512
    per_layer_dim: int = 64
    value_embeddings: str = "alternating"
    card_width: int = 32
    card_hidden: int = 64
    card_layers: int = 2
    card_kernel: int = 3

    def trunk(self) -> TrunkConfig:
        return TrunkConfig(
            d_model=self.d_model, n_layers=self.n_layers, n_heads=self.n_heads, n_kv_heads=self.n_kv_heads,
            d_ff=self.d_ff, per_layer_dim=self.per_layer_dim, value_embeddings=self.value_embeddings,
            input_norm=True,
        )


def _init(module: nn.Module) -> None:
    """N(0, 0.02) weights and zero biases (cardgym/nn/trunk.py:93-101)."""

    if isinstance(module, (nn.Linear, nn.Conv1d)):
        nn.init.normal_(module.weight, std=0.02)
        if module.bias is not None:
            nn.init.zeros_(module.bias)
    elif isinstance(module, nn.Embedding):
        nn.init.normal_(module.weight, std=0.02)


class GridNorm(nn.Module):
    """RMSNorm with a gain (model.py:114-125); evaluated inside the grid kernel."""

    def __init__(self, width: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(width))
        self.eps = eps


class GridBlock(nn.Module):
    """Parameters of one grid block (model.py:128-151); evaluated inside the grid kernel."""

    def __init__(self, width: int, hidden: int, kernel: int) -> None:
        super().__init__()
        self.kernel = kernel
        self.norm = GridNorm(width)
        self.along_rank = nn.Conv1d(width, hidden, kernel)
        self.across_suits = nn.Linear(width, hidden, bias=False)
        self.out = nn.Linear(hidden, width)


class CardGrid(nn.Module):
    """Parameters of the card grid (model.py:180-211)."""

    def __init__(self, config: PiquetModelConfig) -> None:
        super().__init__()
        width = config.card_width
        self.width = width
        self.code = nn.Embedding(CARD_VOCAB, width)
        self.rank = nn.Embedding(NUM_RANKS, width)
        self.blocks = nn.ModuleList(
            GridBlock(width, config.card_hidden, config.card_kernel) for _ in range(config.card_layers)
        )
        self.norm = GridNorm(width)
        self.summary = nn.Linear(NUM_CARDS * width, config.d_model, bias=False)
        for module in (self.code, self.rank, *self.blocks):
            module.apply(_init)
        with torch.no_grad():
            for block in self.blocks:
                block.out.weight.mul_(1.0 / max(len(self.blocks), 1) ** 0.5)
        nn.init.normal_(self.summary.weight, std=0.02 * (NUM_FIELDS / (NUM_CARDS * width)) ** 0.5)


class PiquetEmbedding(ops.Registered, nn.Module):
    """Token fields plus the card-grid summary (model.py:286-341), on the HIP path."""

    def __init__(self, config: PiquetModelConfig, ple_width: int, value_width: int) -> None:
        super().__init__()
        self.config = config
        self.kept: torch.Tensor | None = None
        rows = sum(FIELD_VOCAB)
        self.fields = nn.Embedding(rows, config.d_model)
        _init(self.fields)
        self.ple_fields = nn.Embedding(rows, ple_width) if ple_width else None
        self.value_fields = nn.Embedding(rows, value_width) if value_width else None
        for table in (self.ple_fields, self.value_fields):
            if table is not None:
                nn.init.zeros_(table.weight)
        self.grid = CardGrid(config)
        # bf16 copies of the tables and the grid's matrices, kept current after optimiser
        # steps and load_state_dict (card_playing_gym_amd/nn/derived.py).
        self._handles = HandleCache()
        self.register_load_state_dict_post_hook(after_load_hook)
        self._register_op_key()

    def _params(self) -> list[torch.Tensor]:
        g = self.grid
        out = [self.fields.weight, g.code.weight, g.rank.weight, g.norm.weight, g.summary.weight]
        out += [t.weight for t in (self.ple_fields, self.value_fields) if t is not None]
        for b in g.blocks:
            out += [b.norm.weight, b.along_rank.weight, b.along_rank.bias, b.across_suits.weight, b.out.weight,
                    b.out.bias]
        for t in out:
            if t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError("embedder parameters must be contiguous float32 tensors")
        return out

    def native(self, device: torch.device) -> _NativePiquet:
        params = self._params()
        key = device.index if device.index is not None else torch.cuda.current_device()
        return self._handles.get(key, params, lambda: _NativePiquet(self, params, device), stream_handle(device))

    def refresh_native(self) -> int:
        """Re-derives the bf16 copies now if the parameters changed in place (optimiser steps
        and ``load_state_dict`` do this by themselves)."""

        return self._handles.refresh()

    def _apply(self, fn, *args, **kwargs):
        out = super()._apply(fn, *args, **kwargs)
        handles = self.__dict__.get("_handles")
        if handles is not None:
            handles.retire_moved(lambda key: self._params())
        return out

    def forward(self, tokens: torch.Tensor):
        """(x, ple lookup, value lookup) for [..., 64] tokens; ``kept`` = cards [..., 32, w]."""

        require_device(tokens, self.fields.weight)
        device = tokens.device
        if not (torch.is_autocast_enabled(device.type) and torch.get_autocast_dtype(device.type) == torch.bfloat16):
            raise RuntimeError("the HIP Piquet embedder runs under torch.autocast(device, dtype=torch.bfloat16) only")
        if torch.is_grad_enabled() and any(p.requires_grad for p in self.parameters()):
            # The kernels have no backward: under autograd the tables and the grid would get
            # no gradient, silently.  Rollouts run under no_grad (cardgym/rl/continuous.py:165-179).
            raise RuntimeError(
                "the HIP Piquet embedder is inference-only: call it under torch.no_grad() (rollout), "
                "or train with the reference's PiquetEmbedding (requires_grad parameters under autograd)"
            )
        lead = tokens.shape[:-1]
        flat = tokens.reshape(-1, tokens.shape[-1])
        if flat.shape[1] != NUM_FIELDS + NUM_CARDS:
            raise ValueError("a Piquet token holds 32 fields and 32 card codes")
        flat = flat.to(torch.int64).contiguous()
        c = self.config
        ple_width = 0 if self.ple_fields is None else self.ple_fields.embedding_dim
        value_width = 0 if self.value_fields is None else self.value_fields.embedding_dim
        x, ple, values, cards = ops.piquet_embed(flat, self.op_key, c.d_model, ple_width, value_width, c.card_width)
        self.kept = cards.view(*lead, NUM_CARDS, c.card_width)
        return (
            x.view(*lead, -1),
            None if self.ple_fields is None else ple.view(*lead, -1),
            None if self.value_fields is None else values.view(*lead, -1),
        )

    def _embed_native(self, flat: torch.Tensor):
        """The launch behind ``torch.ops.cardgym_hip.piquet_embed`` (flat int64 tokens [n, 64])."""

        device = flat.device
        n = flat.shape[0]
        c = self.config
        widths = [0 if t is None else t.embedding_dim for t in (self.ple_fields, self.value_fields)]
        x = torch.empty((n, c.d_model), device=device, dtype=torch.bfloat16)
        ple, values = (torch.empty((n, w), device=device, dtype=torch.bfloat16) for w in widths)
        cards = torch.empty((n, NUM_CARDS, c.card_width), device=device, dtype=torch.float32)
        handle = self.native(device)
        nat.call(
            "cg_piquet_embed", handle.handle, flat.data_ptr(), flat.shape[1], n, x.data_ptr(),
            ple.data_ptr() if widths[0] else None, values.data_ptr() if widths[1] else None, cards.data_ptr(), None,
            stream_handle(device),
        )
        return x, ple, values, cards


class _NativePiquet(DerivedCopies):
    """A ``cg_piquet`` handle over the embedder's parameters (bf16 copies of the tables and
    the grid's matrices)."""

    def __init__(self, module: PiquetEmbedding, params: list[torch.Tensor], device: torch.device) -> None:
        super().__init__(params, device)
        c = module.config
        g = module.grid
        cfg = nat.PiquetConfig(
            c.d_model, 0 if module.ple_fields is None else module.ple_fields.embedding_dim,
            0 if module.value_fields is None else module.value_fields.embedding_dim, sum(FIELD_VOCAB),
            c.card_width, c.card_hidden, c.card_kernel, c.card_layers, g.norm.eps,
        )
        blocks = (nat.PiquetBlock * max(len(g.blocks), 1))()
        for i, b in enumerate(g.blocks):
            blocks[i] = nat.PiquetBlock(
                b.norm.weight.data_ptr(), b.along_rank.weight.data_ptr(), b.along_rank.bias.data_ptr(),
                b.across_suits.weight.data_ptr(), b.out.weight.data_ptr(), b.out.bias.data_ptr(),
            )
        offsets = (ctypes.c_int32 * NUM_FIELDS)(*FIELD_OFFSETS)
        handle = ctypes.c_void_p()
        nat.call(
            "cg_piquet_create", ctypes.byref(cfg), offsets, module.fields.weight.data_ptr(),
            None if module.ple_fields is None else module.ple_fields.weight.data_ptr(),
            None if module.value_fields is None else module.value_fields.weight.data_ptr(),
            g.code.weight.data_ptr(), g.rank.weight.data_ptr(), blocks, g.norm.weight.data_ptr(),
            g.summary.weight.data_ptr(), ctypes.byref(handle),
        )
        self.handle = handle

    def _refresh(self, stream: int) -> None:
        nat.call("cg_piquet_refresh", self.handle, stream)

    def close(self) -> None:
        if self.handle:
            try:
                nat.lib().cg_piquet_destroy(self.handle)
            finally:
                self.handle = ctypes.c_void_p()
