"""GQA decoder trunk with a KV-cached ragged step on MI355X (API of cardgym.nn.trunk).

The module tree and parameter names are those of the reference trunk
(cardgym/nn/trunk.py:124-281): ``input_norm``, ``ple_context``, ``blocks[i].ln_attn``,
``.qkv_proj``, ``.out_proj``, ``.ln_mlp``, ``.mlp[0|2]``, ``final_norm``, so a reference
state dict loads unchanged and the collectors' calls keep their meaning.  Every forward
runs on the HIP kernels of libcardgym_hip.so through one ``cg_trunk_forward`` call per
step (all layers, append + attention + projections); there is no PyTorch compute path.

Precision follows the caller's autocast state, as the reference's collectors set it
(cardgym/core/devices.py:32-43): under ``torch.autocast("cuda", dtype=torch.bfloat16)``
the projections run as bf16 x bf16 MFMA with fp32 accumulation, otherwise in fp32.
The KV storage dtype is the cache's own.  Norms, softmax and the residual stream are
always fp32.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Literal

import numpy as np
import torch
from torch import nn

from .. import _native as nat
from . import ops
from .derived import DerivedCopies, HandleCache, after_load_hook
from .kv_cache import KVCache, check_enabled, index_tensor, require_device, stream_handle

ValueEmbeddingMode = Literal["off", "alternating", "all"]


@dataclass(frozen=True)
class TrunkConfig:
    """Fields and derived sizes of cardgym.nn.trunk.TrunkConfig (trunk.py:39-91)."""

    d_model: int = 256
    n_layers: int = 6
    n_heads: int = 8
    n_kv_heads: int = 2
    d_ff: int = 768
    per_layer_dim: int = 0
    value_embeddings: ValueEmbeddingMode = "off"
    input_norm: bool = True

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    @property
    def kv_width(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def value_layers(self) -> tuple[int, ...]:
        """Blocks whose V receives a value embedding: none, all, or the last block and
        every other block before it."""

        if self.value_embeddings == "off":
            return ()
        if self.value_embeddings == "all":
            return tuple(range(self.n_layers))
        last_parity = (self.n_layers - 1) % 2
        return tuple(layer for layer in range(self.n_layers) if layer % 2 == last_parity)

    @property
    def ple_width(self) -> int:
        return self.n_layers * self.per_layer_dim

    @property
    def value_width(self) -> int:
        return len(self.value_layers) * self.kv_width

    def validate(self) -> None:
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads.")
        if self.n_kv_heads > self.n_heads or self.n_heads % self.n_kv_heads:
            raise ValueError("n_kv_heads must divide n_heads.")
        if self.per_layer_dim < 0:
            raise ValueError("per_layer_dim must be non-negative.")
        if self.value_embeddings not in ("off", "alternating", "all"):
            raise ValueError(f"Unknown value_embeddings mode {self.value_embeddings!r}.")


def init_weights(module: nn.Module) -> None:
    """N(0, 0.02) Linear / Embedding weights and zero biases (trunk.py:93-101)."""

    if isinstance(module, nn.Linear):
        nn.init.normal_(module.weight, mean=0.0, std=0.02)
        if module.bias is not None:
            nn.init.zeros_(module.bias)
    elif isinstance(module, nn.Embedding):
        nn.init.normal_(module.weight, mean=0.0, std=0.02)


class RMSNorm(nn.Module):
    """Gain-only RMSNorm (trunk.py:104-115); evaluated by the ``cg_rmsnorm`` kernel."""

    def __init__(self, d: int, eps: float = 1e-5) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        require_device(x)
        # A bf16 input (a game embedder's autocast sum) keeps its dtype: the kernel rounds
        # the normalised value to bf16 before the gain, as .to(x.dtype) does.
        bf16 = x.dtype == torch.bfloat16
        flat = x.reshape(-1, x.shape[-1])
        flat = (flat if bf16 else flat.float()).contiguous()
        return ops.rmsnorm(flat, self.weight, float(self.eps)).view(x.shape)


class DecoderBlock(nn.Module):
    """Parameters of one pre-LN GQA block (trunk.py:124-139).

    The block's computation is fused into the trunk-level kernels; it is not callable
    on its own (run ``Trunk.forward_ragged`` / ``forward_prefill`` / ``forward``).
    """

    def __init__(self, config: TrunkConfig) -> None:
        super().__init__()
        d = config.d_model
        self.n_heads = config.n_heads
        self.kv_heads = config.n_kv_heads
        self.head_dim = config.head_dim
        self.head_group = config.n_heads // config.n_kv_heads
        self.scale = 1.0 / math.sqrt(config.head_dim)
        self.ln_attn = nn.LayerNorm(d)
        self.qkv_proj = nn.Linear(d, (self.n_heads + 2 * self.kv_heads) * self.head_dim, bias=False)
        self.out_proj = nn.Linear(self.n_heads * self.head_dim, d, bias=False)
        self.ln_mlp = nn.LayerNorm(d)
        self.mlp = nn.Sequential(nn.Linear(d, config.d_ff), nn.GELU(), nn.Linear(config.d_ff, d))

    def forward(self, *args, **kwargs):  # pragma: no cover - guidance only
        raise NotImplementedError("Blocks run fused inside Trunk.forward_ragged / forward_prefill / forward.")


def _param(tensor: torch.Tensor) -> torch.Tensor:
    if tensor.dtype != torch.float32 or not tensor.is_contiguous():
        raise ValueError("trunk parameters must be contiguous float32 tensors")
    return tensor


def compute_dtype_code(device: torch.device) -> int:
    """bf16 projections under bf16 autocast on the device, fp32 without autocast.

    fp16 autocast (the reference's ``precision = "fp16"``) is refused rather than run in
    another precision: the kernels have no fp16 projection path.  An fp16 KV pool is
    supported under either precision."""

    if torch.is_autocast_enabled(device.type):
        dtype = torch.get_autocast_dtype(device.type)
        if dtype == torch.bfloat16:
            return nat.CG_BF16
        if dtype == torch.float16:
            raise RuntimeError(
                "fp16 autocast is not supported by the HIP trunk: run under bf16 autocast or fp32 "
                "(an fp16 KV cache works with either)"
            )
    return nat.CG_F32


class _NativeTrunk(DerivedCopies):
    """A ``cg_trunk`` handle over the module's parameters for one compute dtype."""

    def __init__(self, trunk: "Trunk", compute: int, device: torch.device) -> None:
        super().__init__(_trunk_tensors(trunk), device)
        self.compute = compute
        config = trunk.config
        cfg = nat.TrunkConfig(
            config.d_model, config.n_layers, config.n_heads, config.n_kv_heads, config.d_ff,
            config.per_layer_dim, config.value_width, float(trunk.final_norm.eps),
        )
        layers = (nat.LayerParams * config.n_layers)()
        for index, block in enumerate(trunk.blocks):
            layers[index] = nat.LayerParams(
                _param(block.ln_attn.weight).data_ptr(), _param(block.ln_attn.bias).data_ptr(),
                _param(block.qkv_proj.weight).data_ptr(), _param(block.out_proj.weight).data_ptr(),
                _param(block.ln_mlp.weight).data_ptr(), _param(block.ln_mlp.bias).data_ptr(),
                _param(block.mlp[0].weight).data_ptr(), _param(block.mlp[0].bias).data_ptr(),
                _param(block.mlp[2].weight).data_ptr(), _param(block.mlp[2].bias).data_ptr(),
                trunk._value_index.get(index, -1),
            )
        self.layers = layers
        handle = ctypes.c_void_p()
        nat.call(
            "cg_trunk_create", ctypes.byref(cfg), layers, _param(trunk.final_norm.weight).data_ptr(),
            _param(trunk.final_norm.bias).data_ptr(), compute, ctypes.byref(handle),
        )
        self.handle = handle

    def _refresh(self, stream: int) -> None:
        nat.call("cg_trunk_refresh", self.handle, stream)

    def close(self) -> None:
        if self.handle:
            try:
                nat.lib().cg_trunk_destroy(self.handle)
            finally:
                self.handle = ctypes.c_void_p()


def _trunk_tensors(trunk: "Trunk"):
    for block in trunk.blocks:
        yield from (
            block.ln_attn.weight, block.ln_attn.bias, block.qkv_proj.weight, block.out_proj.weight,
            block.ln_mlp.weight, block.ln_mlp.bias, block.mlp[0].weight, block.mlp[0].bias,
            block.mlp[2].weight, block.mlp[2].bias,
        )
    yield trunk.final_norm.weight
    yield trunk.final_norm.bias


class Trunk(ops.Registered, nn.Module):
    def __init__(self, config: TrunkConfig) -> None:
        super().__init__()
        config.validate()
        self.config = config
        d = config.d_model
        self.input_norm = RMSNorm(d) if config.input_norm else None
        self.ple_context = nn.Linear(d, config.ple_width, bias=False) if config.per_layer_dim else None
        self.blocks = nn.ModuleList(DecoderBlock(config) for _ in range(config.n_layers))
        self.final_norm = nn.LayerNorm(d)
        self._value_index = {layer: index for index, layer in enumerate(config.value_layers)}
        self.blocks.apply(init_weights)
        # GPT-2 residual scaling of the two projections that write the stream (trunk.py:276-279).
        residual_scale = 1.0 / math.sqrt(2 * config.n_layers)
        for block in self.blocks:
            block.out_proj.weight.data.mul_(residual_scale)
            block.mlp[2].weight.data.mul_(residual_scale)
        if self.ple_context is not None:
            nn.init.zeros_(self.ple_context.weight)
        # bf16 weight copies per (device, compute dtype), kept current after optimiser steps
        # and load_state_dict (card_playing_gym_amd/nn/derived.py).
        self._handles = HandleCache()
        self.register_load_state_dict_post_hook(after_load_hook)
        # The key naming this trunk inside torch.ops.cardgym_hip.trunk_step.
        self._register_op_key()
        # The reference's fused Metal trunk (trunk.py:274, model.py:108-115) exists only on
        # MPS; callers read `metal` and `uses_metal` to choose that path.  Here the HIP
        # kernels are the path on every call, so there is never a Metal trunk.
        self.metal = None

    def uses_metal(self, device: torch.device, length: int) -> bool:
        """The reference's gate for its MPS-only fused kernels (trunk.py:337-346): never here."""

        return False

    # -- native handle ---------------------------------------------------------

    def native(self, device: torch.device, compute: int | None = None) -> _NativeTrunk:
        """The handle for ``device`` and a compute type (the autocast state's by default)."""

        if compute is None:
            compute = compute_dtype_code(device)
        key = (device.index if device.index is not None else torch.cuda.current_device(), compute)
        return self._handles.get(
            key, list(_trunk_tensors(self)), lambda: _NativeTrunk(self, compute, device), stream_handle(device)
        )

    def refresh_native(self) -> int:
        """Re-derives the bf16 weight copies now, if the parameters changed in place since
        (optimiser steps and ``load_state_dict`` do this by themselves).  Returns the number
        of handles refreshed."""

        return self._handles.refresh()

    def _apply(self, fn, *args, **kwargs):
        out = super()._apply(fn, *args, **kwargs)
        # Handles hold raw pointers: those whose parameters moved are retired (kept alive for
        # graphs captured before the move, no longer used for new calls).
        handles = self.__dict__.get("_handles")
        if handles is not None:
            handles.retire_moved(lambda key: list(_trunk_tensors(self)))
        return out

    # -- conditioning ----------------------------------------------------------

    def condition(self, x: torch.Tensor, ple_lookup: torch.Tensor | None, value_lookup: torch.Tensor | None):
        """Normalise the embedding sum and shape the per-layer streams (trunk.py:285-312)."""

        require_device(x)
        if self._recording(x):
            return self._condition_train(x, ple_lookup, value_lookup)
        if self.input_norm is not None:
            x = self.input_norm(x)
        else:
            x = x.float()
        lead = x.shape[:-1]
        ple = None
        if self.ple_context is not None:
            if ple_lookup is None:
                raise ValueError("This trunk expects a per-layer embedding lookup.")
            flat = x.reshape(-1, x.shape[-1]).contiguous()
            # A bf16 lookup (a game embedder under autocast) is read as bf16 and the sum and
            # its scaling round to bf16, as the reference's bf16 tensor arithmetic does.
            bf16 = ple_lookup.dtype == torch.bfloat16
            lookup = ple_lookup.reshape(flat.shape[0], -1)
            lookup = (lookup if bf16 else lookup.float()).contiguous()
            out = ops.ple_context(flat, self.ple_context.weight, lookup, 1.0 / math.sqrt(2.0),
                                  compute_dtype_code(x.device))
            ple = out.view(*lead, self.config.n_layers, self.config.per_layer_dim)
        values = None
        if self._value_index:
            if value_lookup is None:
                raise ValueError("This trunk expects a value-embedding lookup.")
            values = value_lookup.view(*lead, len(self._value_index), self.config.kv_width)
        return x, ple, values

    def _recording(self, *inputs: torch.Tensor | None) -> bool:
        """Whether autograd records this call (training)."""

        if not torch.is_grad_enabled():
            return False
        return any(t is not None and t.requires_grad for t in inputs) or any(p.requires_grad for p in self.parameters())

    @torch.compiler.disable
    def _condition_train(self, x, ple_lookup, value_lookup):
        from .train import PleContextFunction, RMSNormFunction, train_precision

        bf16 = train_precision(x.device)
        if self.input_norm is not None:
            x = RMSNormFunction.apply(x, self.input_norm.weight, self.input_norm.eps)
        else:
            x = x.float()
        lead = x.shape[:-1]
        ple = None
        if self.ple_context is not None:
            if ple_lookup is None:
                raise ValueError("This trunk expects a per-layer embedding lookup.")
            ple = PleContextFunction.apply(ple_lookup, x, self.ple_context.weight, bf16).view(
                *lead, self.config.n_layers, self.config.per_layer_dim
            )
        values = None
        if self._value_index:
            if value_lookup is None:
                raise ValueError("This trunk expects a value-embedding lookup.")
            values = value_lookup.view(*lead, len(self._value_index), self.config.kv_width)
        return x, ple, values

    # -- execution paths -------------------------------------------------------

    def _run(
        self,
        x: torch.Tensor | None,
        ple: torch.Tensor | None,
        values: torch.Tensor | None,
        cache: KVCache,
        *,
        n_seqs: int,
        T: int,
        seq_start: torch.Tensor | None,
        positions: torch.Tensor,
        rows: torch.Tensor | None,
        readout: torch.Tensor | None,
        span: int | None,
        tokens: tuple[torch.Tensor, torch.Tensor] | None = None,
    ) -> torch.Tensor:
        # (The pool is named by its storage tensors only, never by its per-layer views:
        # see KVCache.pools.)
        if cache.device.type != "cuda":
            raise RuntimeError("the KV pool must live on the GPU")
        config = self.config
        if cache.n_layers != config.n_layers or cache.kv_heads != config.n_kv_heads or cache.head_dim != config.head_dim:
            raise ValueError("cache layout does not match the trunk")
        k_pools, v_pools = cache.pools()
        if tokens is not None:
            # Token ids through a single-field embedding table and the input norm, in the step.
            ids, table = tokens
            require_device(ids)
            norm = self.input_norm
            hidden = ops.trunk_step_tokens(
                ids, table, norm.weight, float(norm.eps), k_pools, v_pools, cache.status, positions, seq_start, rows,
                readout, self.op_key, compute_dtype_code(ids.device), n_seqs, T, 0 if span is None else int(span),
            )
            if check_enabled() and not torch.compiler.is_compiling() and not torch.cuda.is_current_stream_capturing():
                cache.check()
            return hidden
        require_device(x)
        device = x.device
        n_tokens = x.numel() // config.d_model
        flat = x.reshape(n_tokens, config.d_model).float().contiguous()
        ple_flat = None if ple is None else ple.reshape(n_tokens, -1).float().contiguous()
        values_flat = None if values is None else values.reshape(n_tokens, -1).float().contiguous()
        if config.per_layer_dim and ple_flat is None:
            raise ValueError("This trunk expects a per-layer embedding lookup.")
        if self._value_index and values_flat is None:
            raise ValueError("This trunk expects a value-embedding lookup.")
        # One opaque op per step (torch.ops.cardgym_hip.trunk_step): eager, compiled and
        # captured calls all launch the same cg_trunk_forward.
        hidden = ops.trunk_step(
            flat, ple_flat, values_flat, k_pools, v_pools, cache.status, positions, seq_start, rows, readout,
            self.op_key, compute_dtype_code(device), n_seqs, T, 0 if span is None else int(span),
        )
        if check_enabled() and not torch.compiler.is_compiling() and not torch.cuda.is_current_stream_capturing():
            cache.check()
        return hidden

    def forward_ragged(
        self,
        x: torch.Tensor,
        ple: torch.Tensor | None,
        values: torch.Tensor | None,
        cache: KVCache,
        positions: torch.Tensor,
        readout_offsets: torch.Tensor,
        span: int | None = None,
        rows: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Append a padded run of T tokens to rows 0..B-1 (or ``rows``) at their own lengths.

        Same contract as trunk.py:391-429: ``positions[b]`` is row b's length, token t is
        written at ``min(positions[b] + t, max_len - 1)``, query t sees keys below
        ``positions[b] + 1 + t`` (capped by ``span``).  Returns the final-norm hidden
        state of token ``readout_offsets[b]`` of each row, [B, d].  ``span`` is only a cap:
        nothing is read back from the device when it is None.
        """

        batch, length = x.shape[0], x.shape[1]
        device = x.device
        return self._run(
            x, ple, values, cache, n_seqs=batch, T=length, seq_start=None,
            positions=index_tensor(positions, device), rows=None if rows is None else index_tensor(rows, device),
            readout=index_tensor(readout_offsets, device), span=span,
        )

    def forward_packed(
        self,
        x: torch.Tensor,
        ple: torch.Tensor | None,
        values: torch.Tensor | None,
        cache: KVCache,
        positions: torch.Tensor,
        seq_start: torch.Tensor,
        readout_offsets: torch.Tensor | None,
        rows: torch.Tensor | None = None,
        span: int | None = None,
    ) -> torch.Tensor:
        """Packed variable-length chunks (no padding): sequence b owns packed tokens
        ``seq_start[b] .. seq_start[b+1]-1`` of ``x`` [N, d] (the ``[start, end)`` bounds
        convention of cardgym/nn/packing.py:36-40).  Causal inside each chunk, full
        attention to the cached prefix.  ``readout_offsets=None`` returns every token."""

        device = x.device
        starts = index_tensor(seq_start, device)
        return self._run(
            x, ple, values, cache, n_seqs=starts.numel() - 1, T=0, seq_start=starts,
            positions=index_tensor(positions, device), rows=None if rows is None else index_tensor(rows, device),
            readout=None if readout_offsets is None else index_tensor(readout_offsets, device), span=span,
        )

    def tokens_fold(self, width: int) -> bool:
        """Whether a single-field embedder's token ids (``width`` 1) can go into the step itself
        (``cg_trunk_forward_tokens``): an input norm, no per-layer or value embeddings, and
        no autograd recording."""

        return (
            width == 1 and self.input_norm is not None and not self.config.per_layer_dim
            and not self._value_index and not self._recording()
        )

    def forward_ragged_tokens(self, ids, table, cache, positions, readout_offsets, span=None, rows=None):
        """``forward_ragged`` of the rows rms_norm(table[ids]) * input_norm.weight: ids int64
        [B, T] (padded runs), table the embedder's fp32 [vocab, d_model] weight."""

        device = ids.device
        batch, length = ids.shape
        return self._run(
            None, None, None, cache, n_seqs=batch, T=length, seq_start=None,
            positions=index_tensor(positions, device), rows=None if rows is None else index_tensor(rows, device),
            readout=index_tensor(readout_offsets, device), span=span,
            tokens=(ids.reshape(-1).to(torch.int64).contiguous(), table),
        )

    def forward_packed_tokens(self, ids, table, cache, positions, seq_start, readout_offsets, rows=None, span=None):
        """``forward_packed`` of token ids [N] (int64) through ``table`` and the input norm."""

        device = ids.device
        starts = index_tensor(seq_start, device)
        return self._run(
            None, None, None, cache, n_seqs=starts.numel() - 1, T=0, seq_start=starts,
            positions=index_tensor(positions, device), rows=None if rows is None else index_tensor(rows, device),
            readout=None if readout_offsets is None else index_tensor(readout_offsets, device), span=span,
            tokens=(ids.reshape(-1).to(torch.int64).contiguous(), table),
        )

    def forward_prefill_tokens(self, ids, table, cache, rows):
        """``forward_prefill`` of token ids [B, T] (int64) through ``table`` and the input norm."""

        batch, length = ids.shape
        if length > cache.max_len:
            raise IndexError("prefill longer than the pool's max_len")
        device = ids.device
        return self._run(
            None, None, None, cache, n_seqs=batch, T=length, seq_start=None,
            positions=torch.zeros(batch, dtype=torch.int64, device=device),
            rows=None if rows is None else index_tensor(rows, device),
            readout=torch.full((batch,), length - 1, dtype=torch.int64, device=device), span=length,
            tokens=(ids.reshape(-1).to(torch.int64).contiguous(), table),
        )

    def forward_prefill(
        self,
        x: torch.Tensor,
        ple: torch.Tensor | None,
        values: torch.Tensor | None,
        cache: KVCache,
        rows: torch.Tensor | None,
    ) -> torch.Tensor:
        """Encode fresh prefixes into cache ``rows`` at positions 0..T-1; last hidden [B, d]
        (trunk.py:376-389)."""

        batch, length = x.shape[0], x.shape[1]
        if length > cache.max_len:
            raise IndexError("prefill longer than the pool's max_len")
        device = x.device
        positions = torch.zeros(batch, dtype=torch.int64, device=device)
        readout = torch.full((batch,), length - 1, dtype=torch.int64, device=device)
        return self._run(
            x, ple, values, cache, n_seqs=batch, T=length, seq_start=None, positions=positions,
            # Positions start at 0, so no key past the chunk's length is visible: span = length
            # is exact and lets attention size its launch to the chunk.
            rows=None if rows is None else index_tensor(rows, device), readout=readout, span=length,
        )

    def forward(
        self,
        x: torch.Tensor,
        ple: torch.Tensor | None,
        values: torch.Tensor | None,
        bounds: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Full causal forward (trunk.py:348-374), run as a prefill into a scratch pool:
        [B, T, d] -> final-norm hidden states [B, T, d]; with ``bounds`` the input is packed
        rows [N, d] whose row i belongs to the sequence of rows ``[bounds[i, 0],
        bounds[i, 1])`` (cardgym/nn/packing.py:36-40), -> [N, d].

        When autograd records the call (training), it runs the training path
        (card_playing_gym_amd/nn/train.py: the same forward keeping its activations, and a
        HIP backward)."""

        if self._recording(x, ple, values):
            from .train import trunk_train_forward

            return trunk_train_forward(self, x, ple, values, bounds)
        if bounds is not None:
            return self._forward_bounds(x, ple, values, bounds)
        batch, length = x.shape[0], x.shape[1]
        cache = KVCache(
            n_layers=self.config.n_layers, kv_heads=self.config.n_kv_heads, head_dim=self.config.head_dim,
            capacity=batch, max_len=length, device=x.device, dtype=torch.float32,
        )
        positions = torch.zeros(batch, dtype=torch.int64, device=x.device)
        hidden = self._run(
            x, ple, values, cache, n_seqs=batch, T=length, seq_start=None, positions=positions,
            rows=None, readout=None, span=None,
        )
        return hidden.view(batch, length, self.config.d_model)

    @staticmethod
    def _seq_start_of(bounds) -> tuple[torch.Tensor, int]:
        """Host seq_start [S + 1] and the longest sequence of packed-row bounds [N, 2]."""

        # numpy, not torch CPU ops: this runs on the host once per packed training forward while
        # the GPU waits, and numpy does it in a tenth of the time at ten thousand rows.
        b = torch.as_tensor(bounds).to("cpu", torch.int64).numpy()
        if b.ndim != 2 or b.shape[1] != 2:
            raise ValueError("bounds must be [N, 2]")
        n = b.shape[0]
        if n == 0:
            raise ValueError("bounds must hold at least one row")
        starts, ends = b[:, 0], b[:, 1]
        first = np.empty(n, dtype=bool)
        first[0] = True
        np.not_equal(starts[1:], starts[:-1], out=first[1:])
        seq_start = np.append(np.flatnonzero(first), n)
        lengths = np.diff(seq_start)
        if not (np.array_equal(starts, np.repeat(seq_start[:-1], lengths))
                and np.array_equal(ends, np.repeat(seq_start[1:], lengths))):
            raise ValueError("bounds must describe sequences packed back to back (cardgym.nn.packing.Packing)")
        return torch.from_numpy(seq_start), int(lengths.max())

    def _forward_bounds(self, x, ple, values, bounds) -> torch.Tensor:
        n = x.shape[0]
        b = torch.as_tensor(bounds)
        if x.dim() != 2 or b.shape != (n, 2):
            raise ValueError("packed rows take x [N, d] and bounds [N, 2]")
        if n == 0:
            return torch.empty((0, self.config.d_model), device=x.device, dtype=torch.float32)
        seq_start, longest = self._seq_start_of(b)
        lengths = seq_start[1:] - seq_start[:-1]
        cache = KVCache(
            n_layers=self.config.n_layers, kv_heads=self.config.n_kv_heads, head_dim=self.config.head_dim,
            capacity=lengths.numel(), max_len=longest, device=x.device, dtype=torch.float32,
        )
        positions = torch.zeros(lengths.numel(), dtype=torch.int64, device=x.device)
        return self._run(
            x, ple, values, cache, n_seqs=lengths.numel(), T=0, seq_start=seq_start.to(x.device), positions=positions,
            rows=None, readout=None, span=longest,
        )
