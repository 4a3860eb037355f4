"""The HIP entry points of the decode path as torch custom ops (``torch.ops.cardgym_hip.*``).

The reference's collectors compile the decode wave with ``torch.compile(dynamic=True)``
and capture it into a CUDA graph (cardgym/rl/graphs.py:75-104, 137-151;
cardgym/nn/compile.py:26-44), and its one native kernel is a registered op with a fake
implementation (cardgym/nn/cuda_decode.py:172-181).  Here every launch of the wave is such
an op: Dynamo and Inductor see each one as an opaque node whose output shapes come from
its fake implementation, never a ``ctypes`` call on fake tensors, so the wave compiles as
one graph (``fullgraph=True`` holds) and the capture records the kernels themselves.

Ops that need a module's device-side weight copies (the trunk's, the heads', the Piquet
embedder's bf16 fragments) name the module by an integer key from :func:`register`; the
implementation looks the module up at run time and takes its handle for the call's device
and compute type, so the copies stay those the module keeps current (optimiser steps,
``load_state_dict``).  A copied or unpickled module registers again under a new key.

Compute type codes are explicit arguments (0 fp32, 1 bf16): the caller reads its autocast
state while it is traced, which a compiled graph no longer carries when it runs.
"""

import ctypes
import itertools
import weakref
from typing import List, Optional, Tuple

import torch
from torch import Tensor

from .. import _native as nat
from .kv_cache import dtype_code, require_device, stream_handle

# -- module registry --------------------------------------------------------------------

_MODULES: "dict[int, weakref.ref]" = {}
_KEYS = itertools.count(1)


def register(module) -> int:
    """A new key naming ``module`` inside the ops (held weakly)."""

    key = next(_KEYS)
    _MODULES[key] = weakref.ref(module, lambda _ref, key=key: _MODULES.pop(key, None))
    return key


def lookup(key: int):
    ref = _MODULES.get(key)
    module = None if ref is None else ref()
    if module is None:
        raise RuntimeError(f"cardgym_hip: module key {key} names no live module")
    return module


class Registered:
    """Mixin of the modules the ops name: a key at construction and after copy / unpickle."""

    def _register_op_key(self) -> None:
        self.__dict__["op_key"] = register(self)

    def __setstate__(self, state) -> None:
        super().__setstate__(state)
        self._register_op_key()


def _param(tensor: Tensor) -> Tensor:
    if tensor.dtype != torch.float32 or not tensor.is_contiguous():
        raise ValueError("parameters must be contiguous float32 tensors")
    return tensor


# -- KV layer descriptors --------------------------------------------------------------

_LAYER_ARRAYS: dict = {}


def kv_layers(k: List[Tensor], v: List[Tensor]):
    """ctypes array of ``cg_kv_layer`` over the pools ``KVCache.pools()`` returns: one
    stacked [n_layers, capacity, kv_heads, max_len, head_dim] tensor each for k and v, or
    one [capacity, kv_heads, max_len, head_dim] tensor per layer (memoised by storage
    address and shape)."""

    if len(k) != len(v) or not k:
        raise ValueError("k and v must list the same, non-zero number of pools")
    key = tuple((a.data_ptr(), b.data_ptr(), tuple(a.shape), a.dtype) for a, b in zip(k, v))
    array = _LAYER_ARRAYS.get(key)
    if array is not None:
        return array
    layers = []  # (k address, v address, shape, dtype) per layer
    for a, b in zip(k, v):
        if a.shape != b.shape or a.dtype != b.dtype or a.dim() not in (4, 5) or (a.dim() == 5 and len(k) != 1):
            raise ValueError("k and v pools must match: one stacked [n_layers, capacity, kv_heads, max_len, "
                             "head_dim] tensor, or one [capacity, kv_heads, max_len, head_dim] tensor per layer")
        if not (a.is_contiguous() and b.is_contiguous()):
            raise ValueError("k and v pools must be contiguous")
        if a.dim() == 5:
            step = a.stride(0) * a.element_size()
            layers += [(a.data_ptr() + i * step, b.data_ptr() + i * step, a.shape[1:], a.dtype) for i in range(a.shape[0])]
        else:
            layers.append((a.data_ptr(), b.data_ptr(), a.shape, a.dtype))
    array = (nat.KVLayer * len(layers))()
    for index, (ka, va, shape, dtype) in enumerate(layers):
        capacity, heads, max_len, head_dim = shape
        array[index] = nat.KVLayer(ka, va, capacity, heads, max_len, head_dim, dtype_code(dtype))
    if len(_LAYER_ARRAYS) > 64:
        _LAYER_ARRAYS.clear()
    _LAYER_ARRAYS[key] = array
    return array


def _ptr(tensor: Optional[Tensor]):
    return None if tensor is None else tensor.data_ptr()


# -- norms and embedding -----------------------------------------------------------------


@torch.library.custom_op("cardgym_hip::rmsnorm", mutates_args=())
def rmsnorm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """Gain-only RMSNorm of rows x [n, d] (fp32 or bf16) -> fp32 [n, d] (cg_rmsnorm)."""

    out = torch.empty(x.shape, device=x.device, dtype=torch.float32)
    bf16 = x.dtype == torch.bfloat16
    nat.call(
        "cg_rmsnorm", x.data_ptr(), nat.CG_BF16 if bf16 else nat.CG_F32, _param(weight).data_ptr(), float(eps),
        out.data_ptr(), x.shape[0], x.shape[1], stream_handle(x.device),
    )
    return out


@rmsnorm.register_fake
def _(x, weight, eps):
    return x.new_empty(x.shape, dtype=torch.float32)


@torch.library.custom_op("cardgym_hip::embed_rmsnorm", mutates_args=())
def embed_rmsnorm(table: Tensor, ids: Tensor, weight: Tensor, eps: float) -> Tensor:
    """RMSNorm(table[ids]) -> fp32 [n, d] in one launch (cg_embed_rmsnorm)."""

    n, d = ids.numel(), table.shape[1]
    out = torch.empty((n, d), device=ids.device, dtype=torch.float32)
    nat.call(
        "cg_embed_rmsnorm", _param(table).data_ptr(), table.shape[0], ids.data_ptr(), _param(weight).data_ptr(),
        float(eps), out.data_ptr(), n, d, None, stream_handle(ids.device),
    )
    return out


@embed_rmsnorm.register_fake
def _(table, ids, weight, eps):
    return ids.new_empty((ids.numel(), table.shape[1]), dtype=torch.float32)


@torch.library.custom_op("cardgym_hip::ple_context", mutates_args=())
def ple_context(x: Tensor, weight: Tensor, lookup: Tensor, scale: float, compute: int) -> Tensor:
    """(x . weight^T + lookup) * scale -> fp32 [n, ple_width] (cg_linear_add_scale): the
    per-layer embedding context of trunk.py:296-306; ``lookup`` fp32 or bf16."""

    out = torch.empty(lookup.shape, device=lookup.device, dtype=torch.float32)
    bf16 = lookup.dtype == torch.bfloat16
    nat.call(
        "cg_linear_add_scale", x.data_ptr(), _param(weight).data_ptr(), lookup.data_ptr(),
        nat.CG_BF16 if bf16 else nat.CG_F32, out.data_ptr(), x.shape[0], lookup.shape[1], x.shape[1], float(scale),
        int(compute), stream_handle(x.device),
    )
    return out


@ple_context.register_fake
def _(x, weight, lookup, scale, compute):
    return x.new_empty(lookup.shape, dtype=torch.float32)


# -- the trunk step ----------------------------------------------------------------------


@torch.library.custom_op("cardgym_hip::trunk_step", mutates_args=("k", "v", "status"))
def trunk_step(
    x: Tensor,
    ple: Optional[Tensor],
    values: Optional[Tensor],
    k: List[Tensor],
    v: List[Tensor],
    status: Optional[Tensor],
    positions: Tensor,
    seq_start: Optional[Tensor],
    rows: Optional[Tensor],
    readout: Optional[Tensor],
    trunk: int,
    compute: int,
    n_seqs: int,
    T: int,
    span: int,
) -> Tensor:
    """One ``cg_trunk_forward`` over every layer: appends the step's K / V to the pools
    ``k`` / ``v`` (``KVCache.pools()``, mutated) and returns the final-norm hidden rows, fp32 [n_seqs, d] at
    the readout tokens (or [n_tokens, d] without ``readout``).  ``x`` [n_tokens, d],
    ``ple`` [n_tokens, n_layers * per_layer_dim], ``values`` [n_tokens, value_width]
    (fp32, contiguous); index tensors int64 as ``cg_ragged`` takes them.  ``status`` (int32
    [3] on the device, ``KVCache.status``) gets a 1 in word 0 / 1 / 2 when some row is outside
    the pool, some position is negative, some readout offset is outside its sequence."""

    module = lookup(trunk)
    device = x.device
    native = module.native(device, compute)
    n_tokens, d = x.shape
    hidden = torch.empty((n_seqs if readout is not None else n_tokens, d), device=device, dtype=torch.float32)
    size = nat.lib().cg_trunk_workspace_size(native.handle, n_tokens, n_seqs)
    workspace = torch.empty(max(size, 1), device=device, dtype=torch.uint8)
    step = _ragged(status, n_seqs, n_tokens, T, span, seq_start, positions, rows, readout)
    nat.call(
        "cg_trunk_forward", native.handle, kv_layers(k, v), x.data_ptr(), _ptr(ple), _ptr(values), ctypes.byref(step),
        hidden.data_ptr(), workspace.data_ptr(), size, stream_handle(device),
    )
    return hidden


def _ragged(status, n_seqs, n_tokens, T, span, seq_start, positions, rows, readout) -> "nat.Ragged":
    if status is not None and (status.dtype != torch.int32 or status.numel() < 4 or not status.is_contiguous()):
        raise ValueError("status must be a contiguous int32 tensor of 4 words")
    return nat.Ragged(
        n_seqs, n_tokens, T, span, _ptr(seq_start), positions.data_ptr(), _ptr(rows), _ptr(readout), _ptr(status),
    )


@trunk_step.register_fake
def _(x, ple, values, k, v, status, positions, seq_start, rows, readout, trunk, compute, n_seqs, T, span):
    return x.new_empty((n_seqs if readout is not None else x.shape[0], x.shape[1]))


@torch.library.custom_op("cardgym_hip::trunk_step_tokens", mutates_args=("k", "v", "status"))
def trunk_step_tokens(
    ids: Tensor,
    table: Tensor,
    gain: Tensor,
    eps: float,
    k: List[Tensor],
    v: List[Tensor],
    status: Optional[Tensor],
    positions: Tensor,
    seq_start: Optional[Tensor],
    rows: Optional[Tensor],
    readout: Optional[Tensor],
    trunk: int,
    compute: int,
    n_seqs: int,
    T: int,
    span: int,
) -> Tensor:
    """``trunk_step`` of the rows rms_norm(table[ids], eps) * gain (``cg_trunk_forward_tokens``):
    a single-field token embedder and the trunk's input RMSNorm folded into the step.  ``ids``
    int64 [n_tokens]; ``table`` fp32 [vocab, d]; ``gain`` fp32 [d]."""

    require_device(ids, table, gain)
    if table.device != ids.device or gain.device != ids.device:
        raise RuntimeError("token ids, embedding table and gain must be on one device")
    module = lookup(trunk)
    device = ids.device
    native = module.native(device, compute)
    n_tokens, d = ids.numel(), table.shape[1]
    hidden = torch.empty((n_seqs if readout is not None else n_tokens, d), device=device, dtype=torch.float32)
    size = nat.lib().cg_trunk_workspace_size(native.handle, n_tokens, n_seqs)
    workspace = torch.empty(max(size, 1), device=device, dtype=torch.uint8)
    step = _ragged(status, n_seqs, n_tokens, T, span, seq_start, positions, rows, readout)
    nat.call(
        "cg_trunk_forward_tokens", native.handle, kv_layers(k, v), _param(table).data_ptr(), table.shape[0],
        ids.data_ptr(), _param(gain).data_ptr(), float(eps), None, None, ctypes.byref(step), hidden.data_ptr(),
        workspace.data_ptr(), size, stream_handle(device),
    )
    return hidden


@trunk_step_tokens.register_fake
def _(ids, table, gain, eps, k, v, status, positions, seq_start, rows, readout, trunk, compute, n_seqs, T, span):
    return ids.new_empty((n_seqs if readout is not None else ids.numel(), table.shape[1]), dtype=torch.float32)


# -- heads and game embedders -----------------------------------------------------------


@torch.library.custom_op("cardgym_hip::synthetic_heads", mutates_args=())
def synthetic_heads(hidden: Tensor, model: int, compute: int, n_policy: int, n_value: int) -> Tuple[Tensor, Tensor]:
    """Policy logits [m, n_policy] and seat values [m, n_value] (fp32) of the synthetic
    model's heads from hidden rows [m, d] (fp32)."""

    return lookup(model)._run_heads(hidden, compute)


@synthetic_heads.register_fake
def _(hidden, model, compute, n_policy, n_value):
    m = hidden.shape[0]
    return hidden.new_empty((m, n_policy)), hidden.new_empty((m, n_value))


@torch.library.custom_op("cardgym_hip::piquet_embed", mutates_args=())
def piquet_embed(
    tokens: Tensor, module: int, d_model: int, ple_width: int, value_width: int, card_width: int
) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """Piquet token embedding of tokens [n, 64] (int64): x [n, d] bf16, the per-layer and
    value lookups [n, width] bf16 (width 0 when the model has none) and the per-card
    features [n, 32, card_width] fp32 (cg_piquet_embed)."""

    return lookup(module)._embed_native(tokens)


@piquet_embed.register_fake
def _(tokens, module, d_model, ple_width, value_width, card_width):
    n = tokens.shape[0]
    bf16 = torch.bfloat16
    return (
        tokens.new_empty((n, d_model), dtype=bf16),
        tokens.new_empty((n, ple_width), dtype=bf16),
        tokens.new_empty((n, value_width), dtype=bf16),
        tokens.new_empty((n, 32, card_width), dtype=torch.float32),
    )
