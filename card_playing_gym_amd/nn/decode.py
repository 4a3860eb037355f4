"""Ragged GQA decode attention straight from the KV pool (API of cardgym.nn.cuda_decode).

``decode_attention(q, k_cache, v_cache, rows, key_lengths, span, scale)`` keeps the
signature and meaning of cardgym/nn/cuda_decode.py:188-202 -- query t of row b sees keys
below ``key_lengths[b] + t`` of cache row ``rows[b]`` -- and is registered as the custom
op ``cardgym_hip::decode_attention`` with a fake implementation, as the reference
registers ``cardgym::decode_attention`` (cuda_decode.py:172-181), so graph capture and
torch.compile treat it as opaque.  Unlike the reference kernel it takes any span,
head_dim 8 / 16 / 24 / 32 / 64 and fp32 / bf16 / fp16 caches; scores, softmax and
accumulation are fp32.
"""

from __future__ import annotations

import torch

from .. import _native as nat
from .kv_cache import dtype_code, require_device, stream_handle

HEAD_DIMS = (8, 16, 24, 32, 64)


def supported(head_dim: int, span: int, queries: int) -> bool:
    """Shapes the kernel is built for (any span and query count)."""

    return head_dim in HEAD_DIMS


def _layer(k: torch.Tensor, v: torch.Tensor) -> nat.KVLayer:
    if k.shape != v.shape or k.dtype != v.dtype:
        raise ValueError("k and v caches must match in shape and dtype")
    if not (k.is_contiguous() and v.is_contiguous()):
        raise ValueError("k and v caches must be contiguous [capacity, kv_heads, max_len, head_dim]")
    capacity, kv_heads, max_len, head_dim = k.shape
    return nat.KVLayer(k.data_ptr(), v.data_ptr(), capacity, kv_heads, max_len, head_dim, dtype_code(k.dtype))


def attention_into(
    out: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    rows: torch.Tensor | None,
    key_lengths: torch.Tensor,
    span: int,
    scale: float,
    order: torch.Tensor | None = None,
) -> None:
    """Writes attention of q [B, H, T, D] (any strides, unit last stride) into out
    [B, H, T, D] (contiguous).  ``order`` (from :func:`attention_order` for the same rows,
    key lengths, T and span) makes decode runs take the persistent kernel instead of the
    split kernel the trunk step uses (the two stream at the same rate; results agree to
    rounding)."""

    import ctypes

    require_device(q, k, v, out)
    if q.stride(3) != 1:
        q = q.contiguous()
    if rows is not None and (rows.dtype != torch.int64 or not rows.is_contiguous()):
        rows = rows.to(torch.int64).contiguous()
    lengths = key_lengths.to(torch.int64).contiguous()
    batch, heads, steps, _ = q.shape
    layer = _layer(k, v)
    if order is not None and (order.dtype != torch.int32 or order.numel() < batch * k.shape[1]):
        raise ValueError("order must be an int32 tensor of batch * kv_heads entries (attention_order)")
    nat.call(
        "cg_decode_attention_ordered", q.data_ptr(), dtype_code(q.dtype), q.stride(0), q.stride(1), q.stride(2),
        ctypes.byref(layer), None if rows is None else rows.data_ptr(), lengths.data_ptr(), batch, heads,
        steps, int(span), float(scale), out.data_ptr(), dtype_code(out.dtype),
        None if order is None else order.data_ptr(), stream_handle(q.device),
    )


def attention_order(
    k: torch.Tensor,
    rows: torch.Tensor | None,
    key_lengths: torch.Tensor,
    batch: int,
    heads: int,
    steps: int,
    span: int,
) -> torch.Tensor | None:
    """The (row, KV head) units of a padded run sorted by key tiles (int32 [batch * kv_heads]),
    for :func:`attention_into`; None when the persistent kernel does not apply (fp32 pool,
    head_dim other than 32 / 64, more than 16 queries per unit, span below 1024 keys)."""

    import ctypes

    require_device(k, key_lengths)
    if rows is not None and (rows.dtype != torch.int64 or not rows.is_contiguous()):
        rows = rows.to(torch.int64).contiguous()
    lengths = key_lengths.to(torch.int64).contiguous()
    layer = _layer(k, k)
    order = torch.empty(max(batch * k.shape[1], 1), dtype=torch.int32, device=k.device)
    streams = ctypes.c_int32(0)
    nat.call(
        "cg_decode_attention_order", ctypes.byref(layer), None if rows is None else rows.data_ptr(), lengths.data_ptr(),
        batch, heads, steps, int(span), order.data_ptr(), ctypes.byref(streams), stream_handle(k.device),
    )
    return order if streams.value else None


def attention_packed_into(
    out: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    rows: torch.Tensor | None,
    positions: torch.Tensor,
    seq_start: torch.Tensor,
    span: int,
    scale: float,
    order: torch.Tensor | None = None,
) -> None:
    """Packed chunks: q [N, H, D] (unit last stride), sequence b owning tokens
    ``seq_start[b] .. seq_start[b+1]-1`` (packing.py:36-40 bounds) at cache row ``rows[b]``;
    its token t sees keys below ``positions[b] + 1 + t`` (its prefix and its own chunk,
    already in the pool).  Writes out [N, H, D] (contiguous).  ``order`` (from
    :func:`attention_packed_order` for the same rows, positions, bounds and span) deals the
    units longest first, as the trunk step does."""

    import ctypes

    require_device(q, k, v, out)
    if q.stride(2) != 1:
        q = q.contiguous()
    index = lambda t: t.to(torch.int64).contiguous()  # noqa: E731
    rows = None if rows is None else index(rows)
    positions, seq_start = index(positions), index(seq_start)
    layer = _layer(k, v)
    if order is not None and (order.dtype != torch.int32 or order.numel() < positions.numel() * k.shape[1]):
        raise ValueError("order must be an int32 tensor of n_seqs * kv_heads entries (attention_packed_order)")
    nat.call(
        "cg_decode_attention_packed_ordered", q.data_ptr(), dtype_code(q.dtype), q.stride(0), q.stride(1),
        ctypes.byref(layer), None if rows is None else rows.data_ptr(), positions.data_ptr(), seq_start.data_ptr(),
        positions.numel(), q.shape[0], q.shape[1], int(span), float(scale), out.data_ptr(), dtype_code(out.dtype),
        None if order is None else order.data_ptr(), stream_handle(q.device),
    )


def attention_packed_order(
    k: torch.Tensor,
    rows: torch.Tensor | None,
    positions: torch.Tensor,
    seq_start: torch.Tensor,
    n_tokens: int,
    heads: int,
    span: int,
) -> torch.Tensor:
    """The (row, KV head) units of a packed run sorted by work, most first (int32
    [n_seqs * kv_heads]), for :func:`attention_packed_into`."""

    import ctypes

    require_device(k, positions, seq_start)
    index = lambda t: t.to(torch.int64).contiguous()  # noqa: E731
    rows = None if rows is None else index(rows)
    positions, seq_start = index(positions), index(seq_start)
    layer = _layer(k, k)
    order = torch.empty(max(positions.numel() * k.shape[1], 1), dtype=torch.int32, device=k.device)
    nat.call(
        "cg_decode_attention_packed_order", ctypes.byref(layer), None if rows is None else rows.data_ptr(),
        positions.data_ptr(), seq_start.data_ptr(), positions.numel(), int(n_tokens), heads, int(span),
        order.data_ptr(), stream_handle(k.device),
    )
    return order


@torch.library.custom_op("cardgym_hip::decode_attention", mutates_args=())
def _decode_attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rows: torch.Tensor, lengths: torch.Tensor, span: int, scale: float
) -> torch.Tensor:
    out = torch.empty(q.shape, dtype=k.dtype, device=q.device)
    attention_into(out, q, k, v, rows, lengths, span, scale)
    return out


@_decode_attention.register_fake
def _(q, k, v, rows, lengths, span, scale):
    return torch.empty(q.shape, dtype=k.dtype, device=q.device)


def decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    rows: torch.Tensor,
    key_lengths: torch.Tensor,
    span: int,
    scale: float,
) -> torch.Tensor:
    """q [B, H, T, D] against cache rows ``rows`` [B] of k/v [R, KVH, L, D]; returns
    [B, H, T, D] in the cache's dtype."""

    return _decode_attention(q, k_cache, v_cache, rows, key_lengths, span, scale)
