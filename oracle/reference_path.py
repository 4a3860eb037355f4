"""ORACLE -- test infrastructure only.

A CPU-first restatement, in eager PyTorch, of the reference's KV-cached ragged trunk
step.  It is the checker for the HIP kernels and the "reference path" timed beside them;
it is never part of the product.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s baseline leg may import it.

What it restates (paths into maxrlinder/card_playing_gym):
  * ``RefCache``            cardgym/nn/kv_cache.py:19-138 (zero-filled pool, write_range,
                            write_step, gathered read, chunked copy_rows)
  * ``RefTrunk.condition``  cardgym/nn/trunk.py:285-312 (RMSNorm input norm, PLE, VE)
  * ``_add_ple``            cardgym/nn/trunk.py:318-333
  * ``block_ragged``        cardgym/nn/trunk.py:183-223 (fallback branch 216-223)
  * ``grouped_attention``   cardgym/nn/trunk.py:225-256
  * ``block_full``          cardgym/nn/trunk.py:159-164 (SDPA, is_causal, enable_gqa)
  * ``block_prefill``       cardgym/nn/trunk.py:166-181
  * ``forward_ragged``      cardgym/nn/trunk.py:391-429
  * ``forward_prefill``     cardgym/nn/trunk.py:376-389
  * ``forward_full``        cardgym/nn/trunk.py:348-374
  * synthetic heads         cardgym/nn/model.py:12-17 evaluated as cardgym/rl/graphs.py:88-104

Precision modes:
  * ``"fp32"``: every op in float32 (the reference without autocast).
  * ``"bf16"``: the rounding points of the reference under
    ``torch.autocast("cuda", dtype=torch.bfloat16)`` (cardgym/core/devices.py:32-43),
    written as explicit casts so the CPU reproduces the CUDA policy: nn.Linear and ``@``
    take bf16 operands and return bf16; LayerNorm and softmax run in fp32; GELU runs on
    its bf16 input; residual adds promote to fp32.
Independently of the precision, K/V are stored in the cache dtype and the grouped
attention casts q to it (trunk.py:222), so a bf16 cache also rounds scores and
probabilities as the reference does (trunk.py:245, 255).

Parity status of each function is pinned by tests/test_oracle.py (see the header there).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class RefConfig:
    d_model: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    d_ff: int
    per_layer_dim: int = 0
    value_layers: tuple[int, ...] = ()
    input_norm: bool = True
    eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    @property
    def kv_width(self) -> int:
        return self.n_kv_heads * self.head_dim


class RefCache:
    """kv_cache.py:19-138 with per-layer tensors [capacity, kv_heads, max_len, head_dim]."""

    COPY_CHUNK_BYTES = 256 * 1024 * 1024

    def __init__(self, n_layers, kv_heads, head_dim, capacity, max_len, dtype=torch.float32, device="cpu"):
        self.n_layers, self.capacity, self.max_len, self.dtype = n_layers, capacity, max_len, dtype
        self.kv_heads, self.head_dim = kv_heads, head_dim
        shape = (capacity, kv_heads, max_len, head_dim)
        # kv_cache.py:40-41: one stacked tensor up to 2**31-1 elements; only copy_rows' chunk
        # size depends on it (kv_cache.py:124-126).
        self.stacked = n_layers * capacity * kv_heads * max_len * head_dim <= 2**31 - 1
        self.k = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(n_layers)]
        self.v = [torch.zeros(shape, dtype=dtype, device=device) for _ in range(n_layers)]

    def write_range(self, layer, rows, start, k_new, v_new):
        stop = start + k_new.shape[2]
        if rows is None:
            count = k_new.shape[0]
            self.k[layer][:count, :, start:stop] = k_new.to(self.dtype)
            self.v[layer][:count, :, start:stop] = v_new.to(self.dtype)
        else:
            self.k[layer][rows, :, start:stop] = k_new.to(self.dtype)
            self.v[layer][rows, :, start:stop] = v_new.to(self.dtype)

    def write_step(self, layer, rows, positions, k_new, v_new):
        length = k_new.shape[2]
        if positions.dim() == 1:
            if length != 1:
                raise ValueError("A [B] position vector writes exactly one position per row.")
            self.k[layer][rows, :, positions] = k_new[:, :, 0].to(self.dtype)
            self.v[layer][rows, :, positions] = v_new[:, :, 0].to(self.dtype)
            return
        index = rows[:, None]
        self.k[layer][index, :, positions] = k_new.transpose(1, 2).to(self.dtype)
        self.v[layer][index, :, positions] = v_new.transpose(1, 2).to(self.dtype)

    def read(self, layer, rows, length, count=None):
        if rows is None:
            return self.k[layer][:count, :, :length], self.v[layer][:count, :, :length]
        return self.k[layer][rows, :, :length], self.v[layer][rows, :, :length]

    def copy_rows(self, sources, targets, length):
        row_bytes = max(self.kv_heads * length * self.head_dim * self.dtype.itemsize, 1)
        if self.stacked:
            row_bytes *= self.n_layers
        chunk = max(self.COPY_CHUNK_BYTES // row_bytes, 1)
        for start in range(0, sources.shape[0], chunk):
            src, dst = sources[start : start + chunk], targets[start : start + chunk]
            for layer in range(self.n_layers):
                self.k[layer][dst, :, :length] = self.k[layer][src, :, :length]
                self.v[layer][dst, :, :length] = self.v[layer][src, :, :length]


def _is_bf16(precision: str) -> bool:
    if precision not in ("fp32", "bf16"):
        raise ValueError(f"unknown precision {precision!r}")
    return precision == "bf16"


class RefTrunk:
    """The trunk's forward paths over a reference-named state dict (CPU or any device)."""

    def __init__(self, state: dict[str, torch.Tensor], config: RefConfig, precision: str = "fp32", prefix: str = "trunk."):
        self.c = config
        self.bf16 = _is_bf16(precision)
        self.s = {k[len(prefix):]: v for k, v in state.items() if k.startswith(prefix)}
        self.value_index = {layer: i for i, layer in enumerate(config.value_layers)}
        self.scale = 1.0 / math.sqrt(config.head_dim)

    # -- primitives with the precision policy ---------------------------------

    def lin(self, x, weight, bias=None):
        if self.bf16:
            return F.linear(x.bfloat16(), weight.bfloat16(), None if bias is None else bias.bfloat16())
        return F.linear(x, weight, bias)

    def mm(self, a, b):
        if self.bf16:
            return a.bfloat16() @ b.bfloat16()
        return a @ b

    def layer_norm(self, x, name):
        return F.layer_norm(x.float(), (x.shape[-1],), self.s[f"{name}.weight"], self.s[f"{name}.bias"], self.c.eps)

    def p(self, name):
        return self.s[name]

    # -- conditioning (trunk.py:285-333) ---------------------------------------

    def condition(self, x, ple_lookup=None, value_lookup=None):
        c = self.c
        if c.input_norm:
            x = F.rms_norm(x.float(), (x.shape[-1],), eps=1e-5).to(x.dtype) * self.p("input_norm.weight")
        lead = x.shape[:-1]
        ple = None
        if c.per_layer_dim:
            ple = ((ple_lookup + self.lin(x, self.p("ple_context.weight"))) * (1.0 / math.sqrt(2.0))).view(
                *lead, c.n_layers, c.per_layer_dim
            )
        values = None
        if self.value_index:
            values = value_lookup.view(*lead, len(self.value_index), c.kv_width)
        return x, ple, values

    def _value(self, values, layer):
        index = self.value_index.get(layer)
        return None if index is None or values is None else values[..., index, :]

    def _add_ple(self, x, ple, layer):
        if ple is None:
            return x
        update = ple[..., layer, :]
        if update.shape[-1] == x.shape[-1]:
            return x + update
        if x.shape[-1] % update.shape[-1] == 0:
            repeats = x.shape[-1] // update.shape[-1]
            shaped = x.view(*x.shape[:-1], repeats, update.shape[-1])
            shaped = shaped + update.unsqueeze(-2) * (1.0 / math.sqrt(repeats))
            return shaped.reshape_as(x)
        repeats = math.ceil(x.shape[-1] / update.shape[-1])
        expanded = torch.cat([update] * repeats, dim=-1)[..., : x.shape[-1]]
        return x + expanded * (1.0 / math.sqrt(repeats))

    # -- block pieces (trunk.py:141-157) -----------------------------------------

    def qkv(self, layer, h, value_embedding):
        c = self.c
        batch, length, _ = h.shape
        q, k, v = self.lin(h, self.p(f"blocks.{layer}.qkv_proj.weight")).split(
            [c.n_heads * c.head_dim, c.kv_width, c.kv_width], dim=-1
        )
        q = q.view(batch, length, c.n_heads, c.head_dim).transpose(1, 2)
        k = k.view(batch, length, c.n_kv_heads, c.head_dim).transpose(1, 2)
        v = v.view(batch, length, c.n_kv_heads, c.head_dim)
        if value_embedding is not None:
            v = v + value_embedding.view_as(v)
        return q, k, v.transpose(1, 2)

    def finish(self, layer, x, attn):
        batch, _, length, _ = attn.shape
        pre = f"blocks.{layer}."
        x = x + self.lin(attn.transpose(1, 2).reshape(batch, length, -1), self.p(pre + "out_proj.weight"))
        h = self.layer_norm(x, pre + "ln_mlp")
        h = self.lin(h, self.p(pre + "mlp.0.weight"), self.p(pre + "mlp.0.bias"))
        h = F.gelu(h)
        h = self.lin(h, self.p(pre + "mlp.2.weight"), self.p(pre + "mlp.2.bias"))
        return x + h

    def sdpa(self, q, k, v):
        if self.bf16:
            q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
        return F.scaled_dot_product_attention(
            q, k, v, is_causal=True, enable_gqa=self.c.n_kv_heads != self.c.n_heads
        )

    def grouped_attention(self, q, k, v, key_lengths):
        """trunk.py:225-256: q [B, H, T, D] against k, v [B, KVH, span, D]."""

        c = self.c
        group = c.n_heads // c.n_kv_heads
        batch, _, length, _ = q.shape
        grouped = q.reshape(batch, c.n_kv_heads, group * length, c.head_dim)
        scores = self.mm(grouped, k.transpose(-1, -2)) * self.scale
        keys = torch.arange(k.shape[2], device=q.device)
        if length == 1:
            blocked = keys[None, :] >= key_lengths[:, None]
            scores = scores.masked_fill(blocked[:, None, None, :], float("-inf"))
        else:
            limits = key_lengths[:, None] + torch.arange(length, device=q.device)[None, :]
            blocked = keys[None, None, :] >= limits[:, :, None]
            scores = scores.masked_fill(blocked.repeat(1, group, 1)[:, None], float("-inf"))
        weights = scores.float().softmax(dim=-1).to(v.dtype)
        return self.mm(weights, v).view(batch, c.n_heads, length, c.head_dim)

    # -- per-block paths ----------------------------------------------------------

    def block_full(self, layer, x, value_embedding=None):
        q, k, v = self.qkv(layer, self.layer_norm(x, f"blocks.{layer}.ln_attn"), value_embedding)
        return self.finish(layer, x, self.sdpa(q, k, v))

    def block_prefill(self, layer, x, cache, rows, value_embedding=None):
        q, k, v = self.qkv(layer, self.layer_norm(x, f"blocks.{layer}.ln_attn"), value_embedding)
        cache.write_range(layer, rows, 0, k, v)
        return self.finish(layer, x, self.sdpa(q, k, v))

    def block_ragged(self, layer, x, cache, write_positions, key_lengths, span, value_embedding=None, rows=None):
        q, k, v = self.qkv(layer, self.layer_norm(x, f"blocks.{layer}.ln_attn"), value_embedding)
        if rows is None:
            cache.write_step(layer, torch.arange(x.shape[0], device=x.device), write_positions, k, v)
            k_all, v_all = cache.read(layer, None, span, count=x.shape[0])
        else:
            cache.write_step(layer, rows, write_positions, k, v)
            k_all, v_all = cache.read(layer, rows, span)
        attn = self.grouped_attention(q.to(cache.dtype), k_all, v_all, key_lengths)
        return self.finish(layer, x, attn.to(x.dtype))

    # -- trunk paths (trunk.py:348-429) ------------------------------------------

    def final_norm(self, x):
        return self.layer_norm(x, "final_norm")

    def forward_full(self, x, ple=None, values=None):
        for layer in range(self.c.n_layers):
            x = self.block_full(layer, x, self._value(values, layer))
            x = self._add_ple(x, ple, layer)
        return self.final_norm(x)

    def forward_prefill(self, x, ple, values, cache, rows):
        for layer in range(self.c.n_layers):
            x = self.block_prefill(layer, x, cache, rows, self._value(values, layer))
            x = self._add_ple(x, ple, layer)
        return self.final_norm(x[:, -1])

    def forward_ragged(self, x, ple, values, cache, positions, readout_offsets, span=None, rows=None):
        length = x.shape[1]
        batch = torch.arange(x.shape[0], device=x.device)
        steps = torch.arange(length, device=positions.device)[None, :]
        write_positions = (positions[:, None] + steps).clamp(max=cache.max_len - 1)
        if span is None:
            span = int(positions.max()) + length
        span = min(span, cache.max_len)
        for layer in range(self.c.n_layers):
            x = self.block_ragged(layer, x, cache, write_positions, positions + 1, span, self._value(values, layer), rows)
            x = self._add_ple(x, ple, layer)
        return self.final_norm(x[batch, readout_offsets])


class RefSynthetic:
    """The synthetic model: embedding lookup -> trunk -> policy logits and seat values."""

    def __init__(self, state: dict[str, torch.Tensor], config: RefConfig, precision: str = "fp32"):
        self.trunk = RefTrunk(state, config, precision)
        self.state = state
        self.bf16 = self.trunk.bf16

    def prepare(self, tokens):
        x = F.embedding(tokens[..., 0], self.state["embedding.weight"])
        return self.trunk.condition(x)

    def heads(self, hidden):
        s, lin = self.state, self.trunk.lin
        logits = lin(hidden, s["policy_head.weight"], s["policy_head.bias"]).float()
        mid = F.gelu(lin(hidden, s["value_head.0.weight"], s["value_head.0.bias"]))
        values = lin(mid, s["value_head.2.weight"], s["value_head.2.bias"]).float()
        return logits, values

    def forward_ragged(self, tokens, positions, cache, readout_offsets, span=None, rows=None):
        return self.trunk.forward_ragged(*self.prepare(tokens), cache, positions, readout_offsets, span, rows)

    def forward_prefill(self, tokens, cache, rows):
        return self.trunk.forward_prefill(*self.prepare(tokens), cache, rows)

    def forward_hidden(self, tokens):
        return self.trunk.forward_full(*self.prepare(tokens))


def ref_config_of(trunk_config) -> RefConfig:
    """RefConfig from any object with the TrunkConfig fields."""

    return RefConfig(
        d_model=trunk_config.d_model,
        n_layers=trunk_config.n_layers,
        n_heads=trunk_config.n_heads,
        n_kv_heads=trunk_config.n_kv_heads,
        d_ff=trunk_config.d_ff,
        per_layer_dim=trunk_config.per_layer_dim,
        value_layers=tuple(trunk_config.value_layers),
        input_norm=trunk_config.input_norm,
    )
