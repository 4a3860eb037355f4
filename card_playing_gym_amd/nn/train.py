"""Training side of the trunk on the HIP path (fp32, or bf16 autocast): autograd functions
whose forward and backward run the kernels of csrc/train.hip.

What autograd records in the reference (cardgym/nn/trunk.py:104-181, 285-374) is, per
block, LayerNorm -> fused QKV projection (+ value embedding) -> causal GQA attention
(F.scaled_dot_product_attention, is_causal) -> output projection + residual -> LayerNorm ->
Linear -> GELU -> Linear + residual -> per-layer embedding add; then the final LayerNorm,
and before the blocks the input RMSNorm and the per-layer-embedding context projection.
``TrunkFunction`` runs that forward on packed rows (sequences back to back, as
cardgym/nn/packing.py lays them out; a padded [B, T, d] batch is B sequences of T) keeping
the activations the backward needs, and its backward produces the gradients of the
input, of the per-layer and value lookups and of every trunk parameter.
``RMSNormFunction`` and ``PleContextFunction`` cover ``Trunk.condition``.

Precision follows the caller's autocast as the reference's does (cardgym/core/devices.py:32-43,
cardgym/rl/trainer.py): outside autocast everything is fp32; under bf16 autocast every
projection takes bf16-rounded operands and returns a bf16-rounded product (fp32 accumulation),
the attention returns bf16 outputs and gradients, the value embedding is added to v in fp32 and
rounded once, and the residual stream, LayerNorm / RMSNorm and their statistics stay fp32
(metal_trunk.py's statement of the same policy: cardgym/nn/metal_trunk.py:32-35).  Values are
kept in fp32 storage holding bf16 numbers; the products run on bf16 MFMA.

Only the elementwise bookkeeping (allocation, zero fills, copies) uses torch; every
reduction, product, norm and attention is a HIP kernel.
"""

from __future__ import annotations

import ctypes
import math

import torch

from .. import _native as nat
from .kv_cache import stream_handle


def _s(t: torch.Tensor) -> int:
    return stream_handle(t.device)


def _ptr(t: torch.Tensor, offset: int = 0) -> int:
    return t.data_ptr() + 4 * offset


def _gemm(m, n, k, alpha, a, sam, sak, b, sbk, sbn, beta, out, device, bf16=False) -> None:
    size = nat.lib().cg_gemm_workspace_size(m, n, k)
    ws = torch.empty(max(size // 4, 1), device=device) if size else None
    nat.call("cg_gemm_strided", m, n, k, float(alpha), a, sam, sak, b, sbk, sbn, float(beta), out.data_ptr(),
             out.stride(0), nat.CG_BF16 if bf16 else nat.CG_F32, None if ws is None else ws.data_ptr(), size,
             stream_handle(device))


def linear_nt(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor, alpha=1.0, beta=0.0, bf16=False) -> None:
    """out[M, N] = alpha * x[M, K] @ w[N, K]^T + beta * out (contiguous rows); with ``bf16``
    the operands and alpha * product are rounded to bf16 (autocast)."""

    m, k = x.shape
    n = w.shape[0]
    _gemm(m, n, k, alpha, x.data_ptr(), k, 1, w.data_ptr(), 1, k, beta, out, x.device, bf16)


def matmul_nn(dy: torch.Tensor, w: torch.Tensor, out: torch.Tensor, alpha=1.0, beta=0.0, bf16=False) -> None:
    """out[M, K] = alpha * dy[M, N] @ w[N, K] + beta * out."""

    m, n = dy.shape
    k = w.shape[1]
    _gemm(m, k, n, alpha, dy.data_ptr(), dy.stride(0), 1, w.data_ptr(), k, 1, beta, out, dy.device, bf16)


def matmul_tn(dy: torch.Tensor, x: torch.Tensor, out: torch.Tensor, alpha=1.0, beta=0.0, bf16=False) -> None:
    """out[N, K] = alpha * dy[M, N]^T @ x[M, K] + beta * out (weight gradients)."""

    m, n = dy.shape
    k = x.shape[1]
    _gemm(n, k, m, alpha, dy.data_ptr(), 1, dy.stride(0), x.data_ptr(), x.stride(0), 1, beta, out, dy.device, bf16)


def add_(dst: torch.Tensor, src: torch.Tensor, alpha=1.0, rows=None, cols=None, ld_src=None) -> None:
    """dst[r, c] += alpha * src[r, c] over 2-D (possibly column-offset) views."""

    rows = dst.shape[0] if rows is None else rows
    cols = dst.shape[1] if cols is None else cols
    nat.call("cg_add_strided", rows, cols, float(alpha), src.data_ptr(),
             src.stride(0) if ld_src is None else ld_src, dst.data_ptr(), dst.stride(0), _s(dst))


def add_bias_(dst: torch.Tensor, bias: torch.Tensor) -> None:
    nat.call("cg_add_strided", dst.shape[0], dst.shape[1], 1.0, bias.data_ptr(), 0, dst.data_ptr(), dst.stride(0),
             _s(dst))


def column_sum(x: torch.Tensor, out: torch.Tensor, accumulate: bool = False) -> None:
    size = nat.lib().cg_column_sum_workspace_size(x.shape[0], x.shape[1])
    ws = torch.empty(max(size // 4, 1), device=x.device) if size else None
    nat.call("cg_column_sum", x.data_ptr(), x.shape[0], x.shape[1], x.stride(0), out.data_ptr(), int(accumulate),
             None if ws is None else ws.data_ptr(), size, _s(x))


def layernorm_fwd(x, w, b, eps):
    n, d = x.shape
    y = torch.empty_like(x)
    mean = torch.empty(n, device=x.device)
    rstd = torch.empty(n, device=x.device)
    nat.call("cg_layernorm_fwd", x.data_ptr(), w.data_ptr(), b.data_ptr(), float(eps), y.data_ptr(), mean.data_ptr(),
             rstd.data_ptr(), n, d, _s(x))
    return y, mean, rstd


def norm_bwd(x, dy, w, mean, rstd, dw, db, residual=None) -> torch.Tensor:
    """dx of LayerNorm (mean given) or RMSNorm (mean None), plus `residual` when given; dw / db
    receive the sums."""

    n, d = x.shape
    dx = torch.empty_like(x)
    size = nat.lib().cg_norm_bwd_workspace_size(n, d)
    ws = torch.empty(max(size // 4, 1), device=x.device)
    nat.call("cg_norm_bwd", x.data_ptr(), dy.data_ptr(), w.data_ptr(), None if mean is None else mean.data_ptr(),
             rstd.data_ptr(), dx.data_ptr(), None if residual is None else residual.data_ptr(), dw.data_ptr(),
             None if db is None else db.data_ptr(), n, d, ws.data_ptr(), size, 0, _s(x))
    return dx


def gelu_fwd(u):
    g = torch.empty_like(u)
    nat.call("cg_gelu_fwd", u.data_ptr(), g.data_ptr(), u.numel(), _s(u))
    return g


def gelu_bwd(u, dg):
    du = torch.empty_like(u)
    nat.call("cg_gelu_bwd", u.data_ptr(), dg.data_ptr(), du.data_ptr(), u.numel(), _s(u))
    return du


def train_precision(device: torch.device) -> bool:
    """Whether the update runs at bf16 autocast's rounding points (True) or in fp32 (False);
    fp16 autocast is refused (the reference scales fp16 losses, cardgym/rl/trainer.py:409)."""

    if not torch.is_autocast_enabled(device.type):
        return False
    if torch.get_autocast_dtype(device.type) != torch.bfloat16:
        raise RuntimeError("the HIP training path runs in fp32 or under bf16 autocast, not fp16")
    return True


# ---- conditioning ---------------------------------------------------------------------------


class RMSNormFunction(torch.autograd.Function):
    """y = rms_norm(x) * w over the last dim (trunk.py:104-115)."""

    @staticmethod
    def forward(ctx, x, w, eps):
        flat = x.reshape(-1, x.shape[-1]).float().contiguous()
        n, d = flat.shape
        y = torch.empty_like(flat)
        rstd = torch.empty(n, device=x.device)
        nat.call("cg_rmsnorm_fwd", flat.data_ptr(), w.data_ptr(), float(eps), y.data_ptr(), rstd.data_ptr(), n, d,
                 _s(flat))
        ctx.save_for_backward(flat, w, rstd)
        ctx.shape = x.shape
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        flat, w, rstd = ctx.saved_tensors
        dw = torch.empty_like(w)
        dx = norm_bwd(flat, dy.reshape(flat.shape).float().contiguous(), w, None, rstd, dw, None)
        return dx.view(ctx.shape), dw, None


class PleContextFunction(torch.autograd.Function):
    """ple = (lookup + x @ W^T) / sqrt(2) (trunk.py:301-306); under bf16 autocast the product
    is a bf16 projection of bf16-rounded operands, added to the fp32 lookup."""

    @staticmethod
    def forward(ctx, lookup, x, w, bf16=False):
        flat = x.reshape(-1, x.shape[-1]).float().contiguous()
        look = lookup.reshape(flat.shape[0], -1).float().contiguous()
        s = 1.0 / math.sqrt(2.0)
        if bf16:
            proj = torch.empty_like(look)
            linear_nt(flat, w, proj, bf16=True)
            out = torch.zeros_like(look)
            add_(out, look, alpha=s)
            add_(out, proj, alpha=s)
        else:
            out = look.clone()
            linear_nt(flat, w, out, alpha=s, beta=s)
        ctx.save_for_backward(flat, w)
        ctx.shapes = (lookup.shape, x.shape)
        ctx.bf16 = bf16
        return out

    @staticmethod
    def backward(ctx, dple):
        flat, w = ctx.saved_tensors
        s = 1.0 / math.sqrt(2.0)
        dple = dple.reshape(flat.shape[0], -1).float().contiguous()
        dlookup = torch.zeros_like(dple)
        add_(dlookup, dple, alpha=s)
        dx = torch.empty_like(flat)
        dw = torch.empty_like(w)
        if ctx.bf16:  # the projection's gradient s * dple enters both products rounded to bf16
            matmul_nn(dlookup, w, dx, bf16=True)
            matmul_tn(dlookup, flat, dw, bf16=True)
        else:
            matmul_nn(dple, w, dx, alpha=s)
            matmul_tn(dple, flat, dw, alpha=s)
        return dlookup.view(ctx.shapes[0]), dx.view(ctx.shapes[1]), dw, None


# ---- the blocks ------------------------------------------------------------------------------


def block_params(trunk) -> list[torch.Tensor]:
    out = []
    for b in trunk.blocks:
        out += [b.ln_attn.weight, b.ln_attn.bias, b.qkv_proj.weight, b.out_proj.weight, b.ln_mlp.weight,
                b.ln_mlp.bias, b.mlp[0].weight, b.mlp[0].bias, b.mlp[2].weight, b.mlp[2].bias]
    return out + [trunk.final_norm.weight, trunk.final_norm.bias]


class _Native:
    """ctypes views of a trunk's configuration and parameters for the training entry points."""

    def __init__(self, trunk, params: list[torch.Tensor], bf16: bool) -> None:
        c = trunk.config
        self.value_index = (ctypes.c_int32 * max(c.n_layers, 1))(
            *[trunk._value_index.get(layer, -1) for layer in range(c.n_layers)]
        )
        eps = trunk.blocks[0].ln_attn.eps if len(trunk.blocks) else 1e-5
        self.config = nat.TrainConfig(c.d_model, c.n_layers, c.n_heads, c.n_kv_heads, c.d_ff, c.per_layer_dim,
                                      c.ple_width, c.value_width, eps, self.value_index, 1 if bf16 else 0)
        self.blocks = (nat.TrainBlock * max(c.n_layers, 1))()
        for layer in range(c.n_layers):
            self.blocks[layer] = nat.TrainBlock(*(t.data_ptr() for t in params[10 * layer : 10 * layer + 10]))


class TrunkFunction(torch.autograd.Function):
    """Packed-row trunk forward (blocks + final norm) and its backward: two calls of
    cg_trunk_train_forward / cg_trunk_train_backward."""

    @staticmethod
    def forward(ctx, trunk, bf16, seq_start, x, ple, values, *params):
        c = trunk.config
        device = x.device
        n = x.shape[0]
        native = _Native(trunk, list(params), bf16)
        saved_size = nat.lib().cg_train_saved_size(ctypes.byref(native.config), n)
        scratch_size = nat.lib().cg_train_scratch_size(ctypes.byref(native.config), n)
        saved = torch.empty(saved_size, dtype=torch.uint8, device=device)
        scratch = torch.empty(scratch_size, dtype=torch.uint8, device=device)
        hidden = torch.empty((n, c.d_model), device=device)
        L = c.n_layers
        nat.call(
            "cg_trunk_train_forward", ctypes.byref(native.config), native.blocks, params[10 * L].data_ptr(),
            params[10 * L + 1].data_ptr(), x.data_ptr(), None if ple is None else ple.data_ptr(),
            None if values is None else values.data_ptr(), seq_start.data_ptr(), seq_start.numel() - 1, n,
            hidden.data_ptr(), saved.data_ptr(), saved_size, scratch.data_ptr(), scratch_size, _s(x),
        )
        ctx.trunk = trunk
        ctx.bf16 = bf16
        ctx.has_ple, ctx.has_values = ple is not None, values is not None
        ctx.save_for_backward(seq_start, saved, *params)
        return hidden

    @staticmethod
    def backward(ctx, dh):
        trunk = ctx.trunk
        c = trunk.config
        seq_start, saved, *params = ctx.saved_tensors
        device = dh.device
        n = dh.shape[0]
        native = _Native(trunk, params, ctx.bf16)
        grads = [torch.empty_like(p) for p in params]
        L = c.n_layers
        block_grads = (nat.TrainBlockGrads * max(L, 1))()
        for layer in range(L):
            block_grads[layer] = nat.TrainBlockGrads(*(g.data_ptr() for g in grads[10 * layer : 10 * layer + 10]))
        tg = nat.TrainGrads(block_grads, grads[10 * L].data_ptr(), grads[10 * L + 1].data_ptr())
        dx = torch.empty((n, c.d_model), device=device)
        dple = torch.empty((n, c.ple_width), device=device) if ctx.has_ple else None
        dvalues = torch.empty((n, c.value_width), device=device) if ctx.has_values else None
        scratch_size = nat.lib().cg_train_scratch_size(ctypes.byref(native.config), n)
        scratch = torch.empty(scratch_size, dtype=torch.uint8, device=device)
        nat.call(
            "cg_trunk_train_backward", ctypes.byref(native.config), native.blocks, params[10 * L].data_ptr(),
            seq_start.data_ptr(), n, dh.float().contiguous().data_ptr(), saved.data_ptr(), saved.numel(),
            scratch.data_ptr(), scratch_size, ctypes.byref(tg), dx.data_ptr(),
            None if dple is None else dple.data_ptr(), None if dvalues is None else dvalues.data_ptr(), _s(dh),
        )
        return (None, None, None, dx, dple, dvalues, *grads)


@torch.compiler.disable
def trunk_train_forward(trunk, x, ple, values, bounds=None):
    """Trunk.forward under autograd: [B, T, d] (or packed rows [N, d] with ``bounds``) ->
    final-norm hidden states of the same leading shape, differentiable.

    Opaque to torch.compile: the reference trainer compiles ``forward_hidden``
    (cardgym/rl/trainer.py:386, cardgym/nn/compile.py:26-44); dynamo runs this call eagerly
    (its host-side bounds check and the C-ABI calls) and compiles around it."""

    bf16 = train_precision(x.device)
    c = trunk.config
    if bounds is None:
        batch, length = x.shape[0], x.shape[1]
        flat = x.reshape(batch * length, c.d_model)
        seq_start = torch.arange(batch + 1, device=x.device, dtype=torch.int64) * length
        lead = (batch, length)
    else:
        flat = x
        seq_start = trunk._seq_start_of(bounds)[0].to(x.device)
        lead = (x.shape[0],)
    n = flat.shape[0]
    ple_flat = None if ple is None else ple.reshape(n, -1).float().contiguous()
    values_flat = None if values is None else values.reshape(n, -1).float().contiguous()
    hidden = TrunkFunction.apply(trunk, bf16, seq_start, flat.float().contiguous(), ple_flat, values_flat,
                                 *block_params(trunk))
    return hidden.view(*lead, c.d_model)
