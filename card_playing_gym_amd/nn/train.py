"""Training side of the trunk on the HIP path (fp32): autograd functions whose forward and
backward run the kernels of csrc/train.hip.

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


def linear_nt(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor, alpha=1.0, beta=0.0) -> None:
    """out[M, N] = alpha * x[M, K] @ w[N, K]^T + beta * out (contiguous rows)."""

    m, k = x.shape
    n = w.shape[0]
    nat.call("cg_gemm_strided", m, n, k, float(alpha), x.data_ptr(), k, 1, w.data_ptr(), 1, k, float(beta),
             out.data_ptr(), out.stride(0), _s(x))


def matmul_nn(dy: torch.Tensor, w: torch.Tensor, out: torch.Tensor, alpha=1.0, beta=0.0) -> None:
    """out[M, K] = alpha * dy[M, N] @ w[N, K] + beta * out."""

    m, n = dy.shape
    k = w.shape[1]
    nat.call("cg_gemm_strided", m, k, n, float(alpha), dy.data_ptr(), dy.stride(0), 1, w.data_ptr(), k, 1,
             float(beta), out.data_ptr(), out.stride(0), _s(dy))


def matmul_tn(dy: torch.Tensor, x: torch.Tensor, out: torch.Tensor, alpha=1.0, beta=0.0) -> None:
    """out[N, K] = alpha * dy[M, N]^T @ x[M, K] + beta * out (weight gradients)."""

    m, n = dy.shape
    k = x.shape[1]
    nat.call("cg_gemm_strided", n, k, m, float(alpha), dy.data_ptr(), 1, dy.stride(0), x.data_ptr(), x.stride(0), 1,
             float(beta), out.data_ptr(), out.stride(0), _s(dy))


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
    nat.call("cg_column_sum", x.data_ptr(), x.shape[0], x.shape[1], x.stride(0), out.data_ptr(), int(accumulate),
             _s(x))


def layernorm_fwd(x, w, b, eps):
    n, d = x.shape
    y = torch.empty_like(x)
    mean = torch.empty(n, device=x.device)
    rstd = torch.empty(n, device=x.device)
    nat.call("cg_layernorm_fwd", x.data_ptr(), w.data_ptr(), b.data_ptr(), float(eps), y.data_ptr(), mean.data_ptr(),
             rstd.data_ptr(), n, d, _s(x))
    return y, mean, rstd


def norm_bwd(x, dy, w, mean, rstd, dw, db) -> torch.Tensor:
    """dx of LayerNorm (mean given) or RMSNorm (mean None); dw / db receive the sums."""

    n, d = x.shape
    dx = torch.empty_like(x)
    size = nat.lib().cg_norm_bwd_workspace_size(n, d)
    ws = torch.empty(max(size // 4, 1), device=x.device)
    nat.call("cg_norm_bwd", x.data_ptr(), dy.data_ptr(), w.data_ptr(), None if mean is None else mean.data_ptr(),
             rstd.data_ptr(), dx.data_ptr(), dw.data_ptr(), None if db is None else db.data_ptr(), n, d,
             ws.data_ptr(), size, 0, _s(x))
    return dx


def gelu_fwd(u):
    g = torch.empty_like(u)
    nat.call("cg_gelu_fwd", u.data_ptr(), g.data_ptr(), u.numel(), _s(u))
    return g


def gelu_bwd(u, dg):
    du = torch.empty_like(u)
    nat.call("cg_gelu_bwd", u.data_ptr(), dg.data_ptr(), du.data_ptr(), u.numel(), _s(u))
    return du


def _require_fp32(device: torch.device) -> None:
    if torch.is_autocast_enabled(device.type):
        raise RuntimeError("the HIP training path runs in fp32: leave autocast off for the update")


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
    """ple = (lookup + x @ W^T) / sqrt(2) (trunk.py:301-306)."""

    @staticmethod
    def forward(ctx, lookup, x, w):
        flat = x.reshape(-1, x.shape[-1]).float().contiguous()
        look = lookup.reshape(flat.shape[0], -1).float().contiguous()
        s = 1.0 / math.sqrt(2.0)
        out = look.clone()
        linear_nt(flat, w, out, alpha=s, beta=s)
        ctx.save_for_backward(flat, w)
        ctx.shapes = (lookup.shape, x.shape)
        return out

    @staticmethod
    def backward(ctx, dple):
        flat, w = ctx.saved_tensors
        s = 1.0 / math.sqrt(2.0)
        dple = dple.reshape(flat.shape[0], -1).float().contiguous()
        dlookup = torch.zeros_like(dple)
        add_(dlookup, dple, alpha=s)
        dx = torch.empty_like(flat)
        matmul_nn(dple, w, dx, alpha=s)
        dw = torch.empty_like(w)
        matmul_tn(dple, flat, dw, alpha=s)
        return dlookup.view(ctx.shapes[0]), dx.view(ctx.shapes[1]), dw


# ---- the blocks ------------------------------------------------------------------------------


def block_params(trunk) -> list[torch.Tensor]:
    out = []
    for b in trunk.blocks:
        out += [b.ln_attn.weight, b.ln_attn.bias, b.qkv_proj.weight, b.out_proj.weight, b.ln_mlp.weight,
                b.ln_mlp.bias, b.mlp[0].weight, b.mlp[0].bias, b.mlp[2].weight, b.mlp[2].bias]
    return out + [trunk.final_norm.weight, trunk.final_norm.bias]


def _ple_slices(d: int, pd: int):
    """(column offset, width, scale) of each repeat of a per-layer embedding (trunk.py:318-333)."""

    if pd == d:
        return [(0, d, 1.0)]
    repeats = d // pd if d % pd == 0 else math.ceil(d / pd)
    scale = 1.0 / math.sqrt(repeats)
    return [(r * pd, min(pd, d - r * pd), scale) for r in range(repeats)]


class TrunkFunction(torch.autograd.Function):
    """Packed-row trunk forward (blocks + final norm) and its backward."""

    @staticmethod
    def forward(ctx, trunk, seq_start, x, ple, values, *params):
        c = trunk.config
        device = x.device
        n, d = x.shape
        H, KVH, D = c.n_heads, c.n_kv_heads, c.head_dim
        Q, KVW = H * D, KVH * D
        n_seqs = seq_start.numel() - 1
        seq_of = torch.empty(n, dtype=torch.int32, device=device)
        nat.call("cg_seq_of", seq_start.data_ptr(), n_seqs, seq_of.data_ptr(), _s(x))
        eps = trunk.blocks[0].ln_attn.eps if len(trunk.blocks) else 1e-5
        value_index = trunk._value_index
        saved = []
        xl = x.float().contiguous()
        for layer in range(c.n_layers):
            w = params[10 * layer : 10 * layer + 10]
            h1, m1, r1 = layernorm_fwd(xl, w[0], w[1], eps)
            qkv = torch.empty((n, Q + 2 * KVW), device=device)
            linear_nt(h1, w[2], qkv)
            if layer in value_index:
                ve = values[:, value_index[layer] * KVW : (value_index[layer] + 1) * KVW]
                add_(qkv[:, Q + KVW :], ve, rows=n, cols=KVW)
            o = torch.empty((n, Q), device=device)
            lse = torch.empty((n, H), device=device)
            at = nat.AttnTrain(n, H, KVH, D, 1.0 / math.sqrt(D), seq_start.data_ptr(), seq_of.data_ptr(),
                               qkv.data_ptr(), _ptr(qkv, Q), _ptr(qkv, Q + KVW), Q + 2 * KVW, Q + 2 * KVW,
                               Q + 2 * KVW, o.data_ptr(), lse.data_ptr())
            nat.call("cg_attn_train_fwd", ctypes.byref(at), _s(x))
            x1 = xl.clone()
            linear_nt(o, w[3], x1, beta=1.0)
            h2, m2, r2 = layernorm_fwd(x1, w[4], w[5], eps)
            u = torch.empty((n, w[6].shape[0]), device=device)
            linear_nt(h2, w[6], u)
            add_bias_(u, w[7])
            g = gelu_fwd(u)
            x2 = x1.clone()
            linear_nt(g, w[8], x2, beta=1.0)
            add_bias_(x2, w[9])
            if ple is not None:
                pd = c.per_layer_dim
                for off, width, scale in _ple_slices(d, pd):
                    add_(x2[:, off:], ple[:, layer * pd :], alpha=scale, rows=n, cols=width)
            saved += [xl, h1, m1, r1, qkv, o, lse, x1, h2, m2, r2, u]
            xl = x2
        fw, fb = params[10 * c.n_layers], params[10 * c.n_layers + 1]
        hidden, mf, rf = layernorm_fwd(xl, fw, fb, eps)
        ctx.trunk, ctx.eps = trunk, eps
        ctx.has_ple, ctx.has_values = ple is not None, values is not None
        ctx.save_for_backward(seq_start, seq_of, xl, mf, rf, *saved, *params)
        ctx.n_saved = len(saved)
        return hidden

    @staticmethod
    def backward(ctx, dh):
        trunk = ctx.trunk
        c = trunk.config
        t = ctx.saved_tensors
        seq_start, seq_of, x_last, mf, rf = t[:5]
        saved = t[5 : 5 + ctx.n_saved]
        params = t[5 + ctx.n_saved :]
        device = dh.device
        n, d = x_last.shape
        H, KVH, D = c.n_heads, c.n_kv_heads, c.head_dim
        Q, KVW = H * D, KVH * D
        value_index = trunk._value_index
        grads = [torch.empty_like(p) for p in params]
        L = c.n_layers
        dx = norm_bwd(x_last, dh.float().contiguous(), params[10 * L], mf, rf, grads[10 * L], grads[10 * L + 1])
        dple = torch.zeros((n, c.ple_width), device=device) if ctx.has_ple else None
        dvalues = torch.zeros((n, c.value_width), device=device) if ctx.has_values else None
        for layer in reversed(range(L)):
            xl, h1, m1, r1, qkv, o, lse, x1, h2, m2, r2, u = saved[12 * layer : 12 * layer + 12]
            w = params[10 * layer : 10 * layer + 10]
            gw = grads[10 * layer : 10 * layer + 10]
            if dple is not None:
                pd = c.per_layer_dim
                for off, width, scale in _ple_slices(d, pd):
                    add_(dple[:, layer * pd :], dx[:, off:], alpha=scale, rows=n, cols=width)
            # x2 = x1 + GELU(u) W2^T + b2
            g = gelu_fwd(u)
            matmul_tn(dx, g, gw[8])
            column_sum(dx, gw[9])
            dg = torch.empty_like(u)
            matmul_nn(dx, w[8], dg)
            du = gelu_bwd(u, dg)
            matmul_tn(du, h2, gw[6])
            column_sum(du, gw[7])
            dh2 = torch.empty_like(h2)
            matmul_nn(du, w[6], dh2)
            dx1 = norm_bwd(x1, dh2, w[4], m2, r2, gw[4], gw[5])
            add_(dx1, dx)
            # x1 = xl + o Wo^T
            matmul_tn(dx1, o, gw[3])
            do = torch.empty_like(o)
            matmul_nn(dx1, w[3], do)
            dqkv = torch.empty_like(qkv)
            dsum = torch.empty((n, H), device=device)
            at = nat.AttnTrain(n, H, KVH, D, 1.0 / math.sqrt(D), seq_start.data_ptr(), seq_of.data_ptr(),
                               qkv.data_ptr(), _ptr(qkv, Q), _ptr(qkv, Q + KVW), Q + 2 * KVW, Q + 2 * KVW,
                               Q + 2 * KVW, o.data_ptr(), lse.data_ptr())
            nat.call("cg_attn_train_bwd", ctypes.byref(at), do.data_ptr(), dsum.data_ptr(), dqkv.data_ptr(),
                     _ptr(dqkv, Q), _ptr(dqkv, Q + KVW), _s(dh))
            if dvalues is not None and layer in value_index:
                col = value_index[layer] * KVW
                add_(dvalues[:, col:], dqkv[:, Q + KVW :], rows=n, cols=KVW)
            matmul_tn(dqkv, h1, gw[2])
            dh1 = torch.empty_like(h1)
            matmul_nn(dqkv, w[2], dh1)
            dx = norm_bwd(xl, dh1, w[0], m1, r1, gw[0], gw[1])
            add_(dx, dx1)
        return (None, None, dx, dple, dvalues, *grads)


def trunk_train_forward(trunk, x, ple, values, bounds=None):
    """Trunk.forward under autograd: [B, T, d] (or packed rows [N, d] with ``bounds``) ->
    final-norm hidden states of the same leading shape, differentiable."""

    _require_fp32(x.device)
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
    hidden = TrunkFunction.apply(trunk, seq_start, flat, ple_flat, values_flat, *block_params(trunk))
    return hidden.view(*lead, c.d_model)
