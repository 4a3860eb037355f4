"""ctypes binding of libcardgym_hip.so (declared in include/cardgym_hip.h).

The library is the only compute path of this package: there is no CPU or PyTorch
fallback. Loading fails loudly when the shared library is missing, and every call's
status code becomes a Python exception (``ValueError`` for bad arguments, ``IndexError``
for out-of-range sizes, ``RuntimeError`` for HIP errors), like the ``TORCH_CHECK`` /
``RuntimeError`` behaviour of the reference's custom op (cardgym/nn/cuda_decode.py:135-151).
"""

from __future__ import annotations

import ctypes
import os
import re
from functools import lru_cache
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
LIBRARY = PACKAGE / "libcardgym_hip.so"
HEADER = PACKAGE.parent / "include" / "cardgym_hip.h"

CG_OK, CG_ERR_INVALID, CG_ERR_UNSUPPORTED, CG_ERR_RANGE, CG_ERR_HIP = 0, 1, 2, 3, 4
CG_F32, CG_BF16, CG_F16 = 0, 1, 2
CG_ACT_NONE, CG_ACT_GELU = 0, 1
CG_COPY_AUTO, CG_COPY_ORDERED = 0, 1
CG_TRUNK_STATIC_WORKSPACE = 64 << 20

c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64
c_void_p = ctypes.c_void_p
c_float = ctypes.c_float
c_size_t = ctypes.c_size_t


class KVLayer(ctypes.Structure):
    _fields_ = [
        ("k", c_void_p),
        ("v", c_void_p),
        ("capacity", c_int32),
        ("kv_heads", c_int32),
        ("max_len", c_int32),
        ("head_dim", c_int32),
        ("dtype", c_int32),
    ]


class KVSource(ctypes.Structure):
    _fields_ = [
        ("data", c_void_p),
        ("dtype", c_int32),
        ("stride_b", c_int64),
        ("stride_h", c_int64),
        ("stride_t", c_int64),
    ]


class TrunkConfig(ctypes.Structure):
    _fields_ = [
        ("d_model", c_int32),
        ("n_layers", c_int32),
        ("n_heads", c_int32),
        ("n_kv_heads", c_int32),
        ("d_ff", c_int32),
        ("per_layer_dim", c_int32),
        ("value_width", c_int32),
        ("eps", c_float),
    ]


class HeadsConfig(ctypes.Structure):
    _fields_ = [
        ("d_model", c_int32),
        ("n_policy", c_int32),
        ("d_mid", c_int32),
        ("n_value", c_int32),
    ]


class PiquetConfig(ctypes.Structure):
    _fields_ = [
        ("d_model", c_int32),
        ("ple_width", c_int32),
        ("value_width", c_int32),
        ("table_rows", c_int32),
        ("card_width", c_int32),
        ("card_hidden", c_int32),
        ("card_kernel", c_int32),
        ("card_layers", c_int32),
        ("eps", c_float),
    ]


class PiquetBlock(ctypes.Structure):
    _fields_ = [(name, c_void_p) for name in ("norm", "along_w", "along_b", "across_w", "out_w", "out_b")]


class AttnTrain(ctypes.Structure):
    _fields_ = [
        ("n", c_int32), ("H", c_int32), ("KVH", c_int32), ("head_dim", c_int32), ("scale", c_float),
        ("seq_start", c_void_p), ("seq_of", c_void_p), ("q", c_void_p), ("k", c_void_p), ("v", c_void_p),
        ("ldq", c_int64), ("ldk", c_int64), ("ldv", c_int64), ("o", c_void_p), ("lse", c_void_p),
        ("round_bf16", c_int32),
    ]


class TrainConfig(ctypes.Structure):
    _fields_ = [(name, c_int32) for name in ("d_model", "n_layers", "n_heads", "n_kv_heads", "d_ff", "per_layer_dim",
                                             "ple_width", "value_width")] + [("eps", c_float),
                                                                             ("value_index", ctypes.POINTER(c_int32)),
                                                                             ("bf16", c_int32)]


_TRAIN_BLOCK_FIELDS = ("ln_attn_w", "ln_attn_b", "qkv_w", "out_w", "ln_mlp_w", "ln_mlp_b", "up_w", "up_b", "down_w",
                       "down_b")


class TrainBlock(ctypes.Structure):
    _fields_ = [(name, c_void_p) for name in _TRAIN_BLOCK_FIELDS]


class TrainBlockGrads(ctypes.Structure):
    _fields_ = [(name, c_void_p) for name in _TRAIN_BLOCK_FIELDS]


class TrainGrads(ctypes.Structure):
    _fields_ = [("blocks", ctypes.POINTER(TrainBlockGrads)), ("final_dw", c_void_p), ("final_db", c_void_p)]


class LayerParams(ctypes.Structure):
    _fields_ = [
        ("ln_attn_w", c_void_p),
        ("ln_attn_b", c_void_p),
        ("qkv_w", c_void_p),
        ("out_w", c_void_p),
        ("ln_mlp_w", c_void_p),
        ("ln_mlp_b", c_void_p),
        ("mlp_up_w", c_void_p),
        ("mlp_up_b", c_void_p),
        ("mlp_down_w", c_void_p),
        ("mlp_down_b", c_void_p),
        ("value_index", c_int32),
    ]


class Ragged(ctypes.Structure):
    _fields_ = [
        ("n_seqs", c_int32),
        ("n_tokens", c_int32),
        ("T", c_int32),
        ("span", c_int32),
        ("seq_start", c_void_p),
        ("positions", c_void_p),
        ("rows", c_void_p),
        ("readout", c_void_p),
        ("status", c_void_p),
    ]


P = ctypes.POINTER
_SIGNATURES = {
    "cg_version": (c_int32, []),
    "cg_last_error": (c_size_t, [ctypes.c_char_p, c_size_t]),
    "cg_kv_write_step": (c_int32, [P(KVLayer), c_void_p, c_void_p, P(KVSource), P(KVSource), c_int32, c_int32, c_void_p]),
    "cg_kv_write_range": (c_int32, [P(KVLayer), c_void_p, c_int32, P(KVSource), P(KVSource), c_int32, c_int32, c_void_p]),
    "cg_kv_read": (c_int32, [P(KVLayer), c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "cg_kv_copy_rows": (c_int32, [P(KVLayer), c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "cg_kv_copy_workspace_size": (c_size_t, [P(KVLayer), c_int32, c_int32, c_int32]),
    "cg_kv_copy_rows_layers": (
        c_int32, [P(KVLayer), c_int32, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_size_t, c_void_p],
    ),
    "cg_kv_check_indices": (c_int32, [P(KVLayer), c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_void_p]),
    "cg_decode_attention": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_int64, P(KVLayer), c_void_p, c_void_p,
         c_int32, c_int32, c_int32, c_int32, c_float, c_void_p, c_int32, c_void_p],
    ),
    "cg_decode_attention_order": (
        c_int32, [P(KVLayer), c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p],
    ),
    "cg_decode_attention_ordered": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, c_int64, P(KVLayer), c_void_p, c_void_p,
         c_int32, c_int32, c_int32, c_int32, c_float, c_void_p, c_int32, c_void_p, c_void_p],
    ),
    "cg_decode_attention_packed": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, P(KVLayer), c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
         c_int32, c_float, c_void_p, c_int32, c_void_p],
    ),
    "cg_decode_attention_packed_order": (
        c_int32, [P(KVLayer), c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p],
    ),
    "cg_decode_attention_packed_ordered": (
        c_int32,
        [c_void_p, c_int32, c_int64, c_int64, P(KVLayer), c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32,
         c_int32, c_float, c_void_p, c_int32, c_void_p, c_void_p],
    ),
    "cg_trunk_create": (c_int32, [P(TrunkConfig), P(LayerParams), c_void_p, c_void_p, c_int32, P(c_void_p)]),
    "cg_trunk_refresh": (c_int32, [c_void_p, c_void_p]),
    "cg_trunk_destroy": (c_int32, [c_void_p]),
    "cg_trunk_workspace_size": (c_size_t, [c_void_p, c_int32, c_int32]),
    "cg_trunk_forward": (
        c_int32,
        [c_void_p, P(KVLayer), c_void_p, c_void_p, c_void_p, P(Ragged), c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "cg_trunk_forward_tokens": (
        c_int32,
        [c_void_p, P(KVLayer), c_void_p, c_int32, c_void_p, c_void_p, c_float, c_void_p, c_void_p, P(Ragged),
         c_void_p, c_void_p, c_size_t, c_void_p],
    ),
    "cg_trunk_forward_static": (
        c_int32, [c_void_p, P(KVLayer), c_void_p, c_void_p, c_void_p, P(Ragged), c_void_p, c_void_p],
    ),
    "cg_gelu_bf16": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p]),
    "cg_rmsnorm": (c_int32, [c_void_p, c_int32, c_void_p, c_float, c_void_p, c_int32, c_int32, c_void_p]),
    "cg_embed_rmsnorm": (
        c_int32,
        [c_void_p, c_int32, c_void_p, c_void_p, c_float, c_void_p, c_int32, c_int32, c_void_p, c_void_p],
    ),
    "cg_linear": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p],
    ),
    "cg_linear_add_scale": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32, c_float, c_int32, c_void_p],
    ),
    "cg_heads_create": (
        c_int32, [P(HeadsConfig), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, P(c_void_p)],
    ),
    "cg_heads_refresh": (c_int32, [c_void_p, c_void_p]),
    "cg_heads_destroy": (c_int32, [c_void_p]),
    "cg_heads_forward": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p]),
    "cg_masked_probabilities": (
        c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64, c_void_p],
    ),
    "cg_sample_rows": (
        c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int32, c_int32, c_void_p, c_void_p],
    ),
    "cg_advance_positions": (c_int32, [c_void_p, c_int32, c_int64, c_void_p]),
    "cg_piquet_create": (
        c_int32,
        [P(PiquetConfig), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, P(c_void_p)],
    ),
    "cg_piquet_refresh": (c_int32, [c_void_p, c_void_p]),
    "cg_gemm_workspace_size": (c_size_t, [c_int32, c_int32, c_int32]),
    "cg_gemm_strided": (
        c_int32,
        [c_int32, c_int32, c_int32, c_float, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_float,
         c_void_p, c_int64, c_int32, c_void_p, c_size_t, c_void_p],
    ),
    "cg_layernorm_fwd": (
        c_int32, [c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p],
    ),
    "cg_norm_bwd_workspace_size": (c_size_t, [c_int32, c_int32]),
    "cg_norm_bwd": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
         c_int32, c_void_p, c_size_t, c_int32, c_void_p],
    ),
    "cg_column_sum_workspace_size": (c_size_t, [c_int32, c_int32]),
    "cg_column_sum": (c_int32, [c_void_p, c_int32, c_int32, c_int64, c_void_p, c_int32, c_void_p, c_size_t, c_void_p]),
    "cg_gelu_fwd": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p]),
    "cg_gelu_bwd": (c_int32, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "cg_add_strided": (c_int32, [c_int32, c_int32, c_float, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "cg_rmsnorm_fwd": (c_int32, [c_void_p, c_void_p, c_float, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "cg_seq_of": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p]),
    "cg_attn_train_fwd": (c_int32, [P(AttnTrain), c_void_p]),
    "cg_train_saved_size": (c_size_t, [P(TrainConfig), c_int32]),
    "cg_train_scratch_size": (c_size_t, [P(TrainConfig), c_int32]),
    "cg_trunk_train_forward": (
        c_int32,
        [P(TrainConfig), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
         c_void_p, c_void_p, c_size_t, c_void_p, c_size_t, c_void_p],
    ),
    "cg_trunk_train_backward": (
        c_int32,
        [P(TrainConfig), c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_size_t, c_void_p, c_size_t,
         P(TrainGrads), c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "cg_attn_train_bwd": (c_int32, [P(AttnTrain), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "cg_piquet_destroy": (c_int32, [c_void_p]),
    "cg_piquet_embed": (
        c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
}


class NativeLibraryMissing(RuntimeError):
    pass


def declared_symbols() -> list[str]:
    """Every ``cg_*`` function the public header declares."""

    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+\*?\s*(cg_\w+)\s*\(", text, re.M)))


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    """The loaded library with typed signatures; raises when it was not built."""

    path = Path(os.environ.get("CARDGYM_HIP_LIBRARY", LIBRARY))
    if not path.exists():
        raise NativeLibraryMissing(
            f"{path} is missing: build it with `python -m card_playing_gym_amd.csrc.build` "
            "(there is no fallback path)."
        )
    handle = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def last_error() -> str:
    buf = ctypes.create_string_buffer(1024)
    lib().cg_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


_EXCEPTIONS = {
    CG_ERR_INVALID: ValueError,
    CG_ERR_UNSUPPORTED: ValueError,
    CG_ERR_RANGE: IndexError,
    CG_ERR_HIP: RuntimeError,
}


def check(status: int) -> None:
    if status != CG_OK:
        raise _EXCEPTIONS.get(status, RuntimeError)(last_error())


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
