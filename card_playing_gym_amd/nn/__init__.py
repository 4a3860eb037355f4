"""The cardgym.nn API of the KV-cached self-play trunk step, on MI355X kernels."""

from .kv_cache import KVCache
from .model import SequenceModel, value_mlp
from .trunk import DecoderBlock, RMSNorm, Trunk, TrunkConfig, init_weights

__all__ = [
    "DecoderBlock",
    "KVCache",
    "RMSNorm",
    "SequenceModel",
    "Trunk",
    "TrunkConfig",
    "init_weights",
    "value_mlp",
]
