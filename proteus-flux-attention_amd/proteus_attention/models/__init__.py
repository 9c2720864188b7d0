"""ASPA model layer (reference models/__init__.py)."""

from .aspa import (
    MLP,
    AdaptiveSparseAttention,
    AdaptiveSparseAttentionBlock,
    AdaptiveSparseProtoAttention,
    ModelConfig,
    SwitchRouter,
)

__all__ = [
    "AdaptiveSparseAttentionBlock",
    "AdaptiveSparseAttention",
    "AdaptiveSparseProtoAttention",
    "MLP",
    "ModelConfig",
    "SwitchRouter",
]
