"""Proteus attention, MI355X build.

Drop-in for the ``proteus_attention`` package of Proteus-Flux-Attention on
its ASPA forward path: the same module, operator and tool names, computed by
hand-written gfx950 HIP kernels in ``lib/libpfa_hip.so`` (C ABI declared in
``include/pfa_hip.h``).
"""

from .kernels.sparse_attn import aspa_sparse_attention, get_last_backend, get_last_backend_info
from .models.aspa import (
    MLP,
    AdaptiveSparseAttention,
    AdaptiveSparseAttentionBlock,
    AdaptiveSparseProtoAttention,
    ModelConfig,
)
from .modules import CausalASPAMultiheadAttention
from .tools.chunked_shortlist import (
    ChunkedShortlistConfig,
    ChunkedShortlistMetrics,
    ChunkedShortlistResult,
    ChunkedShortlistRunner,
)

__all__ = [
    "AdaptiveSparseAttentionBlock",
    "AdaptiveSparseAttention",
    "AdaptiveSparseProtoAttention",
    "aspa_sparse_attention",
    "CausalASPAMultiheadAttention",
    "MLP",
    "ModelConfig",
    "get_last_backend",
    "get_last_backend_info",
    "ChunkedShortlistConfig",
    "ChunkedShortlistMetrics",
    "ChunkedShortlistResult",
    "ChunkedShortlistRunner",
    "__version__",
]

__version__ = "0.1.0+mi355x"
