"""Drop-in modules (reference modules/__init__.py)."""

from .aspa_multihead import CausalASPAMultiheadAttention
from .sparse_ctl import SparseCtlSnapshot, SparseHeadController
from .transformer_block import CausalASPATransformerBlock

__all__ = [
    "CausalASPAMultiheadAttention",
    "SparseHeadController",
    "SparseCtlSnapshot",
    "CausalASPATransformerBlock",
]
