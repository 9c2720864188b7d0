"""``nn.TransformerEncoderLayer``-shaped block around the ASPA drop-in
(reference modules/transformer_block.py:31-116)."""
from __future__ import annotations

from typing import Callable, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .aspa_multihead import CausalASPAMultiheadAttention

_ACTIVATIONS = {"relu": F.relu, "gelu": F.gelu, "silu": F.silu}


def _get_activation_fn(name: str) -> Callable[[torch.Tensor], torch.Tensor]:
    try:
        return _ACTIVATIONS[name.lower()]
    except KeyError as exc:
        raise ValueError(f"Unsupported activation '{name}'.") from exc


class CausalASPATransformerBlock(nn.Module):
    """Encoder block (post- or pre-norm) whose self-attention is ASPA."""

    def __init__(self, embed_dim: int, num_heads: int, *, dim_feedforward: int = 2048, dropout: float = 0.1,
                 activation: str = "gelu", layer_norm_eps: float = 1e-5, norm_first: bool = False,
                 attention_kwargs: Optional[dict] = None) -> None:
        super().__init__()
        args = dict(attention_kwargs or {})
        args.setdefault("batch_first", True)
        args.setdefault("dropout", dropout)
        self.self_attn = CausalASPAMultiheadAttention(embed_dim=embed_dim, num_heads=num_heads, **args)
        self.linear1 = nn.Linear(embed_dim, dim_feedforward)
        self.activation = _get_activation_fn(activation)
        self.dropout = nn.Dropout(dropout)
        self.linear2 = nn.Linear(dim_feedforward, embed_dim)
        self.norm_first = bool(norm_first)
        self.norm1 = nn.LayerNorm(embed_dim, eps=layer_norm_eps)
        self.norm2 = nn.LayerNorm(embed_dim, eps=layer_norm_eps)
        self.dropout1 = nn.Dropout(dropout)
        self.dropout2 = nn.Dropout(dropout)

    def forward(self, src: torch.Tensor, *, src_mask: Optional[torch.Tensor] = None,
                src_key_padding_mask: Optional[torch.Tensor] = None, return_attn: bool = False, **kwargs):
        residual = src
        h = self.norm1(src) if self.norm_first else src
        attn_out, weights = self.self_attn(h, attn_mask=src_mask, key_padding_mask=src_key_padding_mask,
                                           need_weights=return_attn, **kwargs)
        src = residual + self.dropout1(attn_out)
        if not self.norm_first:
            src = self.norm1(src)
        residual = src
        h = self.norm2(src) if self.norm_first else src
        src = residual + self.dropout2(self.linear2(self.dropout(self.activation(self.linear1(h)))))
        if not self.norm_first:
            src = self.norm2(src)
        return (src, weights) if return_attn else src


__all__ = ["CausalASPATransformerBlock"]
