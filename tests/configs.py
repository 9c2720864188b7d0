"""Shared workload definitions: config kwargs and the seeded input/weight
recipe, used identically by the golden-vector generator (which feeds the
reference implementation) and by the tests and bench (which feed this build).

Mapping of BASELINE.json configs onto the reference's ModelConfig: the
common settings pin k=2 heads per token (attn_h_active/min/max = 2,
attn_router_top_p = 0, attn_linear_head_k = 2), gates == heads, prototype
routing on, no dropout, eval mode, no small-sequence dense path.
"""
from __future__ import annotations

from typing import Dict, Tuple

import torch

COMMON = dict(
    n_layer=1,
    p_dropout=0.0,
    bias=False,
    attn_variant="aspa",
    attn_h_active=2,
    attn_h_active_min=2,
    attn_h_active_max=2,
    attn_router_top_p=0.0,
    attn_linear_head_k=2,
    attn_router_noise_std=0.0,
    attn_force_dense_threshold=None,
    attn_small_seq_dense=0,
    attn_proto_enable=True,
)


def sparse_cfg(T: int, C: int, H: int, keep: float = 0.25) -> Dict:
    """Configs 1/2: token top-k at `keep`, causal attention over all keys
    <= t (linear mode with a full-length window, local policy)."""
    return dict(COMMON, vocab_size=0, n_ctx=T, n_head=H, d_model=C, attn_h_total=H, attn_gates=H,
                attn_token_sparse=True, attn_token_keep_ratio=keep, attn_linear_token_keep_schedule="fixed",
                attn_mode="linear", attn_linear_L=T, attn_linear_L_base=T, attn_linear_L_min=T, attn_linear_L_max=T,
                attn_linear_window=T, attn_linear_anchor_stride=0, attn_linear_policy="local")


def shortlist_cfg(T: int, C: int, H: int, L: int, window: int = 512, stride: int = 256) -> Dict:
    """Configs 3/4: linear shortlist mode, no token sparsity, fixed L,
    local+anchors+proto policy."""
    return dict(COMMON, vocab_size=0, n_ctx=T, n_head=H, d_model=C, attn_h_total=H, attn_gates=H,
                attn_token_sparse=False, attn_mode="linear", attn_linear_L=L, attn_linear_L_base=L,
                attn_linear_L_min=L, attn_linear_L_max=L, attn_linear_L_schedule="fixed", attn_linear_window=window,
                attn_linear_anchor_stride=stride, attn_linear_policy="local+anchors+proto")


def make_inputs(B: int, T: int, C: int, seed: int = 0, outlier_frac: float = 0.0) -> Tuple[torch.Tensor, torch.Generator]:
    """x ~ N(0,1) (f32) from Generator(seed); optional salient outliers:
    round(outlier_frac*T) positions scaled by 4."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, C, generator=g)
    if outlier_frac > 0.0:
        n = int(round(outlier_frac * T))
        idx = torch.randperm(T, generator=g)[:n]
        x[:, idx, :] *= 4.0
    return x, g


def init_weights(module, g: torch.Generator) -> None:
    """Xavier-normal re-init, in a fixed order, from the input generator."""
    with torch.no_grad():
        for t in (module.head_router.linear.weight, module.routing_prototypes, module.qkv.weight, module.proj.weight):
            tmp = torch.empty(t.shape, dtype=torch.float32)
            torch.nn.init.xavier_normal_(tmp, generator=g)
            t.copy_(tmp.to(t.dtype))
        module.routing_usage_ema.zero_()
        module.routing_confidence.zero_()


def state_tensors(module) -> Dict[str, torch.Tensor]:
    return {
        "w_router": module.head_router.linear.weight.detach().float().clone(),
        "protos": module.routing_prototypes.detach().float().clone(),
        "w_qkv": module.qkv.weight.detach().float().clone(),
        "w_proj": module.proj.weight.detach().float().clone(),
    }
