"""Adaptive Sparse Proto Attention (ASPA) module on the MI355X kernels.

Host-side mirror of ``src/proteus_attention/models/aspa.py`` of the
reference: the same ``ModelConfig`` attribute bag, the same constructor
knobs, schedules and telemetry dictionaries, and the same forward semantics.
All per-token and per-row work runs in libpfa_hip.so:

=====================================  ======================================
reference step (aspa.py)               device work here
=====================================  ======================================
router + proto prior (628-690)         ``pfa_router_topk`` (one pass over x)
importance (1521-1530)                 same kernel
head top-k + mask (1590-1606)          same kernel + ``pfa_pack_rows``
token top-k (790-842)                  ``pfa_token_topk``
QKV / out projections                  torch Linear (hipBLASLt GEMMs)
RoPE (606-618)                         ``pfa_rope_qk_inplace`` (in the QKV buffer)
packing (1704-1756)                    ``pfa_pack_rows``
shortlist candidates (1269-1284)       ``pfa_proto_prefix_topk`` + ``pfa_shortlist_build``
sparse attention + scatter (1287-1302,
1802-1807, 1841-1842)                  ``pfa_sparse_attn_fwd`` writing (B,T,H,D)
prototype EMA (692-718)                ``pfa_proto_accumulate`` + reduce
=====================================  ======================================

The attention kernel reads q/k/v straight out of the (B, T, 3, H, D) QKV
projection and writes each active row into its (B, T, H, D) slot, so the
reference's permute/index_select/index_copy/zeros passes disappear.

Out of scope (kept for API compatibility only): the memory bank
(aspa.py:932-1035; its candidates are clamped to the row itself by the
builder, so it never changes outputs — updates are not performed here) and
training-mode attention dropout.
"""
from __future__ import annotations

import gc
import math
import time
import warnings
from typing import Any, Dict, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _hip
from ..kernels import sparse_attn as _sa
from ..kernels.sparse_attn import (
    _record_backend,
    get_last_backend,
    get_last_backend_info,
)


# Side streams (default priority) shared by every module in the process, one
# per (device, role): "fork" carries a forward's second dependency chain,
# "capture" a graph capture's warm-up forward, "copy" the chunked runner's
# host-to-device chunk copies.  torch keeps a GEMM workspace
# (hipBLASLt) for every stream a GEMM has run on until the process ends, so a
# stream per module instance would leave one workspace behind per instance.
# Every use is bracketed by stream waits in both directions, so sharing adds
# no dependency a forward does not already have.
_SIDE_STREAMS: Dict[Tuple[int, str], torch.cuda.Stream] = {}


def _side_stream(device: torch.device, role: str) -> torch.cuda.Stream:
    index = device.index if device.index is not None else torch.cuda.current_device()
    st = _SIDE_STREAMS.get((index, role))
    if st is None:
        st = torch.cuda.Stream(device=torch.device("cuda", index))
        _SIDE_STREAMS[(index, role)] = st
    return st

class ModelConfig:
    """Attribute bag with the reference defaults (aspa.py:33-72)."""

    _DEFAULTS: Dict[str, Any] = {
        "vocab_size": 0,
        "n_ctx": 0,
        "n_layer": 0,
        "n_head": 1,
        "d_model": 0,
        "p_dropout": 0.0,
        "bias": False,
        "attn_variant": "standard",
        "moe_n_experts": 0,
        "attn_mode": "auto",
        "attn_linear_L": 512,
        "attn_linear_window": 512,
        "attn_linear_anchor_stride": 256,
        "attn_linear_head_k": 2,
        "attn_linear_switch_ctx": 20000,
        "attn_linear_latency_budget_ms": None,
        "attn_linear_policy": "local+anchors",
        "attn_use_rope": True,
        "attn_rope_base": 10000.0,
        "attn_router_top_p": 0.9,
    }

    def __init__(self, **kwargs: Any) -> None:
        merged = dict(self._DEFAULTS)
        merged.update(kwargs)
        self.__dict__.update(merged)

    def to_dict(self) -> Dict[str, Any]:
        return dict(self.__dict__)


class LayerNorm(nn.Module):
    """LayerNorm with optional bias (aspa.py:75-85)."""

    def __init__(self, ndim: int, bias: bool, eps: float = 1e-5) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(ndim))
        self.bias = nn.Parameter(torch.zeros(ndim)) if bias else None
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.layer_norm(x, x.shape[-1:], self.weight, self.bias, eps=self.eps)


class RMSNorm(nn.Module):
    """RMS normalisation (aspa.py:88-99)."""

    def __init__(self, ndim: int, eps: float = 1e-6) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(ndim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.weight * (x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + self.eps))


def _build_norm(config: ModelConfig) -> nn.Module:
    kind = str(getattr(config, "norm_type", "layernorm") or "layernorm").lower()
    eps = float(getattr(config, "norm_eps", 1e-5))
    if kind == "rmsnorm":
        return RMSNorm(config.d_model, eps=eps)
    return LayerNorm(config.d_model, bias=bool(getattr(config, "bias", False)), eps=eps)


class MLP(nn.Module):
    """Feed-forward block of AdaptiveSparseAttentionBlock (aspa.py:114-132)."""

    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        hidden = int(getattr(config, "mlp_hidden_mult", 4)) * config.d_model
        self.fc1 = nn.Linear(config.d_model, hidden, bias=bool(config.bias))
        self.act = nn.GELU()
        self.fc2 = nn.Linear(hidden, config.d_model, bias=bool(config.bias))
        self.dropout = nn.Dropout(config.p_dropout)
        self.last_aux_loss: Optional[torch.Tensor] = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.dropout(self.fc2(self.act(self.fc1(x))))


class SwitchRouter(nn.Module):
    """Router parameters (aspa.py:135-157).  Its math runs inside the fused
    router kernel; ``forward`` is kept for API compatibility and runs the
    same computation with torch ops on the module's device."""

    def __init__(self, d_model: int, n_gates: int, noise_std: float = 0.0) -> None:
        super().__init__()
        self.linear = nn.Linear(d_model, n_gates, bias=False)
        self.noise_std = float(noise_std)

    def forward(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        logits = self.linear(x)
        if self.training and self.noise_std > 0.0:
            logits = logits + torch.randn_like(logits) * self.noise_std
        probs = F.softmax(logits, dim=-1)
        scores, indices = torch.max(probs, dim=-1)
        return indices, scores, probs


def pack_router_weights(w_router: torch.Tensor, proto_norm: Optional[torch.Tensor], x_dtype: torch.dtype) -> torch.Tensor:
    """(C, 2*Gp) f32 channel-interleaved router weights for pfa_router_topk:
    column g holds the router weight of gate g at its ``x_dtype`` value,
    column Gp+g the normalised prototype; padding gates are zero."""

    G, C = w_router.shape
    Gp = int(_hip.lib().pfa_router_gate_pad(G))
    packed = torch.zeros(C, 2 * Gp, dtype=torch.float32, device=w_router.device)
    packed[:, :G] = w_router.detach().to(x_dtype).to(torch.float32).t()
    if proto_norm is not None:
        packed[:, Gp:Gp + G] = proto_norm.detach().to(torch.float32).t()
    return packed


def _flag(value: Any) -> bool:
    return bool(value)


def _policy_tokens(raw: str) -> set:
    text = str(raw or "local+anchors").lower().replace("|", ",").replace("+", ",")
    toks = {p.strip() for p in text.split(",") if p.strip()}
    return toks or {"local", "anchors"}


def _lazy_stat(name: str) -> property:
    """Telemetry attribute whose value may still be in flight from the GPU:
    reading it first completes the pending readbacks of earlier forwards, so
    a forward itself never waits on the device for its statistics."""
    key = "_lazy_" + name

    def get(self):
        self._resolve_stats()
        return self.__dict__.get(key)

    def put(self, value):
        self.__dict__[key] = value

    return property(get, put)


class AdaptiveSparseAttention(nn.Module):
    """ASPA layer (reference aspa.py:170-1932) on MI355X kernels."""

    last_head_stats = _lazy_stat("last_head_stats")
    _last_sparse_state = _lazy_stat("_last_sparse_state")
    _last_proto_stats = _lazy_stat("_last_proto_stats")
    _density_ema = _lazy_stat("_density_ema")
    _last_density = _lazy_stat("_last_density")
    _latency_ema = _lazy_stat("_latency_ema")

    def __init__(self, config: ModelConfig):
        super().__init__()
        g = lambda name, default=None: getattr(config, name, default)  # noqa: E731
        self.d_model = config.d_model
        self.bias = _flag(g("bias", False))

        # --- head counts and schedule (aspa.py:183-224) ---
        h_total = int(g("attn_h_total", 0) or g("n_head", 1) or 1)
        if h_total <= 0:
            h_total = max(1, int(g("n_head", 1)))
        self.h_total = h_total
        if self.d_model % self.h_total != 0:
            raise ValueError("d_model must be divisible by the total number of attention heads (attn_h_total)")
        base_active = int(g("attn_h_active", 0))
        if base_active <= 0 or base_active > h_total:
            base_active = max(1, min(4, h_total))
        amax = int(g("attn_h_active_max", 0) or 0)
        amax = min(16, h_total) if amax <= 0 else amax
        amax = max(1, min(amax, h_total))
        amin = int(g("attn_h_active_min", 0) or 0)
        amin = max(1, min(2, amax)) if amin <= 0 else amin
        amin = max(1, min(amin, amax))
        self.h_active_min, self.h_active_max = amin, amax
        self.h_active = max(amin, min(base_active, amax))
        curve = g("attn_active_curve", None)
        try:
            curve_val = float(curve) if curve is not None else 0.25
        except (TypeError, ValueError):
            curve_val = 0.25
        self.h_active_curve = 1.0 if curve_val <= 0.0 else curve_val
        self.force_dense_when_full = _flag(g("attn_force_dense_when_full", False))
        self.d_head = self.d_model // self.h_total

        # --- RoPE (aspa.py:226-247) ---
        self.use_rope = _flag(g("attn_use_rope", True))
        rope_base = float(g("attn_rope_base", 10000.0) or 10000.0)
        self.rope_base = rope_base if rope_base > 0.0 else 10000.0
        if self.use_rope and self.d_head % 2 != 0:
            warnings.warn("Disabling RoPE because attention head dimension is not even.", RuntimeWarning)
            self.use_rope = False
        inv_freq = 1.0 / (self.rope_base ** (torch.arange(0, self.d_head, 2, dtype=torch.float32)
                                             / max(self.d_head, 1)))
        self.register_buffer("_rope_inv_freq", inv_freq, persistent=False)
        self._rope_cache: Dict[Tuple[str, int, str], Tuple[int, torch.Tensor, torch.Tensor]] = {}

        self.dropout = nn.Dropout(config.p_dropout)
        self.use_sdpa = _flag(g("use_sdpa", True))
        self.router_reg_lambda = float(g("attn_router_lambda", 0.0) or 0.0)
        self.router_reg_beta = float(g("attn_router_beta", 1.0) or 1.0)
        self.router_reg_mode = str(g("attn_router_reg_mode", "entropy"))
        try:
            top_p = float(g("attn_router_top_p", 0.0))
        except (TypeError, ValueError):
            top_p = 0.0
        if not math.isfinite(top_p):
            top_p = 0.0
        self.router_top_p = max(0.0, min(top_p, 1.0))
        mode = str(g("attn_mode", "auto") or "auto").lower()
        self.mode_setting = mode if mode in {"auto", "subquad", "linear"} else "auto"

        # --- shortlist length schedule (aspa.py:274-306) ---
        self.linear_L = max(1, int(g("attn_linear_L", 512) or 512))
        sched = str(g("attn_linear_L_schedule", "fixed") or "fixed").lower()
        self.linear_L_schedule = sched if sched in {"fixed", "sqrt", "log", "mem_cap"} else "fixed"
        self.linear_L_base = max(1, int(g("attn_linear_L_base", self.linear_L) or self.linear_L))
        lmin_default = min(64, self.linear_L_base)
        self.linear_L_min = max(1, int(g("attn_linear_L_min", lmin_default) or lmin_default))
        lmax_cfg = g("attn_linear_L_max", self.linear_L)
        self.linear_L_max = max(self.linear_L_min, int(lmax_cfg if lmax_cfg is not None else self.linear_L))
        self.linear_L_scale_init = max(0.1, float(g("attn_linear_L_scale", 1.0) or 1.0))
        smax_default = max(1.0, self.linear_L_scale_init)
        self.linear_L_scale_max = float(g("attn_linear_L_scale_max", smax_default) or smax_default)
        self._linear_scale_min = max(0.05, self.linear_L_min / max(1.0, self.linear_L_base))
        self._linear_L_scale_runtime = self.linear_L_scale_init
        self.linear_latency_shrink = min(max(float(g("attn_linear_latency_shrink", 0.8) or 0.8), 0.1), 0.99)
        self.linear_latency_growth = max(1.0, float(g("attn_linear_latency_growth", 1.05) or 1.05))
        mem_budget = g("attn_linear_mem_budget_mb", None)
        self.linear_mem_budget_mb = float(mem_budget) if mem_budget is not None else None

        # --- piece fractions (aspa.py:307-378) ---
        f_local = max(0.0, min(1.0, float(g("attn_linear_piece_local_frac", 0.6) or 0.6)))
        f_anchor = max(0.0, min(1.0, float(g("attn_linear_piece_anchor_frac", 0.3) or 0.3)))
        f_proto = float(g("attn_linear_piece_proto_frac", max(0.0, 1.0 - f_local - f_anchor)))
        f_proto = max(0.0, min(1.0, f_proto))
        tot = f_local + f_anchor + f_proto
        if tot <= 0.0:
            f_local, f_anchor, f_proto, tot = 1.0, 0.0, 0.0, 1.0
        f_local /= tot
        f_anchor /= tot
        f_proto = max(0.0, 1.0 - f_local - f_anchor)
        window_hint = int(g("attn_linear_window", self.linear_L_base) or self.linear_L_base)
        if window_hint <= 0:
            window_hint = self.linear_L_base
        self.linear_window_base = max(1, window_hint)
        self.linear_window = self.linear_window_base
        stride = int(g("attn_linear_anchor_stride", g("attn_linear_anchors_every", 256)) or 0)
        self.linear_anchor_stride = max(0, stride)
        self.linear_head_k = max(1, min(int(g("attn_linear_head_k", 2) or 2), self.h_total))
        self.linear_switch_ctx = max(0, int(g("attn_linear_switch_ctx", 20000) or 20000))
        lat = g("attn_linear_latency_budget_ms", None)
        self.linear_latency_budget_ms = float(lat) if lat is not None else None
        toks = _policy_tokens(g("attn_linear_policy", "local+anchors"))
        self.linear_policy_tokens = toks
        self.linear_use_anchors = bool(toks & {"anchors", "anchor", "global"})
        self.linear_use_proto = bool(toks & {"proto", "prototype", "semantic", "dna"})
        self.linear_use_local = bool(toks & {"local", "window"}) or not (self.linear_use_anchors or self.linear_use_proto)
        f_local = f_local if self.linear_use_local else 0.0
        f_anchor = f_anchor if self.linear_use_anchors else 0.0
        f_proto = f_proto if self.linear_use_proto else 0.0
        psum = f_local + f_anchor + f_proto
        if psum <= 0.0:
            f_local, f_anchor, f_proto = 1.0, 0.0, 0.0
        else:
            f_local /= psum
            f_anchor /= psum
            f_proto = max(0.0, 1.0 - f_local - f_anchor)
        self.linear_piece_local_frac = f_local
        self.linear_piece_anchor_frac = f_anchor
        self.linear_piece_proto_frac = f_proto
        self._linear_runtime: Optional[dict] = None
        self._linear_runtime_seq_len: Optional[int] = None
        self._linear_runtime_alpha: Optional[float] = None
        self._current_alpha: float = 0.0
        try:
            cutoff = float(g("attn_dense_alpha_cutoff", 0.0))
        except (TypeError, ValueError):
            cutoff = 0.25
        self.dense_alpha_cutoff = float(max(0.0, min(0.95, cutoff)))

        # --- memory bank: accepted, not executed (see module docstring) ---
        self.memory_enabled = _flag(g("attn_memory_enable", False))
        slots = int(g("attn_memory_slots", 0) or 0)
        if slots <= 0:
            self.memory_enabled = False
            slots = 1
        if self.memory_enabled:
            warnings.warn("attn_memory_enable: the memory bank is not executed by the MI355X build; "
                          "its candidates never reach attention in the reference either.", RuntimeWarning)
        self.memory_slots = slots
        self.memory_decay = float(max(0.0, min(1.0, float(g("attn_memory_decay", 0.9) or 0.9))))
        self.register_buffer("memory_keys", torch.zeros(h_total, slots, self.d_head), persistent=False)
        self.register_buffer("memory_values", torch.zeros(h_total, slots, self.d_head), persistent=False)
        self.register_buffer("memory_counts", torch.zeros(h_total, slots), persistent=False)
        self.register_buffer("memory_ptr", torch.zeros(h_total, dtype=torch.long), persistent=False)

        # --- per-head int8 quantisation (aspa.py:395-437) ---
        self.quantize_sparse_int8 = _flag(g("attn_quantize_int8", False))
        qmode = str(g("attn_quantize_int8_mode", "max") or "max").lower()
        self.quantize_sparse_int8_mode = qmode if qmode in {"max", "percentile", "ema_percentile"} else "max"
        self.quantize_sparse_int8_percentile = min(max(float(g("attn_quantize_int8_percentile", 1.0) or 1.0), 0.0), 1.0)
        self.quantize_sparse_int8_ema_decay = min(max(float(g("attn_quantize_int8_ema_decay", 0.9) or 0.9), 0.0), 0.9999)
        for name in ("_quant_ema_q", "_quant_ema_k", "_quant_ema_v"):
            self.register_buffer(name, torch.zeros(h_total), persistent=False)
        self._quant_ema_flags = {"_quant_ema_q": False, "_quant_ema_k": False, "_quant_ema_v": False}

        # --- sequence schedule (aspa.py:438-476) ---
        low = int(g("attn_active_seq_low", 0) or 0)
        high = int(g("attn_active_seq_high", 0) or 0)
        if low <= 0:
            low = max(64, self.d_head)
        if high <= 0:
            high = int(g("n_ctx", 0) or (low * 4))
        if high < low:
            high = low
        self.seq_low, self.seq_high = low, high
        dense_hint = g("attn_small_seq_dense", None)
        try:
            dense_cut = int(dense_hint) if dense_hint is not None else max(0, low // 2)
        except (TypeError, ValueError):
            dense_cut = max(0, low // 2)
        self.small_seq_dense = max(0, dense_cut)
        self._density_ema: Optional[float] = None
        self._last_density: Optional[float] = None
        self._last_target_k: Optional[int] = None
        thr_hint = g("attn_force_dense_threshold", None)
        thr = float(thr_hint) if thr_hint is not None else None
        self._dense_threshold: Optional[float] = thr if (thr is not None and thr > 0.0) else None

        # --- router + gate->head map (aspa.py:478-489) ---
        gates = int(g("attn_gates", 0))
        if gates <= 0:
            gates = max(h_total, self.h_active_max, self.h_active) * 2
        self.attn_gates = max(gates, h_total, self.h_active_max)
        self.head_router = SwitchRouter(self.d_model, self.attn_gates,
                                        noise_std=float(g("attn_router_noise_std", 0.01)))
        gate_to_head = self._default_mapping(self.attn_gates, h_total)
        self.register_buffer("gate_to_head", gate_to_head, persistent=False)
        self.register_buffer("gate_to_head_onehot", F.one_hot(gate_to_head, num_classes=h_total).to(torch.float32),
                             persistent=False)
        self._shortlist_alpha_override: Optional[float] = None

        self.qkv = nn.Linear(self.d_model, 3 * self.d_model, bias=self.bias)
        self.proj = nn.Linear(self.d_model, self.d_model, bias=self.bias)

        # --- telemetry / caches (aspa.py:497-567) ---
        self.last_head_stats: Optional[dict] = None
        self._last_sparse_state: Optional[dict] = None
        self._hip_graph_enabled = _flag(g("attn_hip_graph", False))
        self._hip_graph_static_output = False
        self._hip_graphs: Dict[Any, dict] = {}
        self._hip_graph_pool = None
        self._cached_active_mask: Optional[torch.Tensor] = None
        self._cached_packing = None
        self.last_aux_loss: Optional[torch.Tensor] = None
        self.last_router_reg: Optional[torch.Tensor] = None
        self._latency_ema: Optional[float] = None
        self.track_latency = _flag(g("attn_track_latency", True))
        self.proto_enabled = _flag(g("attn_proto_enable", False))
        self.proto_decay = float(g("attn_proto_decay", 0.97))
        self.proto_threshold = float(g("attn_proto_threshold", 0.25))
        self.proto_blend = float(g("attn_proto_blend", 0.6))
        self.proto_temp = float(max(g("attn_proto_temp", 0.2), 1e-3))
        self.proto_usage_boost = float(max(g("attn_proto_usage_boost", 0.0), 0.0))
        self.proto_init_scale = float(g("attn_proto_init_scale", 0.02))
        if self.proto_enabled:
            self.register_buffer("routing_prototypes",
                                 torch.randn(self.attn_gates, self.d_model, dtype=torch.float32) * self.proto_init_scale)
            self.register_buffer("routing_usage_ema", torch.zeros(self.attn_gates, dtype=torch.float32))
            self.register_buffer("routing_confidence", torch.zeros(self.attn_gates, dtype=torch.float32))
        else:
            self.routing_prototypes = None  # type: ignore[assignment]
            self.routing_usage_ema = None  # type: ignore[assignment]
            self.routing_confidence = None  # type: ignore[assignment]
        self._last_proto_stats: Optional[dict] = None
        self.token_sparse = _flag(g("attn_token_sparse", False))
        keep = min(max(float(g("attn_token_keep_ratio", 1.0) or 1.0), 0.0), 1.0)
        self.token_keep_ratio_base = keep
        self._token_keep_ratio_runtime: Optional[float] = None
        ksched = str(g("attn_linear_token_keep_schedule", "sqrt") or "sqrt").lower()
        self.linear_token_keep_schedule = ksched if ksched in {"fixed", "sqrt", "log"} else "sqrt"
        kmin = float(g("attn_linear_token_keep_min_ratio", 0.2) or 0.2)
        self.linear_token_keep_ratio_min = min(max(kmin, 0.0), keep)
        self.linear_token_keep_ratio_ref = int(g("attn_linear_token_keep_ref", 2048) or 2048)
        min_keep = max(0, int(g("attn_token_keep_min", 0) or 0))
        guard = max(0, int(g("attn_token_keep_guard", 1) or 1))
        self.token_keep_guard = guard
        self.token_keep_min = max(min_keep, guard if self.token_sparse else min_keep)
        self.token_keep_threshold = float(max(0.0, float(g("attn_token_keep_threshold", 0.0) or 0.0)))
        self._last_token_importance: Optional[torch.Tensor] = None
        self._last_token_mask: Optional[torch.Tensor] = None
        self._last_token_blend: Optional[torch.Tensor] = None
        self._last_token_similarity: Optional[torch.Tensor] = None
        self._last_shortlist_backend_info: Optional[Dict[str, object]] = None
        self._last_batch_size: Optional[int] = None
        self.last_head_consensus: Optional[torch.Tensor] = None
        self._last_gate_probs: Optional[torch.Tensor] = None
        self._last_shortlist_lengths: Optional[torch.Tensor] = None
        # per-row candidate counts of the structured shortlist path are
        # telemetry: computed (inside the attention kernel) only on request
        self.record_shortlist_lengths = False
        # structured shortlist path: rotate q rows inside the attention kernel
        # (only k is rotated in the QKV buffer); False rotates q in the buffer
        self.fuse_q_rope = True
        # structured path with anchors: fuse_anchor_pass makes the anchor pass
        # write the zeros of the output rows without a packed row (no zero
        # fill of the output); with fuse_k_rope as well (and q rotated on
        # load) it also rotates k, so no RoPE pass runs either.  Both are off
        # by default: the anchor pass's share of that work costs more than
        # the pass it replaces (measured at configs 3 and 4; config 3 on one
        # box: 0.4037 ms/step unfused, 0.4099 with the zeros in the anchor
        # pass, 0.4425 with k's rotation as well -- each anchor workgroup
        # rotates its class's rows before its first tile).
        self.fuse_anchor_pass = False
        self.fuse_k_rope = False
        # The prototype EMA statistics (sum_t gate * x) are accumulated inside
        # the router pass (x is read from HBM once; MFMA with exact products);
        # False accumulates them by a separate pass over x in the router's
        # tail instead (token-order f32 sums).  Both give the same sums up to
        # f32 rounding, in the same 64-token parts.
        self.fuse_ema_stats = True

    # ------------------------------------------------------------------
    # RoPE tables (aspa.py:576-604)
    # ------------------------------------------------------------------
    @staticmethod
    def _rope_rotate_half(x: torch.Tensor) -> torch.Tensor:
        return torch.stack((-x[..., 1::2], x[..., ::2]), dim=-1).reshape_as(x)

    def _rope_factors(self, seq_len: int, device: torch.device, dtype: torch.dtype):
        if seq_len <= 0:
            raise ValueError("RoPE requires a positive sequence length.")
        key = (device.type, int(device.index) if device.index is not None else -1, str(dtype))
        cached = self._rope_cache.get(key)
        if cached is None or cached[0] < seq_len:
            inv = self._rope_inv_freq.to(device=device)
            pos = torch.arange(seq_len, device=device, dtype=inv.dtype)
            ang = torch.outer(pos, inv)
            cos = torch.repeat_interleave(ang.cos(), 2, dim=-1).to(dtype)
            sin = torch.repeat_interleave(ang.sin(), 2, dim=-1).to(dtype)
            cached = (seq_len, cos, sin)
            self._rope_cache[key] = cached
        return cached[1][:seq_len], cached[2][:seq_len]

    @staticmethod
    def _default_mapping(gates: int, heads: int) -> torch.Tensor:
        heads = max(1, heads)
        idx = torch.arange(gates, dtype=torch.long)
        return torch.clamp((idx * heads) // max(gates, 1), 0, heads - 1)

    # ------------------------------------------------------------------
    # schedules (aspa.py:731-930, 1037-1173) -- host arithmetic
    # ------------------------------------------------------------------
    def _choose_active_k(self, seq_len: int) -> int:
        if seq_len <= self.seq_low:
            target = self.h_active_max
        elif seq_len >= self.seq_high:
            target = self.h_active_min
        else:
            ratio = float(seq_len - self.seq_low) / float(max(1, self.seq_high - self.seq_low))
            if self.h_active_curve != 1.0:
                ratio = max(0.0, min(1.0, ratio)) ** self.h_active_curve
            target = int(math.floor(self.h_active_max - ratio * (self.h_active_max - self.h_active_min) + 1e-6))
        target = max(self.h_active_min, min(target, self.h_active_max))
        self._last_target_k = target
        return target

    def _nucleus_head_count(self, head_probs: torch.Tensor, target_p: float, max_cap: int) -> int:
        if max_cap <= 1:
            return max(1, max_cap)
        probs = head_probs.detach().to(torch.float32)
        if probs.numel() == 0:
            return 1
        mean = probs.mean(dim=(0, 1))
        if mean.numel() == 0:
            return 1
        mean = torch.where(torch.isfinite(mean), mean, torch.zeros_like(mean)).cpu()
        total = float(mean.sum())
        if total <= 0.0:
            return 1
        cum = torch.cumsum(torch.sort(mean, descending=True).values, dim=0)
        keep = int((cum < total * float(target_p)).sum())
        if keep < mean.numel():
            keep += 1
        return min(max_cap, max(1, keep))

    def _defer(self, fn) -> None:
        """Queue a telemetry step that needs device results; it runs at the
        next _resolve_stats (a telemetry read or the next forward) as
        fn(module).  The steps take the module as their argument rather than
        closing over it: a queued closure holding the module would make a
        reference cycle, and a dropped module (with its device buffers and
        graphs) would then live until Python's cycle collector ran."""
        self.__dict__.setdefault("_pending_stats", []).append(fn)

    def _resolve_stats(self) -> None:
        pend = self.__dict__.get("_pending_stats")
        if not pend:
            return
        self.__dict__["_pending_stats"] = []
        for fn in pend:
            fn(self)

    def _update_density(self, value: float) -> None:
        value = float(max(0.0, value))
        self._last_density = value
        self._density_ema = value if self._density_ema is None else 0.8 * self._density_ema + 0.2 * value

    def _density_threshold(self) -> Optional[float]:
        return self._dense_threshold

    def _set_linear_scale(self, value: float) -> None:
        lo = self._linear_scale_min
        hi = max(lo, self.linear_L_scale_max)
        self._linear_L_scale_runtime = float(min(max(value, lo), hi))
        self._linear_runtime_seq_len = None
        self._linear_runtime_alpha = None

    def adjust_linear_L_scale(self, factor: float) -> None:
        if factor == 0.0:
            return
        self._set_linear_scale(self._linear_L_scale_runtime * factor)

    def _linear_token_keep_ratio(self, seq_len: int) -> float:
        if not self.token_sparse:
            return self.token_keep_ratio_base
        base = self.token_keep_ratio_base
        ref = max(1, self.linear_token_keep_ratio_ref)
        seq = max(1, int(seq_len))
        if self.linear_token_keep_schedule == "sqrt":
            ratio = base * math.sqrt(ref / float(seq))
        elif self.linear_token_keep_schedule == "log":
            ratio = base * (math.log2(ref + 1.0) / math.log2(seq + 1.0))
        else:
            ratio = base
        return float(max(min(base, self.linear_token_keep_ratio_min), min(base, ratio)))

    def _get_shortlist_alpha(self, seq_len: int) -> float:
        if self._shortlist_alpha_override is not None:
            return float(max(0.0, min(1.0, self._shortlist_alpha_override)))
        seq_len = int(max(1, seq_len))
        low = max(1, int(self.seq_low))
        high = max(low + 1, int(self.linear_switch_ctx)) if self.linear_switch_ctx > 0 else max(low + 1, seq_len)
        if seq_len <= low:
            return 0.0
        if seq_len >= high:
            return 1.0
        return float((seq_len - low) / (high - low))

    def _compute_cvt_alpha(self, seq_len: int) -> float:
        seq_len = int(max(1, seq_len))
        setting = str(self.mode_setting or "").lower()
        if setting == "linear":
            alpha = 1.0
        elif setting == "subquad":
            alpha = 0.0
        else:
            alpha = self._get_shortlist_alpha(seq_len)
        if self.linear_latency_budget_ms is not None and self._latency_ema is not None:
            budget, lat = self.linear_latency_budget_ms, self._latency_ema
            if lat > budget * 1.05:
                if self._linear_L_scale_runtime > self._linear_scale_min + 1e-3:
                    self.adjust_linear_L_scale(self.linear_latency_shrink)
                alpha = 1.0
            elif lat < budget * 0.80 and seq_len < max(1, self.linear_switch_ctx):
                if self._linear_L_scale_runtime < self.linear_L_scale_max:
                    self.adjust_linear_L_scale(self.linear_latency_growth)
                alpha = min(alpha, 0.0)
        if self.linear_switch_ctx > 0:
            if self._current_alpha >= 0.95 and seq_len >= max(1, int(self.linear_switch_ctx * 0.75)):
                alpha = max(alpha, 0.95)
            if seq_len >= self.linear_switch_ctx:
                alpha = 1.0
        return float(max(0.0, min(1.0, alpha)))

    def set_shortlist_alpha(self, value: float) -> None:
        """Override the shortlist slider (0 = dense, 1 = linear)."""
        self._shortlist_alpha_override = float(max(0.0, min(1.0, value)))
        self._linear_runtime = None
        self._linear_runtime_seq_len = None
        self._linear_runtime_alpha = None

    def _compute_effective_linear_params(self, seq_len: int, batch_size: Optional[int], alpha: float) -> dict:
        seq_len = max(1, int(seq_len))
        coeff = float(max(1.0, self.linear_L_base))
        sched = self.linear_L_schedule
        if sched == "sqrt":
            base_val = coeff * math.sqrt(float(seq_len))
        elif sched == "log":
            base_val = coeff * math.log2(float(seq_len) + 1.0)
        elif sched == "mem_cap" and self.linear_mem_budget_mb:
            heads_est = max(1, int(getattr(self, "_last_target_k", self.linear_head_k)))
            batch_est = max(1, int(batch_size) if batch_size is not None else 1)
            denom = heads_est * batch_est * seq_len * max(1, self.d_head) * 8
            cap = int(self.linear_mem_budget_mb * 1024 * 1024 // denom) if denom > 0 else self.linear_L_max
            base_val = max(1, min(cap, self.linear_L_max))
        else:
            base_val = coeff
        eff = max(self.linear_L_min, min(self.linear_L_max, int(math.ceil(self._linear_L_scale_runtime * max(1.0, base_val)))))
        window = min(self.linear_window_base, eff)
        dense_cap = int(min(seq_len, max(self.linear_L_min, self.linear_window_base + seq_len // 32)))
        dense_cap = max(self.linear_L_min, min(self.linear_L_max, dense_cap))
        eff = max(self.linear_L_min, min(self.linear_L_max, int(alpha * eff + (1.0 - alpha) * dense_cap)))
        window_dense = max(1, min(seq_len, max(self.linear_window_base, seq_len // 8)))
        window = max(1, min(eff, int(alpha * window + (1.0 - alpha) * window_dense)))
        use = (self.linear_use_local, self.linear_use_anchors, self.linear_use_proto)
        dense_w = (0.85 if use[0] else 0.0, 0.10 if use[1] else 0.0, 0.05 if use[2] else 0.0)
        frac = (self.linear_piece_local_frac, self.linear_piece_anchor_frac, self.linear_piece_proto_frac)
        target_w = tuple(f if u else 0.0 for f, u in zip(frac, use))
        w = [(1.0 - alpha) * d + alpha * t for d, t in zip(dense_w, target_w)]
        total = sum(w)
        if total <= 0.0:
            w, total = [1.0, 0.0, 0.0], 1.0
        w_local = w[0] / total
        w_anchor = w[1] / total
        w_proto = max(0.0, 1.0 - w_local - w_anchor)
        caps = [int(round(eff * w_local)) if use[0] else 0,
                int(round(eff * w_anchor)) if use[1] else 0,
                int(round(eff * w_proto)) if use[2] else 0]
        total_caps = sum(caps)
        if total_caps > eff and total_caps > 0:
            caps = [int(max(0, math.floor(c * (eff / total_caps)))) for c in caps]
            total_caps = sum(caps)
        remaining = eff - total_caps
        for i in range(3):
            if remaining <= 0:
                break
            if not use[i]:
                continue
            caps[i] += 1
            remaining -= 1
        if remaining > 0:
            caps[0 if use[0] else 1 if use[1] else 2] += remaining
        if use[0]:
            caps[0] = min(caps[0], window)
            if caps[0] <= 0 and eff > 0:
                caps[0] = min(window, max(1, eff // 4))
        if use[1] and caps[1] < 0:
            caps[1] = 0
        if use[2] and caps[2] < 0:
            caps[2] = 0
        return {
            "effective_L": eff,
            "local_cap": max(0, int(caps[0])),
            "anchor_cap": max(0, int(caps[1])),
            "proto_cap": max(0, int(caps[2])),
            "window": max(1, int(window)),
            "shortlist_alpha": float(alpha),
        }

    def _prepare_linear_runtime(self, seq_len: int, batch_size: Optional[int], alpha: float) -> dict:
        if (self._linear_runtime is not None and self._linear_runtime_seq_len == seq_len
                and self._linear_runtime_alpha is not None and abs(self._linear_runtime_alpha - float(alpha)) < 1e-4):
            return self._linear_runtime
        alpha = float(max(0.0, min(1.0, alpha)))
        p = self._compute_effective_linear_params(seq_len, batch_size, alpha)
        self.linear_L = p["effective_L"]
        self.linear_window = p["window"]
        runtime = dict(p)
        runtime["anchor_stride"] = self.linear_anchor_stride
        self._linear_runtime = runtime
        self._linear_runtime_seq_len = seq_len
        self._linear_runtime_alpha = alpha
        return runtime

    # ------------------------------------------------------------------
    # int8 per-head quantisation (aspa.py:1312-1363)
    # ------------------------------------------------------------------
    def _quantize_per_head_int8(self, tensor: torch.Tensor, ema_buffer: str) -> Tuple[torch.Tensor, torch.Tensor]:
        """(P, T, D) -> int8 (P, T, D) and per-head f32 scales (P,), on the
        device (pfa_quantize_heads_int8)."""
        if tensor.dim() != 3:
            raise ValueError("Expected a rank-3 tensor for per-head quantization")
        device = _hip.require_device(tensor, what="_quantize_per_head_int8")
        x = tensor if tensor.stride(-1) == 1 else tensor.contiguous()
        P, T, D = x.shape
        quant = torch.empty(P, T, D, dtype=torch.int8, device=device)
        scales = torch.empty(P, dtype=torch.float32, device=device)
        self._quantize_heads(_hip.tensor4(x, P), x.dtype, P, T, D, None, P, None, _hip.tensor4(quant, P), torch.int8,
                             scales, ema_buffer)
        return quant, scales

    def _quantize_heads(self, x4, dtype, H, T, D, head_map, P, summary, dst4, dst_dtype, scales, ema_buffer):
        """The reference's quantisation rule (aspa.py:1312-1363) for the P
        active heads of one of q/k/v, with this module's mode and its
        per-head EMA buffer (re-initialised when P changes, as the
        reference's is)."""
        mode = self.quantize_sparse_int8_mode
        ema, valid = None, False
        if mode == "ema_percentile":
            ema = getattr(self, ema_buffer)
            valid = bool(ema is not None and ema.numel() == P and self._quant_ema_flags.get(ema_buffer, False)
                         and ema.device == scales.device and ema.dtype == torch.float32)
            if not valid:
                ema = torch.empty(P, dtype=torch.float32, device=scales.device)
        _sa.quantize_heads_int8(x4, dtype, H, T, D, head_map, P, summary, mode,
                                float(self.quantize_sparse_int8_percentile), float(self.quantize_sparse_int8_ema_decay),
                                ema, valid, dst4, dst_dtype, scales, scales.device)
        if ema is not None:
            setattr(self, ema_buffer, ema)
            self._quant_ema_flags[ema_buffer] = True

    # ------------------------------------------------------------------
    # device stages
    # ------------------------------------------------------------------
    def _router_raw_inputs(self, device: torch.device):
        """The router's weight and prototype-prior buffers as they are:
        (w, protos, confidence, usage, buf_dtype, use_proto)."""
        w = self.head_router.linear.weight.detach()
        if w.device != device:
            w = w.to(device)
        w = w.contiguous()
        use_proto = bool(self.proto_enabled and self.routing_prototypes is not None)
        protos = conf_b = usage_b = None
        buf_dtype = w.dtype
        if use_proto:
            protos = self.routing_prototypes.detach().contiguous()
            buf_dtype = protos.dtype
            if self.routing_confidence is not None:
                conf_b = self.routing_confidence.detach().view(-1).contiguous()
            if self.proto_usage_boost > 0.0 and self.routing_usage_ema is not None:
                usage_b = self.routing_usage_ema.detach().view(-1).contiguous()
            for t in (conf_b, usage_b):
                if t is not None and t.dtype != buf_dtype:
                    raise ValueError("routing_prototypes / routing_confidence / routing_usage_ema must share one dtype")
        return w, protos, conf_b, usage_b, buf_dtype, use_proto

    def _router_inputs(self, device: torch.device, x_dtype: torch.dtype):
        """Router weight table, prototype prior inputs (aspa.py:636-663) in one
        launch (pfa_router_prepare): (w_packed, conf_weight, usage_bias,
        use_proto)."""
        lib = _hip.lib()
        G, C = self.attn_gates, self.d_model
        w, protos, conf_b, usage_b, buf_dtype, use_proto = self._router_raw_inputs(device)
        Gp = int(lib.pfa_router_gate_pad(G))
        wpk = torch.empty(C, 2 * Gp, dtype=torch.float32, device=device)
        conf = torch.empty(G, dtype=torch.float32, device=device) if conf_b is not None else None
        usage = torch.empty(G, dtype=torch.float32, device=device) if usage_b is not None else None
        _hip.check(lib.pfa_router_prepare(_hip.ptr(w), _hip.dtype_tag(w.dtype), _hip.ptr(protos), _hip.ptr(conf_b),
                                          _hip.ptr(usage_b), _hip.dtype_tag(buf_dtype), G, C, _hip.dtype_tag(x_dtype),
                                          _hip.ptr(wpk), _hip.ptr(conf), _hip.ptr(usage), _hip.stream_ptr(device)),
                   "pfa_router_prepare")
        return wpk, conf, usage, use_proto

    def _gate_to_head_i32(self, device: torch.device) -> torch.Tensor:
        # int32 copy, rebuilt when the mapping buffer moves or is modified
        src = self.gate_to_head
        key = (device, src.data_ptr(), src._version)
        cached = getattr(self, "_g2h_cache", None)
        if cached is None or cached[0] != key:
            cached = (key, src.to(device=device, dtype=torch.int32).contiguous())
            self._g2h_cache = cached
        keep = self.__dict__.get("_capture_keep")
        if keep is not None:
            keep.append(cached[1])
        return cached[1]

    def _route_device(self, x2d: torch.Tensor, topk: int, need_head_scores: bool = True):
        """Fused router: gate probs, sim, blend, importance, head top-k."""
        lib = _hip.lib()
        device = x2d.device
        n_tok, C = x2d.shape
        G, H = self.attn_gates, self.h_total
        # bf16 shapes of the MFMA router build their inputs inside the router
        # (pfa_router_topk_raw); the others take pfa_router_prepare first
        w, protos, conf_b, usage_b, buf_dtype, use_proto = self._router_raw_inputs(device)
        raw = bool(lib.pfa_router_raw_supported(_hip.dtype_tag(x2d.dtype), _hip.dtype_tag(w.dtype),
                                                _hip.dtype_tag(buf_dtype), G, C, 1 if use_proto else 0))
        if raw:
            keep = self.__dict__.get("_capture_keep")
            if keep is not None:
                keep.extend(t for t in (w, protos, conf_b, usage_b) if t is not None)
        else:
            wpk, conf, usage, use_proto = self._router_inputs(device, x2d.dtype)
        gate = torch.empty(n_tok, G, dtype=torch.float32, device=device)
        imp = torch.empty(n_tok, dtype=torch.float32, device=device)
        sim = torch.empty(n_tok, dtype=torch.float32, device=device) if use_proto else None
        blend = torch.empty(n_tok, dtype=torch.float32, device=device) if use_proto else None
        hidx = torch.empty(n_tok, topk, dtype=torch.int32, device=device)
        hsc = torch.empty(n_tok, topk, dtype=torch.float32, device=device) if need_head_scores else None
        nblk = _hip.ctypes.c_int(0)
        _hip.check(lib.pfa_router_block_count(n_tok, _hip.ctypes.byref(nblk)), "pfa_router_block_count")
        stats = torch.empty(max(1, nblk.value), 8, dtype=torch.float32, device=device)
        # prototype EMA statistics accumulated in the same pass over x when
        # fuse_ema_stats is set (consumed by _update_routing_prototypes at the
        # end of the forward; otherwise that step accumulates them itself)
        ema = None
        if self._ema_active() and self.fuse_ema_stats:
            ema = torch.empty(max(1, nblk.value), G, C + 1, dtype=torch.float32, device=device)
        self._ema_partial = (ema, x2d.data_ptr(), n_tok) if ema is not None else None
        g2h = self._gate_to_head_i32(device)
        tail = (_hip.ptr(g2h), H, topk, float(self.proto_temp), float(self.proto_threshold),
                float(self.proto_blend), float(self.proto_usage_boost), _hip.ptr(gate), _hip.ptr(sim),
                _hip.ptr(blend), _hip.ptr(imp), _hip.ptr(hidx), _hip.ptr(hsc), _hip.ptr(stats), _hip.ptr(ema),
                _hip.stream_ptr(device))
        with _hip.TIMER.timed("router_topk"):
            if raw and G > 16:
                # 17-64 gates: 16-gate MFMA blocks into a workspace, then the epilogue
                name = "pfa_router_topk_raw_ws"
                nbytes = _sa._size_out(lib.pfa_router_raw_workspace_size, n_tok, G)
                ws = _sa._workspace(nbytes, device)
                rc = lib.pfa_router_topk_raw_ws(
                    _hip.ptr(x2d), _hip.dtype_tag(x2d.dtype), n_tok, C, G, _hip.ptr(w), _hip.dtype_tag(w.dtype),
                    _hip.ptr(protos), _hip.ptr(conf_b), _hip.ptr(usage_b), _hip.dtype_tag(buf_dtype), *tail[:-1],
                    _hip.ptr(ws), ws.numel(), tail[-1])
            elif raw:
                name = "pfa_router_topk_raw"
                rc = lib.pfa_router_topk_raw(
                    _hip.ptr(x2d), _hip.dtype_tag(x2d.dtype), n_tok, C, G, _hip.ptr(w), _hip.dtype_tag(w.dtype),
                    _hip.ptr(protos), _hip.ptr(conf_b), _hip.ptr(usage_b), _hip.dtype_tag(buf_dtype), *tail)
            else:
                name = "pfa_router_topk"
                rc = lib.pfa_router_topk(
                    _hip.ptr(x2d), _hip.dtype_tag(x2d.dtype), n_tok, C, G, _hip.ptr(wpk), 1 if use_proto else 0,
                    _hip.ptr(conf), _hip.ptr(usage), *tail)
        _hip.check(rc, name)
        self._router_stats = stats
        return gate, sim, blend, imp, hidx, hsc

    def _select_active_tokens(self, importance: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
        """Token keep mask (aspa.py:790-842) via pfa_token_topk."""
        if not self.token_sparse or importance is None or importance.dim() != 2:
            return None
        B, T = importance.shape
        if T == 0:
            return None
        ratio = float(self._token_keep_ratio_runtime if self._token_keep_ratio_runtime is not None
                      else self.token_keep_ratio_base)
        device = importance.device
        if ratio >= 0.999 and self.token_keep_threshold <= 0.0:
            mask = torch.ones(B, T, dtype=torch.bool, device=device)
            self._last_token_mask = mask
            self._token_keep_cap = T
            return mask
        guard = min(max(0, self.token_keep_guard), T)
        min_keep = max(min(max(0, self.token_keep_min), T), guard)
        keep = int(torch.tensor(ratio * T, dtype=torch.float32).round().item())
        if min_keep > 0:
            keep = max(keep, min_keep)
        keep = max(1, min(keep, T))
        _hip.require_device(importance, what="_select_active_tokens")
        imp = importance.to(torch.float32).contiguous()
        mask8 = torch.empty(B, T, dtype=torch.uint8, device=device)
        lib = _hip.lib()
        ws = _sa._workspace(_sa._size_out(lib.pfa_token_topk_workspace_size, B, T), device)
        rc = lib.pfa_token_topk(_hip.ptr(imp), B, T, keep, guard, float(self.token_keep_threshold),
                                _hip.ptr(mask8), _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device))
        _hip.check(rc, "pfa_token_topk")
        mask = mask8.view(torch.bool)
        self._last_token_mask = mask
        # kept tokens per batch row: without a threshold, the top `keep`
        # plus at most `guard` leading tokens; with one, data dependent
        self._token_keep_cap = min(T, keep + guard) if self.token_keep_threshold <= 0.0 else None
        return mask

    def _ema_active(self) -> bool:
        return bool(self.proto_enabled and self.routing_prototypes is not None
                    and self.routing_usage_ema is not None and self.routing_confidence is not None)

    def _update_routing_prototypes(self, token_feats: torch.Tensor, gate_probs: torch.Tensor) -> None:
        """Prototype / usage / confidence EMA (aspa.py:692-718)."""
        if not self._ema_active():
            return
        with torch.no_grad():
            lib = _hip.lib()
            x2d = token_feats.detach().reshape(-1, self.d_model)
            if x2d.dtype not in (torch.float32, torch.bfloat16, torch.float16):
                x2d = x2d.to(torch.float32)
            x2d = x2d.contiguous()
            device = x2d.device
            n_tok, C, G = x2d.size(0), self.d_model, self.attn_gates
            fused = getattr(self, "_ema_partial", None)
            self._ema_partial = None
            if fused is not None and fused[1] == x2d.data_ptr() and fused[2] == n_tok:
                # statistics already accumulated by this forward's router pass
                partial = fused[0]
                nparts = partial.size(0)
            else:
                probs = gate_probs.detach().to(torch.float32).reshape(-1, self.attn_gates).contiguous()
                np_c = _hip.ctypes.c_int(0)
                _hip.check(lib.pfa_proto_partial_count(n_tok, _hip.ctypes.byref(np_c)), "pfa_proto_partial_count")
                nparts = np_c.value
                partial = torch.empty(nparts, G, C + 1, dtype=torch.float32, device=device)
                _hip.check(lib.pfa_proto_accumulate(_hip.ptr(x2d), _hip.dtype_tag(x2d.dtype), n_tok, C, G,
                                                    _hip.ptr(probs), _hip.ptr(partial), nparts,
                                                    _hip.stream_ptr(device)), "pfa_proto_accumulate")
            sums = torch.empty(G, C + 1, dtype=torch.float32, device=device)
            _hip.check(lib.pfa_proto_partial_reduce(_hip.ptr(partial), nparts, G, C, _hip.ptr(sums),
                                                    _hip.stream_ptr(device)), "pfa_proto_partial_reduce")
            proto, usage, conf = self.routing_prototypes, self.routing_usage_ema, self.routing_confidence
            if not (proto.dtype == usage.dtype == conf.dtype and proto.is_contiguous()):
                raise ValueError("routing_prototypes / routing_usage_ema / routing_confidence must share one "
                                 "dtype and be contiguous")
            _hip.check(lib.pfa_proto_ema_update(_hip.ptr(sums), G, C, float(self.proto_decay), _hip.ptr(proto),
                                                _hip.ptr(usage), _hip.ptr(conf), _hip.dtype_tag(proto.dtype),
                                                _hip.stream_ptr(device)), "pfa_proto_ema_update")
            self._proto_sums = sums

    # ------------------------------------------------------------------
    def _full_rows(self, B: int, T: int, device: torch.device):
        """All (b, h, t) rows active: packed layout for the dense branches."""
        BH = B * self.h_total
        token_idx = torch.arange(T, device=device, dtype=torch.int32).repeat(BH)
        row_head = torch.arange(BH, device=device, dtype=torch.int32).repeat_interleave(T)
        return token_idx, row_head

    def _masked_rows(self, token_mask: torch.Tensor, B: int, T: int, device: torch.device):
        """Rows of every head for the tokens token_mask keeps, packed on the
        device (pfa_pack_rows with each token's head list = all H heads):
        token_idx / row_head at capacity B*H*T, -1 / 0 past the device row
        count, the compact head list and the packing summary ({P, N, ...})."""
        H = self.h_total
        BH = B * H
        lib = _hip.lib()
        hidx = torch.arange(H, dtype=torch.int32, device=device).repeat(B * T)
        mask8 = torch.empty(BH, T, dtype=torch.uint8, device=device)
        heads = torch.empty(BH, dtype=torch.int32, device=device)
        row_offsets = torch.empty(BH + 1, dtype=torch.int32, device=device)
        token_idx = torch.full((BH * T,), -1, dtype=torch.int32, device=device)
        row_head = torch.zeros(BH * T, dtype=torch.int32, device=device)
        summary = torch.empty(4, dtype=torch.int32, device=device)
        ws = _sa._workspace(_sa._size_out(lib.pfa_pack_workspace_size, B, H, T), device)
        tm8 = token_mask.contiguous().view(torch.uint8)
        rc = lib.pfa_pack_rows(_hip.ptr(hidx), H, _hip.ptr(tm8), B, H, T, _hip.ptr(mask8), _hip.ptr(heads),
                               _hip.ptr(row_offsets), _hip.ptr(token_idx), _hip.ptr(row_head), None,
                               _hip.ptr(summary), _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device))
        _hip.check(rc, "pfa_pack_rows")
        return token_idx, row_head, heads, summary

    def _attend_dense_causal(self, qkv: torch.Tensor, B: int, T: int, out: torch.Tensor,
                             token_mask: Optional[torch.Tensor] = None) -> None:
        """Every head and token, keys 0..t (force-dense / dense fast path).
        Equivalent to the reference's (T,T) triu(-inf) mask without
        materialising it (aspa.py:1664-1677, 1365-1396).  With token_mask
        (B, T) only the rows of the kept tokens are attended and `out`
        keeps its zeros elsewhere: the reference's dense output times the
        token mask (aspa.py:1841-1842) without the multiply."""
        H, D = self.h_total, self.d_head
        head_map = n_dev = None
        if token_mask is None:
            token_idx, row_head = self._full_rows(B, T, qkv.device)
        else:
            token_idx, row_head, head_map, summary = self._masked_rows(token_mask, B, T, qkv.device)
            n_dev = summary[1:2]
        q5 = qkv.view(B, T, 3, H, D)
        out4 = out.view(B, T, H, D)
        t4 = (_hip.tensor4(q5[:, :, 0], H, "bthd"), _hip.tensor4(q5[:, :, 1], H, "bthd"),
              _hip.tensor4(q5[:, :, 2], H, "bthd"), _hip.tensor4(out4, H, "bthd"))
        if out.dtype == qkv.dtype and _sa._mfma_causal_ok(qkv.dtype, D, *t4):
            # flash-style causal tiles on MFMA (64 queries x 64 keys); rows
            # past the device count carry token -1, which the kernel skips
            _sa._causal_attn_mfma(*t4, H, T, D, token_idx, row_head, head_map, qkv.device)
            return
        _sa._attn_launch(_hip.tensor4(q5[:, :, 0], H, "bthd"), _hip.tensor4(q5[:, :, 1], H, "bthd"),
                         _hip.tensor4(q5[:, :, 2], H, "bthd"), qkv.dtype, _hip.tensor4(out4, H, "bthd"), out.dtype,
                         H, T, D, token_idx, row_head, head_map, None, None, None, None, 1.0 / math.sqrt(D),
                         (None, None, None), qkv.device, n_rows_dev=n_dev)

    def _project_qkv(self, x: torch.Tensor) -> torch.Tensor:
        qkv = self.qkv(x).contiguous()  # (B, T, 3C) = (B, T, 3, H, D)
        self._rope_inplace(qkv, rotate_q=True)
        return qkv

    def _rope_inplace(self, qkv: torch.Tensor, rotate_q: bool, rotate_k: bool = True,
                      zero_out: Optional[torch.Tensor] = None):
        """RoPE of the QKV buffer (aspa.py:606-618).  With rotate_q=False only
        k is rotated and the (cos, sin) tables are returned for a kernel that
        rotates q rows as it loads them (pfa_shortlist_attn_fwd); with
        rotate_k=False as well nothing is launched and the tables are
        returned for the fused anchor pass, which rotates k too.  zero_out
        (k alone rotated): the attention output, filled with zeros by the same
        pass (pfa_rope_k_zero_inplace); with RoPE off it is filled here."""
        if not self.use_rope:
            if zero_out is not None:
                zero_out.zero_()
            return None
        B, T = qkv.shape[0], qkv.shape[1]
        cos, sin = self._rope_factors(T, qkv.device, qkv.dtype)
        cos, sin = cos.contiguous(), sin.contiguous()
        keep = self.__dict__.get("_capture_keep")
        if keep is not None:
            keep.extend((cos, sin))
        if not rotate_q and not rotate_k:
            return cos, sin
        if rotate_q and not rotate_k:
            raise ValueError("q alone is never rotated by the RoPE kernels")
        if zero_out is not None and (rotate_q or not rotate_k):
            raise ValueError("the output zero fill rides on the k-only RoPE pass")
        lib = _hip.lib()
        args = (_hip.ptr(qkv), _hip.dtype_tag(qkv.dtype), B, T, self.h_total, self.d_head, _hip.ptr(cos),
                _hip.ptr(sin))
        with _hip.TIMER.timed("rope_qk"):
            if zero_out is not None:
                name = "pfa_rope_k_zero_inplace"
                rc = lib.pfa_rope_k_zero_inplace(*args, _hip.ptr(zero_out), _hip.stream_ptr(qkv.device))
            else:
                name = "pfa_rope_qk_inplace" if rotate_q else "pfa_rope_k_inplace"
                rc = getattr(lib, name)(*args, _hip.stream_ptr(qkv.device))
        _hip.check(rc, name)
        return None if rotate_q else (cos, sin)

    def _forward_dense_fastpath(self, x: torch.Tensor) -> torch.Tensor:
        """Dense causal attention for short sequences (aspa.py:1365-1440)."""
        B, T, C = x.shape
        self._resolve_stats()
        qkv = self._project_qkv(x)
        attn = torch.empty(B, T, C, dtype=qkv.dtype, device=x.device)
        self._attend_dense_causal(qkv, B, T, attn)
        y = self.dropout(self.proj(attn))
        self._last_target_k = self.h_total
        self._last_sparse_state = {
            "mode": "dense_fastpath", "backend": "hip_dense", "max_rows": T, "density": 1.0,
            "target_k": self.h_total,
            "force_dense_threshold": None if self._dense_threshold is None else float(self._dense_threshold),
            "cutoff": int(self.small_seq_dense), "quantized": False, "token_keep_fraction": 1.0,
        }
        self._update_density(1.0)
        self.last_head_stats = {
            "top_k": int(self.h_total), "mean_gate_prob": 1.0, "router_entropy": 0.0,
            "mean_active_per_token": float(self.h_total), "unique_heads": int(self.h_total),
            "active_fraction": 1.0, "max_active_rows": int(T), "max_active_density": 1.0,
            "target_k": int(self.h_total), "seq_len": int(T), "active_min": int(self.h_active_min),
            "active_max": int(self.h_active_max),
            "force_dense_threshold": None if self._dense_threshold is None else float(self._dense_threshold),
            "active_curve": float(self.h_active_curve), "token_keep_fraction": 1.0,
            "router_top_p": float(self.router_top_p), "nucleus_k": int(self.h_total), "top_a_consensus": True,
        }
        self.last_router_reg = None
        return y

    # ------------------------------------------------------------------
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _hip.require_device(x, what="AdaptiveSparseAttention.forward")
        if self.training and float(self.dropout.p) > 0.0:
            raise NotImplementedError("training-mode attention dropout is not provided by the HIP forward path")
        if self._hip_graph_enabled and self._graph_eligible(x):
            return self._forward_graph(x)
        return self._forward_impl(x)

    # ------------------------------------------------------------------
    # HIP graph replay of the forward
    def enable_hip_graph(self, enabled: bool = True, static_output: bool = False) -> None:
        """Replay the forward from a captured HIP graph.

        The first call for an input shape/dtype (and the schedule state that
        fixes the launch sequence) captures every launch of the forward up to
        the attention output, plus the prototype EMA, into one graph; later
        calls copy the input into the graph's static buffer (skipped when the
        caller passes that buffer back), replay it and run the output
        projection eagerly, so the returned tensor is fresh.  Telemetry is
        read back as in the eager forward.  Applies in eval / no-grad mode
        when no host decision depends on device results (no token sparsity,
        density threshold, nucleus head count, memory or latency budget);
        otherwise the eager forward runs.  Tensors the module keeps from the
        last forward (last_head_consensus, _last_gate_probs, ...) are the
        graph's static buffers and change with the next replay.

        static_output=True captures the output projection too: forward()
        then returns the graph's own output buffer, with no launch after the
        replay, and that tensor is overwritten by the next forward of the
        same shape (the usual contract of a captured graph's outputs; clone
        it to keep it)."""
        if bool(static_output) != self._hip_graph_static_output:
            self.reset_hip_graphs()
        self._hip_graph_enabled = bool(enabled)
        self._hip_graph_static_output = bool(static_output) and bool(enabled)
        if not enabled:
            self.reset_hip_graphs()

    def reset_hip_graphs(self) -> None:
        self._resolve_stats()
        self._hip_graphs = {}
        # the graphs' private memory pool goes with the last graph that used
        # it: the next capture opens a new one (capturing into a released
        # pool's handle fails inside the caching allocator)
        self._hip_graph_pool = None

    def hip_graph_input(self, x: torch.Tensor) -> torch.Tensor:
        """The static input buffer of the graph that serves inputs shaped like
        x (capturing it first if needed), filled with x.  A caller that writes
        its next input into this buffer and passes it to forward() skips the
        per-call input copy."""
        if not (self._hip_graph_enabled and self._graph_eligible(x)):
            raise RuntimeError("hip_graph_input: graph mode is off or not applicable to this input")
        key = self._graph_key(x)
        ent = self._hip_graphs.get(key)
        if ent is None:
            ent = self._capture_graph(x, key)
        ent["x"].copy_(x)
        return ent["x"]

    def _graph_eligible(self, x: torch.Tensor) -> bool:
        """No host decision of the forward depends on device results: no
        density threshold, memory or latency budget, int8 mode; the nucleus
        head count only where the head count is already at its floor (its
        readback is skipped there); token masks only without a keep
        threshold (the kept count is bounded on the host) and on the
        materialised-candidate path, which reads the exact row count on the
        device."""
        if not (x.dim() == 3 and not self.training and not torch.is_grad_enabled()
                and self._dense_threshold is None and not self.force_dense_when_full
                and not self.linear_mem_budget_mb and self.linear_latency_budget_ms is None
                and not self.quantize_sparse_int8
                and not (self.small_seq_dense and x.shape[1] <= self.small_seq_dense)
                and x.dtype in (torch.float32, torch.bfloat16, torch.float16)):
            return False
        B, T = int(x.shape[0]), int(x.shape[1])
        if self.router_top_p > 0.0 and self._choose_active_k(T) > self.h_active_min:
            return False
        if self.token_sparse:
            if self.token_keep_threshold > 0.0:
                return False
            sims = bool(self.proto_enabled and self.routing_prototypes is not None)
            if self._shortlist_plan(B, T, self._compute_cvt_alpha(T), x.dtype, sims=sims)["structured"]:
                return False
        return True

    _GRAPH_STATE = ("_last_batch_size", "_current_alpha", "_token_keep_ratio_runtime", "_last_target_k",
                    "_last_gate_probs", "_last_token_similarity", "_last_token_blend", "_last_token_importance",
                    "_last_token_mask", "_router_stats", "_proto_sums", "_last_shortlist_lengths",
                    "_last_shortlist_backend_info", "_cached_active_mask", "_cached_packing", "_pending_summary",
                    "last_head_consensus", "last_router_reg", "last_aux_loss")

    def _graph_key(self, x: torch.Tensor):
        T = int(x.shape[1])
        # the graph reads its own contiguous input buffer, into which any
        # layout of x is copied: the key does not depend on x's strides
        return (tuple(x.shape), x.dtype, x.device, float(self._compute_cvt_alpha(T)),
                int(self.linear_L), float(self._linear_L_scale_runtime), self._shortlist_alpha_override,
                str(self.mode_setting), int(self._choose_active_k(T)),
                (float(self.token_keep_ratio_base), int(self.token_keep_min), int(self.token_keep_guard),
                 str(self.linear_token_keep_schedule), int(self.linear_token_keep_ratio_ref),
                 float(self.linear_token_keep_ratio_min), float(self._linear_token_keep_ratio(T)))
                if self.token_sparse else None)

    def _capture_graph(self, x: torch.Tensor, key) -> dict:
        self._resolve_stats()
        device = x.device
        bufs = {n: b.detach().clone() for n, b in self.named_buffers()}
        xs = x.detach().clone(memory_format=torch.contiguous_format)
        timer_on = _hip.TIMER.enabled
        _hip.TIMER.enabled = False
        try:
            side = _side_stream(device, "capture")
            side.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(side):
                # warm-up: library handles, lazy allocations; with the output
                # projection captured it runs here too, so that its GEMM sets
                # up the library's handle and workspace outside the capture
                attn_w = self._forward_impl(xs, capture=True)[0]
                if self._hip_graph_static_output:
                    self.dropout(self.proj(attn_w))
                del attn_w
            torch.cuda.current_stream(device).wait_stream(side)
            with torch.no_grad():
                for n, b in self.named_buffers():
                    b.copy_(bufs[n])
            # the restore bumped the buffers' versions: refresh the int32 gate
            # map now, so that the capture does not record its rebuild
            self._gate_to_head_i32(device)
            if getattr(self, "_hip_graph_pool", None) is None:
                self._hip_graph_pool = torch.cuda.graph_pool_handle()
            graph = torch.cuda.CUDAGraph()
            # cached tensors the captured kernels read (gate map, RoPE tables)
            # are held by the graph: a later rebuild of a cache must not free
            # memory a replay still reads
            self._capture_keep = []
            # no garbage collection inside the capture: a dead object that
            # owns device resources (pinned host memory, events) would be
            # freed while the stream captures, which is not allowed; dead
            # cycles are collected first
            gc.collect()
            gc_was_on = gc.isenabled()
            gc.disable()
            try:
                with torch.cuda.graph(graph, pool=self._hip_graph_pool):
                    attn, stats_args, label = self._forward_impl(xs, capture=True)
                    y_static = self.dropout(self.proj(attn)) if self._hip_graph_static_output else None
            finally:
                if gc_was_on:
                    gc.enable()
            keep = self._capture_keep
        finally:
            _hip.TIMER.enabled = timer_on
            self._capture_keep = None
        ent = {"graph": graph, "x": xs, "attn": attn, "y": y_static, "stats_args": stats_args, "label": label,
               "state": {k: self.__dict__.get(k) for k in self._GRAPH_STATE},
               "sparse_state": self.__dict__.get("_lazy__last_sparse_state"), "keep": keep}
        self._hip_graphs[key] = ent
        return ent

    def _forward_graph(self, x: torch.Tensor) -> torch.Tensor:
        key = self._graph_key(x)
        ent = self._hip_graphs.get(key)
        if ent is None:
            ent = self._capture_graph(x, key)
        ev0 = ev1 = None
        if self.track_latency:
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            ev0.record()
        xs = ent["x"]
        if x.data_ptr() != xs.data_ptr():
            xs.copy_(x)
        ent["graph"].replay()
        y = ent["y"] if ent["y"] is not None else self.dropout(self.proj(ent["attn"]))
        for k, v in ent["state"].items():
            self.__dict__[k] = v
        st = ent["sparse_state"]
        self._last_sparse_state = dict(st) if st is not None else None
        # the latency's end event, recorded after the telemetry copy, also
        # marks that copy done (one event after the replay instead of two)
        self._finish_stats(*ent["stats_args"], done=ev1)
        self._finish_forward(ent["label"], ev0, ev1, ended=ev1 is not None)
        return y

    # ------------------------------------------------------------------
    def _finish_forward(self, label: str, ev0, ev1, ended: bool = False) -> None:
        """Latency and mode labels of this forward, deferred with its other
        statistics (the latency needs the end event; ended: ev1 is already
        recorded)."""
        st_now = self.__dict__.get("_lazy__last_sparse_state")
        if self.track_latency and ev0 is not None:
            if not ended:
                ev1.record()

            def latency(self, st=st_now):
                ev1.synchronize()
                ms = float(ev0.elapsed_time(ev1))
                prev = self.__dict__.get("_lazy__latency_ema")
                self._latency_ema = ms if prev is None else 0.8 * prev + 0.2 * ms
                hs = self.__dict__.get("_lazy_last_head_stats")
                if hs is not None:
                    hs["latency_ms"] = ms
                if st is not None:
                    st["latency_ms"] = ms

            self._defer(latency)

        def labels(self, st=st_now):
            hs = self.__dict__.get("_lazy_last_head_stats")
            if hs is not None:
                hs["mode_setting"] = self.mode_setting
                hs["mode_selected"] = label
            if st is not None:
                st["mode_selected"] = label

        self._defer(labels)

    def _forward_impl(self, x: torch.Tensor, capture: bool = False):
        """The forward (aspa.py:1442-1932).  With capture=True nothing waits
        on the host and the output projection, statistics and latency are
        left to the caller: returns (attn, stats_args, label)."""
        B, T, C = x.shape
        device = x.device
        self.last_aux_loss = None
        self._last_token_importance = None
        self._last_token_mask = None
        self._last_token_blend = None
        if not self.proto_enabled:
            self._last_token_similarity = None
        ev0 = ev1 = None
        if self.track_latency and not capture:
            ev0 = torch.cuda.Event(enable_timing=True)
            ev1 = torch.cuda.Event(enable_timing=True)
            ev0.record()
        self._last_batch_size = B

        def finish(label: str) -> None:
            self._finish_forward(label, ev0, ev1)

        if self.small_seq_dense and T <= self.small_seq_dense:
            y = self._forward_dense_fastpath(x)
            finish("dense_fastpath")
            return y

        # Two streams: the QKV projection, RoPE, the output zero fill and the
        # anchor pass run on a forked stream while the router, packing, the
        # prototype EMA and the prototype prefix tables run on the calling
        # stream; the main attention pass joins them.
        main_s = torch.cuda.current_stream(device)
        fork_s = self._fork_stream(device)
        fork_s.wait_stream(main_s)
        with torch.cuda.stream(fork_s):
            qkv = self.qkv(x).contiguous()  # (B, T, 3C) = (B, T, 3, H, D)

        alpha = self._compute_cvt_alpha(T)
        self._current_alpha = alpha
        if self.token_sparse:
            blend_ratio = (1.0 - alpha) * float(self.token_keep_ratio_base) + alpha * float(self._linear_token_keep_ratio(T))
            self._token_keep_ratio_runtime = float(max(0.0, min(1.0, blend_ratio)))
        else:
            self._token_keep_ratio_runtime = None

        # head count (aspa.py:1574-1589); nucleus count needs head probs, so
        # the router is run with topk chosen after it when top_p > 0.
        dense_topk = self._choose_active_k(T)
        x2d = x.reshape(B * T, C)
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        if x2d.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise ValueError(f"unsupported input dtype {x.dtype}")
        adaptive_topk = dense_topk
        # One router pass ranks dense_topk heads per token (best first); the
        # nucleus / alpha blend below can only shrink k, and the first k of a
        # ranked list are the top-k under the same total order.
        gate, sim, blend, imp, hidx_all, hsc_all = self._route_device(x2d, dense_topk)
        # (when dense_topk is already the floor h_active_min, the nucleus count
        # cannot change k: max(h_min, min(dense_topk, n)) = dense_topk, and
        # its host readback is skipped)
        if self.router_top_p > 0.0 and dense_topk > self.h_active_min:
            head_probs = gate.view(B, T, -1) @ self.gate_to_head_onehot.to(device=device, dtype=gate.dtype)
            nucleus_k = self._nucleus_head_count(head_probs, self.router_top_p, dense_topk)
            adaptive_topk = max(self.h_active_min, min(dense_topk, nucleus_k))
        linear_topk = max(1, min(adaptive_topk, self.linear_head_k))
        topk = max(1, int(round((1.0 - alpha) * float(adaptive_topk) + alpha * float(linear_topk))))
        topk = min(adaptive_topk, topk)
        self._last_target_k = topk
        if topk == dense_topk:
            hidx, hsc = hidx_all, hsc_all
        else:
            hidx = hidx_all[:, :topk].contiguous()
            hsc = hsc_all[:, :topk].contiguous()
        gate_probs = gate.view(B, T, self.attn_gates)
        self._last_gate_probs = gate_probs
        # the prototype EMA (aspa.py:692-718) reads only this forward's router
        # outputs and is read only by the next forward's router: it is queued
        # last before the streams join (on the structured path beside the
        # anchor and main passes, which run on the forked stream)
        heads64 = [None]

        def ema() -> None:
            # the router's tail: the prototype EMA and the telemetry reduction
            # (both read only router outputs; neither is read in this forward)
            self._update_routing_prototypes(x, gate_probs)
            # the int64 active-head list of the sparse state, made here (off the
            # critical path) rather than when the telemetry is read
            heads64[0] = active_heads.to(torch.int64)
            _hip.check(lib.pfa_router_stats_reduce(_hip.ptr(router_stats), int(router_stats.size(0)), _hip.ptr(comb),
                                                   _hip.stream_ptr(device)), "pfa_router_stats_reduce")
        if sim is not None:
            self._last_token_similarity = sim.view(B, T)
            self._last_token_blend = blend.view(B, T)
        else:
            self._last_token_similarity = None
            self._last_token_blend = None
        self._last_proto_stats = None
        importance = imp.view(B, T)
        self._last_token_importance = importance
        token_mask = self._select_active_tokens(importance)
        self._last_token_mask = token_mask

        router_reg = self._router_regulariser(gate_probs)

        # pack rows on the device (mask, active heads, row offsets)
        lib = _hip.lib()
        H = self.h_total
        BH = B * H
        mask8 = torch.empty(BH, T, dtype=torch.uint8, device=device)
        # telemetry for the host in one small buffer (one device-to-host copy):
        # [0:16) the router statistics as 8 float64, [16:20) the packing
        # summary, [20:20+BH) the active heads
        comb = torch.empty(20 + BH, dtype=torch.int32, device=device)
        active_heads = comb[20:]
        router_stats = self._router_stats
        row_offsets = torch.empty(BH + 1, dtype=torch.int32, device=device)
        token_idx = torch.empty(BH * T, dtype=torch.int32, device=device)
        row_head = torch.empty(BH * T, dtype=torch.int32, device=device)
        row_of = torch.empty(BH, T, dtype=torch.int32, device=device)
        summary = comb[16:20]
        ws = _sa._workspace(_sa._size_out(lib.pfa_pack_workspace_size, B, H, T), device)
        tm8 = token_mask.view(torch.uint8) if token_mask is not None else None
        with _hip.TIMER.timed("pack_rows"):
            rc = lib.pfa_pack_rows(_hip.ptr(hidx), topk, _hip.ptr(tm8), B, H, T, _hip.ptr(mask8), _hip.ptr(active_heads),
                               _hip.ptr(row_offsets), _hip.ptr(token_idx), _hip.ptr(row_head), _hip.ptr(row_of),
                               _hip.ptr(summary),
                               _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device))
        _hip.check(rc, "pfa_pack_rows")
        density_threshold = self._density_threshold()
        # The host needs the packing summary only to decide force-dense by
        # density / fullness or when a token mask makes the row count data
        # dependent; otherwise every token has exactly `topk` active rows and
        # the summary is read back with the telemetry at the end (no stall
        # between the router and the attention launches).
        # The int8 mode needs P on the host as well: its per-head EMA buffers
        # have one entry per active head (aspa.py:1347-1357).
        # With a token mask whose kept count is bounded on the host (no
        # threshold: at most keep + guard tokens per batch row) and the
        # materialised-candidate path, the rows are launched for that bound
        # and the kernels read the exact count from the summary on the
        # device (rows_dev); the structured path takes the exact count.
        use_quant = bool(self.quantize_sparse_int8 and not self.training)
        need_summary = density_threshold is not None or self.force_dense_when_full or use_quant
        rows_dev = None
        plan_early = None
        if token_mask is not None and not need_summary:
            cap = self.__dict__.get("_token_keep_cap")
            plan_early = self._shortlist_plan(B, T, alpha, qkv.dtype)
            if cap is None or plan_early["structured"]:
                need_summary = True
            else:
                rows_dev = summary[1:2]
        if need_summary:
            summ = summary.cpu()
            P, N, max_rows = int(summ[0]), int(summ[1]), int(summ[2])
        elif rows_dev is not None:
            P, N, max_rows = -1, B * cap * topk, -1
        else:
            P, N, max_rows = -1, B * T * topk, -1
        self._pending_summary = None if need_summary else summary
        density_est = float(max_rows) / float(max(1, T)) if max_rows >= 0 else 0.0
        all_rows_active = N == BH * T
        prefer_dense = alpha <= self.dense_alpha_cutoff and not self.quantize_sparse_int8
        force_dense, dense_reason = False, None
        if prefer_dense:
            force_dense, dense_reason = True, "alpha"
        if density_threshold is not None and density_est >= density_threshold:
            force_dense = True
            dense_reason = dense_reason or "density"
        elif all_rows_active and self.force_dense_when_full:
            force_dense = True
            dense_reason = dense_reason or "full"
        if alpha >= 0.95:
            if dense_reason == "alpha":
                dense_reason = None
            force_dense = False

        shortlist_path = not force_dense and not (P == 0 or N == 0 or (not need_summary and B * T == 0))
        plan = (plan_early or self._shortlist_plan(B, T, alpha, qkv.dtype)) if shortlist_path else None
        structured = plan is not None and plan["structured"]
        # The structured kernel rotates q rows as it loads them; with anchors
        # and fuse_anchor_pass its anchor pass (on the forked stream) writes
        # the zeros of the rows without a packed row (no zero fill) and, with
        # fuse_k_rope, rotates k as well (no RoPE pass).
        q_fused = structured and self.fuse_q_rope and not use_quant and self.d_head <= 64
        fuse = 0
        if q_fused and self.d_head == 64 and self.fuse_anchor_pass and plan["stride"] > 0 and plan["slots"] > 0:
            fuse = _sa.FUSE_ZERO | (_sa.FUSE_K_ROPE if (self.use_rope and self.fuse_k_rope) else 0)
        with torch.cuda.stream(fork_s):
            rot_k = not (fuse & _sa.FUSE_K_ROPE)
            if fuse:
                attn = torch.empty(B, T, C, dtype=qkv.dtype, device=device)
                q_rope = self._rope_inplace(qkv, rotate_q=not q_fused, rotate_k=rot_k)
            elif q_fused and rot_k:
                # k rotated alone: the same pass writes the output's zeros
                attn = torch.empty(B, T, C, dtype=qkv.dtype, device=device)
                q_rope = self._rope_inplace(qkv, rotate_q=False, rotate_k=True, zero_out=attn)
            else:
                q_rope = self._rope_inplace(qkv, rotate_q=not q_fused, rotate_k=rot_k)
                attn = torch.zeros(B, T, C, dtype=qkv.dtype, device=device)
        if not capture:
            # the forked stream's tensors are used (and freed) on this stream
            qkv.record_stream(main_s)
            attn.record_stream(main_s)
        # The structured path keeps the two streams apart up to the main pass;
        # the others (and the int8 mode, which quantises q/k/v first) join here.
        join_early = not structured or use_quant
        if join_early:
            ema()
            main_s.wait_stream(fork_s)
        D = self.d_head
        mode_label = "sparse"
        if force_dense:
            self._cached_active_mask = None
            self._cached_packing = None
            # a token mask keeps the rows of the kept tokens only; the others
            # stay zero (attn starts zeroed)
            self._attend_dense_causal(qkv, B, T, attn, token_mask=token_mask)
            if dense_reason == "alpha":
                mode_label = "dense_alpha"
            else:
                mode_label = "dense_auto"  # refined to "dense" once P is read back
            _record_backend("hip_dense", device=str(device), heads=BH, tokens=T, max_rows=T, quantized=False)
            self._last_sparse_state = {
                "mode": mode_label, "backend": get_last_backend(), "max_rows": max_rows, "density": density_est,
                "target_k": int(topk),
                "force_dense_threshold": None if density_threshold is None else float(density_threshold),
                "quantized": False, "token_keep_fraction": None, "mode_setting": self.mode_setting,
                "mode_selected": f"cvt(alpha={alpha:.2f})", "shortlist_alpha": float(alpha),
                "dense_reason": dense_reason,
            }
        elif P == 0 or N == 0 or (not need_summary and B * T == 0):
            dense_reason = None
            self._cached_active_mask = None
            self._cached_packing = None
            self._last_sparse_state = {
                "mode": "dense", "backend": "not_invoked", "max_rows": max_rows, "density": density_est,
                "target_k": int(topk),
                "force_dense_threshold": None if density_threshold is None else float(density_threshold),
                "quantized": False, "token_keep_fraction": None, "mode_setting": self.mode_setting,
                "mode_selected": f"cvt(alpha={alpha:.2f})", "shortlist_alpha": float(alpha),
                "dense_reason": dense_reason,
            }
        else:
            dense_reason = None
            mode_label = "shortlist"
            tok = token_idx[:N]
            rh = row_head[:N]
            heads = active_heads[:P] if P >= 0 else active_heads
            self._run_shortlist_device(qkv, attn, B, T, tok, rh, heads, row_offsets, alpha, row_of, summary,
                                       plan=plan, q_rope=q_rope, streams=None if join_early else (main_s, fork_s),
                                       before_join=None if join_early else ema, rows_dev=rows_dev, fuse=fuse)
            backend_info = self._last_shortlist_backend_info or get_last_backend_info()
            state = {
                "mode": mode_label, "backend": str(backend_info.get("name", "shortlist")),
                "active_head_indices": heads if heads64[0] is None else heads64[0], "head_idx": rh,
                "token_idx": tok,
                "row_offsets": row_offsets, "max_rows": int(max_rows), "density": density_est,
                "target_k": int(topk),
                "force_dense_threshold": None if density_threshold is None else float(density_threshold),
                "cache_hit": False, "quantized": bool(self.quantize_sparse_int8 and not self.training),
                "token_keep_fraction": None, "mode_setting": self.mode_setting,
                "mode_selected": f"cvt(alpha={alpha:.2f})", "shortlist_alpha": float(alpha),
                "linear_L": int(self.linear_L), "linear_window": int(self.linear_window),
                "linear_anchor_stride": int(self.linear_anchor_stride),
            }
            state["linear_shortlist_backend"] = backend_info.get("name")
            det = backend_info.get("details")
            if isinstance(det, dict):
                for key, val in det.items():
                    state[f"linear_shortlist_{key}"] = val
            self._last_sparse_state = state
        self.last_head_consensus = None if self.training else attn.detach()
        self.last_router_reg = router_reg
        stats_args = (token_mask, topk, adaptive_topk, P, N, max_rows, density_threshold, alpha, mode_label,
                      dense_reason, B, T, active_heads, row_offsets, summary, comb)
        label = f"cvt(alpha={alpha:.2f})::{mode_label}"
        if capture:
            return attn, stats_args, label
        y = self.dropout(self.proj(attn))

        # the latency's end event also marks the telemetry copy done
        self._finish_stats(*stats_args, done=ev1)
        self._finish_forward(label, ev0, ev1, ended=ev1 is not None)
        if self.linear_mem_budget_mb and device.type == "cuda":
            allocated = torch.cuda.memory_allocated(device) / (1024 * 1024)
            if allocated > self.linear_mem_budget_mb * 1.1:
                self.adjust_linear_L_scale(self.linear_latency_shrink)
            elif allocated < self.linear_mem_budget_mb * 0.6:
                self.adjust_linear_L_scale(self.linear_latency_growth)
        return y

    def _shortlist_plan(self, B: int, T: int, alpha: float, dtype: torch.dtype,
                        sims: Optional[bool] = None) -> Dict[str, Any]:
        """Shortlist sizes of this forward (aspa.py:1175-1210) and whether the
        structured kernel serves it (bf16, D=64, no row truncated).  `sims`:
        whether the router gives prototype similarities (default: whether
        this forward's router gave them)."""
        D = self.d_head
        if sims is None:
            sims = self._last_token_similarity is not None
        runtime = self._prepare_linear_runtime(T, B, alpha)
        L = int(runtime["effective_L"])
        stride = int(runtime["anchor_stride"])
        local_w, slots, proto_cap_val = _sa._resolve_caps(
            L, runtime["window"], stride, self.linear_use_local, self.linear_use_anchors,
            self.linear_use_proto and sims, T, runtime["local_cap"],
            runtime["anchor_cap"], runtime["proto_cap"])
        K = 0
        if self.linear_use_proto and sims and proto_cap_val > 0:
            K = min(L, proto_cap_val, T)
        use_quant = bool(self.quantize_sparse_int8 and not self.training)
        anchors = stride > 0 and slots > 0
        w_eff = max(1, local_w)
        bound = w_eff + ((min(slots, (T - 1) // stride) + 1) if anchors else 0) + K
        structured = (dtype == torch.bfloat16 and D in _sa.STRUCTURED_HEAD_DIMS and bound <= L and K <= 1024
                      and not _hip.env_flag("PFA_FORCE_GENERIC"))
        return {"L": L, "stride": stride, "local_w": local_w, "slots": slots, "K": K, "use_quant": use_quant,
                "w_eff": w_eff, "structured": structured}

    def _fork_stream(self, device: torch.device) -> torch.cuda.Stream:
        """The forward's second stream on `device` (default priority)."""
        return _side_stream(device, "fork")

    def _run_shortlist_device(self, qkv, attn, B, T, token_idx, row_head, heads, row_offsets, alpha, row_of,
                              summary, plan: Optional[Dict[str, Any]] = None, q_rope=None, streams=None,
                              before_join=None, rows_dev: Optional[torch.Tensor] = None, fuse: int = 0) -> None:
        """Candidate attention (aspa.py:1175-1310).

        When no row can be truncated to L, in bf16 with D in
        STRUCTURED_HEAD_DIMS, the candidate sets are used through their structure (window, strided
        anchors, prototype prefix sets) by pfa_shortlist_attn_fwd; otherwise
        the candidates are materialised (pfa_shortlist_build) and attended by
        pfa_sparse_attn_fwd.  Both give the reference's candidate sets.

        streams = (main, fork): qkv and attn come from work queued on the
        fork stream; the structured path queues its anchor pass there too
        (after the packing on main) and then its main pass (after the
        prototype tables, built on main meanwhile), while `before_join()`
        runs on main beside them; main joins the fork stream at the end.
        The other paths are entered with the fork stream already joined.
        The prototype tables are queued before the anchor pass so that, in a
        captured graph, they follow the packing on its queue instead of
        starting on another one.

        rows_dev (materialised path only): a device int32 row count; the
        token_idx / row_head given are then a capacity, valid up to it.

        fuse (structured path with anchors only): FUSE_* bits of the anchor
        pass -- k still unrotated (FUSE_K_ROPE) and attn not zero-filled
        (FUSE_ZERO): the anchor pass does both."""
        H, D = self.h_total, self.d_head
        device = qkv.device
        if plan is None:
            plan = self._shortlist_plan(B, T, alpha, qkv.dtype)
        L, stride, local_w, slots, K = plan["L"], plan["stride"], plan["local_w"], plan["slots"], plan["K"]
        use_quant, w_eff, structured = plan["use_quant"], plan["w_eff"], plan["structured"]
        if q_rope is not None and not structured:
            raise RuntimeError("q rows left unrotated for a path that does not rotate them")
        if fuse and not (structured and stride > 0 and slots > 0 and not use_quant):
            raise RuntimeError("the anchor-pass fusions need the structured path with anchors")
        q5 = qkv.view(B, T, 3, H, D)
        if structured and rows_dev is not None:
            raise RuntimeError("the structured shortlist path takes the exact row count")
        if structured:
            qkv_scales = None
            if use_quant:
                # int8 values in place, as exact bf16 integers; the kernel
                # applies the scales in its tiles
                qkv_scales = self._quantize_qkv(q5, B, T, heads, q5)
            t4 = (_hip.tensor4(q5[:, :, 0], H, "bthd"), _hip.tensor4(q5[:, :, 1], H, "bthd"),
                  _hip.tensor4(q5[:, :, 2], H, "bthd"), _hip.tensor4(attn.view(B, T, H, D), H, "bthd"))
            args = (H, T, D, token_idx, row_head, heads, summary, row_of, w_eff, stride, slots)
            scale = 1.0 / math.sqrt(D)
            part = None
            anchors = stride > 0 and slots > 0
            if anchors:
                part = _sa.shortlist_partials(int(token_idx.numel()), device, D)
            packed = None
            if anchors and streams is not None:
                packed = torch.cuda.Event()
                packed.record(streams[0])  # the packing is done
            # prototype tables on this stream, queued before the anchor pass
            # (which waits only for the packing, not for them)
            blocks = evict = None
            if K > 0:
                blocks, evict = _sa._proto_prefix_blocks(self._last_token_similarity, K)
            if packed is not None:
                # anchor and main pass back to back on the fork stream (one
                # hardware queue: no cross-queue wait between them); the main
                # pass also waits for the prototype tables, queued on this
                # stream, and `before_join` (the tail) runs here beside both
                fork_s = streams[1]
                fork_s.wait_event(packed)
                with torch.cuda.stream(fork_s):
                    _sa._shortlist_attn_structured(*t4, *args, None, None, scale, device, want_lengths=False,
                                                   q_rope=q_rope, passes=1, part=part, fuse=fuse)
                tables = torch.cuda.Event()
                tables.record(streams[0])
                if before_join is not None:
                    before_join()
                fork_s.wait_event(tables)
                with torch.cuda.stream(fork_s):
                    lens = _sa._shortlist_attn_structured(
                        *t4, *args, blocks, evict, scale, device, want_lengths=bool(self.record_shortlist_lengths),
                        q_rope=q_rope, passes=2, part=part, qkv_scales=qkv_scales, fuse=0)
                if lens is not None and not torch.cuda.is_current_stream_capturing():
                    lens.record_stream(streams[0])  # allocated on the fork stream, used and freed on this one
                # join: the forward ends after the main pass
                streams[0].wait_stream(fork_s)
            else:
                if before_join is not None:
                    before_join()
                if streams is not None:
                    streams[0].wait_stream(streams[1])
                lens = _sa._shortlist_attn_structured(
                    *t4, *args, blocks, evict, scale, device, want_lengths=bool(self.record_shortlist_lengths),
                    q_rope=q_rope, passes=3, part=part, qkv_scales=qkv_scales, fuse=fuse)
            self._last_shortlist_lengths = lens
            _record_backend("hip", device=str(device), tokens=T, rows=int(token_idx.numel()), L=L,
                            quantized=use_quant, candidates=True, structured=True)
            self._last_shortlist_backend_info = get_last_backend_info()
            return
        sets = None
        row_batch = None
        if K > 0:
            sets = _sa._proto_prefix_sets(self._last_token_similarity, K)
            if B > 1:
                # rows past a device row count hold arbitrary values: clamp
                # them into range (the builder does not read those rows)
                rh = row_head.clamp(0, heads.numel() - 1) if rows_dev is not None else row_head
                row_batch = (heads.index_select(0, rh) // H).to(torch.int32)
        cand, lens = _sa._shortlist_build_device(token_idx, row_batch, T, L, local_w, stride, slots, sets,
                                                 n_rows_dev=rows_dev)
        self._last_shortlist_lengths = lens
        out4 = _hip.tensor4(attn.view(B, T, H, D), H, "bthd")
        if use_quant:
            # Per-head int8 of the active heads (aspa.py:1258-1267) into an
            # int8 copy of the QKV layout (only the active heads are written
            # or read), attended with the per-global-head scales.
            q8 = torch.empty(B, T, 3, H, D, dtype=torch.int8, device=device)
            scales = self._quantize_qkv(q5, B, T, heads, q8)
            _sa._attn_launch(_hip.tensor4(q8[:, :, 0], H, "bthd"), _hip.tensor4(q8[:, :, 1], H, "bthd"),
                             _hip.tensor4(q8[:, :, 2], H, "bthd"), torch.int8, out4, qkv.dtype, H, T, D, token_idx,
                             row_head, heads, cand, lens, None, None, 1.0 / math.sqrt(D),
                             (scales[0], scales[1], scales[2]), device, n_rows_dev=rows_dev)
        else:
            _sa._attn_launch(_hip.tensor4(q5[:, :, 0], H, "bthd"), _hip.tensor4(q5[:, :, 1], H, "bthd"),
                             _hip.tensor4(q5[:, :, 2], H, "bthd"), qkv.dtype, out4, qkv.dtype, H, T, D, token_idx,
                             row_head, heads, cand, lens, None, None, 1.0 / math.sqrt(D), (None, None, None), device,
                             n_rows_dev=rows_dev)
        _record_backend("hip", device=str(device), tokens=T, rows=int(token_idx.numel()), L=L,
                        quantized=use_quant, candidates=True, structured=False)
        self._last_shortlist_backend_info = get_last_backend_info()

    def _quantize_qkv(self, q5: torch.Tensor, B: int, T: int, heads: torch.Tensor, dst5: torch.Tensor) -> torch.Tensor:
        """Per-head int8 of the P = heads.numel() active heads of q, k and v
        (the (B, T, 3, H, D) view of the projection) into dst5 (int8, or bf16
        integers -- possibly q5 itself); returns the (3, B*H) f32 scales,
        indexed by global head (b*H + h)."""
        H, D = self.h_total, self.d_head
        P = int(heads.numel())
        scales = torch.empty(3, B * H, dtype=torch.float32, device=q5.device)
        for i, name in enumerate(("_quant_ema_q", "_quant_ema_k", "_quant_ema_v")):
            self._quantize_heads(_hip.tensor4(q5[:, :, i], H, "bthd"), q5.dtype, H, T, D, heads, P, None,
                                 _hip.tensor4(dst5[:, :, i], H, "bthd"), dst5.dtype, scales[i], name)
        return scales

    def _router_regulariser(self, gate_probs: torch.Tensor) -> Optional[torch.Tensor]:
        """Router regularisation terms (aspa.py:1543-1573, 1608-1614)."""
        if self.router_reg_lambda <= 0.0:
            return None
        parts = {p.strip() for p in str(self.router_reg_mode or "").lower().replace("|", ",").replace("+", ",").split(",")
                 if p.strip()} or {"entropy"}
        terms = []
        if parts & {"entropy", "ent"}:
            terms.append((gate_probs.clamp_min(1e-9).log() * gate_probs).sum(dim=-1).mean())
        if parts & {"l1", "l_1"}:
            terms.append((gate_probs.sum(dim=-1) ** self.router_reg_beta).mean())
        if not terms:
            return None
        total = terms[0]
        for t in terms[1:]:
            total = total + t
        return self.router_reg_lambda * total

    def _finish_stats(self, token_mask, topk, adaptive_topk, P, N, max_rows, density_threshold, alpha, mode_label,
                      dense_reason, B, T, active_heads, row_offsets, summary, comb, done=None) -> None:
        """Telemetry dictionaries (aspa.py:1857-1916) from the router's
        statistics and the packing summary.  `comb` (the reduced router
        statistics, the summary and the active heads, under a hundred bytes
        for the usual head counts) is copied into pinned host memory without
        waiting -- a large device-to-host copy would make the host wait for
        the device -- and the dictionaries are built when first read (or at
        the next forward), so the forward never stalls the device queue.
        done: an event of the caller's, not yet recorded, that is recorded
        here after the copy (the caller's latency end event), or None."""
        self._resolve_stats()
        H = self.h_total
        with torch.no_grad():
            # one pinned staging tensor, kept across forwards: the previous
            # forward's values were consumed by _resolve_stats above
            h = self.__dict__.get("_stats_host")
            if h is None or h.shape != comb.shape:
                h = torch.empty(comb.shape, dtype=torch.int32, pin_memory=True)
                self.__dict__["_stats_host"] = h
            h.copy_(comb, non_blocking=True)
            host = (h[:16].view(torch.float64), h[16:20], h[20:])
            if done is None:
                done = self.__dict__.get("_stats_event")
                if done is None:
                    done = torch.cuda.Event()
                    self.__dict__["_stats_event"] = done
            done.record()
        # everything the dictionaries need from the host side, as of now
        st = self.__dict__.get("_lazy__last_sparse_state")
        info = self._last_shortlist_backend_info or get_last_backend_info()
        ctx = dict(
            target_k=int(self._last_target_k or topk), linear=(int(self.linear_L), int(self.linear_window),
                                                           int(self.linear_anchor_stride)),
            proto=self._last_token_similarity is not None, mode_setting=self.mode_setting)

        def build(self) -> None:
            nonlocal mode_label
            done.synchronize()
            part = host[0].tolist()
            summ = host[1].tolist()
            ent_sum, sim_sum, blend_sum, blend_pos, score_sum = part[:5]
            P_, N_, max_rows_ = int(summ[0]), int(summ[1]), int(summ[2])
            heads_list = host[2][:P_].tolist()
            n_tok = max(1, B * T)
            density_est = float(max_rows_) / float(max(1, T))
            self._update_density(density_est)
            keep_frac = float(N_) / float(max(1, topk * B * T)) if token_mask is not None else 1.0
            if mode_label == "dense_auto" and P_ == B * H:
                mode_label = "dense"
            if st is not None:
                st["token_keep_fraction"] = keep_frac
                st["max_rows"] = int(max_rows_)
                st["density"] = density_est
                if st.get("mode") == "dense_auto" and mode_label == "dense":
                    st["mode"] = "dense"
                if "active_head_indices" in st:
                    st["active_head_indices"] = st["active_head_indices"][:P_].to(torch.int64)
                    st["row_offsets"] = st["row_offsets"][:P_ + 1]
                if "token_idx" in st:
                    # launched for a row capacity when the count stayed on the device
                    st["token_idx"] = st["token_idx"][:N_]
                    st["head_idx"] = st["head_idx"][:N_]
            hs = {
                "top_k": int(topk),
                "mean_gate_prob": float(score_sum / max(1.0, float(N_))),
                "router_entropy": float(ent_sum / n_tok),
                "mean_active_per_token": float(N_) / float(n_tok),
                "unique_heads": len({int(hb) % H for hb in heads_list}),
                "active_fraction": float(N_) / float(max(1, B * T * H)),
                "max_active_rows": int(max_rows_),
                "max_active_density": float(density_est),
                "target_k": ctx["target_k"],
                "seq_len": int(T),
                "active_min": int(self.h_active_min),
                "active_max": int(self.h_active_max),
                "force_dense_threshold": None if density_threshold is None else float(density_threshold),
                "active_curve": float(self.h_active_curve),
                "token_keep_fraction": keep_frac,
                "mode": mode_label,
                "mode_selected": f"cvt(alpha={alpha:.2f})",
                "shortlist_alpha": float(alpha),
                "router_top_p": float(self.router_top_p),
                "nucleus_k": int(adaptive_topk),
                "top_a_consensus": True,
            }
            if dense_reason is not None:
                hs["dense_reason"] = dense_reason
            if alpha > 0.0:
                hs["linear_L"], hs["linear_window"], hs["linear_anchor_stride"] = ctx["linear"]
                if info.get("name") is not None:
                    hs["linear_shortlist_backend"] = info.get("name")
                    det = info.get("details")
                    if isinstance(det, dict):
                        for key, val in det.items():
                            hs[f"linear_shortlist_{key}"] = val
            proto_stats = None
            if ctx["proto"]:
                proto_stats = {"max_sim_mean": float(sim_sum / n_tok), "blend_mean": float(blend_sum / n_tok),
                               "active_tokens": int(blend_pos)}
                hs["proto"] = dict(proto_stats)
                hs["dna"] = dict(proto_stats)
            self._last_proto_stats = proto_stats
            self.last_head_stats = hs

        self._defer(build)


class AdaptiveSparseProtoAttention(AdaptiveSparseAttention):
    """AdaptiveSparseAttention with prototype routing enabled (aspa.py:1935-1944)."""

    def __init__(self, config: ModelConfig):
        if not getattr(config, "attn_proto_enable", False):
            try:
                setattr(config, "attn_proto_enable", True)
            except Exception:  # noqa: BLE001
                pass
        super().__init__(config)


class AdaptiveSparseAttentionBlock(nn.Module):
    """Pre-norm block around ASPA (aspa.py:1947-1990)."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.ln1 = _build_norm(config)
        if bool(getattr(config, "attn_proto_enable", False)):
            self.attn = AdaptiveSparseProtoAttention(config)
        else:
            self.attn = AdaptiveSparseAttention(config)
        self.ln2 = _build_norm(config)
        self.mlp = MLP(config)
        self._is_moe = False
        self.last_aux_loss = None
        self.last_moe_stats = None
        self.last_router_reg = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln1(x))
        x = x + self.mlp(self.ln2(x))
        self.last_aux_loss = getattr(self.mlp, "last_aux_loss", None)
        self.last_router_reg = getattr(self.attn, "last_router_reg", None)
        self.last_moe_stats = None
        return x

    @property
    def last_head_stats(self) -> Optional[dict]:
        return getattr(self.attn, "last_head_stats", None)

    @property
    def last_sparse_state(self) -> Optional[dict]:
        return getattr(self.attn, "_last_sparse_state", None)
