"""All-query final pass of the chunked shortlist pipeline over an int8
shortlist.

The reference's final pass attends the reduced sequence to itself
(reference chunked_shortlist.py:710-739).  The all-query form kept here lets
every token of the original sequence attend to the shortlisted keys:

* Q: the final model's query projection of all T tokens, RoPE at their own
  positions (written chunk by chunk while the chunks stream through);
* K, V: projections of the S shortlisted tokens, RoPE on K at the tokens'
  original positions, then symmetric int8 per (head, row):
  ``scale = max(absmax / 127, 1e-6)``, ``q = clamp(round(x / scale), ±127)``
  (the per-head scheme of aspa.py:1312-1363 applied per row);
* attention: causal by original position (key j is visible to query t when
  ``key_pos[j] <= t``), dequantised to bf16 inside each LDS tile, bf16 MFMA,
  f32 online softmax; a query with no visible key gets a zero row;
* output: the final model's output projection, ``(1, T, C)``.

Every step is a HIP kernel of libpfa_hip.so except the two projections
(hipBLASLt GEMMs through torch).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from .. import _hip
from ..kernels.sparse_attn import _size_out, _workspace


def quantize_rows_int8(x: torch.Tensor, heads: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """x (S, H*D) (row stride >= H*D, last dim contiguous) -> (int8 (H, S, D),
    f32 scales (H, S)), one symmetric scale per (head, row)."""

    if x.dim() != 2 or x.stride(-1) != 1:
        raise ValueError("x must be a 2-D tensor with a contiguous last dimension")
    device = _hip.require_device(x, what="quantize_rows_int8")
    S, C = x.shape
    if C % heads != 0:
        raise ValueError(f"row width {C} is not a multiple of heads={heads}")
    D = C // heads
    q = torch.empty(heads, S, D, dtype=torch.int8, device=device)
    s = torch.empty(heads, S, dtype=torch.float32, device=device)
    _hip.check(_hip.lib().pfa_quantize_rows_int8(_hip.ptr(x), _hip.dtype_tag(x.dtype), S, x.stride(0), heads, D,
                                                 _hip.ptr(q), _hip.ptr(s), _hip.stream_ptr(device)),
               "pfa_quantize_rows_int8")
    return q, s


def rope_rows_(x: torch.Tensor, heads: int, cos: torch.Tensor, sin: torch.Tensor,
               positions: Optional[torch.Tensor] = None, offset: int = 0) -> torch.Tensor:
    """RoPE in place on the rows of x (n, H*D): row r uses table row
    positions[r] (or offset + r).  Returns x."""

    if x.dim() != 2 or x.stride(-1) != 1:
        raise ValueError("x must be a 2-D tensor with a contiguous last dimension")
    device = _hip.require_device(x, cos, sin, positions, what="rope_rows_")
    n, C = x.shape
    D = C // heads
    if cos.dtype != x.dtype or sin.dtype != x.dtype or cos.shape[-1] != D:
        raise ValueError("RoPE tables must be (T, D) in the tensor dtype")
    pos = None
    if positions is not None:
        if positions.numel() != n:
            raise ValueError("positions must have one entry per row")
        pos = positions.to(torch.int32).contiguous()
        if n > 0 and not (0 <= int(pos.min()) and int(pos.max()) < cos.shape[0]):
            raise ValueError(f"positions must lie in [0, {cos.shape[0]}) (the RoPE table length)")
    elif not (0 <= int(offset) and int(offset) + n <= cos.shape[0]):
        raise ValueError(f"rows {offset}..{int(offset) + n} exceed the RoPE table length {cos.shape[0]}")
    _hip.check(_hip.lib().pfa_rope_rows_inplace(_hip.ptr(x), _hip.dtype_tag(x.dtype), n, x.stride(0), heads, D,
                                                _hip.ptr(cos.contiguous()), _hip.ptr(sin.contiguous()), _hip.ptr(pos),
                                                int(offset), _hip.stream_ptr(device)), "pfa_rope_rows_inplace")
    return x


def int8_shortlist_attention(q: torch.Tensor, k8: torch.Tensor, v8: torch.Tensor, k_scale: torch.Tensor,
                             v_scale: torch.Tensor, key_pos: torch.Tensor, *, causal: bool = True,
                             scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Attention of every query row of q (T, H, D) bf16 (a strided view is
    fine: last dim contiguous) to the int8 shortlist k8/v8 (H, S, D) with
    scales (H, S) and ascending original positions key_pos (S,).  Returns
    out (T, H, D) bf16."""

    if q.dim() != 3 or q.dtype != torch.bfloat16 or q.stride(-1) != 1:
        raise ValueError("q must be a (T, H, D) bf16 tensor with a contiguous last dimension")
    T, H, D = q.shape
    if k8.shape != v8.shape or k8.dim() != 3 or k8.shape[0] != H or k8.shape[2] != D:
        raise ValueError("k8/v8 must be (H, S, D) int8 matching q")
    if k8.dtype != torch.int8 or v8.dtype != torch.int8:
        raise ValueError("k8/v8 must be int8")
    S = k8.shape[1]
    if k_scale.shape != (H, S) or v_scale.shape != (H, S) or key_pos.numel() != S:
        raise ValueError("scales must be (H, S) and key_pos (S,)")
    device = _hip.require_device(q, k8, v8, k_scale, v_scale, key_pos, what="int8_shortlist_attention")
    if out is None:
        out = torch.empty(T, H, D, dtype=torch.bfloat16, device=device)
    if S == 0:
        return out.zero_()
    sc = float(scale) if scale is not None else 1.0 / math.sqrt(D)
    lib = _hip.lib()
    ws = _workspace(_size_out(lib.pfa_int8_kv_attn_workspace_size, T, H, S), device)
    kp = key_pos.to(torch.int32).contiguous()
    t4q = _hip.Tensor4(_hip.ptr(q), 0, q.stride(1), q.stride(0))
    t4o = _hip.Tensor4(_hip.ptr(out), 0, out.stride(1), out.stride(0))
    with _hip.TIMER.timed("int8_kv_attn_fwd"):
        rc = lib.pfa_int8_kv_attn_fwd(t4q, t4o, T, H, D, _hip.ptr(k8.contiguous()), _hip.ptr(v8.contiguous()),
                                      _hip.ptr(k_scale.to(torch.float32).contiguous()),
                                      _hip.ptr(v_scale.to(torch.float32).contiguous()), _hip.ptr(kp), S,
                                      1 if causal else 0, sc, _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device))
    _hip.check(rc, "pfa_int8_kv_attn_fwd")
    return out


class AllQueryFinalPass:
    """Streams the final model's queries chunk by chunk into a resident
    (1, T, C) buffer, then attends all of them to the int8 shortlist."""

    def __init__(self, model, seq_len: int, device: torch.device, dtype: torch.dtype, *, causal: bool = True):
        if dtype != torch.bfloat16:
            raise ValueError("the all-query final pass computes in bf16")
        self.model = model
        self.T = int(seq_len)
        self.C = int(model.d_model)
        self.H = int(model.h_total)
        self.D = self.C // self.H
        if self.D != 64:
            raise ValueError(f"the all-query final pass needs head dim 64 (got {self.D})")
        self.causal = bool(causal)
        self.q_all = torch.empty(1, self.T, self.C, dtype=dtype, device=device)
        self.w_q = model.qkv.weight[: self.C]
        self.w_kv = model.qkv.weight[self.C:]
        self.cos = self.sin = None
        if model.use_rope:
            self.cos, self.sin = model._rope_factors(self.T, device, dtype)

    def add_chunk(self, x_chunk: torch.Tensor, start: int) -> None:
        """x_chunk (1, n, C): project its queries into q_all[:, start:start+n]."""
        n = x_chunk.size(1)
        dst = self.q_all[0, start:start + n]
        torch.matmul(x_chunk[0], self.w_q.t(), out=dst)
        if self.cos is not None:
            rope_rows_(dst, self.H, self.cos, self.sin, offset=start)

    def finish(self, reduced: torch.Tensor, keep_idx: torch.Tensor) -> torch.Tensor:
        """reduced (1, S, C): the shortlisted tokens (sorted by position
        keep_idx).  Returns the final output (1, T, C)."""
        kv = F.linear(reduced[0], self.w_kv)  # (S, 2C)
        k = kv[:, : self.C]
        v = kv[:, self.C:]
        pos = keep_idx.to(device=kv.device, dtype=torch.int32)
        if self.cos is not None:
            rope_rows_(k, self.H, self.cos, self.sin, positions=pos)
        k8, ks = quantize_rows_int8(k, self.H)
        v8, vs = quantize_rows_int8(v, self.H)
        q = self.q_all[0].view(self.T, self.H, self.D)
        attn = int8_shortlist_attention(q, k8, v8, ks, vs, pos, causal=self.causal)
        self.last_shortlist = (k8, ks, v8, vs, pos)
        self.last_attn = attn
        return self.model.proj(attn.view(1, self.T, self.C))


__all__ = ["AllQueryFinalPass", "int8_shortlist_attention", "quantize_rows_int8", "rope_rows_"]
