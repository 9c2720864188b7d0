"""Timed CPU restatement of the shortlist-mode ASPA forward -- TEST /
BASELINE INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg).

The stages follow the reference forward (aspa.py:1442-1932) with the oracle
functions of this package: router and head top-k, packing, QKV projection
and RoPE, prototype prefix sets + candidate builder (C oracle), candidate
attention (the fallback's per-head gather formulation, sparse_attn.py:
982-1008) and the output projection.  Router, packing and projections run
on every token; the builder and attention run on every `sample_every`-th
packed row and are scaled by the inverse sampled fraction of candidate
work (sum of row lengths).
"""
from __future__ import annotations

import math
import time
from typing import Dict

import numpy as np
import torch
import torch.nn.functional as F

from . import aspa_oracle as O
from . import c_oracle


def shortlist_forward_seconds(x: torch.Tensor, w: Dict[str, torch.Tensor], *, H: int, L: int, local_w: int,
                              stride: int, slots: int, K: int, sample_every: int = 16,
                              row_chunk: int = 2048) -> Dict[str, float]:
    """x: (1, T, C) in the compute dtype.  Returns per-stage and total
    seconds (sampled stages already extrapolated)."""

    B, T, C = x.shape
    D = C // H
    dt = x.dtype
    t = {}
    s0 = time.perf_counter()
    gate, sim, blend, imp = O.route_tokens(x, w["w_router"].to(dt), w["protos"].to(dt), torch.zeros(H, dtype=dt),
                                           None, proto_temp=0.2, proto_threshold=0.25, proto_blend=0.6,
                                           usage_boost=0.0)
    _, hidx = O.topk_lowest(gate.view(B * T, -1), 2)
    t["router"] = time.perf_counter() - s0

    s0 = time.perf_counter()
    mask = torch.zeros(B * T, H, dtype=torch.bool)
    mask.scatter_(1, hidx, True)
    mask = mask.view(B, T, H).permute(0, 2, 1).reshape(B * H, T)
    head_idx, token_idx, offs, _ = O.pack_active_rows(mask)
    t["pack"] = time.perf_counter() - s0

    s0 = time.perf_counter()
    qkv = F.linear(x, w["w_qkv"].to(dt)).view(B, T, 3, H, D)
    cos, sin = O.rope_tables(T, D, 10000.0, dt)
    q = O.apply_rope(qkv[:, :, 0], cos, sin)
    k = O.apply_rope(qkv[:, :, 1], cos, sin)
    v = qkv[:, :, 2]
    qh, kh, vh = (a.permute(0, 2, 1, 3).reshape(B * H, T, D) for a in (q, k, v))
    t["qkv_rope"] = time.perf_counter() - s0

    sel = np.arange(0, token_idx.numel(), sample_every)
    rows = token_idx.numpy().astype(np.int32)[sel]
    s0 = time.perf_counter()
    cand, lens = c_oracle.shortlist_build(rows, None, T, L, local_w, stride, slots, sim.view(B, T).numpy(), K)
    t_build = time.perf_counter() - s0
    frac = len(sel) / token_idx.numel()
    t["builder"] = t_build / frac

    s0 = time.perf_counter()
    hsel = head_idx[sel]
    ct = torch.from_numpy(cand).long()
    lt = torch.from_numpy(lens).long()
    for h in torch.unique(hsel).tolist():
        mh = (hsel == h).nonzero(as_tuple=True)[0]
        # rows in chunks: the gathered K/V of a chunk is chunk * L * D each
        for c0 in range(0, mh.numel(), row_chunk):
            m = mh[c0:c0 + row_chunk]
            toks = token_idx[sel][m]
            qs = qh[h][toks]
            cr, lr = ct[m], lt[m]
            ks, vs = kh[h][cr], vh[h][cr]
            inval = torch.arange(L)[None, :] >= lr[:, None]
            sc = torch.einsum("rd,rld->rl", qs, ks.masked_fill(inval[..., None], 0.0)) * (1.0 / math.sqrt(D))
            p = torch.softmax(sc.masked_fill(inval, float("-inf")), -1)
            torch.bmm(p.unsqueeze(1), vs.masked_fill(inval[..., None], 0.0))
    t["attention"] = (time.perf_counter() - s0) / frac

    s0 = time.perf_counter()
    attn = torch.zeros(B, T, C, dtype=dt)
    F.linear(attn, w["w_proj"].to(dt))
    t["proj"] = time.perf_counter() - s0
    t["total"] = sum(t.values())
    t["sample_fraction"] = frac
    return t
