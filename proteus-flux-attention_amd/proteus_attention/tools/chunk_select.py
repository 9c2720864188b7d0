"""Chunk salience selection and global shortlist merge on the device.

nucleus_select  -- reference chunked_shortlist.py:175-208
finalise        -- reference chunked_shortlist.py:211-254

Both keep the reference's semantics with the tie rule made explicit: equal
scores are ordered by ascending position (the reference's unstable argsort
leaves it open).  Inputs are device tensors; the work is a handful of
device sorts over at most a few thousand (value, index) pairs per call.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch


def _order_desc(values: torch.Tensor) -> torch.Tensor:
    # stable descending sort: ties keep ascending position
    return torch.sort(values, descending=True, stable=True).indices


def nucleus_select(scores: torch.Tensor, max_tokens: int, top_p: float,
                   keep_mask: Optional[torch.Tensor] = None) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
    """Top tokens of one chunk by score with nucleus (top-p) truncation.

    Returns ``(selected_scores, selected_positions)`` in selection order, or
    None when nothing is finite.
    """

    if scores.ndim != 1:
        raise ValueError("scores tensor must be 1-D for nucleus selection.")
    scores = scores.to(torch.float32)
    if keep_mask is not None:
        scores = torch.where(keep_mask.to(torch.bool), scores, torch.full_like(scores, float("-inf")))
    limit = min(int(max_tokens), int(scores.numel()))
    if limit <= 0:
        return None
    finite = torch.isfinite(scores)
    if not bool(finite.any()):
        return None
    safe = torch.where(finite, scores, torch.full_like(scores, -1e9))
    order = _order_desc(safe)
    if top_p >= 1.0:
        keep = limit
    else:
        probs = torch.softmax(safe, dim=-1)[order]
        mass = torch.cumsum(probs, dim=-1)
        keep = int((mass < float(top_p)).sum())
        if keep < order.numel():
            keep += 1
        keep = min(limit, max(1, keep))
    sel = order[:keep]
    return scores[sel], sel


def finalise(scores: torch.Tensor, indices: torch.Tensor, max_tokens: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Global shortlist: one entry per position, the first ``max_tokens``
    entries in descending score order, returned sorted by position (int64,
    with their scores).

    A position listed more than once is represented by its LAST entry in
    score order (its lowest score): the reference sorts the composite key
    ``index*(n+1) - order_position`` ascending and keeps the first of each
    group (chunked_shortlist.py:233-243), which is the latest one.  Chunks
    are disjoint, so in the pipeline itself positions never repeat."""

    order = _order_desc(scores.to(torch.float32))
    s_ord = scores[order]
    i_ord = indices[order].to(torch.long)
    n = i_ord.numel()
    pos = torch.arange(n, device=i_ord.device, dtype=torch.long)
    by_idx = torch.sort(i_ord * (n + 1) - pos).indices
    sorted_idx = i_ord[by_idx]
    first = torch.ones_like(sorted_idx, dtype=torch.bool)
    first[1:] = sorted_idx[1:] != sorted_idx[:-1]
    firsts = torch.sort(by_idx[first]).values[:max_tokens]
    sel_i = i_ord[firsts]
    sel_s = s_ord[firsts]
    back = torch.sort(sel_i).indices
    return sel_i[back], sel_s[back]
