"""Chunk salience selection and global shortlist merge on the device.

nucleus_select  -- reference chunked_shortlist.py:175-208 (and the masking
                   and finite filter of _select_top_tokens, :140-172);
                   nucleus_select_device is the same selection with the
                   count left on the device
finalise        -- reference chunked_shortlist.py:211-254

Both run as HIP kernels of libpfa_hip.so (``pfa_chunk_topk``: radix select
plus an LDS bitonic sort of the selected keys; ``pfa_shortlist_finalise``:
two u64 key sorts and a single-workgroup emit).  The tie rule is made
explicit: equal scores are ordered by ascending position (the reference's
unstable argsort leaves it open).  Inputs are device tensors.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import _hip
from ..kernels.sparse_attn import _size_out, _workspace


def nucleus_select_device(scores: torch.Tensor, max_tokens: int, top_p: float,
                          keep_mask: Optional[torch.Tensor] = None, index_offset: int = 0,
                          drop_nonfinite: bool = False
                          ) -> Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
    """As nucleus_select, with no host synchronisation: (values, indices,
    count) with the buffers sized to min(max_tokens, n) and the count an
    int32 device tensor (entries beyond it are unused), or None when nothing
    can be selected (max_tokens or n is 0)."""

    if scores.ndim != 1:
        raise ValueError("scores tensor must be 1-D for nucleus selection.")
    if not (float(top_p) > 0.0):
        raise ValueError("top_p must be positive")
    device = _hip.require_device(scores, keep_mask, what="nucleus_select")
    n = int(scores.numel())
    limit = min(int(max_tokens), n)
    if limit <= 0:
        return None
    sc = scores.to(torch.float32).contiguous()
    mk = None
    if keep_mask is not None:
        if keep_mask.shape != scores.shape:
            raise ValueError("keep_mask must match scores")
        mk = keep_mask.to(torch.bool).contiguous().view(torch.uint8)
    lib = _hip.lib()
    vals = torch.empty(limit, dtype=torch.float32, device=device)
    idx = torch.empty(limit, dtype=torch.int64, device=device)
    cnt = torch.empty(1, dtype=torch.int32, device=device)
    ws = _workspace(_size_out(lib.pfa_chunk_topk_workspace_size, n, limit), device)
    _hip.check(lib.pfa_chunk_topk(_hip.ptr(sc), _hip.ptr(mk), n, limit, float(top_p), int(index_offset),
                                  1 if drop_nonfinite else 0, _hip.ptr(vals), _hip.ptr(idx), _hip.ptr(cnt),
                                  _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device)), "pfa_chunk_topk")
    return vals, idx, cnt


def nucleus_select(scores: torch.Tensor, max_tokens: int, top_p: float, keep_mask: Optional[torch.Tensor] = None,
                   index_offset: int = 0, drop_nonfinite: bool = False):
    """Reference chunked_shortlist.py:175-208 (+ the masking / finite filter
    of _select_top_tokens, 140-172) on the device: (values, indices) in
    selection order (int64 positions), or None when nothing is finite or
    nothing is selected.  ``drop_nonfinite`` removes selected entries whose
    score is not finite (the filter _select_top_tokens applies).  Reads the
    count back: nucleus_select_device leaves it on the device."""

    out = nucleus_select_device(scores, max_tokens, top_p, keep_mask=keep_mask, index_offset=index_offset,
                                drop_nonfinite=drop_nonfinite)
    if out is None:
        return None
    vals, idx, cnt = out
    c = int(cnt.item())
    if c == 0:
        return None
    return vals[:c], idx[:c]


def finalise(scores: torch.Tensor, indices: torch.Tensor, max_tokens: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Global shortlist: one entry per position, the first ``max_tokens``
    entries in descending score order, returned sorted by position (int64,
    with their scores).

    A position listed more than once is represented by its LAST entry in
    score order (its lowest score): the reference sorts the composite key
    ``index*(n+1) - order_position`` ascending and keeps the first of each
    group (chunked_shortlist.py:233-243), which is the latest one.  Chunks
    are disjoint, so in the pipeline itself positions never repeat."""

    if scores.ndim != 1 or indices.ndim != 1 or scores.numel() != indices.numel():
        raise ValueError("scores and indices must be 1-D tensors of equal length")
    device = _hip.require_device(scores, indices, what="finalise")
    n = int(scores.numel())
    if n == 0:
        raise RuntimeError("No candidate tokens captured during chunking.")
    sc = scores.to(torch.float32).contiguous()
    ix = indices.to(torch.int64).contiguous()
    m = max(0, min(int(max_tokens), n))
    lib = _hip.lib()
    keep_i = torch.empty(max(m, 1), dtype=torch.int64, device=device)
    keep_s = torch.empty(max(m, 1), dtype=torch.float32, device=device)
    cnt = torch.empty(1, dtype=torch.int32, device=device)
    ws = _workspace(_size_out(lib.pfa_shortlist_finalise_workspace_size, n), device)
    _hip.check(lib.pfa_shortlist_finalise(_hip.ptr(sc), _hip.ptr(ix), n, m, _hip.ptr(keep_i), _hip.ptr(keep_s),
                                          _hip.ptr(cnt), _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device)),
               "pfa_shortlist_finalise")
    c = int(cnt.item())
    return keep_i[:c], keep_s[:c]
