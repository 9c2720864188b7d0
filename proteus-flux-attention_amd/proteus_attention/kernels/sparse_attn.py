"""Operator API of the ASPA sparse attention path, backed by libpfa_hip.so.

Public names and argument meaning follow the reference operator module
(``src/proteus_attention/kernels/sparse_attn.py``):

* :func:`aspa_sparse_attention`            (reference sparse_attn.py:1373-1646)
* :func:`build_shortlist_candidates`       (reference sparse_attn.py:376-454)
* :func:`build_packed_shortlist_candidates` (reference sparse_attn.py:457-596)
* :func:`_pack_active_rows`                (reference sparse_attn.py:924-947)
* :func:`get_last_backend` / :func:`get_last_backend_info` (sparse_attn.py:64-85)

All compute runs in hand-written HIP kernels for gfx950.  There is no Triton,
no PyTorch fallback and no CPU execution: CPU tensors raise
:class:`~proteus_attention._hip.HipLibraryError`.  Ties in every top-k go to
the lowest index.  Training-mode attention dropout is not provided (this is
the inference forward path) and raises ``NotImplementedError``.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

from .. import _hip

TRITON_AVAILABLE = False
TRITON_SEQ_LEN_LIMIT = 0

_LAST_BACKEND_INFO: Dict[str, object] = {"name": "uninitialized", "details": {}}


def _record_backend(name: str, **details: object) -> None:
    global _LAST_BACKEND_INFO
    _LAST_BACKEND_INFO = {"name": name, "details": details}


def get_last_backend() -> str:
    """Return the name of the backend used by the most recent call."""

    return str(_LAST_BACKEND_INFO.get("name", "uninitialized"))


def get_last_backend_info() -> Dict[str, object]:
    """Return a shallow copy of the most recent backend metadata."""

    info = dict(_LAST_BACKEND_INFO)
    details = info.get("details")
    if isinstance(details, dict):
        info["details"] = dict(details)
    return info


# ---------------------------------------------------------------------------
# workspace helpers
# ---------------------------------------------------------------------------

def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def _size_out(fn, *args) -> int:
    out = _hip.ctypes.c_size_t(0)
    _hip.check(fn(*args, _hip.ctypes.byref(out)), fn.__name__)
    return int(out.value)


# ---------------------------------------------------------------------------
# packing
# ---------------------------------------------------------------------------

def _pack_mask_i32(mask_bool: torch.Tensor):
    """Pack a (P, T) mask on the device.

    Returns (token_idx int32 (N,), row_head int32 (N,), row_offsets int32
    (P+1,), N, max_rows).  One small device->host copy reads N and max_rows,
    as the reference does with ``.item()``.
    """

    lib = _hip.lib()
    device = mask_bool.device
    P, T = mask_bool.shape
    m8 = mask_bool.to(torch.uint8).contiguous()
    ws = _workspace(_size_out(lib.pfa_pack_workspace_size, 1, P, T), device)
    row_offsets = torch.empty(P + 1, dtype=torch.int32, device=device)
    token_idx = torch.empty(P * T, dtype=torch.int32, device=device)
    row_head = torch.empty(P * T, dtype=torch.int32, device=device)
    summary = torch.empty(4, dtype=torch.int32, device=device)
    rc = lib.pfa_pack_mask(_hip.ptr(m8), P, T, _hip.ptr(row_offsets), _hip.ptr(token_idx), _hip.ptr(row_head),
                           _hip.ptr(summary), _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device))
    _hip.check(rc, "pfa_pack_mask")
    s = summary.cpu()
    n, max_rows = int(s[1]), int(s[2])
    return token_idx[:n], row_head[:n], row_offsets, n, max_rows


def _pack_active_rows(
    active_mask: torch.Tensor,
) -> Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]]:
    """Pack active (head, token) pairs for sparse processing.

    Same contract as the reference (sparse_attn.py:924-947): returns
    ``(head_idx int64, token_idx int64, row_offsets int32, max_rows)`` or
    ``None`` when nothing is active.
    """

    if active_mask.dim() != 2:
        raise ValueError("active_mask must have rank 2 after squeeze")
    _hip.require_device(active_mask, what="_pack_active_rows")
    token_idx, row_head, row_offsets, n, max_rows = _pack_mask_i32(active_mask.to(torch.bool))
    if n == 0:
        return None
    return row_head.to(torch.int64), token_idx.to(torch.int64), row_offsets, max_rows


# ---------------------------------------------------------------------------
# shortlist candidates
# ---------------------------------------------------------------------------

# Largest prototype set the prefix kernels keep (their sorted lists live in
# LDS); the reference accepts any proto_cap (sparse_attn.py:260-300).
MAX_PROTO_CANDIDATES = 2048


def _check_proto_k(K: int) -> None:
    if K > MAX_PROTO_CANDIDATES:
        raise ValueError(f"prototype candidates per row: min(max_candidates, proto_cap, seq_len) = {K} exceeds "
                         f"the {MAX_PROTO_CANDIDATES} this build supports")


def _proto_prefix_sets(scores: torch.Tensor, K: int, with_evict: bool = False):
    """Per (batch, token) the top-min(t+1, K) score positions <= t, sorted.

    scores: (B, T_s) f32 on the device.  Returns (B, T_s, K) int32, and with
    ``with_evict`` also the (B, T_s) int32 eviction tokens.
    """

    _check_proto_k(K)
    lib = _hip.lib()
    device = scores.device
    scores = scores.to(torch.float32).contiguous()
    B, Ts = scores.shape
    ws = _workspace(_size_out(lib.pfa_proto_prefix_workspace_size, B, Ts, K), device)
    sets = torch.empty(B, Ts, K, dtype=torch.int32, device=device)
    evict = torch.empty(B, Ts, dtype=torch.int32, device=device) if with_evict else None
    with _hip.TIMER.timed("proto_prefix_topk"):
        rc = lib.pfa_proto_prefix_topk(_hip.ptr(scores), B, Ts, scores.stride(0), K, _hip.ptr(sets), _hip.ptr(evict),
                                       _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device))
    _hip.check(rc, "pfa_proto_prefix_topk")
    return (sets, evict) if with_evict else sets


def _proto_prefix_blocks(scores: torch.Tensor, K: int):
    """Compact form of the prototype prefix sets: per (batch, 64-token block
    j) the set of token 64j-1 sorted by index (INT32_MAX-padded), and per
    token the eviction token evict[p] (p is in the set of t exactly when
    p <= t < evict[p]).  Returns ((B, ceil(T/64), K), (B, T)) int32."""

    _check_proto_k(K)
    lib = _hip.lib()
    device = scores.device
    scores = scores.to(torch.float32).contiguous()
    B, Ts = scores.shape
    ws = _workspace(_size_out(lib.pfa_proto_prefix_workspace_size, B, Ts, K), device)
    blocks = torch.empty(B, (Ts + 63) // 64, K, dtype=torch.int32, device=device)
    evict = torch.empty(B, Ts, dtype=torch.int32, device=device)
    with _hip.TIMER.timed("proto_prefix_blocks"):
        rc = lib.pfa_proto_prefix_blocks(_hip.ptr(scores), B, Ts, scores.stride(0), K, _hip.ptr(blocks),
                                         _hip.ptr(evict), _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device))
    _hip.check(rc, "pfa_proto_prefix_blocks")
    return blocks, evict


def _resolve_caps(max_candidates, linear_window, anchor_stride, use_local, use_anchors, has_proto, seq_len,
                  local_cap, anchor_cap, proto_cap):
    """Cap resolution of sparse_attn.py:395-397 / 476-490 and the piece
    sizes of sparse_attn.py:411-424."""

    local_cap_val = max(0, int(local_cap)) if local_cap is not None else (max_candidates if use_local else 0)
    anchor_cap_val = max(0, int(anchor_cap)) if anchor_cap is not None else (max_candidates if use_anchors else 0)
    proto_cap_val = max(0, int(proto_cap)) if proto_cap is not None else (max_candidates if has_proto else 0)
    local_w = 0
    if use_local and local_cap_val > 0:
        local_w = max(0, min(int(linear_window), int(max_candidates), local_cap_val))
    slots = 0
    if use_anchors and anchor_stride > 0 and anchor_cap_val > 0:
        slots = max(0, min(anchor_cap_val, int(max_candidates), max(1, int(seq_len))))
    return local_w, slots, proto_cap_val


def _shortlist_build_device(
    rows_i32: torch.Tensor,
    row_batch_i32: Optional[torch.Tensor],
    seq_len: int,
    L: int,
    local_w: int,
    anchor_stride: int,
    slots: int,
    proto_sets: Optional[torch.Tensor],
    extra: Optional[torch.Tensor] = None,
    extra_len: Optional[torch.Tensor] = None,
    out_dtype: torch.dtype = torch.int32,
    len_dtype: torch.dtype = torch.int32,
    n_rows_dev: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Candidate lists of the rows (pfa_shortlist_build).  With n_rows_dev
    (a device int32 row count) only rows [0, min(N, count)) are built; the
    rest of cand / lens is left unwritten."""
    lib = _hip.lib()
    device = rows_i32.device
    N = rows_i32.numel()
    cand = torch.empty(N, L, dtype=out_dtype, device=device)
    lens = torch.empty(N, dtype=len_dtype, device=device)
    K = int(proto_sets.size(2)) if proto_sets is not None else 0
    plen = int(proto_sets.size(1)) if proto_sets is not None else 0
    ew = int(extra.size(1)) if extra is not None else 0
    with _hip.TIMER.timed("shortlist_build"):
        rc = lib.pfa_shortlist_build(
        _hip.ptr(rows_i32), _hip.ptr(row_batch_i32), N, _hip.ptr(n_rows_dev), int(seq_len), int(L), int(local_w), int(anchor_stride),
        int(slots), _hip.ptr(proto_sets), K, plen, _hip.ptr(extra), _hip.ptr(extra_len), ew, _hip.ptr(cand),
        1 if out_dtype == torch.int64 else 0, _hip.ptr(lens), 1 if len_dtype == torch.int64 else 0,
        _hip.stream_ptr(device))
    _hip.check(rc, "pfa_shortlist_build")
    return cand, lens


def _check_rows(rows: torch.Tensor, seq_len: int, what: str) -> None:
    lo, hi = torch.aminmax(rows)
    lo_i, hi_i = int(lo), int(hi)
    if lo_i < 0 or hi_i >= seq_len:
        raise ValueError(f"{what}: rows must lie in [0, seq_len) (got [{lo_i}, {hi_i}] with seq_len={seq_len})")


def build_shortlist_candidates(
    rows: torch.Tensor,
    seq_len: int,
    *,
    max_candidates: int,
    linear_window: int,
    anchor_stride: int,
    use_local: bool,
    use_anchors: bool,
    proto_scores: Optional[torch.Tensor] = None,
    local_cap: Optional[int] = None,
    anchor_cap: Optional[int] = None,
    proto_cap: Optional[int] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row shortlist candidates for one group of rows.

    Reference: sparse_attn.py:376-454.  Output ``(cand (N, max_candidates),
    lengths (N,) int64)``; ``cand`` has ``rows.dtype``.
    """

    if rows.numel() == 0 or max_candidates <= 0:
        empty = rows.new_empty(rows.shape + (0,))
        return empty, rows.new_zeros(rows.shape, dtype=torch.long)
    device = _hip.require_device(rows, proto_scores, what="build_shortlist_candidates")
    _check_rows(rows, seq_len, "build_shortlist_candidates")
    proto = None
    if proto_scores is not None and proto_scores.numel() > 0:
        proto = proto_scores.detach().to(device=device, dtype=torch.float32)[:seq_len]
        proto = proto.reshape(-1) if proto.dim() != 1 else proto
        if proto.numel() == 0:
            proto = None
    local_w, slots, proto_cap_val = _resolve_caps(max_candidates, linear_window, anchor_stride, use_local,
                                                  use_anchors, proto is not None, seq_len, local_cap, anchor_cap,
                                                  proto_cap)
    sets = None
    if proto is not None and proto_cap_val > 0:
        K = min(int(max_candidates), proto_cap_val, proto.numel())
        if K > 0:
            sets = _proto_prefix_sets(proto.unsqueeze(0), K)
    rows_i32 = rows.to(torch.int32).contiguous()
    out_dtype = torch.int64 if rows.dtype == torch.int64 else torch.int32
    cand, lens = _shortlist_build_device(rows_i32, None, seq_len, int(max_candidates), local_w, anchor_stride, slots,
                                         sets, out_dtype=out_dtype, len_dtype=torch.int64)
    if cand.dtype != rows.dtype:
        cand = cand.to(rows.dtype)
    _record_backend("hip", op="build_shortlist_candidates", rows=int(rows.numel()), L=int(max_candidates))
    return cand, lens


def build_packed_shortlist_candidates(
    rows: torch.Tensor,
    row_batch_ids: Optional[torch.Tensor],
    seq_len: int,
    *,
    max_candidates: int,
    linear_window: int,
    anchor_stride: int,
    use_local: bool,
    use_anchors: bool,
    proto_scores: Optional[torch.Tensor] = None,
    local_cap: Optional[int] = None,
    anchor_cap: Optional[int] = None,
    proto_cap: Optional[int] = None,
    chunk_size: int = 4096,
    extra_candidates: Optional[torch.Tensor] = None,
    extra_lengths: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Shortlist candidates for packed rows spanning heads and batches.

    Reference: sparse_attn.py:457-596.  ``row_batch_ids`` selects the row of
    ``proto_scores`` (shape ``(B, T)`` or ``(T,)``) each packed row uses.
    ``chunk_size`` is accepted for signature compatibility; the device
    builder processes every row in one launch.
    """

    if rows.numel() == 0 or max_candidates <= 0:
        empty = rows.new_empty(rows.shape + (0,))
        return empty, rows.new_zeros(rows.shape, dtype=torch.long)
    device = _hip.require_device(rows, row_batch_ids, proto_scores, extra_candidates, what="build_packed_shortlist_candidates")
    _check_rows(rows, seq_len, "build_packed_shortlist_candidates")
    local_w, slots, proto_cap_val = _resolve_caps(max_candidates, linear_window, anchor_stride, use_local,
                                                  use_anchors, proto_scores is not None, seq_len, local_cap,
                                                  anchor_cap, proto_cap)
    sets = None
    rb = None
    if proto_scores is not None and proto_cap_val > 0 and proto_scores.numel() > 0:
        ps = proto_scores.detach().to(device=device, dtype=torch.float32)
        if ps.dim() == 1:
            ps = ps.unsqueeze(0)
        ps = ps[:, :seq_len]
        if row_batch_ids is None:
            rb = None  # batch 0 for every row (reference warns when B > 1)
        else:
            rb = row_batch_ids.to(device=device, dtype=torch.int32).contiguous()
        K = min(int(max_candidates), proto_cap_val, int(seq_len), int(ps.size(1)))
        if K > 0:
            sets = _proto_prefix_sets(ps, K)
    extra = extra_len = None
    if extra_candidates is not None and extra_candidates.numel() > 0:
        extra = extra_candidates.to(device=device, dtype=torch.int32).contiguous()
        if extra_lengths is not None:
            extra_len = extra_lengths.to(device=device, dtype=torch.int32).contiguous()
    rows_i32 = rows.to(torch.int32).contiguous()
    out_dtype = torch.int64 if rows.dtype == torch.int64 else torch.int32
    cand, lens = _shortlist_build_device(rows_i32, rb, seq_len, int(max_candidates), local_w, anchor_stride, slots,
                                         sets, extra, extra_len, out_dtype=out_dtype, len_dtype=torch.int64)
    if cand.dtype != rows.dtype:
        cand = cand.to(rows.dtype)
    _record_backend("hip", op="build_packed_shortlist_candidates", rows=int(rows.numel()), L=int(max_candidates))
    return cand, lens


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def _attn_launch(
    q4: "_hip.Tensor4",
    k4: "_hip.Tensor4",
    v4: "_hip.Tensor4",
    in_dtype: torch.dtype,
    out4: "_hip.Tensor4",
    out_dtype: torch.dtype,
    H: int,
    T: int,
    D: int,
    token_idx: torch.Tensor,
    row_head: torch.Tensor,
    head_map: Optional[torch.Tensor],
    cand: Optional[torch.Tensor],
    cand_len: Optional[torch.Tensor],
    mask: Optional[torch.Tensor],
    head_max: Optional[torch.Tensor],
    scale: float,
    scales: Tuple[Optional[torch.Tensor], Optional[torch.Tensor], Optional[torch.Tensor]],
    device: torch.device,
    n_rows_dev: Optional[torch.Tensor] = None,
) -> None:
    lib = _hip.lib()
    mask_tag = _hip.dtype_tag(mask.dtype) if mask is not None else 0
    with _hip.TIMER.timed("sparse_attn_fwd"):
        rc = lib.pfa_sparse_attn_fwd(
        q4, k4, v4, _hip.dtype_tag(in_dtype), out4, _hip.dtype_tag(out_dtype), int(H), int(T), int(D),
        _hip.ptr(token_idx), _hip.ptr(row_head), _hip.ptr(head_map), int(token_idx.numel()), _hip.ptr(n_rows_dev),
        _hip.ptr(cand),
        int(cand.stride(0)) if cand is not None else 0, _hip.ptr(cand_len), _hip.ptr(mask), mask_tag,
        _hip.ptr(head_max), float(scale), _hip.ptr(scales[0]), _hip.ptr(scales[1]), _hip.ptr(scales[2]),
        _hip.stream_ptr(device))
    _hip.check(rc, "pfa_sparse_attn_fwd")


def shortlist_partials(N: int, device: torch.device, D: int = 64) -> torch.Tensor:
    """f32 (N, pfa_shortlist_attn_part_floats_for(D)) anchor-pass partials."""
    return torch.empty(N, int(_hip.lib().pfa_shortlist_attn_part_floats_for(int(D))), dtype=torch.float32,
                       device=device)


# pfa_shortlist_attn_fwd_fused bits (include/pfa_hip.h)
FUSE_K_ROPE = 1
FUSE_ZERO = 2


def _shortlist_attn_structured(
    q4: "_hip.Tensor4",
    k4: "_hip.Tensor4",
    v4: "_hip.Tensor4",
    out4: "_hip.Tensor4",
    H: int,
    T: int,
    D: int,
    token_idx: torch.Tensor,
    row_head: torch.Tensor,
    head_map: torch.Tensor,
    summary: torch.Tensor,
    row_of: torch.Tensor,
    local_w: int,
    stride: int,
    slots: int,
    blocks: Optional[torch.Tensor],
    evict: Optional[torch.Tensor],
    scale: float,
    device: torch.device,
    want_lengths: bool = True,
    q_rope: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    passes: int = 3,
    part: Optional[torch.Tensor] = None,
    qkv_scales: Optional[torch.Tensor] = None,
    fuse: int = 0,
) -> Optional[torch.Tensor]:
    """Module-path shortlist attention without materialised candidates
    (bf16, D in STRUCTURED_HEAD_DIMS); the prototype sets come as _proto_prefix_blocks tables of
    the T-token scores.  Returns each row's candidate count (int32, (N,)),
    or None when want_lengths is False (the kernel then skips the counting).
    q_rope = (cos, sin) bf16 (T, D) tables (D <= 64): q is still unrotated and its
    rows are rotated as the kernel loads them.  passes = 1 runs only the
    anchor pass and 2 only the main pass (the caller orders them and passes
    the same `part`, from shortlist_partials, to both); 3 runs both.
    qkv_scales: (3, B*H) f32 per-head int8 scales of q, k, v (the tensors
    then hold the int8 values as bf16, from quantize_heads_int8), or None.
    fuse: FUSE_K_ROPE | FUSE_ZERO bits for pfa_shortlist_attn_fwd_fused (the
    anchor pass rotates k of the active heads with the q_rope tables and
    zeroes the out rows without a packed row); needs anchors, passes 1 or 3,
    head_map from the packing (ascending, B*H entries) and no int8 scales."""

    lib = _hip.lib()
    N = int(token_idx.numel())
    lengths = torch.empty(N, dtype=torch.int32, device=device) if (want_lengths and passes & 2) else None
    anchors = stride > 0 and slots > 0
    if anchors and part is None:
        if passes != 3:
            raise ValueError("split anchor/main passes need a shared partials buffer")
        part = shortlist_partials(N, device, D)
    if anchors:
        pw = int(_hip.lib().pfa_shortlist_attn_part_floats_for(int(D)))
        if part.dtype != torch.float32 or part.dim() != 2 or part.size(0) < N or part.size(1) != pw \
                or not part.is_contiguous():
            raise ValueError(f"partials must be contiguous f32 (>= {N}, {pw}) for D = {D}")
    K = 0
    if blocks is not None:
        K = int(blocks.size(2))
        if evict is None or int(evict.size(1)) != int(T) or int(blocks.size(1)) != (int(T) + 63) // 64:
            raise ValueError("prototype block tables must cover the T tokens of the sequence")
    rc_cos = rc_sin = None
    if (q_rope is not None and int(D) > 64) or (fuse and int(D) != 64):
        raise ValueError("q RoPE on load needs D <= 64 and the anchor-pass fusions D = 64")
    if q_rope is not None:
        rc_cos, rc_sin = q_rope
        if (rc_cos.dtype != torch.bfloat16 or rc_sin.dtype != torch.bfloat16 or tuple(rc_cos.shape) != (int(T), int(D))
                or tuple(rc_sin.shape) != (int(T), int(D)) or not rc_cos.is_contiguous()
                or not rc_sin.is_contiguous()):
            raise ValueError("q_rope tables must be contiguous bf16 (T, D)")
    if fuse:
        if qkv_scales is not None:
            raise ValueError("the fused anchor pass has no int8 mode")
        with _hip.TIMER.timed("shortlist_attn_fwd"):
            rc = lib.pfa_shortlist_attn_fwd_fused(
                q4, k4, v4, out4, _hip.PFA_BF16, int(H), int(T), int(D), _hip.ptr(token_idx), _hip.ptr(row_head),
                _hip.ptr(head_map), N, int(head_map.numel()), _hip.ptr(summary), _hip.ptr(row_of), int(local_w),
                int(stride), int(slots), _hip.ptr(blocks), K, _hip.ptr(evict), float(scale), _hip.ptr(part),
                _hip.ptr(lengths), _hip.ptr(rc_cos), _hip.ptr(rc_sin), int(passes), int(fuse),
                _hip.stream_ptr(device))
        _hip.check(rc, "pfa_shortlist_attn_fwd_fused")
        return lengths
    with _hip.TIMER.timed("shortlist_attn_fwd"):
        rc = lib.pfa_shortlist_attn_fwd(
            q4, k4, v4, out4, _hip.PFA_BF16, int(H), int(T), int(D), _hip.ptr(token_idx), _hip.ptr(row_head),
            _hip.ptr(head_map), N, int(head_map.numel()), _hip.ptr(summary), _hip.ptr(row_of), int(local_w),
            int(stride), int(slots), _hip.ptr(blocks), K, _hip.ptr(evict), float(scale), _hip.ptr(part),
            _hip.ptr(lengths), _hip.ptr(rc_cos), _hip.ptr(rc_sin),
            *((None, None, None) if qkv_scales is None else (_hip.ptr(qkv_scales[0]), _hip.ptr(qkv_scales[1]),
                                                             _hip.ptr(qkv_scales[2]))),
            int(passes), _hip.stream_ptr(device))
    _hip.check(rc, "pfa_shortlist_attn_fwd")
    return lengths


# Head dims of the structured MFMA kernel: rows of 16 or 32 elements are
# attended as 64-wide rows whose q dims past D are zero, rows of 128 as two
# 64-dim halves of each tile.
STRUCTURED_HEAD_DIMS = (16, 32, 64, 128)


def _mfma_causal_ok(dtype: torch.dtype, D: int, *t4s: "_hip.Tensor4") -> bool:
    """The structured MFMA kernel serves bf16, D in STRUCTURED_HEAD_DIMS,
    16-byte aligned rows."""
    if dtype != torch.bfloat16 or D not in STRUCTURED_HEAD_DIMS:
        return False
    for t in t4s:
        if int(t.ptr or 0) % 16 or t.s_b % 8 or t.s_h % 8 or t.s_t % 8 or t.s_t <= 0 or t.s_t >= 2 ** 31:
            return False
    return True


def _causal_attn_mfma(q4, k4, v4, out4, H: int, T: int, D: int, token_idx: torch.Tensor, row_head: torch.Tensor,
                      head_map: Optional[torch.Tensor], device: torch.device) -> None:
    """Implicit-causal attention (row r attends to keys 0..token_idx[r] of its
    head) on the structured MFMA kernel: a window that covers the whole
    sequence, no anchors and no prototype keys.  Rows must be ordered by
    (head, token), as the packing writes them; 64 consecutive rows of a head
    form one flash-attention tile of queries that streams its key tiles
    0..t_last once (reference: the causal SDPA of sparse_attn.py:1016-1043
    and the dense paths of aspa.py:1365-1440, 1664-1701)."""

    lib = _hip.lib()
    N = int(token_idx.numel())
    summary = torch.zeros(4, dtype=torch.int32, device=device)  # read only by the anchor pass (off here)
    with _hip.TIMER.timed("causal_attn_mfma"):
        rc = lib.pfa_shortlist_attn_fwd(
            q4, k4, v4, out4, _hip.PFA_BF16, int(H), int(T), int(D), _hip.ptr(token_idx), _hip.ptr(row_head),
            _hip.ptr(head_map), N, 1 if head_map is None else int(head_map.numel()), _hip.ptr(summary), None,
            int(T), 0, 0, None, 0, None, float(1.0 / math.sqrt(D)), None, None, None, None, None, None, None, 2,
            _hip.stream_ptr(device))
    _hip.check(rc, "pfa_shortlist_attn_fwd (causal)")


_QUANT_MODES = {"max": 0, "percentile": 1, "ema_percentile": 2}


def quantize_heads_int8(
    x4: "_hip.Tensor4",
    dtype: torch.dtype,
    H: int,
    T: int,
    D: int,
    head_map: Optional[torch.Tensor],
    P_cap: int,
    summary: Optional[torch.Tensor],
    mode: str,
    percentile: float,
    ema_decay: float,
    ema: Optional[torch.Tensor],
    ema_valid: bool,
    dst4: "_hip.Tensor4",
    dst_dtype: torch.dtype,
    scales: torch.Tensor,
    device: torch.device,
) -> None:
    """Per-head symmetric int8 of the active heads (reference aspa.py:1312-1363)
    on the device: scales[b*H+h] and the int8 values in dst4 (int8, or the
    same integers as bf16 for the structured attention's int8 mode; dst4 may
    be x4 itself then).  mode is "max", "percentile" or "ema_percentile"
    (ema: (P,) f32, updated in place)."""

    lib = _hip.lib()
    m = _QUANT_MODES[mode]
    ws = _workspace(_size_out(lib.pfa_quantize_heads_workspace_size, int(P_cap), int(T), int(D), m), device)
    with _hip.TIMER.timed("quantize_heads_int8"):
        rc = lib.pfa_quantize_heads_int8(x4, _hip.dtype_tag(dtype), int(H), int(T), int(D), _hip.ptr(head_map),
                                         int(P_cap), _hip.ptr(summary), m, float(percentile), float(ema_decay),
                                         _hip.ptr(ema), 1 if ema_valid else 0, dst4, _hip.dtype_tag(dst_dtype),
                                         _hip.ptr(scales), _hip.ptr(ws), ws.numel(), _hip.stream_ptr(device))
    _hip.check(rc, "pfa_quantize_heads_int8")


def aspa_sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    active_mask: Optional[torch.Tensor] = None,
    causal_mask: Optional[torch.Tensor] = None,
    dropout_p: float = 0.0,
    training: bool = False,
    prepacked: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor, int]] = None,
    q_scale: Optional[torch.Tensor] = None,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    out_dtype: Optional[torch.dtype] = None,
    shortlist_candidates: Optional[torch.Tensor] = None,
    shortlist_lengths: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """ASPA packed sparse attention (reference sparse_attn.py:1373-1646).

    q, k, v: ``(B*H, T, D)``.  ``active_mask``: ``(B*H, T[, 1])`` (bool or
    float > 0).  ``causal_mask``: optional additive ``(T, T)`` mask.  With
    ``shortlist_candidates``/``shortlist_lengths`` (``(N, L)``/``(N,)``) each
    active row attends to its own candidate keys; otherwise an active row
    attends to keys ``0..token`` (implicit causal) or, with a mask, to keys
    ``0..max_token_of_head`` with the mask row added.  Inactive rows are 0.
    """

    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, v must be rank-3 tensors of shape (B*H, T, D)")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, v must have matching shapes")
    batch_heads, tokens, head_dim = q.shape
    dropout_p = float(dropout_p)
    if dropout_p < 0.0 or dropout_p >= 1.0:
        raise ValueError("dropout_p must satisfy 0.0 <= dropout_p < 1.0")
    training = bool(training)
    dropout_real = dropout_p if training else 0.0
    _record_backend("uninitialized")
    is_quantized = q.dtype == torch.int8 or k.dtype == torch.int8 or v.dtype == torch.int8
    if out_dtype is None:
        out_dtype = q.dtype if q.dtype.is_floating_point else torch.float32
    scales = (None, None, None)
    if is_quantized:
        if q.dtype != torch.int8 or k.dtype != torch.int8 or v.dtype != torch.int8:
            raise ValueError("Quantized path expects int8 q, k, v tensors")
        if q_scale is None or k_scale is None or v_scale is None:
            raise ValueError("Quantized path requires q_scale, k_scale, and v_scale tensors")
        scales = tuple(s.to(device=q.device, dtype=torch.float32).contiguous().view(-1)
                       for s in (q_scale, k_scale, v_scale))
        if any(s.numel() != batch_heads for s in scales):
            raise ValueError("Scale tensors must have length equal to the number of heads in q/k/v")
    elif q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, v must share one dtype")
    if causal_mask is not None:
        if causal_mask.dim() != 2 or causal_mask.size(0) != tokens or causal_mask.size(1) != tokens:
            raise ValueError("causal_mask must have shape (T, T)")
    if dropout_real > 0.0:
        raise NotImplementedError("attention dropout in training mode is not provided by the HIP forward path")

    device = _hip.require_device(q, k, v, active_mask, causal_mask, shortlist_candidates, what="aspa_sparse_attention")
    if causal_mask is not None:
        causal_mask = causal_mask.to(device=device, dtype=out_dtype if out_dtype != torch.float64 else torch.float32)
        causal_mask = causal_mask.contiguous()
    if active_mask is None:
        mask_bool = torch.ones(batch_heads, tokens, device=device, dtype=torch.bool)
    else:
        if active_mask.dim() == 3 and active_mask.size(2) == 1:
            active_mask = active_mask.squeeze(-1)
        if active_mask.dim() != 2 or active_mask.size(0) != batch_heads or active_mask.size(1) != tokens:
            raise ValueError("active_mask must have shape (B*H, T)")
        mask_bool = active_mask if active_mask.dtype == torch.bool else (active_mask > 0.0)

    if prepacked is not None:
        head_idx_p, token_idx_p, row_offsets, max_rows = prepacked
        if head_idx_p.numel() != token_idx_p.numel():
            raise ValueError("prepacked head_idx and token_idx must have the same length")
        token_idx = token_idx_p.to(device=device, dtype=torch.int32).contiguous()
        row_head = head_idx_p.to(device=device, dtype=torch.int32).contiguous()
        row_offsets = row_offsets.to(device=device, dtype=torch.int32).contiguous()
        n_rows = int(token_idx.numel())
        if n_rows > 0:
            # the kernels index q/k/v/out with these: out-of-range rows are
            # rejected here (the reference's index_copy_ raises IndexError)
            _check_rows(token_idx, tokens, "aspa_sparse_attention: prepacked token_idx")
            _check_rows(row_head, batch_heads, "aspa_sparse_attention: prepacked head_idx")
    else:
        token_idx, row_head, row_offsets, n_rows, max_rows = _pack_mask_i32(mask_bool)
    if n_rows == 0:
        _record_backend("empty", device=str(device), heads=batch_heads, quantized=bool(is_quantized))
        return torch.zeros(q.shape, device=device, dtype=out_dtype)

    cand = lens = None
    if shortlist_candidates is not None or shortlist_lengths is not None:
        if shortlist_candidates is None or shortlist_lengths is None:
            raise ValueError("shortlist_candidates and shortlist_lengths must be provided together.")
        if shortlist_candidates.dim() != 2:
            raise ValueError("shortlist_candidates must have shape (N_active, L_max)")
        if shortlist_lengths.dim() != 1:
            raise ValueError("shortlist_lengths must have shape (N_active,)")
        if shortlist_candidates.size(0) != shortlist_lengths.size(0):
            raise ValueError("shortlist_lengths must align with shortlist_candidate rows")
        if shortlist_candidates.size(0) != n_rows:
            raise ValueError("Shortlist candidates must match the number of active rows")
        if shortlist_candidates.numel() > 0:
            cand = shortlist_candidates.to(device=device, dtype=torch.int32).contiguous()
            lens = shortlist_lengths.to(device=device, dtype=torch.int32).contiguous()

    head_max = None
    if cand is None and causal_mask is not None:
        P = row_offsets.numel() - 1
        head_max = torch.empty(P, dtype=torch.int32, device=device)
        _hip.check(_hip.lib().pfa_head_max_token(_hip.ptr(token_idx), _hip.ptr(row_offsets), P, _hip.ptr(head_max),
                                                 _hip.stream_ptr(device)), "pfa_head_max_token")

    qc = q if q.stride(-1) == 1 else q.contiguous()
    kc = k if k.stride(-1) == 1 else k.contiguous()
    vc = v if v.stride(-1) == 1 else v.contiguous()
    out = torch.zeros(q.shape, device=device, dtype=out_dtype)
    H = batch_heads
    scale = 1.0 / math.sqrt(head_dim)
    t4 = (_hip.tensor4(qc, H), _hip.tensor4(kc, H), _hip.tensor4(vc, H), _hip.tensor4(out, H))
    if (cand is None and causal_mask is None and not is_quantized and out_dtype == q.dtype
            and _mfma_causal_ok(q.dtype, head_dim, *t4)):
        # implicit causal branch on MFMA tiles (rows are packed by (head, token))
        _causal_attn_mfma(*t4, H, tokens, head_dim, token_idx, row_head, None, device)
        _record_backend("hip", device=str(device), heads=batch_heads, tokens=tokens, max_rows=int(max_rows),
                        quantized=False, candidates=False, mfma=True)
        return out
    _attn_launch(_hip.tensor4(qc, H), _hip.tensor4(kc, H), _hip.tensor4(vc, H), q.dtype, _hip.tensor4(out, H),
                 out_dtype, H, tokens, head_dim, token_idx, row_head, None, cand, lens, causal_mask, head_max, scale,
                 scales, device)
    _record_backend("hip", device=str(device), heads=batch_heads, tokens=tokens, max_rows=int(max_rows),
                    quantized=bool(is_quantized), candidates=cand is not None)
    return out


__all__ = [
    "aspa_sparse_attention",
    "get_last_backend",
    "get_last_backend_info",
    "build_shortlist_candidates",
    "build_packed_shortlist_candidates",
]
