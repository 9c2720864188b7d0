"""CPU oracle for the ASPA forward path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
(``proteus_attention``) never calls it.

Each function restates the reference's PyTorch path (file:line under
``src/proteus_attention/`` of Proteus-Flux-Attention) on CPU tensors.  Where
the reference leaves the order of equal values open (``torch.topk`` /
``argsort`` on ties) the oracle uses the contract of this build: ties go to
the lowest index.

Pinning (what checks each function beyond re-reading the formula):
  router / route_tokens        golden vectors written by the reference itself
                               (tests/golden), softmax/normalisation invariants
  topk_lowest                  brute-force sort on tiny inputs
  select_active_tokens         golden vectors + brute force
  pack_active_rows             closed form (nonzero order, bincount, scan)
  proto_prefix_sets            brute force per token on tiny T; C oracle
  proto_prefix_evict           membership p <= t < evict[p] against
                               proto_prefix_sets on small T with ties
  build_shortlist              golden vectors from the reference builders,
                               the reference test's independent restatement
                               semantics (local/anchor closed forms), C oracle
  sparse_attention             closed form softmax(QK^T/sqrt(D)+mask)V per row,
                               SDPA equality, golden vectors
  quantize_per_head_int8       closed form (absmax/127, round, clamp); the
                               percentile rule by hand-interpolated order
                               statistics and the EMA recurrence; golden
                               module vectors of the reference's int8 mode
  effective linear params      known answers from the reference tests
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# selection helpers
# ---------------------------------------------------------------------------

def topk_lowest(values: torch.Tensor, k: int, dim: int = -1) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top-k along ``dim``; equal values ordered by ascending index.
    NaN is treated as the smallest value."""

    v = values.to(torch.float32)
    key = torch.where(torch.isnan(v), torch.full_like(v, float("-inf")), v)
    order = torch.sort(key, dim=dim, descending=True, stable=True).indices
    idx = order.narrow(dim, 0, k)
    return torch.gather(values, dim, idx), idx


# ---------------------------------------------------------------------------
# router (aspa.py:135-157, 628-690, 1521-1530, 1540-1542, 1590-1591)
# ---------------------------------------------------------------------------

def route_tokens(
    x: torch.Tensor,
    w_router: torch.Tensor,
    protos: Optional[torch.Tensor],
    confidence: Optional[torch.Tensor],
    usage: Optional[torch.Tensor],
    *,
    proto_temp: float,
    proto_threshold: float,
    proto_blend: float,
    usage_boost: float,
):
    """Returns (gate_probs f32 (B,T,G), sim (B,T) or None, blend (B,T) or
    None, importance (B,T) f32)."""

    logits = F.linear(x, w_router.to(x.dtype))                  # aspa.py:150
    gate = F.softmax(logits, dim=-1).to(torch.float32)           # aspa.py:155, 631
    sim = blend_s = None
    if protos is not None:
        tok = F.normalize(x.detach().to(torch.float32), dim=-1, eps=1e-6)   # aspa.py:637-638
        pn = F.normalize(protos.to(torch.float32), dim=-1, eps=1e-6)         # aspa.py:639-640
        sims = tok @ pn.t()                                                   # aspa.py:641
        sim = sims.max(dim=-1).values                                         # aspa.py:642
        pp = F.softmax(sims / proto_temp, dim=-1)                             # aspa.py:643
        blend_s = torch.clamp((sim - proto_threshold) / max(1e-6, 1.0 - proto_threshold), 0.0, 1.0)
        if confidence is not None:                                            # aspa.py:650-655
            conf = (confidence.view(1, 1, -1) + 1e-6).to(torch.float32)
            pp = pp * conf
            pp = pp / pp.sum(dim=-1, keepdim=True).clamp_min(1e-6)
        bl = proto_blend * blend_s.unsqueeze(-1)
        gate = gate * (1.0 - bl) + pp * bl                                    # aspa.py:658
        if usage_boost > 0.0 and usage is not None:                           # aspa.py:660-666
            ub = torch.softmax(-(usage + 1e-6), dim=0).to(torch.float32)
            gate = gate + ub.view(1, 1, -1) * ((1.0 - blend_s).unsqueeze(-1) * usage_boost)
        gate = gate.clamp_min(0.0)
        gate = gate / gate.sum(dim=-1, keepdim=True).clamp_min(1e-6)          # aspa.py:667-670
    gmax = gate.amax(dim=-1)
    if sim is not None:
        importance = gmax * (1.0 - blend_s) + sim * blend_s                   # aspa.py:1521-1528
    else:
        importance = gmax
    return gate, sim, blend_s, importance.to(torch.float32)


def head_probs_from_gates(gate: torch.Tensor, gate_to_head: torch.Tensor, H: int) -> torch.Tensor:
    onehot = F.one_hot(gate_to_head.to(torch.long), num_classes=H).to(gate.dtype)
    return gate @ onehot                                                      # aspa.py:1540-1542


def default_gate_map(G: int, H: int) -> torch.Tensor:
    idx = torch.arange(G, dtype=torch.long)                                   # aspa.py:620-626
    return torch.clamp((idx * max(1, H)) // max(G, 1), 0, max(1, H) - 1)


# ---------------------------------------------------------------------------
# token top-k (aspa.py:790-842)
# ---------------------------------------------------------------------------

def select_active_tokens(importance: torch.Tensor, ratio: float, min_keep: int, guard: int,
                         threshold: float) -> torch.Tensor:
    B, T = importance.shape
    if ratio >= 0.999 and threshold <= 0.0:
        return torch.ones(B, T, dtype=torch.bool)
    guard = min(max(0, guard), T)
    min_keep = max(min(max(0, min_keep), T), guard)
    keep = torch.full((B,), ratio * T, dtype=torch.float32).round().to(torch.int64)
    if min_keep > 0:
        keep = torch.clamp(keep, min=min_keep)
    keep = torch.clamp(keep, min=1, max=T)
    imp = importance.to(torch.float32)
    out = torch.zeros(B, T, dtype=torch.bool)
    for b in range(B):
        base = imp[b] >= threshold if threshold > 0.0 else torch.zeros(T, dtype=torch.bool)
        need = max(int(keep[b]), int(base.sum()), guard)
        need = min(max(1, need), T)
        if need >= T:
            base = torch.ones(T, dtype=torch.bool)
        else:
            _, idx = topk_lowest(imp[b], need)
            base[idx] = True
        if guard > 0:
            base[:guard] = True
        out[b] = base
    return out


# ---------------------------------------------------------------------------
# packing (sparse_attn.py:924-947)
# ---------------------------------------------------------------------------

def pack_active_rows(mask: torch.Tensor):
    pos = mask.nonzero(as_tuple=False)
    if pos.numel() == 0:
        return None
    head_idx, token_idx = pos[:, 0], pos[:, 1]
    counts = torch.bincount(head_idx, minlength=mask.size(0)).to(torch.int32)
    offs = torch.zeros(mask.size(0) + 1, dtype=torch.int32)
    offs[1:] = torch.cumsum(counts, 0)
    return head_idx.long(), token_idx.long(), offs, int(counts.max())


# ---------------------------------------------------------------------------
# shortlist candidates (sparse_attn.py:260-596)
# ---------------------------------------------------------------------------

def proto_prefix_sets(scores: torch.Tensor, K: int) -> torch.Tensor:
    """(T,) scores -> (T, K) int64: top-min(t+1,K) of scores[0..t] (ties ->
    lowest index), ascending, padded with t.  Brute force, small T only."""

    T = scores.numel()
    out = torch.empty(T, K, dtype=torch.long)
    for t in range(T):
        c = min(t + 1, K)
        _, idx = topk_lowest(scores[: t + 1], c)
        row = torch.full((K,), t, dtype=torch.long)
        row[:c] = torch.sort(idx).values
        out[t] = row
    return out


def proto_prefix_evict(scores: torch.Tensor, K: int) -> torch.Tensor:
    """(T,) scores -> (T,) int64 evict[p]: the first t at which p is no
    longer in the prefix top-K set S(t) of proto_prefix_sets (sparse_attn.py
    :260-300), p when it never enters, 2^31 - 1 when it is in S(T - 1).

    Under the order of topk_lowest (value descending, then index ascending)
    p is in S(t) exactly while p <= t and fewer than K positions q <= t are
    better than p; that count only grows with t, so p leaves at the position
    of the K-th better element.  The positions of the better elements are
    those seen before p in key order: a Fenwick tree over positions gives the
    K-th smallest of them.  O(T log T), for sequences too long for the brute
    force (pinned against proto_prefix_sets on small T with ties)."""

    v = scores.detach().to(torch.float64).cpu().tolist()
    T = len(v)
    order = sorted(range(T), key=lambda i: (-v[i], i))
    tree = [0] * (T + 1)
    log = 1
    while (1 << log) <= T:
        log += 1
    out = [0] * T
    seen = 0
    big = 2 ** 31 - 1
    for p in order:
        if seen >= K:
            # K-th smallest seen position: binary lifting over the tree
            pos, rem = 0, K
            for b in range(log, -1, -1):
                nxt = pos + (1 << b)
                if nxt <= T and tree[nxt] < rem:
                    pos = nxt
                    rem -= tree[nxt]
            tau = pos  # 0-based position of the K-th better element
            out[p] = tau if tau > p else p
        else:
            out[p] = big
        i = p + 1
        while i <= T:
            tree[i] += 1
            i += i & -i
        seen += 1
    return torch.tensor(out, dtype=torch.long)


def build_shortlist(
    rows: torch.Tensor,
    seq_len: int,
    *,
    max_candidates: int,
    linear_window: int,
    anchor_stride: int,
    use_local: bool,
    use_anchors: bool,
    proto_scores: Optional[torch.Tensor] = None,
    row_batch_ids: Optional[torch.Tensor] = None,
    local_cap: Optional[int] = None,
    anchor_cap: Optional[int] = None,
    proto_cap: Optional[int] = None,
    extra_candidates: Optional[torch.Tensor] = None,
    extra_lengths: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """The reference's concat -> clamp -> min(row) -> append row -> sort ->
    unique -> keep smallest L -> pad procedure (sparse_attn.py:399-454 and
    500-594), proto ties -> lowest index.  proto_scores: (T,) or (B, T)."""

    L = int(max_candidates)
    N = rows.numel()
    if N == 0 or L <= 0:
        return rows.new_empty(rows.shape + (0,)), rows.new_zeros(rows.shape, dtype=torch.long)
    r = rows.to(torch.long)
    lc = max(0, int(local_cap)) if local_cap is not None else (L if use_local else 0)
    ac = max(0, int(anchor_cap)) if anchor_cap is not None else (L if use_anchors else 0)
    pc = max(0, int(proto_cap)) if proto_cap is not None else (L if proto_scores is not None else 0)
    pieces = []
    if use_local and lc > 0:
        w = min(linear_window, L, lc)
        if w > 0:
            steps = torch.arange(w)
            ln = torch.clamp(r + 1, max=w)
            start = torch.clamp(r - ln + 1, min=0)
            loc = start[:, None] + steps[None, :]
            pieces.append(torch.where(steps[None, :] < ln[:, None], loc, r[:, None]))
    if use_anchors and anchor_stride > 0 and ac > 0:
        slots = min(ac, L, max(1, seq_len))
        if slots > 0:
            steps = torch.arange(1, slots + 1)
            pieces.append(torch.clamp(r[:, None] - steps[None, :] * anchor_stride, min=0))
    if proto_scores is not None and pc > 0 and proto_scores.numel() > 0:
        ps = proto_scores.to(torch.float32)
        if ps.dim() == 1:
            ps = ps.unsqueeze(0)
        ps = ps[:, :seq_len]
        K = min(L, pc, seq_len, ps.size(1))
        if K > 0:
            rb = row_batch_ids.to(torch.long) if row_batch_ids is not None else torch.zeros(N, dtype=torch.long)
            proto = r[:, None].expand(N, K).clone()
            for b in torch.unique(rb).tolist():
                sel = (rb == b).nonzero(as_tuple=True)[0]
                sets = _prefix_sets_for_rows(ps[b], r[sel], K)
                proto[sel] = sets
            pieces.append(proto)
    if extra_candidates is not None and extra_candidates.numel() > 0:
        ex = extra_candidates.to(torch.long)
        if extra_lengths is not None:
            valid = torch.arange(ex.size(1))[None, :] < extra_lengths.to(torch.long)[:, None]
            ex = torch.where(valid, ex, r[:, None].expand_as(ex))
        pieces.append(ex)
    cand = torch.cat(pieces, dim=1) if pieces else r[:, None]
    cand = torch.clamp(cand, 0, max(seq_len - 1, 0))
    cand = torch.minimum(cand, r[:, None])
    cand = torch.cat([cand, r[:, None]], dim=1)
    cand = torch.sort(cand, dim=1).values
    keep = torch.ones_like(cand, dtype=torch.bool)
    keep[:, 1:] = cand[:, 1:] != cand[:, :-1]
    uidx = keep.to(torch.long).cumsum(1) - 1
    keep = keep & (uidx < L)
    lengths = torch.clamp(keep.sum(1), min=1)
    out = r[:, None].expand(N, L).clone()
    ri, ci = keep.nonzero(as_tuple=True)
    out[ri, uidx[ri, ci]] = cand[ri, ci]
    return out, lengths


def _prefix_sets_for_rows(scores: torch.Tensor, rows: torch.Tensor, K: int) -> torch.Tensor:
    """Per row t: the top-min(t+1,K) positions <= t (ties lowest), padded
    with t; order within the row is irrelevant to the builder (it sorts)."""

    out = rows[:, None].expand(rows.numel(), K).clone()
    T = scores.numel()
    key = torch.where(torch.isnan(scores), torch.full_like(scores, float("-inf")), scores)
    order = torch.sort(key, descending=True, stable=True).indices   # global rank order
    rank = torch.empty(T, dtype=torch.long)
    rank[order] = torch.arange(T)
    for i, t in enumerate(rows.tolist()):
        tt = min(t, T - 1)
        c = min(t + 1, K)
        pos = torch.arange(tt + 1)
        best = pos[torch.argsort(rank[: tt + 1])[:c]]
        out[i, :c] = best
    return out


# ---------------------------------------------------------------------------
# attention (sparse_attn.py:950-1046 and the operator glue 1373-1646)
# ---------------------------------------------------------------------------

def sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    active_mask: Optional[torch.Tensor] = None,
    causal_mask: Optional[torch.Tensor] = None,
    q_scale: Optional[torch.Tensor] = None,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    out_dtype: Optional[torch.dtype] = None,
    shortlist_candidates: Optional[torch.Tensor] = None,
    shortlist_lengths: Optional[torch.Tensor] = None,
    prepacked=None,
    compute_dtype: Optional[torch.dtype] = None,
) -> torch.Tensor:
    """The reference fallback on CPU.  compute_dtype None reproduces the
    reference (computes in the input dtype); torch.float32 gives the exact-
    arithmetic diagnostic restatement."""

    BH, T, D = q.shape
    quant = q.dtype == torch.int8
    if out_dtype is None:
        out_dtype = q.dtype if q.dtype.is_floating_point else torch.float32
    if quant:
        qd = q.to(torch.float32) * q_scale.view(-1, 1, 1)
        kd = k.to(torch.float32) * k_scale.view(-1, 1, 1)
        vd = v.to(torch.float32) * v_scale.view(-1, 1, 1)
    else:
        qd, kd, vd = q, k, v
    if compute_dtype is not None:
        qd, kd, vd = qd.to(compute_dtype), kd.to(compute_dtype), vd.to(compute_dtype)
    cm = causal_mask.to(dtype=out_dtype) if causal_mask is not None else None
    if active_mask is None:
        mask = torch.ones(BH, T, dtype=torch.bool)
    else:
        am = active_mask.squeeze(-1) if active_mask.dim() == 3 else active_mask
        mask = am if am.dtype == torch.bool else am > 0
    packed = prepacked if prepacked is not None else pack_active_rows(mask)
    if packed is None:
        return torch.zeros(q.shape, dtype=out_dtype)
    head_idx, token_idx, offs, _ = packed
    scale = 1.0 / (D ** 0.5)
    result = torch.zeros(qd.shape, dtype=qd.dtype)
    q_act = qd[head_idx, token_idx]
    use_c = shortlist_candidates is not None and shortlist_lengths is not None and shortlist_candidates.numel() > 0
    for h in range(BH):
        s, e = int(offs[h]), int(offs[h + 1])
        if s == e:
            continue
        toks = token_idx[s:e]
        qs = q_act[s:e]
        if use_c:
            cr = shortlist_candidates[s:e].long()
            lr = shortlist_lengths[s:e].long()
            Lm = cr.size(1)
            cc = cr.clamp(0, T - 1)
            ks, vs = kd[h][cc], vd[h][cc]
            inval = torch.arange(Lm)[None, :] >= lr[:, None]
            ks = ks.masked_fill(inval[..., None], 0.0)
            vs = vs.masked_fill(inval[..., None], 0.0)
            sc = torch.einsum("rd,rld->rl", qs, ks) * scale
            if cm is not None:
                sc = sc + torch.gather(cm.index_select(0, toks), 1, cr.clamp(0, cm.size(1) - 1)).to(sc.dtype)
            sc = sc.masked_fill(inval, float("-inf"))
            p = torch.softmax(sc, dim=-1)
            o = torch.bmm(p.unsqueeze(1), vs).squeeze(1)
        else:
            mt = int(toks.max())
            kk, vv = kd[h, : mt + 1].unsqueeze(0), vd[h, : mt + 1].unsqueeze(0)
            if cm is not None:
                am = cm.index_select(0, toks)[:, : mt + 1].unsqueeze(0)
            else:
                fut = torch.arange(mt + 1)[None, :] > toks[:, None]
                am = torch.zeros(1, toks.numel(), mt + 1, dtype=qs.dtype).masked_fill(fut.unsqueeze(0), float("-inf"))
            o = F.scaled_dot_product_attention(qs.unsqueeze(0), kk, vv, attn_mask=am, dropout_p=0.0).squeeze(0)
        result[h].index_copy_(0, toks, o.to(result.dtype))
    return result.to(out_dtype)


def quantize_per_head_int8(t: torch.Tensor, mode: str = "max", percentile: float = 1.0, ema: Optional[torch.Tensor] = None,
                           ema_decay: float = 0.9) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """Per-head symmetric int8 (aspa.py:1312-1363): base = absmax ("max"),
    torch.quantile of |x| with its absmax when that is 0 ("percentile",
    percentile > 0), and for "ema_percentile" ema = decay*ema + (1-decay)*base
    with ema starting at the absmax (aspa.py:1339-1355); scale =
    clamp(base/127, min=1e-6); q = clamp(round(x/scale), +-127).  Returns
    (q, scales, updated ema or None)."""

    flat = t.to(torch.float32).reshape(t.size(0), -1)
    absf = flat.abs()
    amax = absf.amax(dim=1, keepdim=True)
    if mode == "max" or percentile <= 0.0:
        base = amax
    else:
        base = torch.quantile(absf, percentile, dim=1, keepdim=True)
        base = torch.where(base > 0.0, base, amax)
    new_ema = None
    if mode == "ema_percentile":
        prev = amax.squeeze(1) if ema is None else ema.to(torch.float32)
        new_ema = ema_decay * prev + (1.0 - ema_decay) * base.squeeze(1)
        base = new_ema.unsqueeze(1)
    s = torch.clamp(base / 127.0, min=1e-6)
    qv = torch.clamp((flat / s).round(), -127.0, 127.0).to(torch.int8).view_as(t)
    return qv, s.squeeze(1), new_ema


# ---------------------------------------------------------------------------
# RoPE (aspa.py:576-618)
# ---------------------------------------------------------------------------

def rope_tables(T: int, D: int, base: float, dtype: torch.dtype, freq_dtype: torch.dtype = torch.float32):
    """(cos, sin) of shape (T, D) in `dtype` (aspa.py:240-246, 576-604).
    freq_dtype: the dtype of the module's inverse-frequency buffer, in which
    the positions and angles are computed; a module cast to bf16 holds it in
    bf16 (the buffer follows the module's dtype), so positions above 256
    round before the angles are formed."""
    inv = (1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.float32) / max(D, 1)))).to(freq_dtype)
    ang = torch.outer(torch.arange(T, dtype=freq_dtype), inv)
    return (torch.repeat_interleave(ang.cos(), 2, dim=-1).to(dtype),
            torch.repeat_interleave(ang.sin(), 2, dim=-1).to(dtype))


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x (B, T, H, D)."""
    T, D = x.size(1), x.size(3)
    c = cos.view(1, T, 1, D)
    s = sin.view(1, T, 1, D)
    rot = torch.stack((-x[..., 1::2], x[..., ::2]), dim=-1).reshape_as(x)
    return (x * c) + (rot * s)


def causal_attention_f32(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Dense causal attention in f32 (BH, T, D) -- closed form reference."""
    T = q.size(1)
    s = (q.float() @ k.float().transpose(1, 2)) / math.sqrt(q.size(-1))
    s = s.masked_fill(torch.triu(torch.ones(T, T, dtype=torch.bool), 1), float("-inf"))
    return torch.softmax(s, -1) @ v.float()


# ---------------------------------------------------------------------------
# chunked shortlist selection (tools/chunked_shortlist.py:140-254)
# ---------------------------------------------------------------------------

def nucleus_select(scores: torch.Tensor, max_tokens: int, top_p: float, keep_mask: Optional[torch.Tensor] = None,
                   index_offset: int = 0, drop_nonfinite: bool = False):
    """_nucleus_select (chunked_shortlist.py:175-208) with the masking and
    finite filter of _select_top_tokens (:140-172).  The order is (score
    desc, position asc) -- a stable descending sort; the reference's
    argsort leaves ties open.  Returns (values, positions + offset) or None."""

    s = scores.to(torch.float32).clone()
    if keep_mask is not None:
        s = torch.where(keep_mask.to(torch.bool), s, torch.full_like(s, float("-inf")))
    n = s.numel()
    limit = min(int(max_tokens), n)
    if limit <= 0:
        return None
    finite = torch.isfinite(s)
    if not bool(finite.any()):
        return None
    safe = torch.where(finite, s, torch.full_like(s, -1e9))
    order = torch.sort(safe, descending=True, stable=True).indices
    if top_p >= 1.0:
        keep = limit
    else:
        probs = torch.softmax(safe, dim=-1)[order]
        mass = torch.cumsum(probs, dim=-1)
        keep = int((mass < float(top_p)).sum())
        if keep < n:
            keep += 1
        keep = min(limit, max(1, keep))
    sel = order[:keep]
    vals = s[sel]
    if drop_nonfinite:
        ok = torch.isfinite(vals)
        sel, vals = sel[ok], vals[ok]
        if sel.numel() == 0:
            return None
    return vals, sel + int(index_offset)


def finalise_indices(scores: torch.Tensor, indices: torch.Tensor, max_tokens: int):
    """_finalise_indices (chunked_shortlist.py:211-254): score-descending
    order (stable), one survivor per index -- its last entry in that order
    (the composite key index*(n+1)-position of :233-243) -- the first
    max_tokens survivors, sorted by index.  Returns (indices int64, scores)."""

    sc = scores.to(torch.float32)
    order = torch.sort(sc, descending=True, stable=True).indices
    s_ord, i_ord = sc[order], indices[order].to(torch.long)
    n = i_ord.numel()
    pos = torch.arange(n, dtype=torch.long)
    by_idx = torch.sort(i_ord * (n + 1) - pos, stable=True).indices
    grouped = i_ord[by_idx]
    first = torch.ones(n, dtype=torch.bool)
    first[1:] = grouped[1:] != grouped[:-1]
    keep = torch.sort(by_idx[first]).values[:max_tokens]
    ki, ks = i_ord[keep], s_ord[keep]
    back = torch.sort(ki).indices
    return ki[back], ks[back]


# ---------------------------------------------------------------------------
# all-query final pass over an int8 shortlist (no reference counterpart:
# the reference attends the reduced sequence to itself,
# chunked_shortlist.py:710-739)
# ---------------------------------------------------------------------------

def quantize_rows_int8(x: torch.Tensor, heads: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """x (S, H*D) -> int8 (H, S, D), scales (H, S): quantize_per_head_int8
    applied to every (head, row) slice of D elements."""

    S, C = x.shape
    D = C // heads
    slices = x.reshape(S, heads, D).permute(1, 0, 2).reshape(heads * S, 1, D)
    q, s, _ = quantize_per_head_int8(slices)
    return q.view(heads, S, D), s.view(heads, S)


def int8_kv_attention(q: torch.Tensor, k8: torch.Tensor, v8: torch.Tensor, k_scale: torch.Tensor,
                      v_scale: torch.Tensor, key_pos: torch.Tensor, causal: bool = True,
                      scale: Optional[float] = None, q_pos: Optional[torch.Tensor] = None) -> torch.Tensor:
    """q (T, H, D); k8/v8 (H, S, D) int8 with scales (H, S); key_pos (S,).
    Dequantise in f32, softmax(q k^T * scale + mask) v in f32 with key j
    visible to query t iff key_pos[j] <= t (causal); rows with no visible
    key are zero.  q_pos (T,): the positions of the query rows when q holds
    a subset of the sequence (default 0..T-1).  Returns (T, H, D) f32."""

    T, H, D = q.shape
    sc = (1.0 / math.sqrt(D)) if scale is None else float(scale)
    k = k8.to(torch.float32) * k_scale.to(torch.float32).unsqueeze(-1)
    v = v8.to(torch.float32) * v_scale.to(torch.float32).unsqueeze(-1)
    qh = q.to(torch.float32).permute(1, 0, 2)  # (H, T, D)
    s = (qh @ k.transpose(1, 2)) * sc  # (H, T, S)
    vis = torch.ones(T, k.size(1), dtype=torch.bool)
    if causal:
        qp = torch.arange(T) if q_pos is None else q_pos.to(torch.long)
        vis = key_pos.view(1, -1).to(torch.long) <= qp.view(-1, 1)
    s = s.masked_fill(~vis.unsqueeze(0), float("-inf"))
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)  # all-masked rows -> zero output
    return (p @ v).permute(1, 0, 2).contiguous()
