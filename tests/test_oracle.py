"""CPU: pin the oracle against the reference's golden vectors, brute force
and closed forms.  These tests never touch the product package."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import aspa_oracle as O
from oracle import c_oracle


# ---------------------------------------------------------------------------
# selection helpers
# ---------------------------------------------------------------------------

def test_topk_lowest_brute_force():
    g = torch.Generator().manual_seed(0)
    x = torch.randint(0, 5, (300, 8), generator=g).float()
    _, idx = O.topk_lowest(x, 3)
    for r in range(x.size(0)):
        order = sorted(range(8), key=lambda j: (-x[r, j].item(), j))[:3]
        assert idx[r].tolist() == order


def test_select_active_tokens_matches_golden_when_untied(golden):
    z = golden("module_cfg1")
    imp = torch.from_numpy(z["importance"])
    ref_mask = torch.from_numpy(z["token_mask"]).bool()
    T = imp.size(1)
    mine = O.select_active_tokens(imp, 0.25, 1, 1, 0.0)
    # positions whose value equals the cut value may legitimately differ
    need = int(torch.tensor(0.25 * T, dtype=torch.float32).round())
    cut = torch.sort(imp[0], descending=True).values[need - 1]
    differ = (mine != ref_mask)[0]
    assert int(mine.sum()) == int(ref_mask.sum())
    assert bool((imp[0][differ] == cut).all()) or not bool(differ.any())
    assert mine[0, 0]  # guard


def test_pack_closed_form():
    g = torch.Generator().manual_seed(3)
    m = torch.rand(5, 40, generator=g) > 0.5
    m[2] = False
    h, t, offs, mx = O.pack_active_rows(m)
    assert offs[-1] == int(m.sum())
    for p in range(5):
        toks = t[offs[p]:offs[p + 1]]
        assert toks.tolist() == m[p].nonzero().flatten().tolist()
    assert mx == int(m.sum(1).max())


# ---------------------------------------------------------------------------
# shortlist builder
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("tag", ["l", "la", "lp", "ap"])
def test_builder_small_matches_reference(golden, tag):
    z = golden(f"builder_small_{tag}")
    ul, ua, up = (bool(v) for v in z["use"])
    rows = torch.from_numpy(z["rows"])
    c, l = O.build_shortlist(rows, 64, max_candidates=16, linear_window=12, anchor_stride=4, use_local=ul,
                             use_anchors=ua, proto_scores=torch.from_numpy(z["scores"]) if up else None)
    assert np.array_equal(c.numpy(), z["cand"])
    assert np.array_equal(l.numpy(), z["lengths"])


def test_builder_packed_realistic_matches_reference(golden):
    z = golden("builder_packed_T4096")
    L, w, s, lc, ac, pc = (int(v) for v in z["kw"])
    rows = torch.from_numpy(z["rows"])
    rb = torch.from_numpy(z["row_batch"])
    c, l = O.build_shortlist(rows, 4096, max_candidates=L, linear_window=w, anchor_stride=s, use_local=True,
                             use_anchors=True, proto_scores=torch.from_numpy(z["sims"]), row_batch_ids=rb,
                             local_cap=lc, anchor_cap=ac, proto_cap=pc)
    assert np.array_equal(c.numpy(), z["cand"])
    assert np.array_equal(l.numpy(), z["lengths"])
    # C oracle on the same rows
    K = min(L, pc, 4096)
    cc, cl = c_oracle.shortlist_build(z["rows"].astype(np.int32), z["row_batch"].astype(np.int32), 4096, L,
                                      min(w, L, lc), s, min(ac, L, 4096), z["sims"], K)
    assert np.array_equal(cc, z["cand"])
    assert np.array_equal(cl, z["lengths"])


def test_builder_truncation_matches_reference(golden):
    z = golden("builder_truncate")
    L, w, s, lc, ac, pc = (int(v) for v in z["kw"])
    c, l = O.build_shortlist(torch.from_numpy(z["rows"]), 2048, max_candidates=L, linear_window=w, anchor_stride=s,
                             use_local=True, use_anchors=True, proto_scores=torch.from_numpy(z["sims"]),
                             local_cap=lc, anchor_cap=ac, proto_cap=pc)
    assert np.array_equal(c.numpy(), z["cand"])
    assert np.array_equal(l.numpy(), z["lengths"])
    assert int(l.max()) == L  # the case does truncate


def test_builder_closed_forms():
    """Local window alone is [max(0,t-w+1) .. t]; anchors alone are the
    distinct max(t - s*j, 0) plus t (the reference test's restatement)."""
    rows = torch.tensor([0, 3, 11, 40, 99])
    c, l = O.build_shortlist(rows, 100, max_candidates=20, linear_window=8, anchor_stride=0, use_local=True,
                             use_anchors=False)
    for i, t in enumerate(rows.tolist()):
        exp = list(range(max(0, t - 7), t + 1))
        assert c[i, :len(exp)].tolist() == exp and int(l[i]) == len(exp)
        assert all(v == t for v in c[i, len(exp):].tolist())
    c, l = O.build_shortlist(rows, 100, max_candidates=20, linear_window=1, anchor_stride=7, use_local=False,
                             use_anchors=True)
    for i, t in enumerate(rows.tolist()):
        exp = sorted({max(t - 7 * j, 0) for j in range(1, 21)} | {t})
        assert c[i, :len(exp)].tolist() == exp and int(l[i]) == len(exp)


def test_proto_prefix_sets_brute_force():
    g = torch.Generator().manual_seed(5)
    s = torch.randint(0, 6, (70,), generator=g).float()  # many ties
    K = 9
    sets = O.proto_prefix_sets(s, K)
    for t in range(70):
        c = min(t + 1, K)
        best = sorted(range(t + 1), key=lambda j: (-s[j].item(), j))[:c]
        assert sets[t, :c].tolist() == sorted(best)


def test_proto_prefix_evict_matches_brute_force_sets():
    """p is in S(t) exactly when p <= t < evict[p], for the evict oracle
    against the brute-force sets, with heavy ties, K above and below T; a
    planted mistake (the (K+1)-th better element taken for the K-th) must
    fail."""
    g = torch.Generator().manual_seed(31)
    for T, K in ((300, 7), (130, 64), (200, 200), (65, 1), (257, 64), (90, 300)):
        s = torch.randint(0, 7, (T,), generator=g).float()
        ev = O.proto_prefix_evict(s, K)
        exp = O.proto_prefix_sets(s, K)
        member = torch.zeros(T, T, dtype=torch.bool)
        for t in range(T):
            member[t, exp[t, : min(t + 1, K)]] = True
        pos = torch.arange(T)
        assert torch.equal(member, (pos[None, :] <= pos[:, None]) & (ev[None, :] > pos[:, None])), (T, K)
    # planted mistake: the (K+1)-th better element taken for the K-th
    T, K = 150, 6
    s = torch.randint(0, 4, (T,), generator=g).float()
    exp = O.proto_prefix_sets(s, K)
    member = torch.zeros(T, T, dtype=torch.bool)
    for t in range(T):
        member[t, exp[t, : min(t + 1, K)]] = True
    pos = torch.arange(T)
    off = O.proto_prefix_evict(s, K + 1)
    assert not torch.equal(member, (pos[None, :] <= pos[:, None]) & (off[None, :] > pos[:, None]))


def test_c_oracle_matches_torch_oracle_with_ties():
    g = torch.Generator().manual_seed(9)
    T = 500
    rows = torch.randint(0, T, (300,), generator=g)
    s = torch.randint(0, 7, (T,), generator=g).float()
    c, l = O.build_shortlist(rows, T, max_candidates=64, linear_window=20, anchor_stride=9, use_local=True,
                             use_anchors=True, proto_scores=s, local_cap=20, anchor_cap=30, proto_cap=25)
    cc, cl = c_oracle.shortlist_build(rows.numpy().astype(np.int32), None, T, 64, 20, 9, 30, s.numpy(), 25)
    assert np.array_equal(cc, c.numpy().astype(np.int32))
    assert np.array_equal(cl, l.numpy().astype(np.int32))


def test_oracle_detects_planted_mistake():
    """A plausible slip (anchor offsets starting at j=0) is caught by the
    golden vectors."""
    rows = torch.tensor([5, 17, 33])
    good, _ = O.build_shortlist(rows, 64, max_candidates=16, linear_window=1, anchor_stride=4, use_local=False,
                                use_anchors=True)
    bad = torch.stack([torch.clamp(rows - 4 * j, min=0) for j in range(0, 16)], 1)
    assert not torch.equal(good[:, :5], torch.sort(bad, 1).values[:, :5])


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("tag,tol", [("f32", 2e-5), ("bf16", 0.0)])
def test_sparse_attention_matches_reference(golden, tag, tol):
    z = golden(f"attn_{tag}")
    dt = torch.float32 if tag == "f32" else torch.bfloat16
    q, k, v = (torch.from_numpy(z[n]).to(dt) for n in ("q", "k", "v"))
    mask = torch.from_numpy(z["mask"]).bool()
    T = q.size(1)
    causal = torch.triu(torch.full((T, T), float("-inf")), diagonal=1)
    out = O.sparse_attention(q, k, v, active_mask=mask)
    assert torch.allclose(out.float(), torch.from_numpy(z["out_nocand"]), atol=tol + 1e-6, rtol=0)
    out = O.sparse_attention(q, k, v, active_mask=mask, causal_mask=causal)
    assert torch.allclose(out.float(), torch.from_numpy(z["out_mask"]), atol=tol + 1e-6, rtol=0)
    out = O.sparse_attention(q, k, v, active_mask=mask, shortlist_candidates=torch.from_numpy(z["cand"]),
                             shortlist_lengths=torch.from_numpy(z["lengths"]))
    assert torch.allclose(out.float(), torch.from_numpy(z["out_cand"]), atol=tol + 1e-6, rtol=0)


def test_sparse_attention_closed_form_and_sdpa():
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(3, 6, 5, generator=g) for _ in range(3))
    causal = torch.triu(torch.full((6, 6), float("-inf")), diagonal=1)
    out = O.sparse_attention(q, k, v, causal_mask=causal)
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=causal.unsqueeze(0))
    assert torch.allclose(out, ref, atol=1e-6)
    # manual per-row softmax on a partial mask
    m = torch.rand(3, 6, generator=g) > 0.4
    out = O.sparse_attention(q, k, v, active_mask=m, causal_mask=causal)
    for h in range(3):
        for t in range(6):
            if not m[h, t]:
                assert torch.all(out[h, t] == 0)
            else:
                s = (k[h, : t + 1] @ q[h, t]) / math.sqrt(5)
                exp = torch.softmax(s, 0) @ v[h, : t + 1]
                assert torch.allclose(out[h, t], exp, atol=1e-5)


def test_candidates_covering_prefix_equal_causal():
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(2, 40, 8, generator=g) for _ in range(3))
    rows = torch.arange(40).repeat(2)
    c, l = O.build_shortlist(rows, 40, max_candidates=40, linear_window=40, anchor_stride=0, use_local=True,
                             use_anchors=False)
    out = O.sparse_attention(q, k, v, shortlist_candidates=c, shortlist_lengths=l)
    assert torch.allclose(out, O.causal_attention_f32(q, k, v), atol=1e-5)


def test_quantize_per_head_closed_form():
    g = torch.Generator().manual_seed(4)
    t = torch.randn(3, 10, 4, generator=g)
    qv, s, _ = O.quantize_per_head_int8(t)
    assert torch.allclose(s, t.reshape(3, -1).abs().amax(1) / 127.0)
    assert int(qv.abs().max()) == 127
    assert torch.allclose(qv.float() * s.view(-1, 1, 1), t, atol=float(s.max()) / 2 + 1e-7)


def test_quantize_per_head_percentile_and_ema_closed_forms():
    """Percentile base = the linear interpolation between the two order
    statistics around rank p*(n-1) of |x| (by hand on a small sorted list),
    the absmax when that is 0; ema_percentile = decay*ema + (1-decay)*base,
    seeded with the absmax (aspa.py:1325-1355)."""
    t = torch.tensor([[[0.0, -4.0], [1.0, 2.0], [-3.0, 0.5]], [[0.0, 0.0], [0.0, 0.0], [0.0, 9.0]]])
    # head 0: |x| sorted = 0, .5, 1, 2, 3, 4; p = .5 -> rank 2.5 -> 1 + .5*(2 - 1) = 1.5
    _, s, _ = O.quantize_per_head_int8(t, "percentile", 0.5)
    assert s[0].item() == pytest.approx(1.5 / 127.0, rel=1e-7)
    # head 1: the median of |x| is 0 -> the absmax 9
    assert s[1].item() == pytest.approx(9.0 / 127.0, rel=1e-7)
    # p = 1 is the absmax; p = 0 means "max" (percentile <= 0)
    _, s1, _ = O.quantize_per_head_int8(t, "percentile", 1.0)
    _, s0, _ = O.quantize_per_head_int8(t, "percentile", 0.0)
    assert torch.equal(s1, torch.tensor([4.0, 9.0]) / 127.0) and torch.equal(s0, s1)
    # EMA: first call seeds with the absmax, the second reads the first
    _, s_a, e1 = O.quantize_per_head_int8(t, "ema_percentile", 0.5, None, 0.75)
    assert e1[0].item() == pytest.approx(0.75 * 4.0 + 0.25 * 1.5, rel=1e-7)
    _, s_b, e2 = O.quantize_per_head_int8(t, "ema_percentile", 0.5, e1, 0.75)
    assert e2[0].item() == pytest.approx(0.75 * e1[0].item() + 0.25 * 1.5, rel=1e-7)
    assert s_b[0].item() == pytest.approx(e2[0].item() / 127.0, rel=1e-7)
    # the planted mistake: seeding the EMA with the quantile instead of the
    # absmax gives another value
    assert e1[0].item() != pytest.approx(1.5, rel=1e-3)


# ---------------------------------------------------------------------------
# router
# ---------------------------------------------------------------------------

def _module_weights(B, T, C, H, outlier=0.0):
    from configs import make_inputs

    x, g = make_inputs(B, T, C, seed=0, outlier_frac=outlier)
    ws = []
    for shape in ((H, C), (H, C), (3 * C, C), (C, C)):
        tmp = torch.empty(shape)
        torch.nn.init.xavier_normal_(tmp, generator=g)
        ws.append(tmp)
    return x, ws


def _digest(*ts):
    import hashlib

    h = hashlib.sha256()
    for t in ts:
        h.update(t.float().contiguous().numpy().tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("name,B,T,C,dt,outlier", [
    ("module_cfg1", 1, 1024, 256, torch.float32, 0.0),
    ("module_cfg2_T2048", 2, 2048, 512, torch.bfloat16, 0.0),
    ("module_short_T4096_f32", 1, 4096, 512, torch.float32, 0.01),
    ("module_short_T4096_bf16", 1, 4096, 512, torch.bfloat16, 0.01),
])
def test_router_oracle_matches_reference(golden, name, B, T, C, dt, outlier):
    z = golden(name)
    x, ws = _module_weights(B, T, C, 8, outlier)
    assert _digest(x) == str(z["x_sha256"])
    assert _digest(*ws) == str(z["w_sha256"])
    gate, sim, blend, imp = O.route_tokens(x.to(dt), ws[0].to(dt), ws[1].to(dt), torch.zeros(8, dtype=dt),
                                           None, proto_temp=0.2, proto_threshold=0.25, proto_blend=0.6,
                                           usage_boost=0.0)
    assert torch.allclose(gate, torch.from_numpy(z["gate_probs"]), atol=1e-6, rtol=0)
    assert torch.allclose(imp, torch.from_numpy(z["importance"]), atol=1e-6, rtol=0)
    assert torch.allclose(sim, torch.from_numpy(z["sim"]), atol=1e-6, rtol=0)


# ---------------------------------------------------------------------------
# chunked shortlist selection and the all-query int8 final pass
# ---------------------------------------------------------------------------

def test_chunk_selection_oracle_matches_reference(golden):
    z = golden("chunk_select")
    s = torch.from_numpy(z["scores"])
    v, i = O.nucleus_select(s, 512, 1.0)
    assert np.array_equal(i.numpy(), z["i_p1"]) and np.array_equal(v.numpy(), z["v_p1"])
    v, i = O.nucleus_select(s * 4.0, 512, 0.9)
    assert np.array_equal(i.numpy(), z["i_p09"]) and np.array_equal(v.numpy(), z["v_p09"])
    ki, ks = O.finalise_indices(torch.from_numpy(z["all_scores"]), torch.from_numpy(z["all_idx"]), 4096)
    assert np.array_equal(ki.numpy(), z["keep_idx"]) and np.array_equal(ks.numpy(), z["keep_scores"])


def test_chunk_selection_oracle_brute_force_ties():
    g = torch.Generator().manual_seed(5)
    for trial in range(20):
        n = int(torch.randint(1, 60, (1,), generator=g))
        s = torch.randint(-3, 4, (n,), generator=g).float()
        s[torch.rand(n, generator=g) < 0.15] = float("-inf")
        mask = torch.rand(n, generator=g) < 0.8
        budget = int(torch.randint(1, 70, (1,), generator=g))
        got = O.nucleus_select(s, budget, 1.0, keep_mask=mask, index_offset=100, drop_nonfinite=True)
        ms = torch.where(mask, s, torch.full_like(s, float("-inf")))
        safe = [(v if math.isfinite(v) else -1e9) for v in ms.tolist()]
        order = sorted(range(n), key=lambda j: (-safe[j], j))[:min(budget, n)]
        keep = [j for j in order if math.isfinite(ms[j].item())]
        if not keep:
            assert got is None
            continue
        assert got[1].tolist() == [j + 100 for j in keep]
        assert got[0].tolist() == [ms[j].item() for j in keep]
        # finalise: one survivor per index (its last entry in score order)
        idx = torch.randint(0, 15, (n,), generator=g)
        sc = torch.randint(-2, 3, (n,), generator=g).float()
        m = int(torch.randint(0, 20, (1,), generator=g))
        ki, ks = O.finalise_indices(sc, idx, m)
        order = sorted(range(n), key=lambda j: (-sc[j].item(), j))
        last = {}
        for rank, j in enumerate(order):
            last[idx[j].item()] = rank
        chosen = sorted(last.items(), key=lambda kv: kv[1])[:m]
        expect = sorted((ix, sc[order[r]].item()) for ix, r in chosen)
        assert ki.tolist() == [e[0] for e in expect] and ks.tolist() == [e[1] for e in expect]


def test_quantize_rows_int8_invariants():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(37, 4 * 16, generator=g) * torch.rand(37, 1, generator=g) * 5
    x[3] = 0.0
    q, s = O.quantize_rows_int8(x, 4)
    xr = x.view(37, 4, 16).permute(1, 0, 2)
    amax = xr.abs().amax(-1)
    assert torch.equal(s, torch.clamp(amax / 127.0, min=1e-6))
    # the absmax element maps to +-127, every element within half a step
    assert bool((q.abs().amax(-1)[amax > 0] == 127).all())
    assert float((q.float() * s.unsqueeze(-1) - xr).abs().max()) <= float(s.max()) * 0.5 + 1e-7
    assert int(q[:, 3].abs().max()) == 0


def test_int8_kv_attention_oracle_matches_sdpa_and_brute_force():
    g = torch.Generator().manual_seed(11)
    T, H, D, S = 40, 2, 8, 9
    q = torch.randn(T, H, D, generator=g)
    k8 = torch.randint(-127, 128, (H, S, D), generator=g).to(torch.int8)
    v8 = torch.randint(-127, 128, (H, S, D), generator=g).to(torch.int8)
    ks = torch.rand(H, S, generator=g) * 0.02
    vs = torch.rand(H, S, generator=g) * 0.02
    pos = torch.sort(torch.randperm(T, generator=g)[:S]).values
    pos[0] = 5  # queries 0..4 see no key
    pos = torch.sort(pos).values
    out = O.int8_kv_attention(q, k8, v8, ks, vs, pos, causal=True)
    k = k8.float() * ks.unsqueeze(-1)
    v = v8.float() * vs.unsqueeze(-1)
    vis = pos.view(1, -1) <= torch.arange(T).view(-1, 1)
    ref = F.scaled_dot_product_attention(q.permute(1, 0, 2), k, v, attn_mask=vis)
    rows = vis.any(-1)
    assert torch.allclose(out.permute(1, 0, 2)[:, rows], ref[:, rows], atol=1e-6)
    assert float(out[~rows].abs().max()) == 0.0
    # brute force one query per head, including the last (sees every key)
    for h in range(H):
        for t in (7, T - 1):
            sc = [(q[t, h] @ k[h, j]).item() / math.sqrt(D) for j in range(S) if pos[j] <= t]
            w = torch.softmax(torch.tensor(sc), 0)
            vv = v[h][pos <= t]
            assert torch.allclose(out[t, h], (w.unsqueeze(-1) * vv).sum(0), atol=1e-6)
    # non-causal: every key visible
    nc = O.int8_kv_attention(q, k8, v8, ks, vs, pos, causal=False)
    assert torch.allclose(nc.permute(1, 0, 2), F.scaled_dot_product_attention(q.permute(1, 0, 2), k, v), atol=1e-6)


def _rope_golden(z, D, tag, name):
    arr = torch.from_numpy(np.ascontiguousarray(z[f"D{D}_{tag}_{name}"]))
    return arr.view(torch.bfloat16) if tag == "bf16" else arr


@pytest.mark.parametrize("D", [64, 32])
@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_rope_oracle_and_module_tables_match_reference(golden, D, tag):
    """oracle.rope_tables / apply_rope and the module's _rope_factors bit for
    bit against the reference module's _rope_factors / _apply_rope_embedding
    (aspa.py:226-247, 576-618) in f32 and in bf16 (the cast module computes
    positions and angles in bf16), T = 1024."""
    from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

    z = golden("rope_tables")
    T, base, every = int(z["T"]), float(z["base"]), int(z["every"])
    dt = torch.bfloat16 if tag == "bf16" else torch.float32
    cos, sin = O.rope_tables(T, D, base, dt, freq_dtype=dt)
    assert torch.equal(cos, _rope_golden(z, D, tag, "cos")) and torch.equal(sin, _rope_golden(z, D, tag, "sin"))
    for a, b in (("q", "qo"), ("k", "ko")):
        x = _rope_golden(z, D, tag, a)
        got = O.apply_rope(x, cos[::every], sin[::every])
        assert torch.equal(got, _rope_golden(z, D, tag, b)), (a, D, tag)
    H = 256 // D
    m = AdaptiveSparseAttention(ModelConfig(d_model=256, n_head=H, attn_h_total=H, attn_gates=H)).to(dt)
    mc, ms = m._rope_factors(T, torch.device("cpu"), dt)
    assert torch.equal(mc, cos) and torch.equal(ms, sin)
    if tag == "bf16":
        # planted mistake: angles formed in f32 (the buffer left in f32)
        # round differently above position 256 and must not match
        c32, _ = O.rope_tables(T, D, base, dt, freq_dtype=torch.float32)
        assert not torch.equal(c32, _rope_golden(z, D, tag, "cos"))
