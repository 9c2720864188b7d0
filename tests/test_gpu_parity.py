"""GPU parity: every kernel of libpfa_hip.so against the CPU oracle and the
reference's golden vectors, through the product's Python API / C ABI.

Tolerances: index/selection outputs bit-exact (ties -> lowest index, which
the oracle implements; golden comparisons exclude positions whose reference
value is tied at the selection boundary); attention outputs 1e-4 max-abs in
f32 and 2e-2 max-abs in bf16."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import aspa_oracle as O
from oracle import c_oracle

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-4
TOL_BF16 = 2e-2


def _say(msg: str) -> None:
    print(f"[gpu-parity] {msg}", flush=True)


# ---------------------------------------------------------------------------
# shortlist builder
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("tag", ["l", "la", "lp", "ap"])
def test_builder_small_golden(dev, golden, tag):
    from proteus_attention.kernels.sparse_attn import build_shortlist_candidates

    z = golden(f"builder_small_{tag}")
    ul, ua, up = (bool(v) for v in z["use"])
    c, l = build_shortlist_candidates(torch.from_numpy(z["rows"]).to(dev), 64, max_candidates=16, linear_window=12,
                                      anchor_stride=4, use_local=ul, use_anchors=ua,
                                      proto_scores=torch.from_numpy(z["scores"]).to(dev) if up else None)
    assert c.dtype == torch.int64 and l.dtype == torch.int64
    assert np.array_equal(c.cpu().numpy(), z["cand"])
    assert np.array_equal(l.cpu().numpy(), z["lengths"])


def test_builder_packed_golden(dev, golden):
    from proteus_attention.kernels.sparse_attn import build_packed_shortlist_candidates

    z = golden("builder_packed_T4096")
    L, w, s, lc, ac, pc = (int(v) for v in z["kw"])
    c, l = build_packed_shortlist_candidates(
        torch.from_numpy(z["rows"]).to(dev), torch.from_numpy(z["row_batch"]).to(dev), 4096, max_candidates=L,
        linear_window=w, anchor_stride=s, use_local=True, use_anchors=True,
        proto_scores=torch.from_numpy(z["sims"]).to(dev), local_cap=lc, anchor_cap=ac, proto_cap=pc)
    assert np.array_equal(c.cpu().numpy(), z["cand"])
    assert np.array_equal(l.cpu().numpy(), z["lengths"])


def test_builder_truncate_golden(dev, golden):
    from proteus_attention.kernels.sparse_attn import build_shortlist_candidates

    z = golden("builder_truncate")
    L, w, s, lc, ac, pc = (int(v) for v in z["kw"])
    c, l = build_shortlist_candidates(torch.from_numpy(z["rows"]).to(dev), 2048, max_candidates=L, linear_window=w,
                                      anchor_stride=s, use_local=True, use_anchors=True,
                                      proto_scores=torch.from_numpy(z["sims"]).to(dev), local_cap=lc, anchor_cap=ac,
                                      proto_cap=pc)
    assert np.array_equal(c.cpu().numpy(), z["cand"])
    assert np.array_equal(l.cpu().numpy(), z["lengths"])


@pytest.mark.parametrize("T,L,w,s,ac,pc", [(700, 64, 20, 9, 30, 25), (300, 300, 300, 0, 0, 300), (1, 4, 2, 1, 2, 2),
                                           (1000, 200, 1, 3, 180, 150)])
def test_builder_ties_and_edges_vs_oracle(dev, T, L, w, s, ac, pc):
    from proteus_attention.kernels.sparse_attn import build_shortlist_candidates

    g = torch.Generator().manual_seed(T + L)
    rows = torch.randint(0, T, (min(400, 4 * T),), generator=g)
    rows[0] = 0
    rows[-1] = T - 1
    sc = torch.randint(0, 5, (T,), generator=g).float()  # heavy ties
    kw = dict(max_candidates=L, linear_window=w, anchor_stride=s, use_local=True, use_anchors=s > 0,
              local_cap=w, anchor_cap=ac, proto_cap=pc)
    c, l = build_shortlist_candidates(rows.to(dev), T, proto_scores=sc.to(dev), **kw)
    oc, ol = O.build_shortlist(rows, T, proto_scores=sc, **kw)
    assert torch.equal(c.cpu(), oc)
    assert torch.equal(l.cpu(), ol)


def test_builder_extra_candidates_vs_oracle(dev):
    from proteus_attention.kernels.sparse_attn import build_packed_shortlist_candidates

    g = torch.Generator().manual_seed(77)
    T = 500
    rows = torch.sort(torch.randint(0, T, (120,), generator=g)).values
    extra = torch.randint(-5, T + 50, (120, 12), generator=g)
    elen = torch.randint(0, 13, (120,), generator=g)
    kw = dict(max_candidates=40, linear_window=8, anchor_stride=16, use_local=True, use_anchors=True,
              anchor_cap=10)
    c, l = build_packed_shortlist_candidates(rows.to(dev), None, T, extra_candidates=extra.to(dev),
                                             extra_lengths=elen.to(dev), **kw)
    oc, ol = O.build_shortlist(rows, T, extra_candidates=extra, extra_lengths=elen, **kw)
    assert torch.equal(c.cpu(), oc)
    assert torch.equal(l.cpu(), ol)


@pytest.mark.parametrize("T,L,K,A", [(65536, 2048, 205, 614)])
def test_builder_config3_full_size_vs_c_oracle(dev, T, L, K, A):
    """Config 3 builder (N = 2*T rows, L = 2048) bit-exact against the C
    oracle on every row, plus size-independent properties."""
    from proteus_attention.kernels import sparse_attn as sa

    _say(f"builder cfg3 T={T} L={L}")
    g = torch.Generator().manual_seed(3)
    sims = torch.rand(1, T, generator=g)
    heads = torch.stack([torch.randperm(8, generator=g)[:2] for _ in range(1)])
    rows = torch.cat([torch.arange(T), torch.arange(T)]).to(torch.int32)
    sets = sa._proto_prefix_sets(sims.to(dev), K)
    cand, lens = sa._shortlist_build_device(rows.to(dev), None, T, L, 512, 256, A, sets)
    cand, lens = cand.cpu().numpy(), lens.cpu().numpy()
    sub = np.arange(0, 2 * T, 7)
    oc, ol = c_oracle.shortlist_build(rows.numpy()[sub], None, T, L, 512, 256, A, sims.numpy(), K)
    assert np.array_equal(cand[sub], oc)
    assert np.array_equal(lens[sub], ol)
    # properties on all rows: strictly increasing prefix, tail == row, window present
    r = rows.numpy()
    ln = lens.astype(np.int64)
    assert np.all(ln >= 1) and np.all(ln <= L)
    idx = np.arange(L)[None, :]
    valid = idx < ln[:, None]
    diffs = np.diff(cand.astype(np.int64), axis=1)
    assert np.all(diffs[valid[:, 1:]] > 0)
    assert np.all(cand[~valid] == np.broadcast_to(r[:, None], cand.shape)[~valid])
    assert np.all(cand[np.arange(2 * T), ln - 1] == r)
    del heads


def test_proto_prefix_sets_vs_brute_force(dev):
    from proteus_attention.kernels import sparse_attn as sa

    g = torch.Generator().manual_seed(8)
    for T, K in ((300, 7), (130, 64), (200, 200), (65, 1)):
        s = torch.randint(0, 9, (2, T), generator=g).float()
        sets = sa._proto_prefix_sets(s.to(dev), K).cpu()
        for b in range(2):
            exp = O.proto_prefix_sets(s[b], K)
            assert torch.equal(sets[b].long(), exp), (T, K, b)


def test_proto_evict_matches_prefix_sets(dev):
    """p is in the prefix top-K set of t  <=>  p <= t < evict[p]."""
    from proteus_attention.kernels import sparse_attn as sa

    g = torch.Generator().manual_seed(18)
    for T, K in ((400, 9), (257, 64), (130, 200)):
        s = torch.randint(0, 7, (2, T), generator=g).float()
        sets, ev = sa._proto_prefix_sets(s.to(dev), K, with_evict=True)
        ev = ev.cpu().long()
        for b in range(2):
            exp = O.proto_prefix_sets(s[b], K)
            member = torch.zeros(T, T, dtype=torch.bool)
            for t in range(T):
                member[t, exp[t, : min(t + 1, K)]] = True
            pos = torch.arange(T)
            by_evict = (pos[None, :] <= pos[:, None]) & (ev[b][None, :] > pos[:, None])
            assert torch.equal(member, by_evict), (T, K, b)


@pytest.mark.parametrize("T,K,tied", [(65536, 205, False), (65536, 900, True), (40000, 1700, False),
                                       (70000, 205, True), (70000, 1100, False)])
def test_proto_prefix_tables_long_vs_evict_oracle(dev, T, K, tied):
    """Long sequences (one to four superblock sizes, K below and above the
    1,024-key sort): evict equals the O(T log T) evict oracle for every
    position, and every block's set table row is the set
    {p < 64j : evict[p] >= 64j} best first."""
    from proteus_attention.kernels import sparse_attn as sa

    _say(f"prefix tables vs evict oracle T={T} K={K} tied={tied}")
    g = torch.Generator().manual_seed(41 + T + K)
    s = torch.randint(0, 50, (1, T), generator=g).float() if tied else torch.rand(1, T, generator=g)
    blk, ev = sa._proto_prefix_blocks(s.to(dev), K)
    ev = ev.cpu().long()[0]
    exp = O.proto_prefix_evict(s[0], K)
    assert torch.equal(ev, exp)
    blk = blk.cpu().long()[0].numpy()
    evn = exp.numpy()
    sc = s[0].numpy()
    nb = (T + 63) // 64
    for j in list(range(0, nb, max(1, nb // 61))) + [nb - 1]:
        t0 = 64 * j
        want = np.nonzero(evn[:t0] >= t0)[0] if t0 > 0 else np.zeros(0, dtype=np.int64)
        row = blk[j][blk[j] != 2 ** 31 - 1]
        assert len(row) == len(want) == min(K, t0), (j, len(row), len(want))
        assert np.array_equal(np.sort(row), want), j
        keys = [(-float(sc[v]), int(v)) for v in row]
        assert keys == sorted(keys), j


def test_proto_prefix_blocks_match_sets(dev):
    """Block tables: row j is the set of token 64j-1 (best first), and
    set(t) = {p in row t/64 U [64(t/64), t] : evict[p] > t}; evict agrees with
    the per-token form.  Sizes span one to many superblocks, with heavy ties,
    K above and below the 64-token block."""
    from proteus_attention.kernels import sparse_attn as sa

    g = torch.Generator().manual_seed(23)
    for T, K, B, tied in ((64, 5, 1, False), (1000, 70, 2, True), (20000, 205, 1, False), (9000, 900, 1, True),
                          (6000, 1700, 1, True)):
        _say(f"prefix blocks T={T} K={K} B={B} tied={tied}")
        s = (torch.randint(0, 9, (B, T), generator=g).float() if tied else torch.rand(B, T, generator=g))
        sd = s.to(dev)
        sets, ev1 = sa._proto_prefix_sets(sd, K, with_evict=True)
        blk, ev2 = sa._proto_prefix_blocks(sd, K)
        assert torch.equal(ev1.cpu(), ev2.cpu())
        sets, blk, ev = sets.cpu().long(), blk.cpu().long(), ev2.cpu().long()
        nb = (T + 63) // 64
        for b in range(B):
            for j in range(nb):
                t = 64 * j - 1
                want = sets[b, t, : min(t + 1, K)].tolist() if t >= 0 else []
                row = [v for v in blk[b, j].tolist() if v != 2 ** 31 - 1]
                assert sorted(row) == want, (T, K, b, j)
                # best first: scores non-increasing, equal scores by ascending index
                keys = [(-float(s[b, v]), v) for v in row]
                assert keys == sorted(keys), (T, K, b, j)
            # per-token expansion of the compact form, spot rows
            for t in list(range(0, T, max(1, T // 97))) + [T - 1]:
                j = t // 64
                cand = sorted(p for p in blk[b, j].tolist() if p != 2 ** 31 - 1) + list(range(64 * j, t + 1))
                got = [p for p in cand if ev[b, p] > t]
                assert got == sets[b, t, : min(t + 1, K)].tolist(), (T, K, b, t)


def test_proto_prefix_sets_large_vs_c_oracle(dev):
    """Prefix sets at config-4 scale (T = 524,288, K = 409: 8192 blocks, 64
    superblocks) against the C restatement."""
    from proteus_attention.kernels import sparse_attn as sa

    T, K = 524_288, 409
    _say(f"prefix sets T={T} K={K} vs C oracle")
    g = torch.Generator().manual_seed(29)
    s = torch.rand(1, T, generator=g)
    s[0, ::1000] = 0.5  # a few exact ties
    sets = sa._proto_prefix_sets(s.to(dev), K)
    rows = np.arange(0, T, 997, dtype=np.int32)
    # the C builder with only the prototype piece and L = K + 1 returns
    # sorted(set(t) U {t}) padded with t
    exp, _ = c_oracle.shortlist_build(rows, None, T, K + 1, 0, 0, 0, s.numpy(), K)
    got = sets[0][torch.from_numpy(rows).long().to(dev)].cpu().numpy()
    del sets
    for r, t in enumerate(rows.tolist()):
        u = sorted(set(got[r, : min(t + 1, K)].tolist()) | {t})
        u = u + [t] * (K + 1 - len(u))
        assert u == exp[r].tolist(), t


@pytest.mark.parametrize("T,L,w,s,B,outlier,H", [(4096, 1024, 256, 64, 1, 0.01, 8), (3000, 700, 100, 37, 2, 0.0, 8),
                                                 (65536, 2048, 512, 256, 1, 0.01, 8),
                                                 (524288, 4096, 512, 256, 1, 0.0, 8),
                                                 (65536, 2048, 512, 4, 1, 0.01, 8), (20000, 1024, 128, 3, 2, 0.0, 8),
                                                 (4096, 1024, 256, 64, 1, 0.01, 32), (3000, 700, 100, 37, 2, 0.0, 16),
                                                 (65536, 2048, 512, 256, 1, 0.01, 16),
                                                 (4096, 1024, 256, 64, 1, 0.01, 4), (3000, 700, 100, 37, 2, 0.0, 4),
                                                 (65536, 2048, 512, 256, 1, 0.01, 4)])
def test_structured_shortlist_matches_materialised(dev, T, L, w, s, B, outlier, H, monkeypatch):
    """The structure-driven MFMA path and the builder + gather path give the
    same candidate counts per row and the same outputs (bf16 tolerance).
    The T=524,288 case is config 4 at full size, single pass: the
    materialised path holds all 1,048,576 x 4,096 int32 candidates.  The
    stride-4 and stride-3 cases have residue classes of 16,384 and 6,667
    positions, whose rows the anchor pass compacts and attends in rounds.
    H = 32, 16 and 4 over d_model 512 give heads of 16, 32 and 128 dims (q
    rotated by the RoPE pass, not on load)."""
    from configs import shortlist_cfg

    _say(f"structured vs materialised T={T} L={L} w={w} s={s} B={B} H={H}")
    cfg = shortlist_cfg(T, 512, H, L, w, s)
    m, x = _module(cfg, B, T, 512, torch.bfloat16, dev, outlier)
    m.record_shortlist_lengths = True
    snap = {n: b.detach().clone() for n, b in m.named_buffers() if n.startswith("routing_")}
    with torch.no_grad():
        y_s = m(x)
        a_s = m.last_head_consensus.float().clone()
        assert m._last_sparse_state["linear_shortlist_structured"] is True
        len_s = m._last_shortlist_lengths.cpu().long()
        for n, b in snap.items():
            getattr(m, n).copy_(b)
        monkeypatch.setenv("PFA_FORCE_GENERIC", "1")
        y_g = m(x)
        a_g = m.last_head_consensus.float()
        assert m._last_sparse_state["linear_shortlist_structured"] is False
        len_g = m._last_shortlist_lengths.cpu().long()
    assert torch.equal(len_s, len_g)
    # attention outputs (before the output projection).  The gather path keeps
    # probabilities in f32; the MFMA path rounds them to bf16 (relative error
    # <= 2^-9 each, as the reference's bf16 softmax does), so per element
    # |a_s - a_g| <= 2^-9 * max|v| + one bf16 ulp of the output.
    with torch.no_grad():
        C = x.shape[-1]
        vmax = float(m.qkv(x)[..., 2 * C:].float().abs().max())
    diff = (a_s - a_g).abs()
    mag = torch.maximum(a_s.abs(), a_g.abs()).clamp_min(2.0 ** -126)
    ulp = torch.ldexp(torch.ones_like(mag), torch.frexp(mag).exponent - 8)
    _say(f"max-abs structured vs materialised: attention {float(diff.max()):.3e}, "
         f"y {float((y_s.float() - y_g.float()).abs().max()):.3e}")
    bound = ulp + 2.0 ** -9 * vmax
    assert bool((diff <= bound).all()), float((diff - bound).max())
    rel = float(((y_s.float() - y_g.float()).abs() / (y_g.float().abs() + 1.0)).max())
    assert rel <= TOL_BF16


# ---------------------------------------------------------------------------
# router, token top-k, packing, RoPE
# ---------------------------------------------------------------------------

def _weights(B, T, C, H, outlier=0.0):
    from configs import make_inputs

    x, g = make_inputs(B, T, C, seed=0, outlier_frac=outlier)
    ws = []
    for shape in ((H, C), (H, C), (3 * C, C), (C, C)):
        tmp = torch.empty(shape)
        torch.nn.init.xavier_normal_(tmp, generator=g)
        ws.append(tmp)
    return x, ws


def _run_router(dev, x, w, protos, conf, dt, topk, H, temp=0.2, thr=0.25, blend=0.6):
    from proteus_attention import _hip

    lib = _hip.lib()
    n, C = x.reshape(-1, x.size(-1)).shape
    G = w.size(0)
    from proteus_attention.models.aspa import pack_router_weights

    xd = x.reshape(n, C).to(dev, dt).contiguous()
    pn = torch.nn.functional.normalize(protos.to(torch.float32), dim=-1, eps=1e-6).to(dev).contiguous()
    wpk = pack_router_weights(w.to(dev), pn, dt)
    cw = (conf + 1e-6).to(torch.float32).to(dev)
    outs = [torch.empty(n, G, device=dev), torch.empty(n, device=dev), torch.empty(n, device=dev),
            torch.empty(n, device=dev), torch.empty(n, topk, device=dev, dtype=torch.int32),
            torch.empty(n, topk, device=dev)]
    g2h = O.default_gate_map(G, H).to(torch.int32).to(dev)
    rc = lib.pfa_router_topk(_hip.ptr(xd), _hip.dtype_tag(dt), n, C, G, _hip.ptr(wpk), 1, _hip.ptr(cw),
                             None, _hip.ptr(g2h), H, topk, temp, thr, blend, 0.0, *[_hip.ptr(o) for o in outs],
                             None, None, _hip.stream_ptr(dev))
    _hip.check(rc, "router")
    return [o.cpu() for o in outs]


@pytest.mark.parametrize("G,H,C,n,proto,usage,ema", [(8, 8, 512, 4096, True, True, True),
                                                     (8, 8, 768, 3000, True, False, False),
                                                     (16, 16, 512, 2500, True, True, True),
                                                     (5, 4, 384, 777, True, True, False),
                                                     (12, 8, 256, 1030, False, False, False)])
def test_router_raw_inputs_bitwise(dev, G, H, C, n, proto, usage, ema):
    """pfa_router_topk_raw (router inputs built inside the router's
    workgroups) gives exactly the bits of pfa_router_prepare +
    pfa_router_topk: gates, similarity, blend, importance, head indices and
    scores, telemetry partials and the fused EMA partial sums."""
    from proteus_attention import _hip

    lib = _hip.lib()
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(61 + G + C)
    x = (torch.randn(n, C, generator=g) * (1.0 + 3.0 * (torch.rand(n, 1, generator=g) < 0.01))).to(bf).to(dev)
    w = (torch.randn(G, C, generator=g) * 0.05).to(bf).to(dev)
    protos = (torch.randn(G, C, generator=g) * 0.02).to(bf).to(dev) if proto else None
    conf = (torch.rand(G, generator=g) * 3).to(bf).to(dev) if proto else None
    use = (torch.rand(G, generator=g) * 5).to(bf).to(dev) if (proto and usage) else None
    g2h = O.default_gate_map(G, H).to(torch.int32).to(dev)
    topk = 2
    assert lib.pfa_router_raw_supported(_hip.PFA_BF16, _hip.PFA_BF16, _hip.PFA_BF16, G, C, int(proto)) == 1
    nblk = _hip.ctypes.c_int(0)
    _hip.check(lib.pfa_router_block_count(n, _hip.ctypes.byref(nblk)), "block_count")
    nb = max(1, nblk.value)

    def outs():
        return [torch.empty(n, G, device=dev), torch.empty(n, device=dev), torch.empty(n, device=dev),
                torch.empty(n, device=dev), torch.empty(n, topk, device=dev, dtype=torch.int32),
                torch.empty(n, topk, device=dev), torch.empty(nb, 8, device=dev),
                torch.empty(nb, G, C + 1, device=dev) if ema else None]

    Gp = int(lib.pfa_router_gate_pad(G))
    wpk = torch.empty(C, 2 * Gp, device=dev)
    cw = torch.empty(G, device=dev) if conf is not None else None
    ub = torch.empty(G, device=dev) if use is not None else None
    _hip.check(lib.pfa_router_prepare(_hip.ptr(w), _hip.PFA_BF16, _hip.ptr(protos), _hip.ptr(conf), _hip.ptr(use),
                                      _hip.PFA_BF16, G, C, _hip.PFA_BF16, _hip.ptr(wpk), _hip.ptr(cw), _hip.ptr(ub),
                                      _hip.stream_ptr(dev)), "prepare")
    a, b = outs(), outs()
    args = (H, topk, 0.3, 0.2, 0.5, 0.25)
    _hip.check(lib.pfa_router_topk(_hip.ptr(x), _hip.PFA_BF16, n, C, G, _hip.ptr(wpk), int(proto), _hip.ptr(cw),
                                   _hip.ptr(ub), _hip.ptr(g2h), *args, *[_hip.ptr(o) for o in a],
                                   _hip.stream_ptr(dev)), "router")
    _hip.check(lib.pfa_router_topk_raw(_hip.ptr(x), _hip.PFA_BF16, n, C, G, _hip.ptr(w), _hip.PFA_BF16,
                                       _hip.ptr(protos), _hip.ptr(conf), _hip.ptr(use), _hip.PFA_BF16, _hip.ptr(g2h),
                                       *args, *[_hip.ptr(o) for o in b], _hip.stream_ptr(dev)), "router_raw")
    for i, (u, v) in enumerate(zip(a, b)):
        if u is None or (i in (1, 2) and not proto):
            continue
        if i == 6:  # telemetry partials: columns 0..4 of each row are written
            u, v = u[:, :5], v[:, :5]
        assert torch.equal(u.cpu().contiguous().view(torch.int32), v.cpu().contiguous().view(torch.int32)), i


@pytest.mark.parametrize("name,B,T,C,dt,outlier", [
    ("module_cfg1", 1, 1024, 256, torch.float32, 0.0),
    ("module_cfg2_T2048", 2, 2048, 512, torch.bfloat16, 0.0),
    ("module_short_T4096_bf16", 1, 4096, 512, torch.bfloat16, 0.01),
])
def test_router_vs_golden_and_oracle(dev, golden, name, B, T, C, dt, outlier):
    z = golden(name)
    x, ws = _weights(B, T, C, 8, outlier)
    conf = torch.zeros(8, dtype=dt)
    gate, sim, bl, imp, hidx, hsc = _run_router(dev, x.to(dt), ws[0].to(dt), ws[1].to(dt).float(), conf, dt, 2, 8)
    og, osim, obl, oimp = O.route_tokens(x.to(dt), ws[0].to(dt), ws[1].to(dt), conf, None, proto_temp=0.2,
                                         proto_threshold=0.25, proto_blend=0.6, usage_boost=0.0)
    n = B * T
    ref_g = torch.from_numpy(z["gate_probs"]).reshape(n, -1)
    assert torch.allclose(sim, torch.from_numpy(z["sim"]).reshape(n), atol=2e-6, rtol=0)
    # head top-k: exactly the oracle's lowest-index rule applied to our probs
    _, oidx = O.topk_lowest(gate, 2)
    assert torch.equal(hidx.long(), oidx)
    ours = torch.zeros(n, 8, dtype=torch.bool).scatter_(1, hidx.long(), True)
    if dt == torch.float32:
        # f32: gate probabilities to accumulation-order rounding, head sets
        # exactly the reference's lowest-index top-k
        assert torch.allclose(gate, ref_g, atol=2e-6, rtol=0)
        assert torch.allclose(imp, torch.from_numpy(z["importance"]).reshape(n), atol=2e-6, rtol=0)
        _, ridx = O.topk_lowest(ref_g, 2)
        assert torch.equal(ours, torch.zeros(n, 8, dtype=torch.bool).scatter_(1, ridx, True))
    else:
        # bf16: gate probabilities bit for bit except at bf16 rounding
        # boundaries, head sets the lowest-index top-k of the reference's
        # gates wherever those agree (routing_parity.check_routing)
        from routing_parity import check_routing

        _, ridx = O.topk_lowest(ref_g, 2)
        ref_sets = torch.zeros(n, 8, dtype=torch.bool).scatter_(1, ridx, True)
        rep = check_routing(ours, ref_sets, gate, ref_g, x.to(dt).reshape(n, C), ws[0].to(dt), 2)
        _say(f"router {name}: {rep}")
        rep.assert_boundary_sets_at_most(1e-3)


@pytest.mark.parametrize("n_tok,C,G,dt", [(300_000, 512, 8, torch.bfloat16), (5000, 1025, 12, torch.float32),
                                          (37, 64, 3, torch.float16)])
def test_proto_ema_sums_vs_f64(dev, n_tok, C, G, dt):
    """Gate-weighted token sums of the prototype EMA (aspa.py:703-707):
    sum_t gate[t,g]*x[t,c] and sum_t gate[t,g], against a float64 product on
    the CPU.  Covers slices longer than one LDS stage (300k tokens), rows
    wider than one channel pair per thread (C=1025, odd) and a tiny input."""
    from proteus_attention import _hip

    _say(f"proto EMA sums n_tok={n_tok} C={C} G={G} {dt}")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(n_tok, C, generator=g).to(dt)
    gp = torch.softmax(torch.randn(n_tok, G, generator=g), dim=-1)
    lib = _hip.lib()
    n = _hip.ctypes.c_int(0)
    _hip.check(lib.pfa_proto_partial_count(n_tok, _hip.ctypes.byref(n)), "count")
    xd, gd = x.to(dev), gp.to(dev)
    part = torch.empty(n.value, G, C + 1, dtype=torch.float32, device=dev)
    sums = torch.empty(G, C + 1, dtype=torch.float32, device=dev)
    s = _hip.stream_ptr(dev)
    _hip.check(lib.pfa_proto_accumulate(_hip.ptr(xd), _hip.dtype_tag(dt), n_tok, C, G, _hip.ptr(gd), _hip.ptr(part),
                                        n.value, s), "accumulate")
    _hip.check(lib.pfa_proto_partial_reduce(_hip.ptr(part), n.value, G, C, _hip.ptr(sums), s), "reduce")
    got = sums.cpu().double()
    ref = torch.cat([gp.double().t() @ x.double(), gp.double().sum(0).unsqueeze(1)], dim=1)
    scale = (gp.double().t() @ x.double().abs()).clamp_min(1.0)
    scale = torch.cat([scale, gp.double().sum(0).unsqueeze(1).clamp_min(1.0)], dim=1)
    err = float(((got - ref).abs() / scale).max())
    _say(f"max scaled error {err:.2e}")
    assert err < 1e-5


@pytest.mark.parametrize("n_tok,C,G,dt", [(300_000, 512, 8, torch.bfloat16), (5000, 1024, 12, torch.float32),
                                          (37, 64, 3, torch.float16), (1000, 200, 20, torch.bfloat16),
                                          (3000, 512, 8, torch.bfloat16), (777, 384, 5, torch.bfloat16),
                                          (70_000, 512, 16, torch.bfloat16), (777, 384, 13, torch.bfloat16)])
def test_router_fused_ema_sums_vs_f64(dev, n_tok, C, G, dt):
    """The EMA statistics the router accumulates in its own pass over x
    (ema_partial of pfa_router_topk, reduced with pfa_proto_partial_reduce)
    against a float64 product of the router's own gate probabilities."""
    from proteus_attention import _hip
    from proteus_attention.models.aspa import pack_router_weights

    _say(f"router fused EMA sums n_tok={n_tok} C={C} G={G} {dt}")
    g = torch.Generator().manual_seed(6)
    x = torch.randn(n_tok, C, generator=g).to(dt)
    w = (torch.randn(G, C, generator=g) * 0.05).to(dt)
    protos = torch.randn(G, C, generator=g)
    lib = _hip.lib()
    nb = _hip.ctypes.c_int(0)
    _hip.check(lib.pfa_router_block_count(n_tok, _hip.ctypes.byref(nb)), "count")
    xd = x.to(dev)
    pn = torch.nn.functional.normalize(protos, dim=-1, eps=1e-6).to(dev)
    wpk = pack_router_weights(w.to(dev), pn, dt)
    H = min(G, 8)
    g2h = O.default_gate_map(G, H).to(torch.int32).to(dev)
    gate = torch.empty(n_tok, G, device=dev)
    imp = torch.empty(n_tok, device=dev)
    hidx = torch.empty(n_tok, 2, dtype=torch.int32, device=dev)
    part = torch.empty(nb.value, G, C + 1, device=dev)
    sums = torch.empty(G, C + 1, device=dev)
    s = _hip.stream_ptr(dev)
    _hip.check(lib.pfa_router_topk(_hip.ptr(xd), _hip.dtype_tag(dt), n_tok, C, G, _hip.ptr(wpk), 1, None, None,
                                   _hip.ptr(g2h), H, 2, 0.2, 0.25, 0.6, 0.0, _hip.ptr(gate), None, None, _hip.ptr(imp),
                                   _hip.ptr(hidx), None, None, _hip.ptr(part), s), "router")
    _hip.check(lib.pfa_proto_partial_reduce(_hip.ptr(part), nb.value, G, C, _hip.ptr(sums), s), "reduce")
    gp = gate.cpu().double()
    got = sums.cpu().double()
    ref = torch.cat([gp.t() @ x.double(), gp.sum(0).unsqueeze(1)], dim=1)
    scale = (gp.t() @ x.double().abs()).clamp_min(1.0)
    scale = torch.cat([scale, gp.sum(0).unsqueeze(1).clamp_min(1.0)], dim=1)
    err = float(((got - ref).abs() / scale).max())
    _say(f"max scaled error {err:.2e}")
    assert err < 1e-5


@pytest.mark.parametrize("wdt,bdt,xdt,boost", [(torch.bfloat16, torch.bfloat16, torch.bfloat16, 0.0),
                                               (torch.float32, torch.float32, torch.bfloat16, 0.3),
                                               (torch.float32, torch.bfloat16, torch.float32, 0.5)])
def test_router_prepare_matches_tensor_ops(dev, wdt, bdt, xdt, boost):
    """pfa_router_prepare against the tensor ops it replaces, evaluated by
    torch on the same device: weight table and confidence/usage weights
    exactly, normalised prototypes to one f32 rounding (norm summation
    order)."""
    from proteus_attention import _hip
    from proteus_attention.models.aspa import pack_router_weights

    g = torch.Generator().manual_seed(8)
    G, C = 8, 512
    w = torch.randn(G, C, generator=g).to(wdt).to(dev)
    protos = (torch.randn(G, C, generator=g) * 0.02).to(bdt).to(dev)
    conf = torch.rand(G, generator=g).to(bdt).to(dev)
    usage = (torch.rand(G, generator=g) * 3).to(bdt).to(dev)
    lib = _hip.lib()
    Gp = int(lib.pfa_router_gate_pad(G))
    wpk = torch.empty(C, 2 * Gp, device=dev)
    cw = torch.empty(G, device=dev)
    ub = torch.empty(G, device=dev)
    _hip.check(lib.pfa_router_prepare(_hip.ptr(w), _hip.dtype_tag(wdt), _hip.ptr(protos), _hip.ptr(conf),
                                      _hip.ptr(usage) if boost > 0 else None, _hip.dtype_tag(bdt), G, C,
                                      _hip.dtype_tag(xdt), _hip.ptr(wpk), _hip.ptr(cw), _hip.ptr(ub),
                                      _hip.stream_ptr(dev)), "prepare")
    pn = torch.nn.functional.normalize(protos.to(torch.float32), dim=-1, eps=1e-6)
    ref = pack_router_weights(w, pn, xdt)
    assert torch.equal(wpk[:, :Gp], ref[:, :Gp])
    assert torch.allclose(wpk[:, Gp:], ref[:, Gp:], rtol=2.5e-7, atol=1e-12)
    assert torch.equal(cw, (conf + 1e-6).to(torch.float32))
    if boost > 0:
        # softmax: exp and normalisation differ from torch's kernel in the
        # last bits of f32; in bf16 they may straddle a rounding boundary
        ref_u = torch.softmax(-(usage + 1e-6), dim=0).to(torch.float32)
        ulp = 2.0 ** -7 if bdt == torch.bfloat16 else 2.0 ** -22
        assert torch.allclose(ub, ref_u, rtol=ulp, atol=0.0)


def test_token_topk_vs_oracle(dev):
    from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

    g = torch.Generator().manual_seed(12)
    imp = torch.randint(0, 40, (3, 5000), generator=g).float() / 40.0  # many ties
    m = AdaptiveSparseAttention(ModelConfig(d_model=64, n_head=4, attn_h_total=4, attn_token_sparse=True,
                                            attn_token_keep_ratio=0.25, attn_token_keep_guard=3,
                                            attn_token_keep_threshold=0.9))
    m._token_keep_ratio_runtime = 0.25
    mask = m._select_active_tokens(imp.to(dev)).cpu()
    exp = O.select_active_tokens(imp, 0.25, m.token_keep_min, 3, 0.9)
    assert torch.equal(mask, exp)


@pytest.mark.parametrize("B,T,ratio,guard,threshold,levels", [
    (2, 70000, 0.1, 4, 0.0, 40), (1, 65536, 0.25, 0, 0.0, 0), (3, 1000, 0.5, 7, 0.95, 10), (1, 1, 0.5, 0, 0.0, 0),
    (2, 300000, 0.02, 16, 0.999, 1000)])
def test_token_topk_sizes_vs_oracle(dev, B, T, ratio, guard, threshold, levels):
    """The multi-workgroup selection at sizes from one token to several
    hundred workgroups: heavy ties (values on a grid of `levels`, or
    continuous with levels = 0), a guard, a threshold."""
    from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

    _say(f"token top-k B={B} T={T} ratio={ratio} guard={guard} threshold={threshold}")
    g = torch.Generator().manual_seed(T + B)
    imp = torch.rand(B, T, generator=g)
    if levels:
        imp = torch.floor(imp * levels) / levels
    m = AdaptiveSparseAttention(ModelConfig(d_model=64, n_head=4, attn_h_total=4, attn_token_sparse=True,
                                            attn_token_keep_ratio=ratio, attn_token_keep_guard=guard,
                                            attn_token_keep_threshold=threshold))
    m._token_keep_ratio_runtime = ratio
    mask = m._select_active_tokens(imp.to(dev)).cpu()
    exp = O.select_active_tokens(imp, ratio, m.token_keep_min, guard, threshold)
    assert torch.equal(mask, exp)


def test_token_topk_golden(dev, golden):
    from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

    z = golden("module_cfg2_T2048")
    imp = torch.from_numpy(z["importance"])
    m = AdaptiveSparseAttention(ModelConfig(d_model=64, n_head=4, attn_h_total=4, attn_token_sparse=True,
                                            attn_token_keep_ratio=0.25))
    m._token_keep_ratio_runtime = 0.25
    mask = m._select_active_tokens(imp.to(dev)).cpu()
    ref = torch.from_numpy(z["token_mask"]).bool()
    assert torch.equal(mask.sum(1), ref.sum(1))
    need = int(torch.tensor(0.25 * imp.size(1), dtype=torch.float32).round())
    for b in range(imp.size(0)):
        diff = mask[b] != ref[b]
        if diff.any():  # only tokens tied at the cut value may differ
            cut = torch.sort(imp[b], descending=True).values[need - 1]
            assert bool((imp[b][diff] == cut).all())


def test_pack_vs_oracle(dev):
    from proteus_attention.kernels.sparse_attn import _pack_active_rows

    g = torch.Generator().manual_seed(13)
    for P, T, p in ((5, 3000, 0.3), (16, 700, 0.05), (3, 1, 1.0), (7, 2049, 0.0)):
        m = torch.rand(P, T, generator=g) < p
        got = _pack_active_rows(m.to(dev))
        exp = O.pack_active_rows(m)
        if exp is None:
            assert got is None
            continue
        assert torch.equal(got[0].cpu(), exp[0]) and torch.equal(got[1].cpu(), exp[1])
        assert torch.equal(got[2].cpu(), exp[2]) and got[3] == exp[3]


@pytest.mark.parametrize("B,T,H,topk,masked", [(1, 5000, 8, 2, False), (2, 3001, 8, 3, True), (2, 1500, 20, 4, False),
                                                 (1, 700, 16, 1, True), (3, 64, 5, 5, False),
                                                 (2, 70000, 32, 2, True)])
def test_pack_rows_routed_vs_oracle(dev, B, T, H, topk, masked):
    """pfa_pack_rows from per-token head lists (the module's packing; H <= 16
    and H > 16 take different count kernels, and B*H*ceil(T/1024) above 4096
    -- the last case -- takes the separate scan launch): the row mask, the active heads,
    the compacted rows and row_of against the oracle's packing of the same
    mask restricted to its non-empty rows."""
    from proteus_attention import _hip
    from proteus_attention.kernels import sparse_attn as sa

    g = torch.Generator().manual_seed(B * 1000 + T + H)
    scores = torch.rand(B * T, H, generator=g)
    if H > 6:
        scores[:, 3] -= 2.0  # a head nobody picks (a compacted-away row)
    hidx = torch.topk(scores, topk, dim=1).indices.to(torch.int32)
    tmask = (torch.rand(B, T, generator=g) < 0.7) if masked else None
    BH = B * H
    sel = torch.zeros(B, T, H, dtype=torch.bool)
    sel.scatter_(2, hidx.long().view(B, T, topk), True)
    if tmask is not None:
        sel &= tmask[:, :, None]
    mask = sel.permute(0, 2, 1).reshape(BH, T)
    lib = _hip.lib()
    mask8 = torch.empty(BH, T, dtype=torch.uint8, device=dev)
    heads = torch.empty(BH, dtype=torch.int32, device=dev)
    offs = torch.empty(BH + 1, dtype=torch.int32, device=dev)
    tok = torch.empty(BH * T, dtype=torch.int32, device=dev)
    rh = torch.empty(BH * T, dtype=torch.int32, device=dev)
    row_of = torch.empty(BH, T, dtype=torch.int32, device=dev)
    summ = torch.empty(4, dtype=torch.int32, device=dev)
    ws = sa._workspace(sa._size_out(lib.pfa_pack_workspace_size, B, H, T), dev)
    hd = hidx.to(dev)
    tm = tmask.to(torch.uint8).to(dev) if tmask is not None else None
    rc = lib.pfa_pack_rows(_hip.ptr(hd), topk, _hip.ptr(tm), B, H, T, _hip.ptr(mask8), _hip.ptr(heads), _hip.ptr(offs),
                           _hip.ptr(tok), _hip.ptr(rh), _hip.ptr(row_of), _hip.ptr(summ), _hip.ptr(ws), ws.numel(),
                           _hip.stream_ptr(dev))
    _hip.check(rc, "pfa_pack_rows")
    assert torch.equal(mask8.cpu().bool(), mask)
    active = mask.any(dim=1).nonzero().flatten()
    P = int(active.numel())
    s_ = summ.cpu().tolist()
    assert s_[0] == P and s_[1] == int(mask.sum())
    assert torch.equal(heads.cpu()[:P].long(), active)
    exp = O.pack_active_rows(mask[active])
    row_head, tok_e, offs_e, max_rows = exp
    N = int(tok_e.numel())
    assert s_[2] == max_rows
    assert torch.equal(offs.cpu()[:P + 1], offs_e)
    assert torch.equal(tok.cpu()[:N].long(), tok_e)
    assert torch.equal(rh.cpu()[:N].long(), row_head)
    ro = torch.full((BH, T), -1, dtype=torch.long)
    ro[active[row_head], tok_e] = torch.arange(N)
    assert torch.equal(row_of.cpu().long(), ro)


@pytest.mark.parametrize("k_only", [False, True])
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,H,D", [(2, 37, 4, 16), (2, 300, 8, 64), (1, 70, 3, 64), (1, 50, 2, 12),
                                     (1, 21, 40, 64)])
def test_rope_kernel_bitwise(dev, dt, B, T, H, D, k_only):
    """pfa_rope_qk_inplace (and its k-only form pfa_rope_k_inplace) against
    the reference's elementwise ops; covers the D=64 token-row kernel (several
    rows per workgroup, a partial last workgroup, and H=40 rows wider than a
    workgroup), the 8-wide kernel (D=16) and the per-pair kernel (D=12)."""
    from proteus_attention import _hip

    g = torch.Generator().manual_seed(14)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(dt)
    cos, sin = O.rope_tables(T, D, 10000.0, dt)
    d = qkv.to(dev).contiguous()
    cd, sd = cos.to(dev), sin.to(dev)  # keep the device tables alive across the launch
    fn = _hip.lib().pfa_rope_k_inplace if k_only else _hip.lib().pfa_rope_qk_inplace
    rc = fn(_hip.ptr(d), _hip.dtype_tag(dt), B, T, H, D, _hip.ptr(cd), _hip.ptr(sd), _hip.stream_ptr(dev))
    _hip.check(rc, "rope")
    got = d.cpu().view(B, T, 3, H, D)
    ref = qkv.view(B, T, 3, H, D)
    if k_only:
        assert torch.equal(got[:, :, 0], ref[:, :, 0])
    else:
        assert torch.equal(got[:, :, 0], O.apply_rope(ref[:, :, 0], cos, sin))
    assert torch.equal(got[:, :, 1], O.apply_rope(ref[:, :, 1], cos, sin))
    assert torch.equal(got[:, :, 2], ref[:, :, 2])


@pytest.mark.parametrize("dt,B,T,H,D", [(torch.bfloat16, 1, 4099, 8, 64), (torch.bfloat16, 2, 333, 40, 64),
                                         (torch.float32, 1, 517, 4, 64), (torch.bfloat16, 1, 300, 4, 16),
                                         (torch.float16, 2, 77, 3, 12)])
def test_rope_k_zero_bitwise(dev, dt, B, T, H, D):
    """pfa_rope_k_zero_inplace: k gets exactly the bits of pfa_rope_k_inplace
    and the (B, T, H*D) output, poisoned with NaN, comes out all zeros; the
    D=64 token-row kernel writes the zeros itself (H=40: rows wider than a
    workgroup), other shapes rotate and then fill."""
    from proteus_attention import _hip

    g = torch.Generator().manual_seed(15)
    qkv = torch.randn(B, T, 3 * H * D, generator=g).to(dt)
    cos, sin = O.rope_tables(T, D, 10000.0, dt)
    cd, sd = cos.to(dev), sin.to(dev)
    a = qkv.to(dev).contiguous()
    b = qkv.to(dev).contiguous()
    out = torch.full((B, T, H * D), float("nan"), dtype=dt, device=dev)
    lib = _hip.lib()
    _hip.check(lib.pfa_rope_k_inplace(_hip.ptr(a), _hip.dtype_tag(dt), B, T, H, D, _hip.ptr(cd), _hip.ptr(sd),
                                      _hip.stream_ptr(dev)), "rope_k")
    _hip.check(lib.pfa_rope_k_zero_inplace(_hip.ptr(b), _hip.dtype_tag(dt), B, T, H, D, _hip.ptr(cd), _hip.ptr(sd),
                                           _hip.ptr(out), _hip.stream_ptr(dev)), "rope_k_zero")
    assert torch.equal(a.cpu().view(torch.int8), b.cpu().view(torch.int8))
    assert bool((out == 0).all())
    assert torch.equal(b.cpu().view(B, T, 3, H, D)[:, :, 1], O.apply_rope(qkv.view(B, T, 3, H, D)[:, :, 1], cos, sin))


@pytest.mark.parametrize("T,B", [(4096, 1), (3000, 2)])
def test_ema_stats_fused_or_separate(dev, T, B):
    """The prototype EMA statistics accumulated inside the router pass (on
    MFMA, exact products) or by the separate pass in the router's tail
    (token-order f32 sums) give the same prototypes, usage and confidence to
    f32 rounding, and the same routing."""
    from configs import shortlist_cfg

    _say(f"EMA stats fused vs separate T={T} B={B}")
    cfg = shortlist_cfg(T, 512, 8, 1024, 256, 64)
    m, x = _module(cfg, B, T, 512, torch.bfloat16, dev, 0.01)
    snap = {n: b.detach().clone() for n, b in m.named_buffers() if n.startswith("routing_")}
    got = []
    with torch.no_grad():
        for fused in (True, False):
            for n, b in snap.items():
                getattr(m, n).copy_(b)
            m.fuse_ema_stats = fused
            y = m(x)
            got.append(({n: getattr(m, n).float().clone() for n in snap}, y.clone(),
                        m.last_head_consensus.clone()))
    assert not torch.equal(got[0][0]["routing_prototypes"], snap["routing_prototypes"].float())
    for n in snap:
        torch.testing.assert_close(got[0][0][n], got[1][0][n], rtol=1e-5, atol=1e-6, msg=n)
    # this forward's routing does not depend on the statistics (they feed the next one)
    assert torch.equal(got[0][1], got[1][1])
    assert torch.equal(got[0][2], got[1][2])


@pytest.mark.parametrize("T,L,w,s,B", [(4096, 1024, 256, 64, 1), (3000, 700, 100, 37, 2)])
def test_structured_fused_q_rope_bitwise(dev, T, L, w, s, B):
    """q rows rotated as the structured kernel loads them give exactly the
    attention (and output) bits of rotating the q tensor first."""
    from configs import shortlist_cfg

    _say(f"fused q RoPE T={T} B={B}")
    cfg = shortlist_cfg(T, 512, 8, L, w, s)
    m, x = _module(cfg, B, T, 512, torch.bfloat16, dev, 0.01)
    snap = {n: b.detach().clone() for n, b in m.named_buffers() if n.startswith("routing_")}
    outs = []
    with torch.no_grad():
        for fuse in (True, False):
            for n, b in snap.items():
                getattr(m, n).copy_(b)
            m.fuse_q_rope = fuse
            y = m(x)
            assert m._last_sparse_state["linear_shortlist_structured"] is True
            outs.append((y.clone(), m.last_head_consensus.clone()))
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][0], outs[1][0])


@pytest.mark.parametrize("T,L,w,s,B,heads,krope", [(4096, 1024, 256, 64, 1, None, True),
                                                    (3000, 700, 100, 37, 2, 3, True),
                                                    (3000, 700, 100, 37, 2, 3, False),
                                                    (65536, 2048, 512, 256, 1, None, True),
                                                    (65536, 2048, 512, 256, 1, None, False)])
def test_structured_fused_anchor_pass_bitwise(dev, T, L, w, s, B, heads, krope):
    """The anchor pass that writes the zeros of the rows without a packed
    row, and (krope) rotates k (pfa_shortlist_attn_fwd_fused), gives exactly
    the bits of the separate zero fill and RoPE pass: attention rows,
    output, and the zeros.  With the gates mapped onto the first `heads`
    heads the other heads have no rows at all (the workgroups past the
    active heads zero them); the output buffer is left to start from NaN
    garbage."""
    import torch.nn.functional as F

    from configs import shortlist_cfg

    _say(f"fused anchor pass T={T} B={B} heads={heads} k-rope={krope}")
    cfg = shortlist_cfg(T, 512, 8, L, w, s)
    m, x = _module(cfg, B, T, 512, torch.bfloat16, dev, 0.01)
    if heads is not None:
        with torch.no_grad():
            m.gate_to_head.copy_(torch.arange(m.attn_gates, device=dev) % heads)
            m.gate_to_head_onehot.copy_(F.one_hot(m.gate_to_head, 8).to(m.gate_to_head_onehot.dtype))
    snap = {n: b.detach().clone() for n, b in m.named_buffers() if n.startswith("routing_")}
    outs = []
    with torch.no_grad():
        for fuse in (True, False):
            for n, b in snap.items():
                getattr(m, n).copy_(b)
            m.fuse_anchor_pass = fuse
            m.fuse_k_rope = fuse and krope
            # NaN in the allocator's free blocks: an output row the fused
            # pass failed to write would keep it
            junk = torch.full((4 * B * T * 512,), float("nan"), dtype=torch.bfloat16, device=dev)
            del junk
            y = m(x)
            st = m._last_sparse_state
            assert st["linear_shortlist_structured"] is True
            outs.append((y.clone(), m.last_head_consensus.clone(), st["active_head_indices"].cpu().clone()))
    assert torch.equal(outs[0][2], outs[1][2])
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.equal(outs[0][0], outs[1][0])
    if heads is not None:
        act = outs[0][2].tolist()
        assert len(act) == B * heads and all(bh % 8 < heads for bh in act)
        attn4 = outs[0][1].view(B, T, 8, 64)
        assert bool((attn4[:, :, heads:] == 0).all())


# ---------------------------------------------------------------------------
# attention operator
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_attention_vs_golden(dev, golden, tag):
    from proteus_attention.kernels.sparse_attn import aspa_sparse_attention, get_last_backend

    z = golden(f"attn_{tag}")
    dt = torch.float32 if tag == "f32" else torch.bfloat16
    tol = TOL_F32 if tag == "f32" else TOL_BF16
    q, k, v = (torch.from_numpy(z[n]).to(dt).to(dev) for n in ("q", "k", "v"))
    mask = torch.from_numpy(z["mask"]).bool().to(dev)
    T = q.size(1)
    causal = torch.triu(torch.full((T, T), float("-inf")), diagonal=1).to(dev)
    out = aspa_sparse_attention(q, k, v, active_mask=mask.unsqueeze(-1))
    assert get_last_backend() == "hip" and out.dtype == dt
    assert (out.float().cpu() - torch.from_numpy(z["out_nocand"])).abs().max() <= tol
    out = aspa_sparse_attention(q, k, v, active_mask=mask.unsqueeze(-1), causal_mask=causal)
    assert (out.float().cpu() - torch.from_numpy(z["out_mask"])).abs().max() <= tol
    out = aspa_sparse_attention(q, k, v, active_mask=mask.unsqueeze(-1),
                                shortlist_candidates=torch.from_numpy(z["cand"]).to(dev),
                                shortlist_lengths=torch.from_numpy(z["lengths"]).to(dev))
    assert (out.float().cpu() - torch.from_numpy(z["out_cand"])).abs().max() <= tol
    # f32 restatement of the same operator (diagnostic: tighter for bf16)
    ref32 = O.sparse_attention(q.cpu(), k.cpu(), v.cpu(), active_mask=mask.cpu(),
                               shortlist_candidates=torch.from_numpy(z["cand"]),
                               shortlist_lengths=torch.from_numpy(z["lengths"]), compute_dtype=torch.float32)
    assert (out.float().cpu() - ref32.float()).abs().max() <= (2e-5 if tag == "f32" else 8e-3)


@pytest.mark.parametrize("D", [16, 32, 64, 128, 5, 24])
def test_attention_head_dims_vs_oracle(dev, D):
    from proteus_attention.kernels.sparse_attn import aspa_sparse_attention

    g = torch.Generator().manual_seed(D)
    BH, T = 3, 150
    q, k, v = (torch.randn(BH, T, D, generator=g) for _ in range(3))
    m = torch.rand(BH, T, generator=g) > 0.5
    causal = torch.triu(torch.full((T, T), float("-inf")), diagonal=1)
    out = aspa_sparse_attention(q.to(dev), k.to(dev), v.to(dev), active_mask=m.to(dev), causal_mask=causal.to(dev))
    ref = O.sparse_attention(q, k, v, active_mask=m, causal_mask=causal)
    assert (out.cpu() - ref).abs().max() <= TOL_F32


def test_attention_int8_vs_oracle(dev):
    from proteus_attention.kernels.sparse_attn import aspa_sparse_attention

    g = torch.Generator().manual_seed(42)
    q, k, v = (torch.randn(4, 33, 16, generator=g) for _ in range(3))
    m = torch.rand(4, 33, generator=g) > 0.4
    causal = torch.triu(torch.full((33, 33), float("-inf")), diagonal=1)
    (qi, qs, _), (ki, ks, _), (vi, vs, _) = (O.quantize_per_head_int8(t) for t in (q, k, v))
    out = aspa_sparse_attention(qi.to(dev), ki.to(dev), vi.to(dev), active_mask=m.to(dev),
                                causal_mask=causal.to(dev), q_scale=qs.to(dev), k_scale=ks.to(dev),
                                v_scale=vs.to(dev), out_dtype=torch.float32)
    ref = O.sparse_attention(qi, ki, vi, active_mask=m, causal_mask=causal, q_scale=qs, k_scale=ks, v_scale=vs,
                             out_dtype=torch.float32)
    assert (out.cpu() - ref).abs().max() <= TOL_F32
    fp = O.sparse_attention(q, k, v, active_mask=m, causal_mask=causal)
    d = (out.cpu() - fp).abs()
    assert d.mean() < 0.05 and d.max() < 0.2  # reference tests/test_aspa.py:250-305 bound


def test_attention_all_inactive_and_empty(dev):
    from proteus_attention.kernels.sparse_attn import aspa_sparse_attention, get_last_backend

    q = torch.randn(2, 9, 32, device=dev)
    out = aspa_sparse_attention(q, q, q, active_mask=torch.zeros(2, 9, 1, device=dev))
    assert get_last_backend() == "empty" and torch.count_nonzero(out) == 0


# ---------------------------------------------------------------------------
# module forward
# ---------------------------------------------------------------------------

def _module(cfg, B, T, C, dt, dev, outlier=0.0):
    from configs import init_weights, make_inputs

    from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

    torch.manual_seed(1234)
    m = AdaptiveSparseAttention(ModelConfig(**cfg))
    x, g = make_inputs(B, T, C, seed=0, outlier_frac=outlier)
    init_weights(m, g)
    m = m.to(device=dev, dtype=dt).eval()
    return m, x.to(dt).to(dev)


def _active_heads_per_token(token_idx, row_offsets, heads, B, H, T):
    act = torch.zeros(B * H, T, dtype=torch.bool)
    offs = row_offsets.tolist()
    for p, bh in enumerate(heads.tolist()):
        act[bh, token_idx[offs[p]:offs[p + 1]]] = True
    return act.view(B, H, T).permute(0, 2, 1)  # (B, T, H)


@pytest.mark.parametrize("name,maker,B,T,C,dt,outlier", [
    ("module_cfg1", "sparse", 1, 1024, 256, torch.float32, 0.0),
    ("module_cfg2_T2048", "sparse", 2, 2048, 512, torch.bfloat16, 0.0),
    ("module_cfg2_full", "sparse", 2, 8192, 512, torch.bfloat16, 0.0),
    ("module_short_T4096_f32", "short", 1, 4096, 512, torch.float32, 0.01),
    ("module_short_T4096_bf16", "short", 1, 4096, 512, torch.bfloat16, 0.01),
])
def test_module_forward_vs_golden(dev, golden, name, maker, B, T, C, dt, outlier):
    from configs import shortlist_cfg, sparse_cfg

    _say(f"module {name}")
    z = golden(name)
    cfg = sparse_cfg(T, C, 8) if maker == "sparse" else shortlist_cfg(T, C, 8, 1024, 256, 64)
    m, x = _module(cfg, B, T, C, dt, dev, outlier)
    with torch.no_grad():
        y = m(x)
    assert m.last_head_stats["mode"] == str(z["mode"]) == "shortlist"
    st = m._last_sparse_state
    ours = _active_heads_per_token(st["token_idx"].cpu().long(), st["row_offsets"].cpu().long(),
                                   st["active_head_indices"].cpu(), B, 8, T)
    ref = _active_heads_per_token(torch.from_numpy(z["packed_token_idx"]), torch.from_numpy(z["packed_row_offsets"]),
                                  torch.from_numpy(z["active_head_indices"]), B, 8, T)
    same_tok = (ours == ref).all(-1)  # (B, T)
    if dt == torch.float32:
        assert bool(same_tok.all())
    else:
        # every token routed differently is a tie of the reference's gate
        # probabilities broken to the lowest head index, or a token at a
        # bf16 rounding boundary (routing_parity.check_routing)
        from routing_parity import check_routing

        tm = None
        if "token_mask" in z:
            tm = torch.from_numpy(z["token_mask"]).bool().reshape(-1)
            assert torch.equal(m._last_token_mask.cpu().reshape(-1), tm)
        rep = check_routing(ours.reshape(B * T, 8), ref.reshape(B * T, 8), m._last_gate_probs.float().cpu().reshape(B * T, 8),
                            torch.from_numpy(z["gate_probs"]).reshape(B * T, 8), x.cpu().reshape(B * T, C),
                            m.head_router.linear.weight.detach().cpu(), 2, tm)
        _say(f"{name}: {rep}")
        rep.assert_boundary_sets_at_most(1e-3)
    stride = int(z["token_stride"])
    yr = torch.from_numpy(z["y"])
    yo = y.float().cpu()[:, ::stride]
    sel = same_tok[:, ::stride]
    tol = TOL_F32 if dt == torch.float32 else TOL_BF16
    err = (yo - yr).abs().amax(-1)[sel].max()
    _say(f"{name}: max-abs err on matched tokens {float(err):.3e}")
    assert float(err) <= tol
    # post-forward prototype EMA state
    assert torch.allclose(m.routing_prototypes.float().cpu(), torch.from_numpy(z["protos_after"]), atol=1e-5,
                          rtol=1e-4 if dt == torch.float32 else 1e-2)
    assert torch.allclose(m.routing_usage_ema.float().cpu(), torch.from_numpy(z["usage_after"]), rtol=1e-4,
                          atol=1e-4 if dt == torch.float32 else 1e-1)


def test_module_telemetry_deferred(dev):
    """Statistics (aspa.py:1857-1916) are read back after the forward without
    a device wait; reading them gives the values of the latest forward, and
    they agree with closed forms over the forward's own router outputs."""
    from configs import shortlist_cfg

    _say("telemetry after two forwards of different length")
    cfg = shortlist_cfg(4096, 512, 8, 1024, 256, 64)
    m, x = _module(cfg, 1, 4096, 512, torch.bfloat16, dev, 0.01)
    with torch.no_grad():
        m(x)
        m(x[:, :2048].contiguous())
        gate = m._last_gate_probs.double().cpu()
        sim = m._last_token_similarity.double().cpu()
    hs = m.last_head_stats
    assert hs["seq_len"] == 2048 and hs["mode"] == "shortlist"
    assert hs["mean_active_per_token"] == pytest.approx(2.0)
    assert hs["latency_ms"] > 0.0 and hs["mode_selected"].startswith("cvt(")
    ent = float(-(gate.clamp_min(1e-9).log() * gate).sum(-1).mean())
    assert hs["router_entropy"] == pytest.approx(ent, rel=1e-4, abs=1e-6)
    assert hs["proto"]["max_sim_mean"] == pytest.approx(float(sim.mean()), rel=1e-4, abs=1e-6)
    st = m._last_sparse_state
    assert st["max_rows"] == hs["max_active_rows"] and st["latency_ms"] == hs["latency_ms"]
    assert st["active_head_indices"].numel() == 8 and st["row_offsets"].numel() == 9
    assert m._density_ema is not None and m._latency_ema is not None


def test_module_hip_graph_replay_matches_eager(dev):
    """Graph mode: every replay equals the eager forward on the same inputs
    and state (the prototype EMA carries over between forwards), with eager
    device work and synchronisations between replays; a second input shape
    captures its own graph without disturbing the first."""
    from configs import shortlist_cfg

    _say("hip graph replay vs eager, T=4096 and T=2048")
    cfg = shortlist_cfg(4096, 512, 8, 1024, 256, 64)
    m, x = _module(cfg, 1, 4096, 512, torch.bfloat16, dev, 0.01)
    init = {n: b.detach().clone() for n, b in m.named_buffers()}
    xs = [x, (x * 0.5).contiguous(), torch.roll(x, 7, dims=1).contiguous(), x[:, :2048].contiguous(), x]

    def run(graph: bool):
        for n, b in m.named_buffers():
            b.copy_(init[n])
        m.enable_hip_graph(graph)
        outs = []
        with torch.no_grad():
            for i, xi in enumerate(xs):
                y = m(xi)
                a = m.last_head_consensus.clone()
                ent = m.last_head_stats["router_entropy"]
                junk = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
                torch.cuda.synchronize()
                outs.append((y.float().cpu(), a.float().cpu(), ent, m.routing_prototypes.float().cpu().clone(),
                             float(junk)))
        return outs

    eager = run(False)
    graph = run(True)
    assert len(m._hip_graphs) == 2
    for i, (e, g) in enumerate(zip(eager, graph)):
        assert torch.equal(e[1], g[1]), f"forward {i}: attention output differs"
        assert torch.equal(e[3], g[3]), f"forward {i}: prototype EMA differs"
        assert (e[0] - g[0]).abs().max() <= TOL_BF16 * (1.0 + e[0].abs().max())
        assert g[2] == pytest.approx(e[2], rel=1e-6)
    m.enable_hip_graph(False)
    assert not m._hip_graphs


def test_module_hip_graph_static_output_matches_eager(dev):
    """Graph mode with the output projection captured (static_output): every
    replay's returned buffer equals the eager forward's output on the same
    inputs and state, with eager device work between the replays."""
    from configs import shortlist_cfg

    _say("hip graph static output vs eager")
    cfg = shortlist_cfg(4096, 512, 8, 1024, 256, 64)
    m, x = _module(cfg, 1, 4096, 512, torch.bfloat16, dev, 0.01)
    init = {n: b.detach().clone() for n, b in m.named_buffers()}
    xs = [x, (x * 0.5).contiguous(), torch.roll(x, 3, dims=1).contiguous(), x]

    def run(graph: bool):
        for n, b in m.named_buffers():
            b.copy_(init[n])
        m.enable_hip_graph(graph, static_output=graph)
        outs = []
        with torch.no_grad():
            for xi in xs:
                y = m(xi).float().cpu()
                junk = torch.randn(1 << 20, device=dev).sum()
                torch.cuda.synchronize()
                outs.append((y, float(junk)))
        return outs

    eager = run(False)
    graph = run(True)
    for i, (e, g) in enumerate(zip(eager, graph)):
        assert torch.equal(e[0], g[0]), f"forward {i}: output differs"
    m.enable_hip_graph(False)
    # graph mode switched off and on again, with and without the captured
    # projection, captures anew each time (each capture after a reset opens
    # a new memory pool)
    for static in (False, True, False):
        for n, b in m.named_buffers():
            b.copy_(init[n])
        m.enable_hip_graph(True, static_output=static)
        with torch.no_grad():
            for i, xi in enumerate(xs):
                y = m(xi).float().cpu()
                assert torch.equal(y, eager[i][0]), f"recapture (static={static}) forward {i}: output differs"
        m.enable_hip_graph(False)


def test_module_hip_graph_token_mask_matches_eager(dev):
    """Graph mode with a token mask (the chunked pipeline's chunk model:
    token top-k without a threshold, materialised candidates, top-p routing
    at the head-count floor): the forward reads no count back, so it is
    captured; every replay's importance, mask, attention output, prototype
    EMA and returned buffer equal the eager forward's, and the deferred
    telemetry trims the packed rows to the device count.  At T = 24,576 the
    window plus anchors exceed L = 256, so the candidates are materialised
    (shorter chunks take the structured path, which reads the exact count
    and stays eager)."""
    from proteus_attention.models.aspa import AdaptiveSparseAttention
    from proteus_attention.tools.chunked_shortlist import _build_model_config

    T, C, H = 24576, 512, 8
    _say(f"hip graph token mask vs eager, T={T}")
    torch.manual_seed(0)
    m = AdaptiveSparseAttention(_build_model_config(T, C, heads=H, sparse_ratio=0.05, shortlist_alpha=0.0,
                                                    router_top_p=1.0)).to(dev, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, T, C, generator=g).to(torch.bfloat16).to(dev)
    with torch.no_grad():
        assert m._graph_eligible(x)
        assert not m._graph_eligible(x[:, :4096])  # structured: eager
    init = {n: b.detach().clone() for n, b in m.named_buffers()}
    xs = [x, (x * 0.5).contiguous(), torch.roll(x, 11, dims=1).contiguous(), x]

    def run(graph: bool):
        for n, b in m.named_buffers():
            b.copy_(init[n])
        m.enable_hip_graph(graph, static_output=graph)
        outs = []
        with torch.no_grad():
            for xi in xs:
                y = m(xi).float().cpu()
                imp = m._last_token_importance.float().cpu().clone()
                mask = m._last_token_mask.cpu().clone()
                a = m.last_head_consensus.float().cpu().clone()
                st = m._last_sparse_state
                rows = (int(st["token_idx"].numel()), float(m.last_head_stats["mean_active_per_token"]),
                        int(m._last_target_k))
                junk = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
                torch.cuda.synchronize()
                outs.append((y, imp, mask, a, m.routing_prototypes.float().cpu().clone(), rows, float(junk)))
        return outs

    eager = run(False)
    graph = run(True)
    assert len(m._hip_graphs) == 1
    assert m._last_sparse_state["mode"] == "shortlist"
    for i, (e, gr) in enumerate(zip(eager, graph)):
        for j, what in enumerate(("output", "importance", "mask", "attention", "prototype EMA")):
            assert torch.equal(e[j], gr[j]), f"forward {i}: {what} differs"
        assert e[5] == gr[5], f"forward {i}: packed rows {e[5]} vs {gr[5]}"
        kept = int(e[2].sum())
        assert e[5][0] == kept * e[5][2]  # every kept token has its top-k heads
    m.enable_hip_graph(False)


def test_module_dense_paths_vs_oracle(dev):
    """subquad mode (force-dense) and the small-sequence dense fast path
    equal dense causal attention of the projected q/k/v."""
    from configs import COMMON

    from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

    g = torch.Generator().manual_seed(5)
    B, T, C, H = 2, 96, 64, 4
    base = dict(COMMON, d_model=C, n_head=H, attn_h_total=H, attn_gates=H, attn_use_rope=False,
                attn_token_sparse=False)
    x = torch.randn(B, T, C, generator=g)
    for cfg in (dict(base, attn_mode="subquad"), dict(base, attn_small_seq_dense=128)):
        torch.manual_seed(0)
        m = AdaptiveSparseAttention(ModelConfig(**cfg)).eval()
        with torch.no_grad():
            qkv = m.qkv(x).view(B, T, 3, H, C // H)
            q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3).reshape(B * H, T, C // H) for i in range(3))
            att = O.causal_attention_f32(q, k, v).view(B, H, T, C // H).permute(0, 2, 1, 3).reshape(B, T, C)
            exp = m.proj(att)
            y = m.to(dev)(x.to(dev)).cpu()
        assert (y - exp).abs().max() <= TOL_F32


def test_dropin_mha_gpu(dev):
    from proteus_attention import CausalASPAMultiheadAttention

    torch.manual_seed(0)
    mha = CausalASPAMultiheadAttention(64, 4, attn_mode="linear", attn_linear_L=64, attn_linear_window=32).to(dev)
    x = torch.randn(2, 50, 64, device=dev)
    pad = torch.zeros(2, 50, dtype=torch.bool, device=dev)
    pad[1, 40:] = True
    out, w = mha(x, key_padding_mask=pad, need_weights=True)
    assert out.shape == x.shape and w.shape == (2, 50, 50)
    assert torch.count_nonzero(out[1, 40:]) == 0
    assert torch.isfinite(out).all()


# ---------------------------------------------------------------------------
# chunk selection
# ---------------------------------------------------------------------------

def test_chunk_select_vs_golden(dev, golden):
    from proteus_attention.tools import chunk_select

    z = golden("chunk_select")
    s = torch.from_numpy(z["scores"]).to(dev)
    v, i = chunk_select.nucleus_select(s, 512, 1.0)
    assert np.array_equal(i.cpu().numpy(), z["i_p1"]) and np.array_equal(v.cpu().numpy(), z["v_p1"])
    v, i = chunk_select.nucleus_select(s * 4.0, 512, 0.9)
    assert np.array_equal(i.cpu().numpy(), z["i_p09"])
    ki, ks = chunk_select.finalise(torch.from_numpy(z["all_scores"]).to(dev), torch.from_numpy(z["all_idx"]).to(dev),
                                   4096)
    assert np.array_equal(ki.cpu().numpy(), z["keep_idx"]) and np.array_equal(ks.cpu().numpy(), z["keep_scores"])


def test_chunked_runner_small_gpu(dev):
    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig, ChunkedShortlistRunner

    cfg = ChunkedShortlistConfig(seq_len=4096, d_model=64, chunk_len=1024, buffer_tokens=256, per_chunk_budget=128,
                                 device=dev, heads=4, nucleus_top_p=1.0, storage="cpu")
    res = ChunkedShortlistRunner(cfg).run()
    k = res.keep_indices
    assert k.numel() <= 256 and torch.all(k[1:] > k[:-1])
    seq = torch.randn(1, 4096, 64, generator=torch.Generator().manual_seed(7))
    assert res.metrics.used_fallback is False
    assert res.final_output is not None and torch.isfinite(res.final_output).all()
    del seq


def _head_probs(gate: torch.Tensor, G: int, H: int) -> torch.Tensor:
    """gate_probs @ onehot(gate_to_head), summed gate by gate in index order
    (the order the router's epilogue adds them)."""
    g2h = O.default_gate_map(G, H)
    hp = torch.zeros(gate.size(0), H, dtype=torch.float32)
    for gi in range(G):
        hp[:, int(g2h[gi])] += gate[:, gi]
    return hp


@pytest.mark.parametrize("dt,G", [(torch.float32, 8), (torch.bfloat16, 8), (torch.bfloat16, 16),
                                  (torch.bfloat16, 12)])
def test_router_without_prototypes_vs_oracle(dev, dt, G):
    """use_proto == 0: gates are the router softmax alone; the packed table
    keeps its (C, 2*Gp) layout and only the weight columns are read.  3000
    tokens leave the last 64-token group partial (and, in bf16, the last
    workgroup with a group past the end).  16 and 12 gates (two gates per
    head on 8 heads) take the 16-gate MFMA tables."""
    from proteus_attention import _hip
    from proteus_attention.models.aspa import pack_router_weights

    g = torch.Generator().manual_seed(12)
    n, C, H = 3000, 512, 8
    x = torch.randn(n, C, generator=g).to(dt)
    w = (torch.randn(G, C, generator=g) * 0.05).to(dt)
    lib = _hip.lib()
    wpk = pack_router_weights(w.to(dev), None, dt)
    g2h = O.default_gate_map(G, H).to(torch.int32).to(dev)
    gate = torch.empty(n, G, device=dev)
    imp = torch.empty(n, device=dev)
    hidx = torch.empty(n, 2, dtype=torch.int32, device=dev)
    _hip.check(lib.pfa_router_topk(_hip.ptr(x.to(dev)), _hip.dtype_tag(dt), n, C, G, _hip.ptr(wpk), 0, None, None,
                                   _hip.ptr(g2h), H, 2, 0.2, 0.25, 0.6, 0.0, _hip.ptr(gate), None, None, _hip.ptr(imp),
                                   _hip.ptr(hidx), None, None, None, _hip.stream_ptr(dev)), "router")
    og, _, _, oimp = O.route_tokens(x, w, None, None, None, proto_temp=0.2, proto_threshold=0.25, proto_blend=0.6,
                                    usage_boost=0.0)
    if dt == torch.float32:
        assert torch.allclose(gate.cpu(), og, atol=2e-6, rtol=0)
        assert torch.allclose(imp.cpu(), oimp, atol=2e-6, rtol=0)
    else:
        # gates bit for bit except at a bf16 rounding boundary of a logit or
        # a softmax output (the f32 dot in another order)
        from routing_parity import _at_boundary

        bad = (gate.cpu() != og).any(1)
        assert int((bad & ~torch.from_numpy(_at_boundary(x, w))).sum()) == 0
    _, oidx = O.topk_lowest(_head_probs(gate.cpu(), G, H), 2)
    assert torch.equal(hidx.cpu().long(), oidx)


@pytest.mark.parametrize("n,C,G", [(3000, 512, 16), (4096, 384, 13), (1000, 128, 9), (130, 512, 16)])
def test_router_sixteen_gates_bf16_vs_oracle(dev, n, C, G):
    """bf16 router with 9-16 gates and prototypes (the 16-gate MFMA tables:
    weights, and the hi / mid / lo parts of each prototype, in four 16-row
    tables) against the oracle.  The first tokens are made close to a
    prototype so that their prior blend is live.  Prototype similarities to
    f32 accumulation order; gates bit for bit where the blend is zero (the
    router softmax alone) except at a bf16 rounding boundary, within 1e-5
    where it is live; head top-k exactly the lowest-index top-k of the
    router's own head probabilities."""
    from routing_parity import _at_boundary

    H, topk = 8, 2
    _say(f"router G={G} n={n} C={C} bf16")
    g = torch.Generator().manual_seed(40 + G)
    x = torch.randn(n, C, generator=g).to(torch.bfloat16)
    w = (torch.randn(G, C, generator=g) * 0.05).to(torch.bfloat16)
    protos = torch.randn(G, C, generator=g).to(torch.bfloat16)
    near = min(4, G)
    protos[:near] = (x[:near].float() + 0.3 * torch.randn(near, C, generator=g)).to(torch.bfloat16)
    conf = torch.zeros(G, dtype=torch.bfloat16)
    gate, sim, bl, imp, hidx, hsc = _run_router(dev, x, w, protos.float(), conf, torch.bfloat16, topk, H)
    og, osim, obl, oimp = O.route_tokens(x, w, protos, conf, None, proto_temp=0.2, proto_threshold=0.25,
                                         proto_blend=0.6, usage_boost=0.0)
    og, osim, obl, oimp = og.reshape(n, G), osim.reshape(n), obl.reshape(n), oimp.reshape(n)
    assert torch.allclose(sim, osim, atol=2e-6, rtol=0)
    assert torch.allclose(bl, obl, atol=1e-5, rtol=0)
    live = (bl > 0) | (obl > 0)
    assert bool(live[:near].all())
    bad = (gate != og).any(1) & ~live
    assert int((bad & ~torch.from_numpy(_at_boundary(x, w))).sum()) == 0
    assert torch.allclose(gate[live], og[live], atol=1e-5, rtol=0)
    # importance (largest gate, blended with the similarity) wherever the
    # gates agree; the rest are the bf16 rounding-boundary tokens
    close = (gate - og).abs().amax(1) <= 1e-5
    assert float(close.float().mean()) > 0.9
    assert torch.allclose(imp[close], oimp[close], atol=1e-5, rtol=0)
    hp = _head_probs(gate, G, H)
    hv, oidx = O.topk_lowest(hp, topk)
    assert torch.equal(hidx.long(), oidx)
    assert torch.equal(hsc, hv)


def _router_raw_ws(dev, x, w, protos, conf, use, g2h, H, topk, args, ema):
    """pfa_router_topk_raw_ws on bf16 device tensors: (gate, sim, blend,
    importance, head_idx, head_score, telemetry partials, EMA partials)."""
    from proteus_attention import _hip
    from proteus_attention.kernels.sparse_attn import _size_out, _workspace

    lib = _hip.lib()
    n, C = x.shape
    G = w.size(0)
    nblk = _hip.ctypes.c_int(0)
    _hip.check(lib.pfa_router_block_count(n, _hip.ctypes.byref(nblk)), "block_count")
    nb = max(1, nblk.value)
    out = [torch.empty(n, G, device=dev), torch.empty(n, device=dev), torch.empty(n, device=dev),
           torch.empty(n, device=dev), torch.empty(n, topk, device=dev, dtype=torch.int32),
           torch.empty(n, topk, device=dev), torch.empty(nb, 8, device=dev),
           torch.empty(nb, G, C + 1, device=dev) if ema else None]
    ws = _workspace(_size_out(lib.pfa_router_raw_workspace_size, n, G), dev)
    bf = _hip.PFA_BF16
    _hip.check(lib.pfa_router_topk_raw_ws(_hip.ptr(x), bf, n, C, G, _hip.ptr(w), bf, _hip.ptr(protos), _hip.ptr(conf),
                                          _hip.ptr(use), bf, _hip.ptr(g2h), H, topk, *args,
                                          *[_hip.ptr(o) for o in out], _hip.ptr(ws), ws.numel(),
                                          _hip.stream_ptr(dev)), "router_raw_ws")
    return out


@pytest.mark.parametrize("n,C,G,H,ema", [(3000, 512, 64, 32, True), (2500, 384, 32, 16, True),
                                         (1000, 256, 24, 8, False), (4097, 512, 48, 16, True),
                                         (130, 128, 17, 8, True), (20_000, 512, 64, 32, True)])
def test_router_gate_blocks_bf16_vs_oracle(dev, n, C, G, H, ema):
    """bf16 router with 17-64 gates (pfa_router_topk_raw_ws: the 16-gate
    MFMA tables once per block of 16 gates, then the epilogue) against the
    oracle, as the 16-gate router is tested: prototype similarities to f32
    accumulation order, gates bit for bit where the blend is zero except at
    a bf16 rounding boundary of a logit or softmax output, within 1e-5
    where it is live, head top-k exactly the lowest-index top-k of the
    router's own head probabilities; the fused EMA statistics against a
    float64 product of the router's own gates; and the same head sets as
    the VALU router (pfa_router_prepare + pfa_router_topk) wherever the two
    routers' gates agree."""
    from proteus_attention import _hip
    from routing_parity import _at_boundary

    _say(f"router gate blocks G={G} H={H} n={n} C={C} bf16")
    lib = _hip.lib()
    bf = torch.bfloat16
    topk = 2
    g = torch.Generator().manual_seed(70 + G)
    x = torch.randn(n, C, generator=g).to(bf)
    w = (torch.randn(G, C, generator=g) * 0.05).to(bf)
    protos = torch.randn(G, C, generator=g).to(bf)
    near = 4
    protos[:near] = (x[:near].float() + 0.3 * torch.randn(near, C, generator=g)).to(bf)
    conf = (torch.rand(G, generator=g) * 3).to(bf)
    use = (torch.rand(G, generator=g) * 5).to(bf)
    assert lib.pfa_router_raw_supported(_hip.PFA_BF16, _hip.PFA_BF16, _hip.PFA_BF16, G, C, 1) == 1
    g2h = O.default_gate_map(G, H).to(torch.int32).to(dev)
    xd, wd, pd, cd, ud = (t.to(dev) for t in (x, w, protos, conf, use))
    args = (0.2, 0.25, 0.6, 0.0)
    out = _router_raw_ws(dev, xd, wd, pd, cd, ud, g2h, H, topk, args, ema)
    gate, sim, bl, imp, hidx, hsc = (o.cpu() for o in out[:6])
    og, osim, obl, oimp = O.route_tokens(x, w, protos, conf, None, proto_temp=0.2, proto_threshold=0.25,
                                         proto_blend=0.6, usage_boost=0.0)
    og, osim, obl, oimp = og.reshape(n, G), osim.reshape(n), obl.reshape(n), oimp.reshape(n)
    assert torch.allclose(sim, osim, atol=2e-6, rtol=0)
    assert torch.allclose(bl, obl, atol=1e-5, rtol=0)
    live = (bl > 0) | (obl > 0)
    assert bool(live[:near].all())
    bad = (gate != og).any(1) & ~live
    assert int((bad & ~torch.from_numpy(_at_boundary(x, w))).sum()) == 0
    assert torch.allclose(gate[live], og[live], atol=1e-5, rtol=0)
    close = (gate - og).abs().amax(1) <= 1e-5
    assert float(close.float().mean()) > 0.9
    assert torch.allclose(imp[close], oimp[close], atol=1e-5, rtol=0)
    hv, oidx = O.topk_lowest(_head_probs(gate, G, H), topk)
    assert torch.equal(hidx.long(), oidx)
    assert torch.equal(hsc, hv)
    if ema:
        nb = out[7].size(0)
        sums = torch.empty(G, C + 1, device=dev)
        _hip.check(lib.pfa_proto_partial_reduce(_hip.ptr(out[7]), nb, G, C, _hip.ptr(sums), _hip.stream_ptr(dev)),
                   "reduce")
        gp, got = gate.double(), sums.cpu().double()
        ref = torch.cat([gp.t() @ x.double(), gp.sum(0).unsqueeze(1)], dim=1)
        scale = torch.cat([(gp.t() @ x.double().abs()).clamp_min(1.0), gp.sum(0).unsqueeze(1).clamp_min(1.0)], dim=1)
        err = float(((got - ref).abs() / scale).max())
        _say(f"EMA sums max scaled error {err:.2e}")
        assert err < 1e-5
    # the VALU router on the same inputs (usage bias on, conf weights on)
    Gp = int(lib.pfa_router_gate_pad(G))
    wpk = torch.empty(C, 2 * Gp, device=dev)
    cw, ub = torch.empty(G, device=dev), torch.empty(G, device=dev)
    _hip.check(lib.pfa_router_prepare(_hip.ptr(wd), _hip.PFA_BF16, _hip.ptr(pd), _hip.ptr(cd), _hip.ptr(ud),
                                      _hip.PFA_BF16, G, C, _hip.PFA_BF16, _hip.ptr(wpk), _hip.ptr(cw), _hip.ptr(ub),
                                      _hip.stream_ptr(dev)), "prepare")
    args_u = (0.2, 0.25, 0.6, 0.3)
    mine = _router_raw_ws(dev, xd, wd, pd, cd, ud, g2h, H, topk, args_u, False)
    valu = [torch.empty_like(t) if t is not None else None for t in mine]
    _hip.check(lib.pfa_router_topk(_hip.ptr(xd), _hip.PFA_BF16, n, C, G, _hip.ptr(wpk), 1, _hip.ptr(cw), _hip.ptr(ub),
                                   _hip.ptr(g2h), H, topk, *args_u, *[_hip.ptr(o) for o in valu],
                                   _hip.stream_ptr(dev)), "router_valu")
    ga, gb_ = mine[0].cpu(), valu[0].cpu()
    agree = (ga - gb_).abs().amax(1) <= 1e-5
    _say(f"gates within 1e-5 of the VALU router on {float(agree.float().mean()):.4f} of tokens")
    assert float(agree.float().mean()) > 0.9
    assert torch.allclose(mine[1].cpu(), valu[1].cpu(), atol=2e-6, rtol=0)
    same = (ga == gb_).all(1)
    assert torch.equal(mine[4].cpu()[same], valu[4].cpu()[same])


# ---------------------------------------------------------------------------
# drop-in nn.MultiheadAttention replacement (reference tests/test_dropin_attention.py)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name,T,kw", [("dropin_mha_auto", 96, {}),
                                       ("dropin_mha_linear", 300, dict(attn_mode="linear", attn_linear_L=64,
                                                                       attn_linear_window=32))])
def test_dropin_mha_matches_reference(dev, golden, name, T, kw):
    """CausalASPAMultiheadAttention with the reference's state dict on the
    reference's input and key padding mask: the output values, the zero
    attention weights of the reference's shape, zero rows where padded, and
    the head count its nucleus rule (router_top_p 0.9) chose."""
    from proteus_attention import CausalASPAMultiheadAttention

    z = golden(name)
    torch.manual_seed(0)
    mha = CausalASPAMultiheadAttention(embed_dim=64, num_heads=4, batch_first=True, **kw)
    sd = {k[4:]: torch.from_numpy(v) for k, v in z.items() if k.startswith("sd::")}
    missing, unexpected = mha.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all(k.startswith("attention._") or "rope" in k for k in missing), missing
    mha = mha.to(dev).eval()
    x = torch.from_numpy(z["x"]).to(dev)
    pad = torch.from_numpy(z["pad"]).bool().to(dev)
    with torch.no_grad():
        out, w = mha(x, key_padding_mask=pad, need_weights=True)
    hs = mha.attention.last_head_stats
    assert hs["top_k"] == int(z["top_k"]) and hs["nucleus_k"] == int(z["nucleus_k"])
    assert hs["mode"] == str(z["mode"])
    assert tuple(w.shape) == tuple(z["weights_shape"]) and torch.count_nonzero(w) == 0
    err = float((out.cpu() - torch.from_numpy(z["out"])).abs().max())
    _say(f"{name}: mode {hs['mode']} top_k {hs['top_k']} max-abs err {err:.3e}")
    assert err <= TOL_F32
    assert torch.count_nonzero(out[pad]) == 0


def test_dropin_mha_fallbacks_match_torch(dev):
    """Cross attention and a custom (non-causal) mask go to the wrapped
    nn.MultiheadAttention, equal to a torch module with the same weights
    (reference tests/test_dropin_attention.py:55-113); the standard causal
    mask stays on the ASPA path; an entirely padded batch row gives zeros."""
    import torch.nn as nn

    from proteus_attention import CausalASPAMultiheadAttention

    torch.manual_seed(1)
    mha = CausalASPAMultiheadAttention(embed_dim=16, num_heads=4, batch_first=True, dropout=0.0,
                                       return_stats_default=True).to(dev)
    ref = nn.MultiheadAttention(embed_dim=16, num_heads=4, batch_first=True, dropout=0.0).to(dev)
    ref.load_state_dict(mha.fallback_attention.state_dict())
    q, k = torch.randn(2, 5, 16, device=dev), torch.randn(2, 7, 16, device=dev)
    out, w = mha(q, key=k, value=k, need_weights=True)
    eo, ew = ref(q, k, k, need_weights=True)
    assert torch.allclose(out, eo, atol=1e-6) and torch.allclose(w, ew, atol=1e-6)
    assert mha.last_runtime_stats["shortlist_backend"]["name"] == "torch.nn.MultiheadAttention"
    x = torch.randn(3, 6, 16, device=dev)
    custom = torch.full((6, 6), float("-inf"), device=dev).triu_(1)
    custom[0, 3] = 0.0
    out, w = mha(x, attn_mask=custom, need_weights=True, average_attn_weights=False, is_causal=False)
    eo, ew = ref(x, x, x, attn_mask=custom, need_weights=True, average_attn_weights=False, is_causal=False)
    assert torch.allclose(out, eo, atol=1e-6) and torch.allclose(w, ew, atol=1e-6)
    causal = torch.triu(torch.ones(6, 6, dtype=torch.bool, device=dev), diagonal=1)
    out, _ = mha(x, attn_mask=causal, need_weights=False)
    assert mha.last_runtime_stats["shortlist_backend"]["name"] != "torch.nn.MultiheadAttention"
    pad = torch.zeros(3, 6, dtype=torch.bool, device=dev)
    pad[2] = True
    out, _ = mha(x, key_padding_mask=pad, need_weights=False)
    assert torch.count_nonzero(out[2]) == 0 and torch.isfinite(out).all()
    # batch_first=False: (T, B, C) in and out, weights (B, T, T)
    mha_t = CausalASPAMultiheadAttention(embed_dim=16, num_heads=4, batch_first=False).to(dev)
    out, w = mha_t(x.transpose(0, 1), need_weights=True)
    assert out.shape == (6, 3, 16) and w.shape == (3, 6, 6)


# ---------------------------------------------------------------------------
# dense causal attention on MFMA tiles (force-dense / dense fast path /
# the operator's implicit-causal branch)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("BH,T,p,D", [(8, 8192, 1.0, 64), (6, 3001, 0.35, 64), (3, 65, 1.0, 64),
                                       (5, 3001, 0.5, 16), (4, 2049, 0.7, 32), (2, 40, 1.0, 16),
                                       (3, 3001, 0.5, 128), (2, 65, 1.0, 128)])
def test_operator_causal_branch_mfma_vs_oracle(dev, BH, T, p, D):
    """aspa_sparse_attention without candidates or mask (each active row
    attends to keys 0..t, sparse_attn.py:1016-1043) in bf16, D = 16, 32, 64
    or 128, runs the MFMA causal tiles; every active row against f32 causal
    attention, inactive rows zero."""
    from proteus_attention.kernels.sparse_attn import aspa_sparse_attention, get_last_backend_info

    _say(f"operator causal mfma BH={BH} T={T} p={p} D={D}")
    g = torch.Generator().manual_seed(T + BH)
    q, k, v = (torch.randn(BH, T, D, generator=g).to(torch.bfloat16) for _ in range(3))
    mask = torch.rand(BH, T, generator=g) < p
    out = aspa_sparse_attention(q.to(dev), k.to(dev), v.to(dev), active_mask=mask.to(dev))
    info = get_last_backend_info()
    assert info["name"] == "hip" and info["details"].get("mfma") is True
    ref = O.causal_attention_f32(q, k, v)
    o = out.float().cpu()
    err = float((o - ref)[mask].abs().max())
    _say(f"max-abs err {err:.3e}")
    assert err <= TOL_BF16
    assert torch.count_nonzero(o[~mask]) == 0


@pytest.mark.parametrize("B,T,dt,keep", [(1, 8192, torch.bfloat16, None), (2, 4096, torch.bfloat16, 0.3),
                                         (2, 2048, torch.float32, 0.3)])
def test_module_force_dense_mfma_vs_oracle(dev, B, T, dt, keep):
    """subquad mode (force-dense, aspa.py:1624-1677): the attention output
    equals causal attention of the module's own projected and rotated
    q/k/v (bf16 on the MFMA causal tiles, f32 on the row kernel).  With
    token sparsity (keep) only the kept tokens' rows are attended and the
    others are exactly zero: the reference's dense output times the token
    mask (aspa.py:1841-1842)."""
    from configs import COMMON

    from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

    C, H = 512, 8
    _say(f"module force-dense B={B} T={T} {dt} keep={keep}")
    torch.manual_seed(0)
    extra = dict(attn_token_sparse=False) if keep is None else dict(
        attn_token_sparse=True, attn_token_keep_ratio=keep, attn_linear_token_keep_schedule="fixed")
    m = AdaptiveSparseAttention(ModelConfig(**dict(COMMON, d_model=C, n_head=H, attn_h_total=H, attn_gates=H,
                                                   attn_mode="subquad", **extra)))
    m = m.to(dev, dt).eval()
    x = torch.randn(B, T, C, generator=torch.Generator().manual_seed(3)).to(dt).to(dev)
    with torch.no_grad():
        m(x)
        qkv = m.qkv(x).view(B, T, 3, H, 64).cpu()
    assert m._last_sparse_state["mode"].startswith("dense")
    cos, sin = (t.cpu() for t in m._rope_factors(T, dev, dt))
    q = O.apply_rope(qkv[:, :, 0], cos, sin)
    k = O.apply_rope(qkv[:, :, 1], cos, sin)
    qh, kh, vh = (a.permute(0, 2, 1, 3).reshape(B * H, T, 64) for a in (q, k, qkv[:, :, 2]))
    ref = O.causal_attention_f32(qh, kh, vh).view(B, H, T, 64).permute(0, 2, 1, 3).reshape(B, T, C)
    got = m.last_head_consensus.float().cpu()
    if keep is not None:
        tm = m._last_token_mask.cpu()
        assert 0 < int(tm.sum()) < B * T
        ref = ref * tm.view(B, T, 1).float()
        assert bool((got[~tm] == 0).all())
    err = float((got - ref).abs().max())
    _say(f"max-abs err {err:.3e}")
    assert err <= (TOL_BF16 if dt == torch.bfloat16 else TOL_F32)


def test_operator_rejects_out_of_range_prepacked_rows(dev):
    """Caller-supplied prepacked rows outside [0, T) / [0, B*H) raise
    ValueError before any kernel runs."""
    from proteus_attention.kernels.sparse_attn import aspa_sparse_attention

    q = torch.randn(2, 16, 64, device=dev, dtype=torch.bfloat16)
    offs = torch.tensor([0, 2, 3], dtype=torch.int32, device=dev)
    for heads, toks in (([0, 0, 1], [3, 16, 2]), ([0, 0, 2], [3, 4, 2]), ([0, 0, -1], [3, 4, 2])):
        pre = (torch.tensor(heads, device=dev), torch.tensor(toks, device=dev), offs, 2)
        with pytest.raises(ValueError, match="prepacked"):
            aspa_sparse_attention(q, q, q, prepacked=pre)


def test_builder_rejects_prototype_sets_beyond_the_limit(dev):
    """min(max_candidates, proto_cap, seq_len) above MAX_PROTO_CANDIDATES
    (2048) is rejected with ValueError; 2048 itself is served."""
    from proteus_attention.kernels.sparse_attn import MAX_PROTO_CANDIDATES, build_shortlist_candidates

    T = 4096
    rows = torch.arange(0, T, 97, device=dev)
    sims = torch.rand(T, device=dev)
    kw = dict(linear_window=16, anchor_stride=0, use_local=True, use_anchors=False, proto_scores=sims)
    with pytest.raises(ValueError, match="exceeds"):
        build_shortlist_candidates(rows, T, max_candidates=3000, proto_cap=MAX_PROTO_CANDIDATES + 1, **kw)
    cand, lens = build_shortlist_candidates(rows, T, max_candidates=3000, proto_cap=MAX_PROTO_CANDIDATES, **kw)
    oc, ol = O.build_shortlist(rows.cpu(), T, max_candidates=3000, proto_cap=MAX_PROTO_CANDIDATES,
                               linear_window=16, anchor_stride=0, use_local=True, use_anchors=False,
                               proto_scores=sims.cpu())
    assert torch.equal(cand.cpu(), oc) and torch.equal(lens.cpu(), ol)
