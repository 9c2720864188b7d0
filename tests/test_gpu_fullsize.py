"""GPU: the BASELINE configs at their full size against the CPU oracle.

config 3 (T=65,536, L=2048) and config 4 (T=524,288, L=4096, single pass):
  * routing: head sets per token against the oracle router (torch CPU, the
    reference's own arithmetic), proven token by token (routing_parity);
  * prototype similarities to f32 rounding;
  * candidate lengths: every row (config 3) or every 16th row (config 4)
    against the C oracle builder fed this forward's similarities and packed
    rows -- integer work, so exact, and the sum over the checked rows too;
  * attention: a sample of packed rows against an f32 restatement of the
    candidate attention over the oracle's candidate lists, within the bf16
    tolerance.
config 5 (T=1,048,576, chunked): every chunk's promoted tokens against the
  oracle's nucleus selection of the same importances, the global shortlist
  against the oracle's merge, and a sample of all-query final-pass rows
  against the oracle's int8 attention.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import aspa_oracle as O
from oracle import c_oracle

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2


def _say(msg: str) -> None:
    print(f"[fullsize] {msg}", flush=True)


def _module(cfg, B, T, C, dt, dev, outlier):
    from configs import init_weights, make_inputs

    from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

    torch.manual_seed(1234)
    m = AdaptiveSparseAttention(ModelConfig(**cfg))
    x, g = make_inputs(B, T, C, seed=0, outlier_frac=outlier)
    init_weights(m, g)
    m = m.to(device=dev, dtype=dt).eval()
    return m, x.to(dt)


@pytest.mark.parametrize("T,L,row_every,attn_every", [(65536, 2048, 1, 64), (524288, 4096, 16, 512)])
def test_shortlist_forward_full_size_vs_oracle(dev, T, L, row_every, attn_every):
    _check_shortlist_forward(dev, T, L, row_every, attn_every, H=8, G=8, window=512, stride=256,
                             outlier=0.01 if T == 65536 else 0.0)


@pytest.mark.parametrize("T,H,G,window,stride", [(16384, 32, 64, 256, 64), (16384, 4, 4, 512, 128),
                                                 (16384, 16, 32, 256, 64)])
def test_shortlist_forward_head_shapes_vs_oracle(dev, T, H, G, window, stride):
    """The same checks at the shapes off the BASELINE configs: 32 heads of
    16 dims with 64 gates (the reference's tinytoy recipe,
    kernels/tinytoy.py:307-325), 4 heads of 128 dims, 16 heads of 32 dims
    with 32 gates -- the MFMA router in 16-gate blocks and the structured
    attention at those head widths."""
    _check_shortlist_forward(dev, T, 1024, 1, 16, H=H, G=G, window=window, stride=stride, outlier=0.01)


def _check_shortlist_forward(dev, T, L, row_every, attn_every, H, G, window, stride, outlier):
    from configs import shortlist_cfg
    from routing_parity import check_routing

    B, C = 1, 512
    D = C // H
    _say(f"shortlist forward T={T} L={L} H={H} D={D} G={G}")
    cfg = shortlist_cfg(T, C, H, L, window, stride)
    cfg["attn_gates"] = G
    m, x = _module(cfg, B, T, C, torch.bfloat16, dev, outlier)
    m.record_shortlist_lengths = True
    w_router = m.head_router.linear.weight.detach().cpu()
    protos = m.routing_prototypes.detach().cpu()
    conf = m.routing_confidence.detach().cpu()
    xd = x.to(dev)
    with torch.no_grad():
        m(xd)
        qkv = m.qkv(xd).view(B, T, 3, H, D).cpu()  # the forward's projection (same GEMM)
    torch.cuda.synchronize()
    st = m._last_sparse_state
    assert st["mode"] == "shortlist" and st["linear_shortlist_structured"] is True
    tok = st["token_idx"].cpu().long()
    offs = st["row_offsets"].cpu().long()
    heads = st["active_head_indices"].cpu().long()
    lens = m._last_shortlist_lengths.cpu().numpy()
    sims = m._last_token_similarity.float().cpu()
    gates = m._last_gate_probs.float().cpu().reshape(B * T, G)
    g2h = m.gate_to_head.cpu()
    attn = m.last_head_consensus.view(B, T, H, D).float().cpu()

    # routing against the oracle router on the same inputs
    og, osim, _, _ = O.route_tokens(x, w_router, protos, conf, None, proto_temp=float(m.proto_temp),
                                    proto_threshold=float(m.proto_threshold), proto_blend=float(m.proto_blend),
                                    usage_boost=float(m.proto_usage_boost))
    assert torch.allclose(sims.reshape(-1), osim.reshape(-1), atol=2e-6, rtol=0)
    row_head = torch.repeat_interleave(torch.arange(heads.numel()), offs[1:] - offs[:-1])
    ours = torch.zeros(B * H, T, dtype=torch.bool)
    ours[heads[row_head], tok] = True
    ours = ours.view(B, H, T).permute(0, 2, 1).reshape(B * T, H)
    _, oidx = O.topk_lowest(O.head_probs_from_gates(og.reshape(B * T, G), g2h, H), 2)
    ref = torch.zeros(B * T, H, dtype=torch.bool).scatter_(1, oidx, True)
    rep = check_routing(ours, ref, gates, og.reshape(B * T, G), x.reshape(B * T, C), w_router, 2,
                        gate_to_head=None if G == H else g2h, sum_ulps=0 if G <= 8 else G)
    _say(f"T={T} routing vs oracle: {rep}")
    rep.assert_boundary_sets_at_most(1e-3)
    N = int(tok.numel())
    assert N == 2 * B * T

    # candidate lengths: the C oracle builder on this forward's rows and sims
    plan = m._shortlist_plan(B, T, 1.0, torch.bfloat16)
    assert plan["structured"] and plan["L"] == L
    sel = np.arange(0, N, row_every)
    rows = tok.numpy().astype(np.int32)[sel]
    cand, olens = c_oracle.shortlist_build(rows, None, T, L, plan["local_w"], plan["stride"], plan["slots"],
                                           sims.numpy(), plan["K"])
    assert np.array_equal(lens[sel], olens)
    _say(f"T={T} candidate lengths exact on {sel.size} rows; sum {int(olens.astype(np.int64).sum())}")

    # attention rows: f32 restatement over the oracle's candidates, q/k/v
    # from the same projection, rotated by the oracle's RoPE with the
    # module's own tables (its inverse frequencies are a buffer in the
    # module's dtype, as in the reference)
    cos, sin = (t.cpu() for t in m._rope_factors(T, dev, torch.bfloat16))
    sub = np.arange(0, sel.size, max(1, attn_every // row_every))
    r_tok = tok[sel[sub]]
    r_bh = heads[row_head[sel[sub]]]
    max_err = 0.0
    scale = 1.0 / math.sqrt(D)
    for j, i in enumerate(sub):
        t, h = int(r_tok[j]), int(r_bh[j]) % H
        c = torch.from_numpy(cand[i, :olens[i]]).long()
        q_r = O.apply_rope(qkv[:, t:t + 1, 0, h:h + 1], cos[t:t + 1], sin[t:t + 1]).reshape(D).float()
        k_r = O.apply_rope(qkv[:, c, 1, h:h + 1], cos[c], sin[c]).reshape(-1, D).float()
        v_r = qkv[0, c, 2, h].float()
        p = torch.softmax((k_r @ q_r) * scale, dim=0)
        max_err = max(max_err, float((attn[0, t, h] - p @ v_r).abs().max()))
    _say(f"T={T} attention on {sub.size} sampled rows: max-abs err {max_err:.3e}")
    assert max_err <= TOL_BF16


def test_chunked_pipeline_config5_vs_oracle(dev, monkeypatch):
    """Config 5 end to end: T = 2^20 in 16 chunks of 65,536, top-512 per
    chunk (nucleus_top_p = 1), an 8,192-token global shortlist, int8 (per
    head and row) K/V, all-query final pass."""
    from proteus_attention.tools import chunked_shortlist as cs
    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig, ChunkedShortlistRunner

    T, C, H, chunk, budget, buf = 1 << 20, 512, 8, 65536, 512, 8192
    _say(f"chunked pipeline T={T}")
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, T, C, generator=g).to(torch.bfloat16).to(dev)
    seen = []
    orig = cs._select_top_tokens

    def spy(model, offset, **kw):
        imp = model._last_token_importance.squeeze(0).float().cpu()
        mask = model._last_token_mask.squeeze(0).cpu()
        out = orig(model, offset, **kw)
        c = None if out is None else int(out[2].item())
        seen.append((offset, imp, mask, None if out is None else (out[0][:c].cpu(), out[1][:c].cpu())))
        return out

    monkeypatch.setattr(cs, "_select_top_tokens", spy)
    cfg = ChunkedShortlistConfig(seq_len=T, d_model=C, chunk_len=chunk, buffer_tokens=buf, per_chunk_budget=budget,
                                 device=dev, heads=H, nucleus_top_p=1.0, final_mode="all_queries")
    runner = ChunkedShortlistRunner(cfg)
    res = runner.run(x)
    assert len(seen) == T // chunk
    all_s, all_i = [], []
    for offset, imp, mask, got in seen:
        exp = O.nucleus_select(imp, budget, 1.0, keep_mask=mask, index_offset=offset, drop_nonfinite=True)
        assert got is not None and exp is not None
        ev, ei = exp
        assert torch.equal(got[1], ei) and torch.equal(got[0], ev), f"chunk at {offset}"
        all_s.append(ev)
        all_i.append(ei)
    ki, ks = O.finalise_indices(torch.cat(all_s), torch.cat(all_i), buf)
    assert torch.equal(res.keep_indices.cpu(), ki) and torch.equal(res.keep_scores.cpu(), ks)
    assert ki.numel() == buf
    _say(f"chunk selections and the {buf}-token shortlist exact")
    # final pass: sampled queries against the oracle's int8 attention
    fp = runner.last_final_pass
    k8, ksc, v8, vsc, pos = (t.cpu() for t in fp.last_shortlist)
    qsel = torch.arange(0, T, 1024)
    q = fp.q_all[0].view(T, H, 64)[qsel.to(dev)].cpu()
    ref = O.int8_kv_attention(q, k8, v8, ksc, vsc, pos, q_pos=qsel)
    got = fp.last_attn.view(T, H, 64)[qsel.to(dev)].float().cpu()
    err = float((got - ref).abs().max())
    _say(f"final pass on {qsel.numel()} sampled queries: max-abs err {err:.3e}")
    assert err <= TOL_BF16
    assert res.final_output.shape == (1, T, C) and bool(torch.isfinite(res.final_output.float()).all())


def test_config5_final_pass_with_outlier_rows_vs_oracle(dev):
    """Config 5 on config 3's outlier recipe: 1% of the input rows scaled by
    4, so query-key scores between outlier rows are ~16x those of N(0,1)
    rows and single keys dominate their queries' softmax.  The all-query
    final pass scores against the exact int8 keys with f32 scales, takes
    the exact row maximum and adds a dominant key's weight unrounded, so
    the dominant-key rows must still meet the bf16 bound (a single bf16
    copy of the scaled K moved such scores by tenths and the outputs by
    ~0.1).  The pipeline runs at full size (T = 2^20);
    the sampled queries are every 1024th token plus the first 1,024 outlier
    tokens."""
    from configs import make_inputs

    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig, ChunkedShortlistRunner

    T, C, H, chunk, budget, buf = 1 << 20, 512, 8, 65536, 512, 8192
    _say(f"chunked pipeline T={T} with 1% outlier rows x4")
    x, g = make_inputs(1, T, C, seed=5, outlier_frac=0.01)
    # the outlier positions, regenerated from the recipe (randperm after randn)
    g2 = torch.Generator().manual_seed(5)
    torch.randn(1, T, C, generator=g2)
    outliers = torch.sort(torch.randperm(T, generator=g2)[: int(round(0.01 * T))]).values
    xd = x.to(torch.bfloat16).to(dev)
    del x
    torch.manual_seed(7)
    cfg = ChunkedShortlistConfig(seq_len=T, d_model=C, chunk_len=chunk, buffer_tokens=buf, per_chunk_budget=budget,
                                 device=dev, heads=H, nucleus_top_p=1.0, final_mode="all_queries")
    runner = ChunkedShortlistRunner(cfg)
    res = runner.run(xd)
    fp = runner.last_final_pass
    k8, ksc, v8, vsc, pos = (t.cpu() for t in fp.last_shortlist)
    kept_out = int(torch.isin(pos.long(), outliers).sum())
    qsel = torch.unique(torch.cat([torch.arange(0, T, 1024), outliers[:1024]]))
    q = fp.q_all[0].view(T, H, 64)[qsel.to(dev)].cpu()
    ref = O.int8_kv_attention(q, k8, v8, ksc, vsc, pos, q_pos=qsel)
    got = fp.last_attn.view(T, H, 64)[qsel.to(dev)].float().cpu()
    # The output is bf16: around |out| = 8..10 its grid spacing is 2^-4, so
    # the bf16 value nearest to the f32 result may itself be 2^-5 away.  Each
    # element is held to the bf16 bound plus half the bf16 spacing at its
    # reference value (the output's own rounding).
    d = (got - ref).abs()
    half_ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -126))) - 8.0)
    excess = float((d - half_ulp).max())
    err = float(d.max())
    wi = int(d.argmax())
    qmax = float(q.float().abs().max())
    _say(f"outlier final pass: {kept_out} outlier tokens in the shortlist, |q| max {qmax:.2f}, "
         f"{qsel.numel()} sampled queries: max-abs err {err:.3e} (got {float(got.flatten()[wi]):.5f}, "
         f"ref {float(ref.flatten()[wi]):.5f}), |ref| max {float(ref.abs().max()):.3f}; beyond the output's own "
         f"rounding {excess:.3e}; elements above 2e-2: {int((d > TOL_BF16).sum())} of {d.numel()}")
    assert excess <= TOL_BF16
    assert bool(torch.isfinite(res.final_output.float()).all())
