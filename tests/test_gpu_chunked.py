"""GPU parity of the chunked shortlist pipeline's device stages: chunk
salience top-k, global shortlist merge, per-row int8 quantisation, RoPE on
rows and the all-query int8 attention, each against the CPU oracle (and the
reference's golden vectors where they exist)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import aspa_oracle as O

pytestmark = pytest.mark.gpu


def _same(got, ref):
    if ref is None:
        return got is None
    assert got is not None
    return torch.equal(got[0].cpu(), ref[0]) and torch.equal(got[1].cpu(), ref[1])


def test_chunk_topk_golden(dev, golden):
    from proteus_attention.tools import chunk_select

    z = golden("chunk_select")
    s = torch.from_numpy(z["scores"]).to(dev)
    v, i = chunk_select.nucleus_select(s, 512, 1.0)
    assert np.array_equal(i.cpu().numpy(), z["i_p1"]) and np.array_equal(v.cpu().numpy(), z["v_p1"])
    v, i = chunk_select.nucleus_select(s * 4.0, 512, 0.9)
    assert np.array_equal(i.cpu().numpy(), z["i_p09"]) and np.array_equal(v.cpu().numpy(), z["v_p09"])


@pytest.mark.parametrize("n,budget,top_p,ties,masked", [
    (4096, 512, 1.0, False, True), (65536, 512, 1.0, False, True), (65536, 512, 1.0, True, True),
    (1000, 5000, 1.0, True, False), (70000, 9000, 1.0, True, True), (3000, 700, 0.5, False, True),
    (1, 1, 1.0, False, False), (257, 3, 0.999, True, True), (20000, 3000, 0.95, True, True),
    (262144, 512, 1.0, False, False)])
def test_chunk_topk_vs_oracle(dev, n, budget, top_p, ties, masked):
    from proteus_attention.tools import chunk_select

    g = torch.Generator().manual_seed(n + budget)
    s = torch.randint(-20, 20, (n,), generator=g).float() if ties else torch.randn(n, generator=g)
    s[torch.rand(n, generator=g) < 0.05] = float("-inf")
    mask = (torch.rand(n, generator=g) < 0.7) if masked else None
    print(f"chunk_topk n={n} budget={budget} top_p={top_p}", flush=True)
    for drop in (False, True):
        got = chunk_select.nucleus_select(s.to(dev), budget, top_p, keep_mask=None if mask is None else mask.to(dev),
                                          index_offset=12345, drop_nonfinite=drop)
        ref = O.nucleus_select(s, budget, top_p, keep_mask=mask, index_offset=12345, drop_nonfinite=drop)
        assert _same(got, ref)


def test_chunk_topk_all_masked_is_none(dev):
    from proteus_attention.tools import chunk_select

    s = torch.randn(300, device=dev)
    assert chunk_select.nucleus_select(s, 10, 1.0, keep_mask=torch.zeros(300, dtype=torch.bool, device=dev)) is None
    assert chunk_select.nucleus_select(torch.full((50,), float("-inf"), device=dev), 10, 1.0) is None


def test_finalise_golden(dev, golden):
    from proteus_attention.tools import chunk_select

    z = golden("chunk_select")
    ki, ks = chunk_select.finalise(torch.from_numpy(z["all_scores"]).to(dev), torch.from_numpy(z["all_idx"]).to(dev),
                                   4096)
    assert np.array_equal(ki.cpu().numpy(), z["keep_idx"]) and np.array_equal(ks.cpu().numpy(), z["keep_scores"])


@pytest.mark.parametrize("n,span,m", [(8192, 60000, 8192), (20000, 3000, 1500), (5, 3, 10), (40000, 10 ** 6, 8192)])
def test_finalise_vs_oracle(dev, n, span, m):
    from proteus_attention.tools import chunk_select

    g = torch.Generator().manual_seed(n)
    sc = torch.randint(-50, 50, (n,), generator=g).float() / 7.0
    idx = torch.randint(0, span, (n,), generator=g)
    print(f"finalise n={n} span={span} m={m}", flush=True)
    ki, ks = chunk_select.finalise(sc.to(dev), idx.to(dev), m)
    ri, rs = O.finalise_indices(sc, idx, m)
    assert torch.equal(ki.cpu(), ri) and torch.equal(ks.cpu(), rs)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_quantize_rows_bitwise(dev, dt):
    from proteus_attention.tools.final_pass import quantize_rows_int8

    g = torch.Generator().manual_seed(3)
    S, H, D = 777, 8, 64
    full = (torch.randn(S, 2 * H * D, generator=g) * torch.rand(S, 1, generator=g) * 4).to(dt)
    full[5, : H * D] = 0
    x = full[:, : H * D]  # row stride 2*H*D, as the K half of a (S, 2C) projection
    q, s = quantize_rows_int8(x.to(dev), H)
    rq, rs = O.quantize_rows_int8(x.float(), H)
    assert torch.equal(s.cpu(), rs) and torch.equal(q.cpu(), rq)


@pytest.mark.parametrize("dt,D,pad", [(torch.float32, 64, 0), (torch.bfloat16, 64, 0), (torch.bfloat16, 24, 0),
                                      (torch.bfloat16, 64, 2), (torch.float32, 20, 0), (torch.float16, 64, 0)])
def test_rope_rows_bitwise(dev, dt, D, pad):
    """RoPE on strided rows: the 8-element vector kernel (D a multiple of 8,
    16-byte aligned rows) and the per-pair kernel (D = 20, or a row stride
    that is not a multiple of 8 elements) both give the oracle's bits."""
    from proteus_attention.tools.final_pass import rope_rows_

    g = torch.Generator().manual_seed(4)
    T, H, n = 5000, 4, 300
    cos, sin = O.rope_tables(T, D, 10000.0, dt)
    x = torch.randn(n, 2 * H * D + pad, generator=g).to(dt)
    pos = torch.randint(0, T, (n,), generator=g)
    xd = x.to(dev)
    rope_rows_(xd[:, : H * D], H, cos.to(dev), sin.to(dev), positions=pos.to(dev))
    ref = O.apply_rope(x[:, : H * D].reshape(1, n, H, D), cos[pos], sin[pos]).reshape(n, H * D)
    assert torch.equal(xd[:, : H * D].cpu(), ref)
    assert torch.equal(xd[:, H * D:].cpu(), x[:, H * D:])
    # contiguous slice with an offset: rows start..start+n-1
    y = torch.randn(n, H * D, generator=g).to(dt)
    yd = y.to(dev)
    rope_rows_(yd, H, cos.to(dev), sin.to(dev), offset=1234)
    refy = O.apply_rope(y.view(1, n, H, D), cos[1234:1234 + n], sin[1234:1234 + n]).view(n, H * D)
    assert torch.equal(yd.cpu(), refy)


@pytest.mark.parametrize("T,H,S,causal,first", [(1000, 3, 77, True, 0), (4096, 8, 512, True, 300),
                                                (3000, 2, 130, False, 0), (700, 1, 1, True, 10),
                                                (513, 2, 513, True, 0)])
def test_int8_attention_vs_oracle(dev, T, H, S, causal, first):
    from proteus_attention.tools.final_pass import int8_shortlist_attention, quantize_rows_int8

    g = torch.Generator().manual_seed(T + S)
    D = 64
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(S, H * D, generator=g).to(torch.bfloat16)
    v = torch.randn(S, H * D, generator=g).to(torch.bfloat16)
    pos = torch.sort(torch.randperm(T - first, generator=g)[:S] + first).values
    print(f"int8 attention T={T} H={H} S={S} causal={causal}", flush=True)
    k8, ks = quantize_rows_int8(k.to(dev), H)
    v8, vs = quantize_rows_int8(v.to(dev), H)
    out = int8_shortlist_attention(q.to(dev), k8, v8, ks, vs, pos.to(dev), causal=causal)
    ref = O.int8_kv_attention(q, k8.cpu(), v8.cpu(), ks.cpu(), vs.cpu(), pos, causal=causal)
    err = float((out.float().cpu() - ref).abs().max())
    assert err <= 2e-2, err
    if causal and first > 0:
        assert float(out[:first].float().abs().max()) == 0.0


@pytest.mark.parametrize("T,H,S,boost", [(4096, 4, 300, 6.0), (2000, 2, 1000, 4.0)])
def test_int8_attention_dominant_keys_vs_oracle(dev, T, H, S, boost):
    """Queries and keys of 5% of the rows scaled up, so that single keys
    dominate the softmax of the scaled queries.  A dominant key's weight
    P * v_scale must reach the output unrounded (the kernel's lo parts):
    each element is held to 4e-3 beyond the bf16 output's own rounding (one
    bf16 rounding of that weight moves outputs of |v| ~ 10 by ~2e-2)."""
    from proteus_attention.tools.final_pass import int8_shortlist_attention, quantize_rows_int8

    g = torch.Generator().manual_seed(T * 7 + S)
    D = 64
    q = torch.randn(T, H, D, generator=g)
    q[torch.randperm(T, generator=g)[: T // 20]] *= boost
    k = torch.randn(S, H * D, generator=g)
    v = torch.randn(S, H * D, generator=g)
    hot = torch.randperm(S, generator=g)[: max(1, S // 20)]
    k[hot] *= boost
    v[hot] *= boost
    q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    pos = torch.sort(torch.randperm(T, generator=g)[:S]).values
    print(f"int8 attention, dominant keys: T={T} H={H} S={S} boost={boost}", flush=True)
    k8, ks = quantize_rows_int8(k.to(dev), H)
    v8, vs = quantize_rows_int8(v.to(dev), H)
    out = int8_shortlist_attention(q.to(dev), k8, v8, ks, vs, pos.to(dev))
    ref = O.int8_kv_attention(q, k8.cpu(), v8.cpu(), ks.cpu(), vs.cpu(), pos)
    d = (out.float().cpu() - ref).abs()
    half_ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(2.0 ** -126))) - 8.0)
    excess = float((d - half_ulp).max())
    assert float(ref.abs().max()) > 8.0  # the regime the test is for
    assert excess <= 4e-3, excess


def test_chunked_runner_all_queries_gpu(dev):
    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig, ChunkedShortlistRunner

    g = torch.Generator().manual_seed(21)
    T, C = 8192, 512
    x = torch.randn(1, T, C, generator=g).to(torch.bfloat16).to(dev)
    cfg = ChunkedShortlistConfig(seq_len=T, d_model=C, chunk_len=2048, buffer_tokens=512, per_chunk_budget=128,
                                 device=dev, heads=8, nucleus_top_p=1.0, final_mode="all_queries")
    runner = ChunkedShortlistRunner(cfg)
    res = runner.run(x)
    k = res.keep_indices
    # each chunk promotes min(budget, its token-kept count) tokens (the chunk
    # model keeps ~5% of 2048 tokens); the buffer holds them all
    promoted = sum(len(ch.promoted) for ch in res.chunks)
    assert all(1 <= len(ch.promoted) <= 128 for ch in res.chunks)
    assert k.numel() == min(512, promoted) and bool(torch.all(k[1:] > k[:-1]))
    assert res.final_output.shape == (1, T, C) and bool(torch.isfinite(res.final_output.float()).all())
    assert torch.equal(res.reduced_sequence.cpu(), x[:, k.to(dev)].cpu())
    fp = runner.last_final_pass
    k8, ks, v8, vs, pos = fp.last_shortlist
    ref = O.int8_kv_attention(fp.q_all[0].view(T, 8, 64).cpu(), k8.cpu(), v8.cpu(), ks.cpu(), vs.cpu(), pos.cpu())
    err = float((fp.last_attn.float().cpu() - ref).abs().max())
    assert err <= 2e-2, err
    for ch in res.chunks:
        assert all(ch.start <= p < ch.end for p in ch.promoted)


@pytest.mark.parametrize("source", ["cpu_tensor", "disk_tensor", "generated_cpu"])
def test_chunked_runner_host_staging_matches_device(dev, source):
    """Host-staged runs (a CPU tensor staged in pinned RAM, the same tensor
    staged in a disk memmap, and the runner's own seeded sequence) stream
    their chunks through the double-buffered stager and select exactly what
    the device-resident run over the same values selects."""
    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig, ChunkedShortlistRunner

    T, C = 8192, 512
    print(f"chunked runner staging {source}", flush=True)
    kw = dict(seq_len=T, d_model=C, chunk_len=2048, buffer_tokens=512, per_chunk_budget=128, device=dev, heads=8,
              nucleus_top_p=1.0, run_final_pass=False, seed=7)
    if source == "generated_cpu":
        gen = torch.Generator(device="cpu").manual_seed(7)
        x = torch.randn(1, T, C, generator=gen)  # the runner's own sequence (default dtype)
        torch.manual_seed(5)  # the chunk model's initial weights
        res = ChunkedShortlistRunner(ChunkedShortlistConfig(storage="cpu", **kw)).run(None)
    else:
        x = torch.randn(1, T, C, generator=torch.Generator().manual_seed(21)).to(torch.bfloat16)
        storage = "disk" if source == "disk_tensor" else "cpu"
        torch.manual_seed(5)
        res = ChunkedShortlistRunner(ChunkedShortlistConfig(storage=storage, **kw)).run(x)
        assert res.metrics.storage_mode == storage
    torch.manual_seed(5)
    ref = ChunkedShortlistRunner(ChunkedShortlistConfig(storage="cpu", **kw)).run(x.to(dev))
    assert ref.metrics.storage_mode == "device" and ref.metrics.h2d_time_ms is None
    assert torch.equal(res.keep_indices, ref.keep_indices)
    assert torch.equal(res.keep_scores, ref.keep_scores)
    assert torch.equal(res.reduced_sequence.cpu(), ref.reduced_sequence.cpu())
    assert [c.promoted for c in res.chunks] == [c.promoted for c in ref.chunks]
    assert res.metrics.h2d_time_ms is not None and res.metrics.h2d_time_ms > 0.0
    assert res.metrics.h2d_stall_ms is not None and res.metrics.h2d_stall_ms >= 0.0


@pytest.mark.parametrize("storage", ["device", "cpu", "disk"])
def test_chunked_runner_norm_fallback(dev, monkeypatch, storage):
    """A chunk whose selection is empty (count 0, known only after the chunk
    loop) and a chunk with no importance (known at once) both take the
    reference's token-norm fallback (chunked_shortlist.py:632-646): the
    first on its data fetched again from the staging, the second on the
    chunk in hand.  Every other chunk keeps its importance selection."""
    from proteus_attention.tools import chunked_shortlist as cs
    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig, ChunkedShortlistRunner

    T, C, chunk, budget = 8192, 512, 2048, 128
    print(f"chunked runner norm fallback storage={storage}", flush=True)
    x = torch.randn(1, T, C, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16)
    orig = cs._select_top_tokens
    seen = {}

    def patched(model, offset, **kw):
        out = orig(model, offset, **kw)
        c = int(out[2].item())
        seen[offset] = (out[0][:c].cpu(), out[1][:c].cpu())
        if offset == 0:
            return out[0], out[1], torch.zeros_like(out[2])
        if offset == 2 * chunk:
            return None
        return out

    monkeypatch.setattr(cs, "_select_top_tokens", patched)
    kw = dict(seq_len=T, d_model=C, chunk_len=chunk, buffer_tokens=T, per_chunk_budget=budget, device=dev, heads=8,
              nucleus_top_p=1.0, run_final_pass=False)
    src = x.to(dev) if storage == "device" else x
    res = ChunkedShortlistRunner(ChunkedShortlistConfig(storage="cpu" if storage == "device" else storage,
                                                        **kw)).run(src)
    assert res.metrics.storage_mode == storage and res.metrics.used_fallback
    assert [ch.index for ch in res.chunks] == [0, 1, 2, 3]
    xd = x.to(dev)
    all_s, all_i = [], []
    for ch in res.chunks:
        s = ch.start
        if s in (0, 2 * chunk):
            norms = xd[0, s:s + chunk].norm(dim=-1).to(torch.float32).cpu()
            ev, ei = O.nucleus_select(norms, budget, 1.0, index_offset=s)
        else:
            ev, ei = seen[s]
        assert ch.promoted == ei.tolist(), f"chunk at {s}"
        assert torch.equal(torch.tensor(ch.scores, dtype=torch.float32), ev), f"chunk at {s}"
        all_s.append(ev)
        all_i.append(ei)
    ki, ks = O.finalise_indices(torch.cat(all_s), torch.cat(all_i), T)
    assert torch.equal(res.keep_indices.cpu(), ki) and torch.equal(res.keep_scores.cpu(), ks)


@pytest.mark.parametrize("storage", ["device", "cpu"])
def test_chunked_runner_graph_matches_eager(dev, storage):
    """The chunk model replayed from a captured HIP graph selects exactly
    what the eager chunk model selects, chunk by chunk, and gives the same
    shortlist and final output.  60,000 tokens in chunks of 24,576: the two
    full chunks replay the graph (materialised candidates); the 10,848-token
    last chunk takes the structured path, which reads its row count, and
    runs eagerly between them and the selection.  With the sequence staged
    from host memory the chunk model stays eager (graph replays slowed the
    staging copies), so the flag changes nothing there."""
    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig, ChunkedShortlistRunner

    T, C, chunk = 60000, 512, 24576
    print(f"chunked runner graph vs eager storage={storage}", flush=True)
    x = torch.randn(1, T, C, generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    kw = dict(seq_len=T, d_model=C, chunk_len=chunk, buffer_tokens=600, per_chunk_budget=256, device=dev, heads=8,
              nucleus_top_p=1.0, final_mode="all_queries", storage="cpu")
    src = x.to(dev) if storage == "device" else x
    res, graphs = {}, {}
    for graph in (False, True):
        torch.manual_seed(5)
        runner = ChunkedShortlistRunner(ChunkedShortlistConfig(chunk_graph=graph, **kw))
        res[graph] = runner.run(src)
        graphs[graph] = len(runner.last_chunk_model._hip_graphs)
    assert graphs[True] == (1 if storage == "device" else 0) and graphs[False] == 0
    assert res[True].metrics.storage_mode == storage
    for a, b in zip(res[False].chunks, res[True].chunks):
        assert a.promoted == b.promoted and a.scores == b.scores, f"chunk {a.index}"
    assert torch.equal(res[False].keep_indices, res[True].keep_indices)
    assert torch.equal(res[False].keep_scores, res[True].keep_scores)
    assert torch.equal(res[False].final_output.cpu(), res[True].final_output.cpu())



@pytest.mark.parametrize("storage", ["device", "cpu", "disk"])
def test_chunked_runner_frees_its_models_without_cycle_collector(dev, storage):
    """A finished run leaves no reference cycle behind: with Python's cycle
    collector off, dropping the runner and its result returns every device
    byte the run allocated (chunk and final models, captured graph, staging
    buffers) by reference counting alone.  A cycle would keep each run's
    models alive until the collector happened to run, so back-to-back runs
    would grow the device footprint run by run."""
    import gc
    import weakref

    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig, ChunkedShortlistRunner

    T, C, chunk = 60000, 512, 24576
    print(f"chunked runner frees its models storage={storage}", flush=True)
    x = torch.randn(1, T, C, generator=torch.Generator().manual_seed(29)).to(torch.bfloat16)
    cfg = ChunkedShortlistConfig(seq_len=T, d_model=C, chunk_len=chunk, buffer_tokens=600, per_chunk_budget=256,
                                 device=dev, heads=8, nucleus_top_p=1.0, final_mode="all_queries",
                                 storage="disk" if storage == "disk" else "cpu")
    src = x.to(dev) if storage == "device" else x
    ChunkedShortlistRunner(cfg).run(src)  # warm-up: library workspaces, GEMM handles
    gc.collect()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated(dev)
    gc.disable()
    try:
        runner = ChunkedShortlistRunner(cfg)
        res = runner.run(src)
        assert res.keep_indices.numel() > 0
        model = weakref.ref(runner.last_chunk_model)
        del runner, res
        torch.cuda.synchronize()
        assert model() is None
        assert torch.cuda.memory_allocated(dev) == base
    finally:
        gc.enable()


def test_module_freed_without_cycle_collector(dev):
    """Dropping a module after eager or graph-replayed forwards returns
    every device byte its forwards allocated, by reference counting alone:
    the telemetry steps a forward defers (run at the next forward or
    telemetry read) do not keep the module alive, and its side streams are
    shared, so no per-instance GEMM workspace stays behind."""
    import gc
    import weakref

    from proteus_attention.models.aspa import AdaptiveSparseAttention
    from proteus_attention.tools.chunked_shortlist import _build_model_config

    T = 24576
    x = torch.randn(1, T, 512, generator=torch.Generator().manual_seed(31)).to(torch.bfloat16).to(dev)

    def make():
        m = AdaptiveSparseAttention(_build_model_config(T, 512, heads=8, sparse_ratio=0.05, shortlist_alpha=0.0,
                                                        router_top_p=1.0)).to(dev, torch.bfloat16).eval()
        m.use_sdpa = False
        return m

    for graph in (False, True):
        print(f"module freed without cycle collector graph={graph}", flush=True)
        warm = make()
        warm.enable_hip_graph(graph)
        with torch.inference_mode():
            warm(x)  # library handles and workspaces
        del warm
        gc.collect()
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated(dev)
        gc.disable()
        try:
            m = make()
            if graph:
                with torch.no_grad():
                    assert m._graph_eligible(x)
            m.enable_hip_graph(graph)
            with torch.inference_mode():
                for _ in range(3):
                    m(x)
            assert len(m._hip_graphs) == (1 if graph else 0)
            assert m.__dict__.get("_pending_stats")
            ref = weakref.ref(m)
            del m
            torch.cuda.synchronize()
            assert ref() is None
            assert torch.cuda.memory_allocated(dev) == base
        finally:
            gc.enable()
