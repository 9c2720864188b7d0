"""Write golden vectors by running the reference implementation on CPU.

Run in the development container only (the reference tree is not shipped):

    python tests/golden/make_golden.py [/path/to/reference]

It imports Proteus-Flux-Attention from <reference>/src and records, for
seeded inputs, what the reference computes for the functions no closed form
or reference test pins exactly: the bf16/f32 router as executed by torch on
CPU, the token and head selections it makes, full module forwards under the
BASELINE config mapping (including the post-forward prototype EMA state),
the packed builder with prototype candidates at realistic sizes, the
operator's fallback outputs, and the chunk-selection orderings.  Only data
(inputs and outputs) is written, as .npz files next to this script.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))  # tests/ (configs)
from configs import init_weights, make_inputs, shortlist_cfg, sparse_cfg, state_tensors  # noqa: E402


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.numpy()


def _digest(*tensors: torch.Tensor) -> str:
    import hashlib

    h = hashlib.sha256()
    for t in tensors:
        h.update(t.detach().cpu().float().contiguous().numpy().tobytes())
    return h.hexdigest()


def _save(name: str, **arrays) -> None:
    path = HERE / f"{name}.npz"
    np.savez_compressed(path, **{k: (_np(v) if isinstance(v, torch.Tensor) else np.asarray(v)) for k, v in arrays.items()})
    print(f"wrote {path.name} ({path.stat().st_size / 1024:.0f} KiB)")


def module_case(ref, name: str, cfg: dict, B: int, T: int, C: int, dtype: torch.dtype, outlier: float = 0.0,
                token_stride: int = 1, n_forward: int = 1) -> None:
    ModelConfig = ref.models.aspa.ModelConfig
    ASPA = ref.models.aspa.AdaptiveSparseAttention
    torch.manual_seed(1234)
    m = ASPA(ModelConfig(**cfg))
    x, g = make_inputs(B, T, C, seed=0, outlier_frac=outlier)
    init_weights(m, g)
    w = state_tensors(m)
    m = m.to(dtype=dtype).eval()
    xd = x.to(dtype)
    gate_probs = {}

    orig_route = m._route_tokens

    def spy(inp):
        out = orig_route(inp)
        gate_probs["g"] = out.detach().clone()
        return out

    m._route_tokens = spy
    extra = {}
    with torch.no_grad():
        y = m(xd)
        for i in range(1, n_forward):
            # later forwards see the EMA state the earlier ones left
            extra[f"y_first{i}"] = y[:, ::token_stride].float()
            y = m(xd)
    for nm in ("_quant_ema_q", "_quant_ema_k", "_quant_ema_v"):
        t = getattr(m, nm, None)
        if isinstance(t, torch.Tensor):
            extra[nm.lstrip("_")] = t.detach().float()
    st = m._last_sparse_state or {}
    # x and the weights are regenerated from the seed by the tests; their
    # digests pin the regeneration.
    arrays = dict(
        x_sha256=np.array(_digest(x)), w_sha256=np.array(_digest(*w.values())),
        y=y[:, ::token_stride].float(), token_stride=np.int64(token_stride),
        gate_probs=gate_probs["g"].float(), importance=m._last_token_importance.float(),
        sim=m._last_token_similarity.float(), blend=m._last_token_blend.float(),
        protos_after=m.routing_prototypes.detach().float(), usage_after=m.routing_usage_ema.detach().float(),
        conf_after=m.routing_confidence.detach().float(),
        linear_L=np.int64(m.linear_L), linear_window=np.int64(m.linear_window),
        mode=np.array(str(m.last_head_stats.get("mode"))), n_forward=np.int64(n_forward), **extra,
    )
    if m._last_token_mask is not None:
        arrays["token_mask"] = m._last_token_mask.to(torch.uint8)
    if "token_idx" in st:
        arrays["packed_token_idx"] = st["token_idx"].to(torch.int64)
        arrays["packed_row_offsets"] = st["row_offsets"].to(torch.int64)
        arrays["active_head_indices"] = st["active_head_indices"].to(torch.int64)
    _save(name, **arrays)


def dropin_case(ref, name: str, T: int, pad_from: int, **kw) -> None:
    """CausalASPAMultiheadAttention (reference modules/aspa_multihead.py) in
    eval mode on a seeded input with a key padding mask: its state dict, its
    output and the head statistics of its attention layer (the default
    router_top_p = 0.9 takes every forward through the nucleus head count,
    aspa.py:749-780, 1574-1589)."""
    MHA = ref.modules.CausalASPAMultiheadAttention
    torch.manual_seed(4321)
    mha = MHA(embed_dim=64, num_heads=4, batch_first=True, **kw).eval()
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, T, 64, generator=g)
    pad = torch.zeros(2, T, dtype=torch.bool)
    pad[1, pad_from:] = True
    # the state before the forward (the forward moves the prototype EMA)
    arrays = {f"sd::{k}": v.detach().clone() for k, v in mha.state_dict().items()}
    with torch.no_grad():
        out, w = mha(x, key_padding_mask=pad, need_weights=True)
    hs = mha.attention.last_head_stats or {}
    arrays.update(x=x, pad=pad.to(torch.uint8), out=out, weights_shape=np.array(w.shape),
                  top_k=np.int64(hs.get("top_k", -1)), nucleus_k=np.int64(hs.get("nucleus_k", -1)),
                  mode=np.array(str(hs.get("mode"))), kw=np.array(repr(sorted(kw.items()))))
    _save(name, **arrays)


def nucleus_case(ref) -> None:
    """_nucleus_head_count (aspa.py:749-780) on seeded head probabilities:
    softmax rows with a temperature sweep (mass spread from one head to all),
    a target_p sweep and a cap sweep."""
    ASPA = ref.models.aspa.AdaptiveSparseAttention
    m = ASPA(ref.models.aspa.ModelConfig(d_model=64, n_head=8, attn_h_total=8, attn_gates=8))
    g = torch.Generator().manual_seed(13)
    probs, ks = [], []
    for temp in (0.05, 0.3, 1.0, 4.0):
        # a per-head bias so the mean mass is uneven across heads
        bias = torch.linspace(3.0, -3.0, 8)[torch.randperm(8, generator=g)]
        p = torch.softmax((torch.randn(2, 50, 8, generator=g) + bias) / temp, dim=-1)
        probs.append(p)
        row = [m._nucleus_head_count(p, tp, cap) for tp in (0.0, 0.5, 0.9, 0.99, 1.0) for cap in (1, 3, 8)]
        ks.append(row)
    _save("nucleus_head_count", probs=torch.stack(probs), k=torch.tensor(ks), target_p=np.array([0.0, 0.5, 0.9, 0.99, 1.0]),
          caps=np.array([1, 3, 8]))


def builder_cases(ref) -> None:
    sa = ref.kernels.sparse_attn
    g = torch.Generator().manual_seed(11)
    # reference-test-sized cases (seq 64, L 16, window 12, stride 4)
    rows = torch.randint(0, 64, (16,), generator=g)
    scores = torch.rand(64, generator=g)
    for tag, (ul, ua, up) in {"l": (1, 0, 0), "la": (1, 1, 0), "lp": (1, 0, 1), "ap": (0, 1, 1)}.items():
        c, l = sa.build_shortlist_candidates(rows, 64, max_candidates=16, linear_window=12, anchor_stride=4,
                                             use_local=bool(ul), use_anchors=bool(ua),
                                             proto_scores=scores if up else None)
        _save(f"builder_small_{tag}", rows=rows, scores=scores, use=np.array([ul, ua, up]), cand=c, lengths=l)
    # packed, two batches, realistic proto sizes, distinct scores
    T = 4096
    sims = torch.rand(2, T, generator=g)
    toks = []
    rb = []
    for b in range(2):
        for h in range(3):
            sel = torch.sort(torch.randperm(T, generator=g)[: 700]).values
            toks.append(sel)
            rb.append(torch.full_like(sel, b))
    rows = torch.cat(toks)
    row_batch = torch.cat(rb)
    kw = dict(max_candidates=1024, linear_window=256, anchor_stride=64, use_local=True, use_anchors=True,
              local_cap=256, anchor_cap=307, proto_cap=102)
    c, l = sa.build_packed_shortlist_candidates(rows, row_batch, T, proto_scores=sims, **kw)
    _save("builder_packed_T4096", rows=rows, row_batch=row_batch, sims=sims, cand=c.to(torch.int32), lengths=l,
          kw=np.array([1024, 256, 64, 256, 307, 102]))
    # truncation case: more unique candidates than L
    rows = torch.sort(torch.randperm(2048, generator=g)[:400]).values
    sims1 = torch.rand(2048, generator=g)
    c, l = sa.build_shortlist_candidates(rows, 2048, max_candidates=96, linear_window=64, anchor_stride=16,
                                         use_local=True, use_anchors=True, proto_scores=sims1, local_cap=64,
                                         anchor_cap=64, proto_cap=64)
    _save("builder_truncate", rows=rows, sims=sims1, cand=c, lengths=l, kw=np.array([96, 64, 16, 64, 64, 64]))


def attention_cases(ref) -> None:
    sa = ref.kernels.sparse_attn
    g = torch.Generator().manual_seed(21)
    for dtype, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
        BH, T, D = 6, 257, 64
        q = torch.randn(BH, T, D, generator=g)
        k = torch.randn(BH, T, D, generator=g)
        v = torch.randn(BH, T, D, generator=g)
        mask = torch.rand(BH, T, generator=g) > 0.6
        mask[0] = False
        causal = torch.triu(torch.full((T, T), float("-inf")), diagonal=1)
        out_nc = sa.aspa_sparse_attention(q.to(dtype), k.to(dtype), v.to(dtype), active_mask=mask.unsqueeze(-1))
        out_m = sa.aspa_sparse_attention(q.to(dtype), k.to(dtype), v.to(dtype), active_mask=mask.unsqueeze(-1),
                                         causal_mask=causal)
        packed = sa._pack_active_rows(mask)
        rows = packed[1]
        cand, lens = sa.build_shortlist_candidates(rows, T, max_candidates=48, linear_window=16, anchor_stride=8,
                                                   use_local=True, use_anchors=True, anchor_cap=20)
        out_c = sa.aspa_sparse_attention(q.to(dtype), k.to(dtype), v.to(dtype), active_mask=mask.unsqueeze(-1),
                                         prepacked=packed, shortlist_candidates=cand, shortlist_lengths=lens)
        _save(f"attn_{tag}", q=q, k=k, v=v, mask=mask.to(torch.uint8), out_nocand=out_nc.float(),
              out_mask=out_m.float(), cand=cand, lengths=lens, out_cand=out_c.float())


def chunk_cases(ref) -> None:
    cs = ref.tools.chunked_shortlist
    g = torch.Generator().manual_seed(31)
    scores = torch.randn(4096, generator=g)
    scores[::97] = float("-inf")
    v1, i1 = cs._nucleus_select(scores, 512, 1.0)
    v2, i2 = cs._nucleus_select(scores * 4.0, 512, 0.9)
    allsc = torch.randn(16 * 512, generator=g)
    allidx = torch.randint(0, 60000, (16 * 512,), generator=g)
    ki, ks = cs._finalise_indices(allsc, allidx, max_tokens=4096)
    _save("chunk_select", scores=scores, v_p1=v1, i_p1=i1, v_p09=v2, i_p09=i2, all_scores=allsc, all_idx=allidx,
          keep_idx=ki, keep_scores=ks)


def rope_case(ref) -> None:
    """RoPE tables and rotation (aspa.py:226-247, 576-618) as the reference
    module computes them on CPU: _rope_factors and _apply_rope_embedding of
    modules cast to f32 and to bf16 (the cast turns the inverse-frequency
    buffer into bf16 too, so positions above 256 round), head dims 64 and 32,
    T = 1024.  The tables are stored whole; the seeded q/k (1, T, 2, D) and
    their rotations at every 8th position.  bf16 arrays are stored as their
    int16 bit patterns."""
    ModelConfig = ref.models.aspa.ModelConfig
    ASPA = ref.models.aspa.AdaptiveSparseAttention
    g = torch.Generator().manual_seed(17)
    T = 1024

    def bits(t: torch.Tensor) -> np.ndarray:
        t = t.detach().cpu().contiguous()
        return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()

    arrays = {}
    for D in (64, 32):
        H = 256 // D
        for dtype, tag in ((torch.float32, "f32"), (torch.bfloat16, "bf16")):
            m = ASPA(ModelConfig(d_model=256, n_head=H, attn_h_total=H, attn_gates=H)).to(dtype=dtype).eval()
            cos, sin = m._rope_factors(T, torch.device("cpu"), dtype)
            q = torch.randn(1, T, 2, D, generator=g).to(dtype)
            k = torch.randn(1, T, 2, D, generator=g).to(dtype)
            m.d_head = D
            with torch.no_grad():
                qo, ko = m._apply_rope_embedding(q, k)
            key = f"D{D}_{tag}"
            arrays.update({f"{key}_cos": bits(cos), f"{key}_sin": bits(sin), f"{key}_q": bits(q[:, ::8]),
                           f"{key}_k": bits(k[:, ::8]), f"{key}_qo": bits(qo[:, ::8]), f"{key}_ko": bits(ko[:, ::8])})
    _save("rope_tables", T=np.int64(T), base=np.float64(10000.0), every=np.int64(8), **arrays)


def main() -> None:
    ref_root = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    sys.path.insert(0, str(ref_root / "src"))
    import proteus_attention.kernels.sparse_attn  # noqa: F401
    import proteus_attention.models.aspa  # noqa: F401
    import proteus_attention.tools.chunked_shortlist  # noqa: F401
    import proteus_attention.modules  # noqa: F401
    import proteus_attention as ref

    torch.set_num_threads(8)
    cases = module_cases()
    only = [a for a in sys.argv[2:]]
    if only:
        # the named cases only (every other fixture left as it is)
        for name in only:
            cases[name](ref)
        return
    builder_cases(ref)
    attention_cases(ref)
    chunk_cases(ref)
    for name, fn in cases.items():
        if name not in FULL_SIZE_CASES:
            fn(ref)


# Cases at a BASELINE config's full size take minutes of CPU time in the
# reference; they are written only when named on the command line.
FULL_SIZE_CASES = ("module_cfg2_full",)


def module_cases():
    short = shortlist_cfg(2048, 512, 8, 512, 128, 32)
    return {
        # config 1 exactly (f32), token-sparse causal
        "module_cfg1": lambda ref: module_case(ref, "module_cfg1", sparse_cfg(1024, 256, 8), 1, 1024, 256,
                                               torch.float32),
        # config 2 shape reduced in T (bf16), token-sparse causal; every 4th token stored
        "module_cfg2_T2048": lambda ref: module_case(ref, "module_cfg2_T2048", sparse_cfg(2048, 512, 8), 2, 2048, 512,
                                                     torch.bfloat16, token_stride=4),
        # config 2 at its BASELINE size (B=2, T=8192), every 16th token stored
        "module_cfg2_full": lambda ref: module_case(ref, "module_cfg2_full", sparse_cfg(8192, 512, 8), 2, 8192, 512,
                                                    torch.bfloat16, token_stride=16),
        # shortlist mode (config 3 recipe at T=4096, L=1024, window 256, stride 64), f32 and bf16
        "module_short_T4096_f32": lambda ref: module_case(ref, "module_short_T4096_f32",
                                                          shortlist_cfg(4096, 512, 8, 1024, 256, 64), 1, 4096, 512,
                                                          torch.float32, outlier=0.01, token_stride=4),
        "module_short_T4096_bf16": lambda ref: module_case(ref, "module_short_T4096_bf16",
                                                           shortlist_cfg(4096, 512, 8, 1024, 256, 64), 1, 4096, 512,
                                                           torch.bfloat16, outlier=0.01, token_stride=4),
        # per-head int8 mode (aspa.py:1258-1267, 1312-1363) in its three base
        # rules: absmax and percentile in bf16, EMA of the percentile in f32
        # over two forwards (the second reads the EMA the first left)
        "module_int8_max_bf16": lambda ref: module_case(ref, "module_int8_max_bf16",
                                                        dict(short, attn_quantize_int8=True), 1, 2048, 512,
                                                        torch.bfloat16, outlier=0.01, token_stride=8),
        "module_int8_pct_bf16": lambda ref: module_case(
            ref, "module_int8_pct_bf16", dict(short, attn_quantize_int8=True, attn_quantize_int8_mode="percentile",
                                              attn_quantize_int8_percentile=0.995), 1, 2048, 512, torch.bfloat16,
            outlier=0.01, token_stride=8),
        # the drop-in module with its defaults, and in linear (shortlist) mode
        "nucleus_head_count": nucleus_case,
        "rope_tables": rope_case,
        "dropin_mha_auto": lambda ref: dropin_case(ref, "dropin_mha_auto", 96, 70),
        "dropin_mha_linear": lambda ref: dropin_case(ref, "dropin_mha_linear", 300, 250, attn_mode="linear",
                                                     attn_linear_L=64, attn_linear_window=32),
        "module_int8_ema_f32": lambda ref: module_case(
            ref, "module_int8_ema_f32", dict(short, attn_quantize_int8=True, attn_quantize_int8_mode="ema_percentile",
                                             attn_quantize_int8_percentile=0.99, attn_quantize_int8_ema_decay=0.8),
            1, 2048, 512, torch.float32, outlier=0.01, token_stride=8, n_forward=2),
    }


if __name__ == "__main__":
    main()
