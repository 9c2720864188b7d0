"""CPU: host logic of the product package and the C ABI surface (no kernel
launches -- there is no GPU here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from proteus_attention import _hip
from proteus_attention.models.aspa import AdaptiveSparseAttention, ModelConfig

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "pfa_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pfa_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_hip.library_path()))
    declared = _declared_symbols()
    assert len(declared) >= 15
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_hip.EXPORTED_SYMBOLS)
    assert _hip.load_library().pfa_version() >= 100


def test_library_reports_argument_errors_without_gpu():
    lib = _hip.load_library()
    rc = lib.pfa_shortlist_build(None, None, 4, None, 0, 0, 0, 0, 0, None, 0, 0, None, None, 0, None, 0, None, 0, None)
    assert rc == -1
    assert b"bad sizes" in lib.pfa_last_error_string()
    size = ctypes.c_size_t(0)
    assert lib.pfa_pack_workspace_size(2, 8, 8192, ctypes.byref(size)) == 0 and size.value > 0


def test_cpu_tensors_fail_loudly():
    from proteus_attention.kernels.sparse_attn import aspa_sparse_attention, build_shortlist_candidates

    q = torch.randn(2, 5, 8)
    with pytest.raises(_hip.HipLibraryError):
        aspa_sparse_attention(q, q, q)
    with pytest.raises(_hip.HipLibraryError):
        build_shortlist_candidates(torch.arange(5), 5, max_candidates=4, linear_window=2, anchor_stride=0,
                                   use_local=True, use_anchors=False)


def test_operator_validation_messages():
    from proteus_attention.kernels.sparse_attn import aspa_sparse_attention

    q = torch.randn(2, 5, 8)
    with pytest.raises(ValueError, match="rank-3"):
        aspa_sparse_attention(q[0], q[0], q[0])
    with pytest.raises(ValueError, match="matching shapes"):
        aspa_sparse_attention(q, q[:, :4], q)
    with pytest.raises(ValueError, match="dropout_p"):
        aspa_sparse_attention(q, q, q, dropout_p=1.0)
    with pytest.raises(ValueError, match="causal_mask must have shape"):
        aspa_sparse_attention(q, q, q, causal_mask=torch.zeros(4, 4))
    with pytest.raises(ValueError, match="int8"):
        aspa_sparse_attention(q.to(torch.int8), q, q)


def test_active_head_schedule_known_answers():
    """Reference tests/test_aspa.py:718-747."""
    cfg = ModelConfig(vocab_size=32, n_ctx=4096, n_layer=1, n_head=8, d_model=64, attn_variant="aspa",
                      attn_h_total=32, attn_h_active=8, attn_h_active_min=2, attn_h_active_max=16,
                      attn_active_seq_low=512, attn_active_seq_high=4096)
    m = AdaptiveSparseAttention(cfg)
    assert m.h_active_curve == pytest.approx(0.25)
    got = [m._choose_active_k(s) for s in (64, 512, 1024, 2048, 4096, 8192)]
    assert got == [16, 16, 7, 4, 2, 2]


def test_latency_budget_alpha_switch():
    """Reference tests/test_aspa.py:579-606."""
    cfg = ModelConfig(vocab_size=16, n_ctx=128, n_layer=1, n_head=4, d_model=32, attn_variant="aspa",
                      attn_h_total=4, attn_h_active=4, attn_h_active_min=2, attn_h_active_max=4, attn_mode="auto",
                      attn_linear_switch_ctx=1024, attn_linear_latency_budget_ms=0.0, attn_token_sparse=False)
    m = AdaptiveSparseAttention(cfg)
    m._latency_ema = 5.0
    assert m._compute_cvt_alpha(128) == pytest.approx(1.0)
    m._latency_ema = 0.0
    m._current_alpha = 1.0
    assert m._compute_cvt_alpha(64) == pytest.approx(0.0)


def test_shortlist_caps_at_config3():
    from configs import shortlist_cfg

    m = AdaptiveSparseAttention(ModelConfig(**shortlist_cfg(65536, 512, 8, 2048)))
    rt = m._prepare_linear_runtime(65536, 1, m._compute_cvt_alpha(65536))
    assert rt["effective_L"] == 2048 and rt["window"] == 512
    assert (rt["local_cap"], rt["anchor_cap"], rt["proto_cap"]) == (512, 614, 205)
    m4 = AdaptiveSparseAttention(ModelConfig(**shortlist_cfg(524288, 512, 8, 4096)))
    rt4 = m4._prepare_linear_runtime(524288, 1, 1.0)
    # 2458+1229+410 > 4096 is scaled down and re-distributed: proto gets 409
    assert (rt4["local_cap"], rt4["anchor_cap"], rt4["proto_cap"]) == (512, 1229, 409)


def test_linear_params_match_reference_formulas_across_alpha():
    """Spot values of _compute_effective_linear_params for partial alpha
    (hand-evaluated from aspa.py:1037-1145)."""
    m = AdaptiveSparseAttention(ModelConfig(d_model=64, n_head=4, attn_h_total=4, attn_linear_L=256,
                                            attn_linear_window=64, attn_linear_policy="local+anchors+proto"))
    p = m._compute_effective_linear_params(4096, 1, 0.5)
    # eff = int(.5*256 + .5*min(256, max(64, 64+128))) = int(128 + 96) = 224
    assert p["effective_L"] == 224
    # window = int(.5*64 + .5*max(1,min(4096,max(64,512)))) = int(32+256) = 288 -> min(eff) = 224
    assert p["window"] == 224
    assert (p["local_cap"], p["anchor_cap"], p["proto_cap"]) == (162, 45, 17)


def test_module_state_dict_keys_match_reference_layout():
    m = AdaptiveSparseAttention(ModelConfig(d_model=64, n_head=4, attn_h_total=4, attn_gates=8,
                                            attn_proto_enable=True))
    keys = set(m.state_dict().keys())
    assert keys == {"head_router.linear.weight", "qkv.weight", "proj.weight", "routing_prototypes",
                    "routing_usage_ema", "routing_confidence"}


def test_dropin_constructs_and_masks_are_classified():
    from proteus_attention import CausalASPAMultiheadAttention

    mha = CausalASPAMultiheadAttention(32, 4)
    T = 6
    causal = torch.triu(torch.full((T, T), float("-inf")), diagonal=1)
    assert mha._is_supported_attn_mask(None, T, torch.device("cpu"))
    assert mha._is_supported_attn_mask(causal, T, torch.device("cpu"))
    assert not mha._is_supported_attn_mask(torch.zeros(T, T), T, torch.device("cpu"))
    # cross-attention goes to nn.MultiheadAttention exactly as the reference
    x = torch.randn(2, T, 32)
    out, w = mha(x, torch.randn(2, T, 32), torch.randn(2, T, 32))
    assert out.shape == x.shape


def test_chunked_config_validation():
    from proteus_attention.tools.chunked_shortlist import ChunkedShortlistConfig

    with pytest.raises(ValueError):
        ChunkedShortlistConfig(seq_len=0, d_model=8, chunk_len=4, buffer_tokens=2, per_chunk_budget=1,
                               device=torch.device("cpu")).validate()
    with pytest.raises(ValueError):
        ChunkedShortlistConfig(seq_len=8, d_model=8, chunk_len=70000, buffer_tokens=2, per_chunk_budget=1,
                               device=torch.device("cpu")).validate()


def test_nucleus_head_count_matches_reference(golden):
    """_nucleus_head_count (reference aspa.py:749-780) against the
    reference's own answers on seeded head probabilities, over target_p in
    {0, .5, .9, .99, 1} and caps {1, 3, 8}."""
    z = golden("nucleus_head_count")
    m = AdaptiveSparseAttention(ModelConfig(d_model=64, n_head=8, attn_h_total=8, attn_gates=8))
    probs = torch.from_numpy(z["probs"])
    got = [[m._nucleus_head_count(p, float(tp), int(cap)) for tp in z["target_p"] for cap in z["caps"]]
           for p in probs]
    assert got == z["k"].tolist()


def test_graph_eligibility_follows_host_decisions():
    """A forward is captured in a HIP graph only when no host decision reads
    a device result: the chunked pipeline's chunk model at 65,536 tokens
    (token mask without a keep threshold, materialised candidates, top-p
    routing with the head count at its floor) is eligible; a keep
    threshold, a head count above its floor with top-p routing, a length
    served by the structured kernel (which reads the exact row count), a
    density threshold or grad mode are not."""
    from proteus_attention.tools.chunked_shortlist import _build_model_config

    def model(T, **over):
        cfg = _build_model_config(T, 512, heads=8, sparse_ratio=0.05, shortlist_alpha=0.0, router_top_p=1.0)
        for k, v in over.items():
            setattr(cfg, k, v)
        return AdaptiveSparseAttention(cfg).to(torch.bfloat16).eval()

    x = torch.zeros(1, 65536, 512, dtype=torch.bfloat16)
    with torch.no_grad():
        assert model(65536)._graph_eligible(x)
        assert not model(65536, attn_token_keep_threshold=0.5)._graph_eligible(x)
        # a floor of 2 heads: at 65,536 tokens (>= seq_high) k is the floor and
        # the nucleus count is skipped; with seq_high beyond T, k stays above it
        assert model(65536, attn_h_active_min=2)._graph_eligible(x)
        assert not model(65536, attn_h_active_min=2, attn_active_seq_high=1 << 20)._graph_eligible(x)
        assert not model(65536, attn_force_dense_threshold=0.9)._graph_eligible(x)
        # 4,096 tokens: window + anchors fit in L, the structured kernel serves it
        assert not model(4096)._graph_eligible(torch.zeros(1, 4096, 512, dtype=torch.bfloat16))
        m = model(65536)
        m.token_sparse = False
        m.router_top_p = 0.0
        assert m._graph_eligible(x)
    assert not model(65536)._graph_eligible(x)  # grad mode on


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32, torch.float64])
def test_disk_staging_rows_equal_float32_round_trip(tmp_path, dt):
    """The disk memmap keeps bf16/fp16/fp32 rows in their own dtype and
    other dtypes in float32: every fetched row (a slice or a gather) equals
    the reference's float32 memmap round trip (chunked_shortlist.py:506-553)
    bit for bit."""
    import numpy as np

    from proteus_attention.tools import chunked_shortlist as CS

    x = (torch.randn(1, 1000, 48, dtype=torch.float64, generator=torch.Generator().manual_seed(3)) * 300).to(dt)
    x[0, 3, :4] = torch.tensor([float("inf"), float("-inf"), -0.0, 1e-30], dtype=torch.float64).to(dt)
    store = dt if dt in CS._MEMMAP_NP else torch.float32
    mm = np.memmap(tmp_path / "rows.mmap", dtype=CS._MEMMAP_NP[store], mode="w+", shape=(1000, 48))
    mm[:] = CS._memmap_view(x.squeeze(0).to(store))
    assert mm.dtype.itemsize == (4 if store == torch.float32 else 2)
    ref = x[0].to(torch.float32).to(dt)
    got = CS._memmap_rows(mm[10:500], store).to(dt)
    assert torch.equal(got.view(torch.uint8), ref[10:500].contiguous().view(torch.uint8))
    idx = torch.tensor([5, 999, 0, 3, 7])
    got = CS._memmap_rows(mm[idx.numpy()], store).to(dt)
    assert torch.equal(got.view(torch.uint8), ref[idx].contiguous().view(torch.uint8))


def test_graph_key_follows_token_keep_schedule_knobs():
    """A captured graph fixes the token keep count of a token-masked
    forward; the key it is stored under changes with every knob the keep
    ratio reads (linear_token_keep_ratio_ref and _min included), so a
    changed knob captures a new graph instead of replaying the old count."""
    from proteus_attention.tools.chunked_shortlist import _build_model_config

    T = 24576
    m = AdaptiveSparseAttention(_build_model_config(T, 512, heads=8, sparse_ratio=0.05, shortlist_alpha=0.0,
                                                    router_top_p=1.0))
    m.linear_token_keep_schedule = "sqrt"
    m.linear_token_keep_ratio_min = 0.001
    m.linear_token_keep_ratio_ref = 2048
    x = torch.zeros(1, T, 512)
    k0 = m._graph_key(x)
    r0 = m._linear_token_keep_ratio(T)
    m.linear_token_keep_ratio_ref = 4 * 2048
    r1 = m._linear_token_keep_ratio(T)
    assert r1 != r0 and m._graph_key(x) != k0
    k1 = m._graph_key(x)
    m.linear_token_keep_ratio_min = 0.04
    assert m._linear_token_keep_ratio(T) != r1 and m._graph_key(x) != k1
