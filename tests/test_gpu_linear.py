"""The projection GEMM entry point (pfa_linear, hipBLASLt with the kernel
chosen by timing per shape) against an f32 product of the same bf16
operands, bit-for-bit repeatability, graph replays against the eager call,
and the error paths.  The reference computes these projections with
nn.Linear (aspa.py:1641, 1853)."""
import ctypes

import pytest
import torch

from proteus_attention import _hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _call(x, w, b, y, stream=None):
    K, N = x.shape[-1], w.shape[0]
    return _hip.lib().pfa_linear(_hip.ptr(x), _hip.PFA_BF16, x.numel() // K, K, _hip.ptr(w), N,
                                 None if b is None else _hip.ptr(b), _hip.ptr(y),
                                 stream if stream is not None else _hip.stream_ptr(x.device))


@pytest.mark.parametrize("M,K,N,bias", [(65536, 512, 1536, False), (65536, 512, 512, True), (1000, 256, 768, True),
                                        (3, 64, 64, False), (4097, 96, 40, True)])
def test_linear_vs_f32_product(dev, M, K, N, bias):
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16)
    b = torch.randn(N, generator=g).to(torch.bfloat16) if bias else None
    print(f"pfa_linear M={M} K={K} N={N} bias={bias}", flush=True)
    xd, wd = x.to(dev), w.to(dev)
    bd = None if b is None else b.to(dev)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    assert _call(xd, wd, bd, y) == 0, _hip.lib().pfa_last_error_string()
    assert _hip.lib().pfa_linear_tuned(M, N, K, int(bias)) == 1
    ref = x.float() @ w.float().t()
    if b is not None:
        ref += b.float()
    got = y.float().cpu()
    # f32 accumulation in any order, one bf16 rounding of the output
    bound = ref.abs() * 2.0 ** -8 + 1e-3 * K ** 0.5
    assert bool(((got - ref).abs() <= bound).all()), float((got - ref).abs().max())
    y2 = torch.empty_like(y)
    assert _call(xd, wd, bd, y2) == 0
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_linear_graph_replays_match_eager(dev):
    g = torch.Generator().manual_seed(5)
    M, K, N = 8192, 512, 1536
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
    y_eager = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    assert _call(x, w, None, y_eager) == 0
    y = torch.empty_like(y_eager)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            rc = _call(x, w, None, y, stream=ctypes.c_void_p(s.cuda_stream).value)
    torch.cuda.current_stream(dev).wait_stream(s)
    assert rc == 0
    for _ in range(3):
        y.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), y_eager.view(torch.int16))


def test_linear_errors(dev):
    lib = _hip.lib()
    x = torch.zeros(4, 8, dtype=torch.float32, device=dev)
    w = torch.zeros(8, 8, dtype=torch.float32, device=dev)
    y = torch.zeros(4, 8, dtype=torch.float32, device=dev)
    assert lib.pfa_linear(_hip.ptr(x), _hip.PFA_F32, 4, 8, _hip.ptr(w), 8, None, _hip.ptr(y),
                          _hip.stream_ptr(dev)) == -2
    assert b"bf16" in lib.pfa_last_error_string()
    assert lib.pfa_linear(None, _hip.PFA_BF16, 4, 8, None, 8, None, None, _hip.stream_ptr(dev)) == -1
    assert lib.pfa_linear(None, _hip.PFA_BF16, 0, 8, None, 8, None, None, _hip.stream_ptr(dev)) == 0  # empty
