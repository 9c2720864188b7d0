"""pfa_pack_rows_static: the packing entry point that allocates nothing.

Its per-(head, block) counts live in a static device array instead of a
caller workspace.  The GPU test calls it through the C ABI and checks every
output against pfa_pack_rows on the same input, on calls in a row, each
smaller than the one before (stale scratch contents of an earlier call
would show), with sizes on both sides of the fused-scan limit (4,096
(head, block) counts), so that the totals and compact-id regions of the
static array are exercised as well as the block counts.  The CPU test
checks that sizes beyond the static maximum are rejected before any device
work.
"""
from __future__ import annotations

import ctypes

import pytest
import torch


def _routing(B, T, H, topk, masked, seed):
    g = torch.Generator().manual_seed(seed)
    scores = torch.rand(B * T, H, generator=g)
    scores[:, 1] -= 2.0  # a head nobody picks: compacted away
    hidx = torch.topk(scores, topk, dim=1).indices.to(torch.int32)
    tmask = (torch.rand(B, T, generator=g) < 0.6).to(torch.uint8) if masked else None
    return hidx, tmask


def _outputs(B, H, T, dev):
    BH = B * H
    # sentinel-filled, identically for both entry points
    return dict(mask8=torch.full((BH, T), 7, dtype=torch.uint8, device=dev),
                heads=torch.full((BH,), -5, dtype=torch.int32, device=dev),
                offs=torch.full((BH + 1,), -5, dtype=torch.int32, device=dev),
                tok=torch.full((BH * T,), -5, dtype=torch.int32, device=dev),
                rh=torch.full((BH * T,), -5, dtype=torch.int32, device=dev),
                row_of=torch.full((BH, T), -5, dtype=torch.int32, device=dev),
                summ=torch.full((4,), -5, dtype=torch.int32, device=dev))


def _call(lib, _hip, static, hidx, tmask, topk, B, H, T, dev):
    o = _outputs(B, H, T, dev)
    hd = hidx.to(dev)
    tm = tmask.to(dev) if tmask is not None else None
    args = (_hip.ptr(hd), topk, _hip.ptr(tm), B, H, T, _hip.ptr(o["mask8"]), _hip.ptr(o["heads"]),
            _hip.ptr(o["offs"]), _hip.ptr(o["tok"]), _hip.ptr(o["rh"]), _hip.ptr(o["row_of"]), _hip.ptr(o["summ"]))
    if static:
        rc = lib.pfa_pack_rows_static(*args, _hip.stream_ptr(dev))
        _hip.check(rc, "pfa_pack_rows_static")
    else:
        from proteus_attention.kernels import sparse_attn as sa

        ws = sa._workspace(sa._size_out(lib.pfa_pack_workspace_size, B, H, T), dev)
        rc = lib.pfa_pack_rows(*args, _hip.ptr(ws), ws.numel(), _hip.stream_ptr(dev))
        _hip.check(rc, "pfa_pack_rows")
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in o.items()}


@pytest.mark.gpu
def test_pack_rows_static_matches_workspace_entry_point(dev):
    from proteus_attention import _hip

    lib = _hip.lib()
    # each call smaller than the one before it (fewer heads, blocks or
    # rows); the first two take the separate scan kernel (more than 4,096
    # (head, block) counts: 4,688 and 4,416), the rest the fused scan
    for B, T, H, topk, masked, seed in ((1, 600_000, 8, 2, True, 4), (4, 70_000, 16, 3, False, 5),
                                        (2, 70_000, 8, 2, True, 1), (1, 3001, 6, 3, False, 2),
                                        (1, 65_536, 8, 2, False, 3)):
        print(f"[no_alloc] pack B={B} T={T} H={H} topk={topk} masked={masked}", flush=True)
        hidx, tmask = _routing(B, T, H, topk, masked, seed)
        ref = _call(lib, _hip, False, hidx, tmask, topk, B, H, T, dev)
        got = _call(lib, _hip, True, hidx, tmask, topk, B, H, T, dev)
        for k in ref:
            assert torch.equal(got[k], ref[k]), f"{k} differs at B={B} T={T} H={H}"
        P, N = int(ref["summ"][0]), int(ref["summ"][1])
        assert 0 < P <= B * H and N > 0


def test_pack_rows_static_rejects_sizes_beyond_its_scratch():
    from proteus_attention import _hip

    lib = _hip.lib()
    cap = 1 << 20
    dummy = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    # 512 heads x 1024 token blocks of counts = 2 MiB > the 1 MiB array
    rc = lib.pfa_pack_rows_static(dummy, 2, None, 64, 8, 1024 * 1024, dummy, dummy, dummy, dummy, dummy, dummy,
                                  dummy, None)
    assert rc == -1
    msg = lib.pfa_last_error_string().decode()
    assert "static maximum" in msg and str(cap) in msg
