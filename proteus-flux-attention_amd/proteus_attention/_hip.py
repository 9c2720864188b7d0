"""ctypes binding of libpfa_hip.so (declared in include/pfa_hip.h).

The library is the only compute backend of this package: there is no
PyTorch or CPU fallback.  Loading fails loudly when the library is missing
or when a call is made with tensors that are not on a ROCm device.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libpfa_hip.so"

PFA_F32, PFA_BF16, PFA_F16, PFA_I8 = 0, 1, 2, 3

_DTYPE_TAG = {
    torch.float32: PFA_F32,
    torch.bfloat16: PFA_BF16,
    torch.float16: PFA_F16,
    torch.int8: PFA_I8,
}

EXPORTED_SYMBOLS = (
    "pfa_version",
    "pfa_last_error_string",
    "pfa_router_gate_pad",
    "pfa_router_block_count",
    "pfa_router_prepare",
    "pfa_router_topk",
    "pfa_router_raw_supported",
    "pfa_router_topk_raw",
    "pfa_router_raw_workspace_size",
    "pfa_router_topk_raw_ws",
    "pfa_proto_ema_update",
    "pfa_proto_partial_count",
    "pfa_proto_accumulate",
    "pfa_proto_partial_reduce",
    "pfa_token_topk_workspace_size",
    "pfa_token_topk",
    "pfa_pack_workspace_size",
    "pfa_pack_rows",
    "pfa_pack_rows_static",
    "pfa_pack_mask",
    "pfa_proto_prefix_workspace_size",
    "pfa_proto_prefix_topk",
    "pfa_proto_prefix_blocks",
    "pfa_shortlist_build",
    "pfa_sparse_attn_fwd",
    "pfa_shortlist_attn_part_floats",
    "pfa_shortlist_attn_part_floats_for",
    "pfa_shortlist_attn_fwd",
    "pfa_shortlist_attn_fwd_fused",
    "pfa_head_max_token",
    "pfa_quantize_heads_workspace_size",
    "pfa_quantize_heads_int8",
    "pfa_rope_qk_inplace",
    "pfa_rope_k_inplace",
    "pfa_rope_k_zero_inplace",
    "pfa_router_stats_reduce",
    "pfa_zero_fill",
    "pfa_chunk_topk_workspace_size",
    "pfa_chunk_topk",
    "pfa_shortlist_finalise_workspace_size",
    "pfa_shortlist_finalise",
    "pfa_quantize_rows_int8",
    "pfa_rope_rows_inplace",
    "pfa_int8_kv_attn_workspace_size",
    "pfa_int8_kv_attn_fwd",
)


class Tensor4(ctypes.Structure):
    """pfa_tensor4: base pointer plus element strides for [b][h][t][d]."""

    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("s_b", ctypes.c_int64),
        ("s_h", ctypes.c_int64),
        ("s_t", ctypes.c_int64),
    ]


class HipLibraryError(RuntimeError):
    """Raised when libpfa_hip.so cannot be loaded or a call fails."""


_LIB: Optional[ctypes.CDLL] = None

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

_SIGNATURES = {
    "pfa_version": ([], _i32),
    "pfa_last_error_string": ([], ctypes.c_char_p),
    "pfa_router_gate_pad": ([_i32], _i32),
    "pfa_router_block_count": ([_i64, ctypes.POINTER(_i32)], _i32),
    "pfa_router_prepare": ([_vp, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "pfa_router_topk": ([_vp, _i32, _i64, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _i32, _i32,
                         _f32, _f32, _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "pfa_router_raw_supported": ([_i32, _i32, _i32, _i32, _i32, _i32], _i32),
    "pfa_router_topk_raw": ([_vp, _i32, _i64, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _i32, _i32,
                             _f32, _f32, _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "pfa_router_raw_workspace_size": ([_i64, _i32, ctypes.POINTER(_sz)], _i32),
    "pfa_router_topk_raw_ws": ([_vp, _i32, _i64, _i32, _i32, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _i32, _i32,
                                _f32, _f32, _f32, _f32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
                               _i32),
    "pfa_proto_ema_update": ([_vp, _i32, _i32, _f32, _vp, _vp, _vp, _i32, _vp], _i32),
    "pfa_proto_partial_count": ([_i64, ctypes.POINTER(_i32)], _i32),
    "pfa_proto_accumulate": ([_vp, _i32, _i64, _i32, _i32, _vp, _vp, _i32, _vp], _i32),
    "pfa_proto_partial_reduce": ([_vp, _i32, _i32, _i32, _vp, _vp], _i32),
    "pfa_token_topk_workspace_size": ([_i32, _i64, ctypes.POINTER(_sz)], _i32),
    "pfa_token_topk": ([_vp, _i32, _i64, _i64, _i32, _f32, _vp, _vp, _sz, _vp], _i32),
    "pfa_pack_workspace_size": ([_i32, _i32, _i64, ctypes.POINTER(_sz)], _i32),
    "pfa_pack_rows": ([_vp, _i32, _vp, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp], _i32),
    "pfa_pack_rows_static": ([_vp, _i32, _vp, _i32, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp], _i32),
    "pfa_pack_mask": ([_vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _sz, _vp], _i32),
    "pfa_proto_prefix_workspace_size": ([_i32, _i64, _i32, ctypes.POINTER(_sz)], _i32),
    "pfa_proto_prefix_topk": ([_vp, _i32, _i64, _i64, _i32, _vp, _vp, _vp, _sz, _vp], _i32),
    "pfa_proto_prefix_blocks": ([_vp, _i32, _i64, _i64, _i32, _vp, _vp, _vp, _sz, _vp], _i32),
    "pfa_shortlist_build": ([_vp, _vp, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _vp, _i32, _i64, _vp, _vp, _i32,
                             _vp, _i32, _vp, _i32, _vp], _i32),
    "pfa_sparse_attn_fwd": ([Tensor4, Tensor4, Tensor4, _i32, Tensor4, _i32, _i32, _i64, _i32, _vp, _vp, _vp,
                             _i64, _vp, _vp, _i64, _vp, _vp, _i32, _vp, _f32, _vp, _vp, _vp, _vp], _i32),
    "pfa_shortlist_attn_part_floats": ([], _i32),
    "pfa_shortlist_attn_part_floats_for": ([_i32], _i32),
    "pfa_shortlist_attn_fwd": ([Tensor4, Tensor4, Tensor4, Tensor4, _i32, _i32, _i64, _i32, _vp, _vp, _vp, _i64,
                                _i32, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _vp, _f32, _vp, _vp, _vp, _vp, _vp,
                                _vp, _vp, _i32, _vp], _i32),
    "pfa_shortlist_attn_fwd_fused": ([Tensor4, Tensor4, Tensor4, Tensor4, _i32, _i32, _i64, _i32, _vp, _vp, _vp,
                                      _i64, _i32, _vp, _vp, _i32, _i32, _i32, _vp, _i32, _vp, _f32, _vp, _vp, _vp,
                                      _vp, _i32, _i32, _vp], _i32),
    "pfa_head_max_token": ([_vp, _vp, _i32, _vp, _vp], _i32),
    "pfa_quantize_heads_workspace_size": ([_i32, _i64, _i32, _i32, ctypes.POINTER(_sz)], _i32),
    "pfa_quantize_heads_int8": ([Tensor4, _i32, _i32, _i64, _i32, _vp, _i32, _vp, _i32, _f32, ctypes.c_double, _vp,
                                 _i32, Tensor4, _i32, _vp, _vp, _sz, _vp], _i32),
    "pfa_rope_qk_inplace": ([_vp, _i32, _i32, _i64, _i32, _i32, _vp, _vp, _vp], _i32),
    "pfa_rope_k_inplace": ([_vp, _i32, _i32, _i64, _i32, _i32, _vp, _vp, _vp], _i32),
    "pfa_rope_k_zero_inplace": ([_vp, _i32, _i32, _i64, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "pfa_router_stats_reduce": ([_vp, _i32, _vp, _vp], _i32),
    "pfa_zero_fill": ([_vp, _sz, _vp], _i32),
    "pfa_chunk_topk_workspace_size": ([_i64, _i32, ctypes.POINTER(_sz)], _i32),
    "pfa_chunk_topk": ([_vp, _vp, _i64, _i32, _f32, _i64, _i32, _vp, _vp, _vp, _vp, _sz, _vp], _i32),
    "pfa_shortlist_finalise_workspace_size": ([_i64, ctypes.POINTER(_sz)], _i32),
    "pfa_shortlist_finalise": ([_vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp], _i32),
    "pfa_quantize_rows_int8": ([_vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _vp], _i32),
    "pfa_rope_rows_inplace": ([_vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _i64, _vp], _i32),
    "pfa_int8_kv_attn_workspace_size": ([_i64, _i32, _i32, ctypes.POINTER(_sz)], _i32),
    "pfa_int8_kv_attn_fwd": ([Tensor4, Tensor4, _i64, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp,
                              _sz, _vp], _i32),
}


def library_path() -> Path:
    return LIB_PATH


def load_library() -> ctypes.CDLL:
    """Load libpfa_hip.so (once).  Raises HipLibraryError when it is absent."""

    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise HipLibraryError(
            f"{LIB_PATH} is missing: build it with `python proteus-flux-attention_amd/build_hip.py` "
            "(or __graft_entry__.build()); this package has no CPU fallback."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (args, res) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _LIB = lib
    return lib


def lib() -> ctypes.CDLL:
    return load_library()


def check(rc: int, name: str) -> None:
    if rc != 0:
        msg = load_library().pfa_last_error_string()
        text = msg.decode("utf-8", "replace") if msg else ""
        if rc == -1:
            raise ValueError(f"{name}: {text}")
        raise HipLibraryError(f"{name} failed (status {rc}): {text}")


def dtype_tag(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_TAG[dtype]
    except KeyError as exc:
        raise ValueError(f"unsupported dtype {dtype} for the HIP kernels") from exc


def stream_ptr(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None:
        return None
    return int(t.data_ptr())


def require_device(*tensors: Optional[torch.Tensor], what: str) -> torch.device:
    """All tensors must live on one ROCm device; CPU tensors are rejected."""

    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise HipLibraryError(
                f"{what}: tensors must be on a ROCm device (got {t.device}); "
                "the MI355X build has no CPU execution path"
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"{what}: tensors on different devices ({device} vs {t.device})")
    if device is None:
        raise ValueError(f"{what}: no tensor given")
    load_library()
    return device


def tensor4(t: torch.Tensor, H: int, layout: str = "bhtd") -> Tensor4:
    """Describe a tensor for pfa_sparse_attn_fwd.

    layout "bhtd": t is (B*H, T, D) (or (P, T, D) with H == P).
    layout "bthd": t is a (B, T, H, D)-shaped strided view (for example a
    slice of the (B, T, 3, H, D) QKV projection).
    """

    if layout == "bhtd":
        if t.stride(-1) != 1:
            raise ValueError("last dimension must be contiguous")
        s_bh, s_t = t.stride(0), t.stride(1)
        return Tensor4(ptr(t), s_bh * H, s_bh, s_t)
    if layout == "bthd":
        if t.stride(-1) != 1:
            raise ValueError("last dimension must be contiguous")
        return Tensor4(ptr(t), t.stride(0), t.stride(2), t.stride(1))
    raise ValueError(layout)


def is_available() -> bool:
    try:
        load_library()
    except HipLibraryError:
        return False
    return bool(torch.cuda.is_available())


class _TimedBlock:
    """One ``_KernelTimer.timed`` block: an event pair on the current stream
    when the timer is enabled, nothing otherwise."""

    __slots__ = ("timer", "name", "e0")

    def __init__(self, timer: "_KernelTimer", name: str) -> None:
        self.timer, self.name, self.e0 = timer, name, None

    def __enter__(self):
        if self.timer.enabled:
            self.e0 = torch.cuda.Event(enable_timing=True)
            self.e0.record()
        return self

    def __exit__(self, *exc):
        if self.e0 is not None:
            e1 = torch.cuda.Event(enable_timing=True)
            e1.record()
            self.timer.events.setdefault(self.name, []).append((self.e0, e1))
        return False


class _KernelTimer:
    """Optional per-stage HIP event timing on torch's current stream (the
    stream every launch of this package uses).  Disabled by default; when
    enabled each ``timed(name)`` block records a start/end event pair."""

    def __init__(self) -> None:
        self.enabled = False
        self.events: dict = {}

    def reset(self) -> None:
        self.events = {}

    def timed(self, name: str) -> _TimedBlock:
        return _TimedBlock(self, name)

    def summary_ms(self) -> dict:
        torch.cuda.synchronize()
        return {k: [a.elapsed_time(b) for a, b in v] for k, v in self.events.items()}


TIMER = _KernelTimer()


def env_flag(name: str) -> bool:
    return os.getenv(name, "").strip().lower() in {"1", "true", "yes", "on"}
