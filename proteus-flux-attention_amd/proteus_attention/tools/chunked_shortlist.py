"""Chunked Shortlist pipeline (reference tools/chunked_shortlist.py:88-827).

Two passes over a long sequence: every chunk runs an ASPA forward on the
device, promotes its most salient tokens, the promoted tokens of all chunks
are merged into a global shortlist (sorted by position), and a final ASPA
pass runs over the reduced sequence.

Same configuration, result and metric types as the reference.  Host staging
(pinned RAM or a disk memmap) follows the reference.  Chunks reach the device
through two device buffers filled on a copy stream (_ChunkStager): the copy
of chunk i+1 runs while chunk i is computed, and with disk staging a worker
thread reads chunk i+2 from the memmap into one of two pinned buffers
meanwhile.  Chunk salience is the router importance of the chunk model
(device tensors); the reference's norm-score fallback only applies when no
importance is available.
"""
from __future__ import annotations

import concurrent.futures as cf
import contextlib
import logging
import math
import os
import tempfile
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Dict, Iterable, List, Literal, Optional, Sequence, Tuple

import numpy as np
import torch

from ..kernels.sparse_attn import _record_backend, get_last_backend_info
from ..models.aspa import AdaptiveSparseAttention, ModelConfig, _side_stream
from . import chunk_select
from .final_pass import AllQueryFinalPass

LOGGER = logging.getLogger(__name__)

# The reference caps chunks at 65,536 tokens because of a Triton/ROCm compiler
# limit (reference chunked_shortlist.py:51-53).  The HIP kernels have no such
# limit; the constant and its validation are kept for configuration parity.
MAX_SHORTLIST_CHUNK_TOKENS = 65_536
BYTES_PER_MB = 1024.0 * 1024.0


def _system_available_ram() -> Optional[int]:
    try:
        import psutil  # type: ignore

        return int(psutil.virtual_memory().available)
    except Exception:  # noqa: BLE001
        pass
    try:
        return int(os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_AVPHYS_PAGES"))
    except (AttributeError, ValueError, TypeError, OSError):
        return None


def _sanitize_mapping(mapping: Dict[str, Any]) -> Dict[str, Any]:
    out: Dict[str, Any] = {}
    for key, value in mapping.items():
        if isinstance(value, torch.Tensor):
            out[key] = value.detach().cpu().item() if value.numel() == 1 else value.detach().cpu().tolist()
        elif isinstance(value, dict):
            out[key] = _sanitize_mapping(value)
        else:
            out[key] = value
    return out


def _build_model_config(seq_len: int, d_model: int, *, heads: int, sparse_ratio: float, shortlist_alpha: float,
                        router_top_p: float) -> ModelConfig:
    """Chunk / final model recipe (reference chunked_shortlist.py:88-137)."""

    return ModelConfig(
        vocab_size=0, n_ctx=seq_len, n_layer=1, n_head=heads, d_model=d_model, p_dropout=0.0, bias=False,
        attn_variant="aspa", attn_h_total=heads, attn_h_active=heads, attn_h_active_min=heads,
        attn_h_active_max=heads, attn_active_seq_low=max(128, seq_len // 4), attn_active_seq_high=seq_len,
        attn_mode="linear", attn_token_sparse=True, attn_token_keep_ratio=max(0.0, min(1.0, sparse_ratio)),
        attn_token_keep_min=max(4, int(seq_len * sparse_ratio * 0.5)), attn_token_keep_guard=4,
        attn_token_keep_threshold=0.0, attn_linear_L=256, attn_linear_L_base=256, attn_linear_L_min=64,
        attn_linear_L_max=256, attn_linear_switch_ctx=max(512, min(seq_len, 4096)),
        attn_linear_policy="local+anchors", attn_proto_enable=True, attn_proto_threshold=0.2, attn_proto_blend=0.5,
        attn_proto_temp=0.3, attn_linear_token_keep_schedule="sqrt", attn_linear_token_keep_min_ratio=0.05,
        attn_track_latency=False, attn_small_seq_dense=0, use_sdpa=False, attn_shortlist_alpha=shortlist_alpha,
        attn_router_top_p=router_top_p,
    )


def _select_top_tokens(model: AdaptiveSparseAttention, global_offset: int, *, per_chunk_budget: int,
                       nucleus_top_p: float) -> Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
    """Chunk salience (reference chunked_shortlist.py:140-172): the chunk
    model's importance, non-kept tokens at -inf, nucleus-selected.  Returns
    (values, positions, count) with the count left on the device (the first
    ``count`` entries are the selection; a count of 0 is the reference's
    "nothing finite selected" case), or None without importance or budget."""

    importance = getattr(model, "_last_token_importance", None)
    if importance is None or importance.device.type != "cuda":
        return None
    scores = importance.squeeze(0).to(torch.float32)
    mask = getattr(model, "_last_token_mask", None)
    # masking, nucleus selection and the finite filter run in one kernel
    # (pfa_chunk_topk)
    return chunk_select.nucleus_select_device(scores, per_chunk_budget, nucleus_top_p,
                                              keep_mask=mask.squeeze(0) if mask is not None else None,
                                              index_offset=int(global_offset), drop_nonfinite=True)


def _nucleus_select(scores: torch.Tensor, max_tokens: int, top_p: float):
    """Reference chunked_shortlist.py:175-208 (device kernel)."""

    if scores.ndim != 1:
        raise ValueError("scores tensor must be 1-D for nucleus selection.")
    return chunk_select.nucleus_select(scores, max_tokens, top_p)


def _finalise_indices(scores: torch.Tensor, indices: torch.Tensor, *, max_tokens: int):
    """Reference chunked_shortlist.py:211-254 (device kernel)."""

    if scores.numel() == 0 or indices.numel() == 0:
        raise RuntimeError("No candidate tokens captured during chunking.")
    keep_idx, keep_scores = chunk_select.finalise(scores, indices, max_tokens)
    return keep_idx.to("cpu"), keep_scores.to("cpu")


def _chunk_iter(total_len: int, chunk_len: int) -> Iterable[Tuple[int, int]]:
    for start in range(0, total_len, chunk_len):
        yield start, min(total_len, start + chunk_len)


@dataclass
class ChunkSummary:
    index: int
    start: int
    end: int
    promoted: Sequence[int] = field(default_factory=list)
    scores: Sequence[float] = field(default_factory=list)


@dataclass
class ChunkedShortlistMetrics:
    original_tokens: int
    retained_tokens: int
    retention_ratio: float
    chunk_count: int
    device: str
    chunk_time_ms: Optional[float] = None
    final_time_ms: Optional[float] = None
    total_time_ms: Optional[float] = None
    peak_memory_mb: Optional[float] = None
    used_fallback: bool = False
    chunk_tokens_per_s: Optional[float] = None
    final_tokens_per_s: Optional[float] = None
    total_tokens_per_s: Optional[float] = None
    storage_mode: str = "cpu"
    host_required_mb: Optional[float] = None
    host_allocated_mb: Optional[float] = None
    host_limit_mb: Optional[float] = None
    storage_reason: Optional[str] = None
    # host-staged runs: total host-to-device copy time (on the copy stream)
    # and the part of it the compute stream waited for (not hidden behind
    # the previous chunk's compute)
    h2d_time_ms: Optional[float] = None
    h2d_stall_ms: Optional[float] = None


@dataclass
class ChunkedShortlistResult:
    keep_indices: torch.Tensor
    keep_scores: torch.Tensor
    reduced_sequence: torch.Tensor
    metrics: ChunkedShortlistMetrics
    chunks: Sequence[ChunkSummary]
    final_output: Optional[torch.Tensor] = None
    final_stats: Optional[Dict[str, Any]] = None
    backend_info: Optional[Dict[str, Any]] = None


@dataclass
class ChunkedShortlistConfig:
    seq_len: int
    d_model: int
    chunk_len: int
    buffer_tokens: int
    per_chunk_budget: int
    device: torch.device
    heads: int = 8
    nucleus_top_p: float = 0.9
    chunk_sparse_ratio: float = 0.05
    final_sparse_ratio: float = 0.5
    seed: Optional[int] = 7
    report_latency: bool = False
    progress: bool = False
    run_final_pass: bool = True
    shortlist_alpha: float = 1.0
    storage: Literal["cpu", "disk", "auto"] = "auto"
    temp_dir: Optional[Path] = None
    ram_limit_bytes: Optional[int] = None
    # "reduced": the reference's final pass (final model over the reduced
    # sequence).  "all_queries": every token of the sequence attends to the
    # int8 (per head and row) shortlist, causal by original position when
    # final_causal (tools/final_pass.py).
    final_mode: Literal["reduced", "all_queries"] = "reduced"
    final_causal: bool = True
    # replay the chunk model's forward from a captured HIP graph (one
    # capture per chunk length, during the warm-up forward) where the
    # forward has no host decision on device results and the sequence is
    # resident on the device; otherwise it runs eagerly (with host staging
    # the stage is bound by the chunk copies, and graph replays beside them
    # slowed the copies from pinned memory, measured 19.2 -> 23.4 ms for
    # 1 GiB, the chunk stage 20.0 -> 24.4 ms)
    chunk_graph: bool = True

    def validate(self) -> None:
        """Reference chunked_shortlist.py:337-366."""
        if self.seq_len <= 0:
            raise ValueError("seq_len must be positive.")
        if self.d_model <= 0:
            raise ValueError("d_model must be positive.")
        if self.chunk_len <= 0:
            raise ValueError("chunk_len must be positive.")
        if self.chunk_len > MAX_SHORTLIST_CHUNK_TOKENS:
            raise ValueError(f"chunk_len={self.chunk_len} exceeds MAX_SHORTLIST_CHUNK_TOKENS="
                             f"{MAX_SHORTLIST_CHUNK_TOKENS}.")
        if self.buffer_tokens <= 0:
            raise ValueError("buffer_tokens must be positive.")
        if self.per_chunk_budget <= 0:
            raise ValueError("per_chunk_budget must be positive.")
        if not (0.0 < float(self.nucleus_top_p) <= 1.0):
            raise ValueError("nucleus_top_p must be within (0, 1].")
        if self.chunk_sparse_ratio <= 0.0:
            raise ValueError("chunk_sparse_ratio must be positive.")
        if self.final_sparse_ratio <= 0.0:
            raise ValueError("final_sparse_ratio must be positive.")
        if not (0.0 <= self.shortlist_alpha <= 1.0):
            raise ValueError("shortlist_alpha must be within [0, 1].")
        if self.storage not in {"cpu", "disk", "auto"}:
            raise ValueError("storage must be 'cpu', 'disk', or 'auto'.")
        if self.ram_limit_bytes is not None and self.ram_limit_bytes <= 0:
            raise ValueError("ram_limit_bytes must be positive when provided.")
        if self.final_mode not in {"reduced", "all_queries"}:
            raise ValueError("final_mode must be 'reduced' or 'all_queries'.")


# memmap element types for rows stored in their own dtype (bf16 as its raw
# 16-bit pattern)
_MEMMAP_NP = {torch.float32: np.float32, torch.float16: np.float16, torch.bfloat16: np.int16}


def _memmap_view(t: torch.Tensor) -> np.ndarray:
    """A (rows, d_model) CPU tensor as the memmap's element type."""
    return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


def _memmap_rows(a: np.ndarray, store: torch.dtype) -> torch.Tensor:
    """Memmap rows as a CPU tensor of the stored dtype."""
    t = torch.from_numpy(np.asarray(a))
    return t.view(torch.bfloat16) if store == torch.bfloat16 else t

class _ChunkStager:
    """Double-buffered host-to-device chunk streaming (reference
    chunked_shortlist.py:617-625, 688-689 copy each chunk with a blocking
    .to(device)).

    Two device buffers take alternate chunks.  start(i) queues chunk i's copy
    on a copy stream (default priority) after the compute stream has
    released that buffer (chunk i-2); take(i) makes the compute stream wait
    for it; release(i) marks the compute stream's use of the buffer done.
    Pinned staging ("cpu" mode) copies straight from the pinned sequence;
    disk staging reads chunk rows from the memmap into pinned buffers on a
    worker thread, up to HOST_BUFFERS chunks ahead of the copies, each
    buffer reused only after its previous copy is done (with two buffers
    the worker ran one chunk ahead and the copies waited on its reads).
    Copy time and the compute stream's waits are measured with events."""

    HOST_BUFFERS = 3
    # threads that copy one chunk's rows out of the memmap (numpy copies,
    # which release the GIL and block when idle: torch's own CPU copy runs
    # on its OpenMP pool, whose threads spin between regions and slowed the
    # host's launches, measured 39.7 ms chunk stage against 27.8 ms with
    # the pool made passive)
    FILL_THREADS = 4

    def __init__(self, st: Dict[str, Any], chunks: List[Tuple[int, int]], chunk_len: int, d_model: int,
                 device: torch.device, dtype: torch.dtype) -> None:
        self.st, self.chunks, self.device = st, chunks, device
        self.bufs = [torch.empty(1, chunk_len, d_model, device=device, dtype=dtype) for _ in range(2)]
        # one copy stream per device for the process: with a fresh pool
        # stream per run, some runs' copies and the chunk model's kernels
        # waited on each other (chunk stage 20.4-29.9 ms over six runs,
        # 20.0 ms in every run with the one stream)
        self.copy_s = _side_stream(device, "copy")
        self.ready = [torch.cuda.Event() for _ in range(2)]
        self.freed = [None, None]
        self.copy_ev = []
        self.wait_ev = []
        self.disk = st.get("memmap") is not None
        self.pool = None
        if self.disk:
            nh = self.HOST_BUFFERS
            self.host = [torch.empty(1, chunk_len, d_model, dtype=dtype, pin_memory=True) for _ in range(nh)]
            self.h2d_done: List[Optional[torch.cuda.Event]] = [None] * nh
            # numpy views of the pinned buffers (bf16 as its 16-bit pattern,
            # the memmap's element type for bf16 rows); None for a dtype
            # numpy has no type for, which takes torch's copy
            try:
                self.host_np = [_memmap_view(h[0]) for h in self.host]
            except TypeError:
                self.host_np = None
            self.pool = cf.ThreadPoolExecutor(max_workers=1)
            self.copiers = cf.ThreadPoolExecutor(max_workers=self.FILL_THREADS)
            self.fills: Dict[int, cf.Future] = {}
            for j in range(nh):
                self._fill(j)

    def _fill(self, i: int) -> None:
        if i >= len(self.chunks) or i in self.fills:
            return
        s, e = self.chunks[i]
        slot = i % self.HOST_BUFFERS
        done = self.h2d_done[slot]  # the copy of chunk i - HOST_BUFFERS

        def work() -> None:
            if done is not None:
                done.synchronize()  # the previous copy out of this pinned buffer
            if self.host_np is None:
                self.host[slot][:, :e - s].copy_(self.st["rows"](s, e).unsqueeze(0))
                return
            src, dst, n = self.st["memmap"], self.host_np[slot], e - s
            step = -(-n // self.FILL_THREADS)
            parts = [self.copiers.submit(np.copyto, dst[a:min(n, a + step)], src[s + a:s + min(n, a + step)])
                     for a in range(0, n, step)]
            for f in parts:
                f.result()

        self.fills[i] = self.pool.submit(work)

    def start(self, i: int) -> None:
        s, e = self.chunks[i]
        slot = i % 2
        if self.disk:
            self._fill(i)
            self.fills.pop(i).result()
            src = self.host[i % self.HOST_BUFFERS][:, :e - s]
        else:
            src = self.st["fetch"](s, e)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(self.copy_s):
            if self.freed[slot] is not None:
                self.copy_s.wait_event(self.freed[slot])
            e0.record(self.copy_s)
            self.bufs[slot][:, :e - s].copy_(src, non_blocking=True)
            e1.record(self.copy_s)
            self.ready[slot].record(self.copy_s)
        self.copy_ev.append((e0, e1))
        if self.disk:
            ev = torch.cuda.Event()
            ev.record(self.copy_s)
            self.h2d_done[i % self.HOST_BUFFERS] = ev
            self._fill(i + self.HOST_BUFFERS)

    def take(self, i: int) -> torch.Tensor:
        s, e = self.chunks[i]
        slot = i % 2
        cur = torch.cuda.current_stream(self.device)
        w0, w1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0.record(cur)
        cur.wait_event(self.ready[slot])
        w1.record(cur)
        self.wait_ev.append((w0, w1))
        return self.bufs[slot][:, :e - s]

    def release(self, i: int) -> None:
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self.freed[i % 2] = ev

    def timings_ms(self) -> Tuple[float, float]:
        torch.cuda.synchronize(self.device)
        copy = sum(a.elapsed_time(b) for a, b in self.copy_ev)
        stall = sum(a.elapsed_time(b) for a, b in self.wait_ev)
        return float(copy), float(stall)

    def close(self) -> None:
        if self.pool is not None:
            self.pool.shutdown(wait=True)
            self.copiers.shutdown(wait=True)


class ChunkedShortlistRunner:
    """Runs the two-pass pipeline (reference chunked_shortlist.py:369-827)."""

    def __init__(self, config: ChunkedShortlistConfig, *, logger: Optional[logging.Logger] = None) -> None:
        self.config = config
        self.config.validate()
        self.logger = logger or LOGGER

    def _final_model(self, seq_len: int, dtype: torch.dtype) -> AdaptiveSparseAttention:
        """Final-pass model recipe (reference chunked_shortlist.py:712-727)."""
        cfg = self.config
        model = AdaptiveSparseAttention(_build_model_config(
            seq_len, cfg.d_model, heads=cfg.heads, sparse_ratio=cfg.final_sparse_ratio,
            shortlist_alpha=cfg.shortlist_alpha, router_top_p=cfg.nucleus_top_p)).to(
                device=cfg.device, dtype=dtype).eval()
        model.use_sdpa = False
        model.set_shortlist_alpha(float(cfg.shortlist_alpha))
        return model

    def _stage(self, sequence: Optional[torch.Tensor]):
        """Host staging (reference chunked_shortlist.py:417-560)."""
        cfg = self.config
        if sequence is not None:
            if sequence.dim() != 3:
                raise ValueError("sequence tensor must have shape (B, T, D)")
            if sequence.size(1) < cfg.seq_len:
                raise ValueError(f"sequence length {sequence.size(1)} smaller than configured seq_len {cfg.seq_len}")
            if sequence.size(2) != cfg.d_model:
                raise ValueError(f"sequence hidden size {sequence.size(2)} does not match d_model={cfg.d_model}")
            if sequence.size(0) != 1:
                raise ValueError("Chunked Shortlist runner currently expects batch size of 1.")
            source = sequence[:, :cfg.seq_len].detach()
            base_dtype = source.dtype
            if source.device.type == "cuda":
                # already resident in HBM: chunks are views, the shortlist a
                # device gather (no host staging, no copies)
                if source.device != cfg.device:
                    raise ValueError(f"sequence on {source.device} but the runner targets {cfg.device}")
                src = source.contiguous()
                size = int(src.numel() * src.element_size())
                return {"mode": "device", "reason": "sequence resident in device memory", "required": size,
                        "limit": None, "dtype": base_dtype, "memmap": None, "path": None, "pinned": False,
                        "allocated": 0, "dataset": size, "fetch": lambda s, e: src[:, s:e],
                        "gather": lambda idx: src.index_select(1, idx.to(device=src.device, dtype=torch.long))}
        else:
            source = None
            base_dtype = torch.get_default_dtype()
        elem = torch.tensor([], dtype=base_dtype).element_size()
        required = int(cfg.seq_len * cfg.d_model * elem)
        available = _system_available_ram()
        limit = cfg.ram_limit_bytes if cfg.ram_limit_bytes is not None else available
        mode, reason = cfg.storage, None
        if mode == "auto":
            if limit is not None and required > limit:
                mode, reason = "disk", f"required={required:,}B exceeds limit={limit:,}B; staging on disk"
            else:
                mode = "cpu"
                if limit is not None:
                    reason = f"limit={limit:,}B, required={required:,}B"
        elif mode == "cpu":
            if cfg.ram_limit_bytes is not None and required > cfg.ram_limit_bytes:
                mode, reason = "disk", (f"required={required:,}B exceeds ram_limit={cfg.ram_limit_bytes:,}B; "
                                        "staging on disk")
        else:
            mode = "disk"
        st = {"mode": mode, "reason": reason, "required": required, "limit": limit, "dtype": base_dtype,
              "memmap": None, "path": None, "pinned": False}
        on_gpu = cfg.device.type == "cuda"
        if mode == "cpu":
            if source is not None:
                base = source.to("cpu", dtype=base_dtype)
            else:
                gen = torch.Generator(device="cpu")
                if cfg.seed is not None:
                    gen.manual_seed(int(cfg.seed))
                base = torch.randn(1, cfg.seq_len, cfg.d_model, generator=gen).to(base_dtype)
            st["allocated"] = int(base.numel() * base.element_size())
            if on_gpu:
                base = base.pin_memory()
                st["pinned"] = True
            st["fetch"] = lambda s, e: base[:, s:e]
            st["gather"] = lambda idx: base[:, idx]
            st["dataset"] = required
        else:
            tmp_dir = Path(cfg.temp_dir) if cfg.temp_dir is not None else Path(tempfile.gettempdir())
            tmp_dir.mkdir(parents=True, exist_ok=True)
            handle = tempfile.NamedTemporaryFile(dir=tmp_dir, prefix="chunked_shortlist_", suffix=".mmap",
                                                 delete=False)
            handle.close()
            path = Path(handle.name)
            # rows are stored in the sequence's own dtype where a float32
            # round trip (the reference's float32 memmap) is exact -- bf16,
            # fp16, fp32: the same values in half the bytes for 16-bit
            # sequences -- and in float32 otherwise (its rounding kept)
            store = base_dtype if base_dtype in _MEMMAP_NP else torch.float32
            mm = np.memmap(path, dtype=_MEMMAP_NP[store], mode="w+", shape=(cfg.seq_len, cfg.d_model))
            item = mm.dtype.itemsize
            rows = max(1, min(cfg.chunk_len, int((64 * 1024 * 1024) / max(cfg.d_model * item, 1))))
            gen = torch.Generator(device="cpu")
            if cfg.seed is not None:
                gen.manual_seed(int(cfg.seed))
            for s in range(0, cfg.seq_len, rows):
                e = min(cfg.seq_len, s + rows)
                if source is not None:
                    block = source[:, s:e].to("cpu").squeeze(0)
                else:
                    block = torch.randn(e - s, cfg.d_model, generator=gen)
                mm[s:e] = _memmap_view(block.to(store))
            mm.flush()
            st.update(memmap=mm, path=path, allocated=int(rows * cfg.d_model * item),
                      dataset=int(cfg.seq_len * cfg.d_model * item))
            st["rows"] = lambda s, e: _memmap_rows(mm[s:e], store)
            st["fetch"] = lambda s, e: _memmap_rows(mm[s:e], store).to(base_dtype).unsqueeze(0)
            st["gather"] = lambda idx: _memmap_rows(mm[idx.cpu().numpy()], store).to(base_dtype).unsqueeze(0)
        return st

    def run(self, sequence: Optional[torch.Tensor] = None) -> ChunkedShortlistResult:
        cfg = self.config
        device = cfg.device
        st = self._stage(sequence)
        base_dtype = st["dtype"]
        self.logger.info("Host staging: %s (%s)", st["mode"], st["reason"])
        try:
            chunk_model = AdaptiveSparseAttention(_build_model_config(
                cfg.chunk_len, cfg.d_model, heads=cfg.heads, sparse_ratio=cfg.chunk_sparse_ratio,
                shortlist_alpha=cfg.shortlist_alpha, router_top_p=cfg.nucleus_top_p)).to(device=device,
                                                                                         dtype=base_dtype).eval()
            chunk_model.use_sdpa = False
            chunk_model.set_shortlist_alpha(float(cfg.shortlist_alpha))
            if cfg.chunk_graph and device.type == "cuda" and st["mode"] == "device":
                # the forward's output is the graph's own buffer (unused here)
                chunk_model.enable_hip_graph(True, static_output=True)
            direct = st["mode"] == "device"
            chunks = list(_chunk_iter(cfg.seq_len, cfg.chunk_len))
            final_model = None
            all_q = None
            if cfg.run_final_pass and cfg.final_mode == "all_queries":
                final_model = self._final_model(cfg.buffer_tokens, base_dtype)
                all_q = AllQueryFinalPass(final_model, cfg.seq_len, device, base_dtype, causal=cfg.final_causal)
            self.last_final_pass = all_q
            self.last_chunk_model = chunk_model
            with torch.inference_mode():
                chunk_model(torch.randn(1, cfg.chunk_len, cfg.d_model, device=device, dtype=base_dtype))
                tail = cfg.seq_len % cfg.chunk_len
                if tail and cfg.seq_len > cfg.chunk_len and chunk_model._hip_graph_enabled:
                    # capture the short last chunk's graph now, not inside the
                    # chunk loop (capturing restores the module state: no
                    # prototype update)
                    xt = torch.zeros(1, tail, cfg.d_model, device=device, dtype=base_dtype)
                    if chunk_model._graph_eligible(xt):
                        chunk_model.hip_graph_input(xt)
            if device.type == "cuda":
                torch.cuda.synchronize()
            summaries: List[ChunkSummary] = []
            # (chunk, start, end, values, positions, count or None): a chunk's
            # selection count stays on the device until the loop is done, so
            # no chunk waits for its own selection
            pending: List[Tuple[int, int, int, torch.Tensor, torch.Tensor, Optional[torch.Tensor]]] = []
            used_fallback = False
            ev_c0 = ev_c1 = None
            if cfg.report_latency and device.type == "cuda":
                ev_c0, ev_c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                ev_c0.record()
            t_start = time.perf_counter()
            t_chunks = t_start
            stager = None
            if not direct:
                if device.type != "cuda":
                    raise RuntimeError("host-staged chunks need a ROCm device")
                stager = _ChunkStager(st, chunks, cfg.chunk_len, cfg.d_model, device, base_dtype)
                st["stager"] = stager
                stager.start(0)

            def norm_fallback(ci: int, xc: torch.Tensor) -> None:
                # reference chunked_shortlist.py:632-646: the chunk's token
                # norms when its importance selects nothing
                nonlocal used_fallback
                s, e = chunks[ci]
                sel = _nucleus_select(xc[0].detach().norm(dim=-1).to(torch.float32),
                                      cfg.per_chunk_budget, cfg.nucleus_top_p)
                if sel is not None:
                    vals, rel = sel
                    pending.append((ci, s, e, vals, rel.to(torch.long) + s, None))
                    used_fallback = True

            for ci, (s, e) in enumerate(chunks):
                if direct:
                    xc = st["fetch"](s, e)
                else:
                    if ci + 1 < len(chunks):
                        stager.start(ci + 1)  # its copy overlaps this chunk's compute
                    xc = stager.take(ci)
                with torch.inference_mode():
                    chunk_model(xc)
                    if all_q is not None:
                        all_q.add_chunk(xc, s)
                promoted = _select_top_tokens(chunk_model, s, per_chunk_budget=cfg.per_chunk_budget,
                                              nucleus_top_p=cfg.nucleus_top_p)
                if promoted is None:
                    norm_fallback(ci, xc)
                else:
                    pending.append((ci, s, e) + tuple(promoted))
                if stager is not None:
                    stager.release(ci)
                t_chunks = time.perf_counter()
            if ev_c1 is not None:
                ev_c1.record()
            # one readback for every chunk's count; a chunk whose selection is
            # empty takes the norm fallback on its data fetched again
            dev_counts = [p[5] for p in pending if p[5] is not None]
            counts = torch.cat(dev_counts).tolist() if dev_counts else []
            selected: List[Tuple[int, int, int, torch.Tensor, torch.Tensor]] = []
            redo: List[int] = []
            for p_ci, p_s, p_e, p_sc, p_ix, p_cnt in pending:
                if p_cnt is None:
                    selected.append((p_ci, p_s, p_e, p_sc, p_ix))
                    continue
                c = int(counts.pop(0))
                if c > 0:
                    selected.append((p_ci, p_s, p_e, p_sc[:c], p_ix[:c]))
                else:
                    redo.append(p_ci)
            if redo:
                pending.clear()
                for ci in redo:
                    s, e = chunks[ci]
                    with torch.inference_mode():
                        norm_fallback(ci, st["fetch"](s, e).to(device))
                selected.extend((p[0], p[1], p[2], p[3], p[4]) for p in pending)
                selected.sort(key=lambda p: p[0])
                if ev_c1 is not None:
                    ev_c1.record()
            if not selected:
                raise RuntimeError("Chunked pipeline selected zero tokens; adjust per_chunk_budget or sparse ratios.")
            for p_ci, p_s, p_e, p_sc, p_ix in selected:
                summaries.append(ChunkSummary(index=p_ci, start=p_s, end=p_e, promoted=p_ix.tolist(),
                                              scores=[float(v) for v in p_sc.tolist()]))
            scores_all = [p[3] for p in selected]
            idx_all = [p[4] for p in selected]
            keep_idx, keep_scores = _finalise_indices(torch.cat(scores_all), torch.cat(idx_all),
                                                      max_tokens=cfg.buffer_tokens)
            reduced = st["gather"](keep_idx.to(torch.long)).to(device, non_blocking=st["pinned"])
            chunk_ms = None
            if ev_c0 is not None:
                torch.cuda.synchronize()
                chunk_ms = float(ev_c0.elapsed_time(ev_c1))
            if chunk_ms is None:
                chunk_ms = float((t_chunks - t_start) * 1000.0)
            chunk_tps = float(cfg.seq_len * 1000.0 / chunk_ms) if chunk_ms > 0 else None
            final_out = final_stats = backend_info = None
            final_ms = peak_mb = final_tps = None
            t_final_end = t_chunks
            if cfg.run_final_pass:
                t_f0 = time.perf_counter()
                if final_model is None:
                    final_model = self._final_model(reduced.size(1), base_dtype)
                ev_f0 = ev_f1 = None
                if device.type == "cuda":
                    torch.cuda.reset_peak_memory_stats(device)
                    if cfg.report_latency:
                        ev_f0, ev_f1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        ev_f0.record()
                with torch.inference_mode():
                    if all_q is not None:
                        final_out = all_q.finish(reduced, keep_idx).detach()
                        _record_backend("hip_int8_all_queries", device=str(device), tokens=cfg.seq_len,
                                        shortlist=int(keep_idx.numel()), causal=bool(cfg.final_causal),
                                        quantized=True)
                    else:
                        final_out = final_model(reduced).detach()
                t_final_end = time.perf_counter()
                backend_info = get_last_backend_info()
                raw = getattr(final_model, "last_head_stats", {}) or {}
                state = getattr(final_model, "_last_sparse_state", {}) or {}
                final_stats = _sanitize_mapping(raw) if isinstance(raw, dict) else {}
                if isinstance(state, dict) and state:
                    final_stats = dict(final_stats or {})
                    final_stats["sparse_state"] = _sanitize_mapping(state)
                if ev_f1 is not None:
                    ev_f1.record()
                if device.type == "cuda":
                    torch.cuda.synchronize()
                    peak_mb = torch.cuda.max_memory_allocated(device) / BYTES_PER_MB
                    if ev_f0 is not None:
                        final_ms = float(ev_f0.elapsed_time(ev_f1))
                if final_ms is None:
                    final_ms = float((t_final_end - t_f0) * 1000.0)
                if final_ms and final_ms > 0:
                    final_tok = cfg.seq_len if all_q is not None else keep_idx.numel()
                    final_tps = float(final_tok * 1000.0 / final_ms)
            total = t_final_end - t_start
            h2d_ms = h2d_stall = None
            if stager is not None:
                h2d_ms, h2d_stall = stager.timings_ms()
            metrics = ChunkedShortlistMetrics(
                original_tokens=cfg.seq_len, retained_tokens=int(keep_idx.numel()),
                retention_ratio=float(keep_idx.numel() / max(cfg.seq_len, 1)), chunk_count=len(summaries),
                device=str(device), chunk_time_ms=chunk_ms, final_time_ms=final_ms, total_time_ms=float(total * 1e3),
                peak_memory_mb=peak_mb, used_fallback=used_fallback, chunk_tokens_per_s=chunk_tps,
                final_tokens_per_s=final_tps, total_tokens_per_s=float(cfg.seq_len / total) if total > 0 else None,
                storage_mode=st["mode"], host_required_mb=st["dataset"] / BYTES_PER_MB,
                host_allocated_mb=st["allocated"] / BYTES_PER_MB if st.get("allocated") is not None else None,
                host_limit_mb=st["limit"] / BYTES_PER_MB if st["limit"] is not None else None,
                storage_reason=st["reason"], h2d_time_ms=h2d_ms, h2d_stall_ms=h2d_stall)
            self.logger.info("Chunked Shortlist retained %s/%s tokens (%.3f) across %s chunks",
                             metrics.retained_tokens, metrics.original_tokens, metrics.retention_ratio,
                             metrics.chunk_count)
            return ChunkedShortlistResult(keep_indices=keep_idx, keep_scores=keep_scores, reduced_sequence=reduced,
                                          metrics=metrics, chunks=summaries, final_output=final_out,
                                          final_stats=final_stats, backend_info=backend_info)
        finally:
            # the stager refers back to st: take it out so that neither
            # outlives this call in a reference cycle (holding pinned memory
            # and events until a garbage collection)
            stager_ = st.pop("stager", None)
            if stager_ is not None:
                stager_.close()
                stager_.st = None
            if st.get("memmap") is not None:
                st["memmap"].flush()
            if st.get("path") is not None:
                with contextlib.suppress(OSError):
                    os.remove(st["path"])


__all__ = [
    "ChunkedShortlistConfig",
    "ChunkedShortlistMetrics",
    "ChunkedShortlistResult",
    "ChunkedShortlistRunner",
    "ChunkSummary",
    "MAX_SHORTLIST_CHUNK_TOKENS",
]
