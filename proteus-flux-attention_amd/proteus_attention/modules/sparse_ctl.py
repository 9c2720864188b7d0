"""Head-budget feedback controller (reference modules/sparse_ctl.py:23-161).

Pure host logic: it reads ``last_head_stats["max_active_density"]`` after
each forward and nudges the layer's ``h_active_min``/``h_active_max``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, List, Optional

import torch.nn as nn


@dataclass
class SparseCtlSnapshot:
    """One controller decision."""

    density: float
    action: str
    min_heads: int
    max_heads: int
    step: int


class SparseHeadController:
    """Moves the active-head budget toward ``target_density`` (+- tolerance),
    deciding once every ``cooldown`` observations."""

    def __init__(
        self,
        attention_layer: nn.Module,
        *,
        target_density: float = 0.28,
        tolerance: float = 0.03,
        cooldown: int = 4,
        min_heads: Optional[int] = None,
        max_heads: Optional[int] = None,
        dense_threshold: Optional[float] = None,
        verbose: bool = False,
    ) -> None:
        self._layer = attention_layer
        self.target_density = float(max(0.0, min(target_density, 1.0)))
        self.tolerance = float(max(0.0, tolerance))
        self.cooldown = max(1, int(cooldown))
        self.verbose = verbose
        self._global_min = min_heads if (min_heads and min_heads > 0) else None
        self._global_max = max_heads if (max_heads and max_heads > 0) else None
        self._dense_threshold = dense_threshold
        self._step = 0
        self._since_adjust = 0
        self._history: List[float] = []
        self._last_snapshot: Optional[SparseCtlSnapshot] = None
        self._apply_bounds(self._global_min, self._global_max)
        if self._dense_threshold is not None:
            self._layer._dense_threshold = float(max(0.0, min(self._dense_threshold, 1.0)))

    @property
    def last_snapshot(self) -> Optional[SparseCtlSnapshot]:
        return self._last_snapshot

    def reset(self) -> None:
        self._step = 0
        self._since_adjust = 0
        self._history.clear()
        self._last_snapshot = None

    def observe(self, head_stats: Optional[Dict[str, Any]]) -> Optional[SparseCtlSnapshot]:
        self._step += 1
        density = head_stats.get("max_active_density") if isinstance(head_stats, dict) else None
        if density is None:
            self._history.clear()
            return None
        self._history.append(float(density))
        self._since_adjust += 1
        if self._since_adjust < self.cooldown:
            return None
        avg = sum(self._history) / max(1, len(self._history))
        if avg > self.target_density + self.tolerance:
            action = "decrease"
            self._adjust_heads(-1)
        elif avg < max(0.0, self.target_density - self.tolerance):
            action = "increase"
            self._adjust_heads(+1)
        else:
            action = "steady"
        snap = SparseCtlSnapshot(density=avg, action=action,
                                 min_heads=int(getattr(self._layer, "h_active_min", 0)),
                                 max_heads=int(getattr(self._layer, "h_active_max", 0)), step=self._step)
        self._last_snapshot = snap
        self._history.clear()
        self._since_adjust = 0
        if self.verbose:
            print(f"[SparseCtl] step={snap.step} density={snap.density:.3f} action={snap.action} "
                  f"min={snap.min_heads} max={snap.max_heads}")
        return snap

    def _apply_bounds(self, min_heads: Optional[int], max_heads: Optional[int]) -> None:
        layer = self._layer
        total = getattr(layer, "h_total", None)
        if total is None:
            return
        if min_heads is not None:
            layer.h_active_min = max(1, min(int(min_heads), int(total)))
        if max_heads is not None:
            layer.h_active_max = max(layer.h_active_min, min(int(max_heads), int(total)))
        layer.h_active = max(layer.h_active_min, min(layer.h_active, layer.h_active_max))

    def _adjust_heads(self, delta: int) -> None:
        layer = self._layer
        total = int(getattr(layer, "h_total", 1))
        new_max = max(1, min(int(getattr(layer, "h_active_max", 1)) + delta, total))
        if self._global_max is not None:
            new_max = min(new_max, self._global_max)
        if self._global_min is not None:
            new_min = max(1, min(self._global_min, new_max))
        else:
            new_min = min(layer.h_active_min, new_max)
        # The reference's _apply_bounds returns None, so the L-scale nudge
        # that follows it there never fires; the same holds here.
        self._apply_bounds(new_min, new_max)
