"""Tools (reference tools/__init__.py)."""

from .chunked_shortlist import (
    ChunkedShortlistConfig,
    ChunkedShortlistMetrics,
    ChunkedShortlistResult,
    ChunkedShortlistRunner,
    ChunkSummary,
)

__all__ = [
    "ChunkedShortlistConfig",
    "ChunkedShortlistMetrics",
    "ChunkedShortlistResult",
    "ChunkedShortlistRunner",
    "ChunkSummary",
]
