"""Tuned library-GEMM choices for the two projections on MI355X.

The QKV and output projections stay library GEMMs (hipBLASLt / rocBLAS
through torch).  ``gemm_mi355x.csv`` is a PyTorch TunableOp results table
recorded on an MI355X (gfx950) for the projection shapes of the benchmark
workloads (T = 65,536 and 524,288 tokens at d_model 512, the chunked
pipeline's shapes at T = 1,048,576).  :func:`use_tuned_gemms` makes torch
look GEMMs of those shapes up in it instead of using its default heuristic;
shapes that are not in the table keep the default.  Nothing is tuned at run
time, and the table is ignored when its validators (torch, HIP, hipBLASLt,
rocBLAS versions and GPU architecture) do not match the running system.
"""
from __future__ import annotations

import os
import tempfile
from pathlib import Path
from typing import Optional

import torch

TABLE = Path(__file__).resolve().parent / "gemm_mi355x.csv"


def use_tuned_gemms(path: Optional[str] = None) -> bool:
    """Enable TunableOp lookups from the shipped table (no run-time tuning).
    Returns True when the table was accepted."""

    if not torch.cuda.is_available():
        return False
    import torch.cuda.tunable as tunable

    tunable.enable(True)
    tunable.tuning_enable(False)
    tunable.record_untuned_enable(False)
    # results are written back at exit to this file, never into the package
    tunable.set_filename(os.path.join(tempfile.gettempdir(), f"pfa_tunableop_{os.getpid()}.csv"))
    return bool(tunable.read_file(str(path or TABLE)))


__all__ = ["TABLE", "use_tuned_gemms"]
