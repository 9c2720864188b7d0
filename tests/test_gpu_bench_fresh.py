"""bench.py's default run (config 3, graph-replayed forward with the output
projection captured) in a fresh process, where nothing has set up the
libraries before the first capture: every library call the capture records
must have run once in the forward's warm-up.  (A capture that met a
GEMM library's first call inside it failed with "operation not permitted
when stream is capturing".)"""
import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def test_bench_default_run_in_fresh_process():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print("bench.py --steps 3 --warmup 1 --no-cpu-baseline in a child process", flush=True)
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--steps", "3", "--warmup", "1",
                          "--no-cpu-baseline"], cwd=str(ROOT), capture_output=True, text=True, timeout=240)
    assert res.returncode == 0, res.stderr[-2000:]
    line = json.loads(res.stdout.strip().splitlines()[-1])
    assert line["steps"] == 3 and line["value"] > 0 and line["ms_per_step"] > 0
