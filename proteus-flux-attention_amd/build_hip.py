"""Build libpfa_hip.so (gfx950) from csrc/*.hip with hipcc.

Each translation unit is compiled to an object in parallel, then linked into
``proteus_attention/lib/libpfa_hip.so`` inside the source tree, so the built
library travels with the tree.  Always rebuilds when called.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT_DIR = ROOT / "proteus_attention" / "lib"
LIB_NAME = "libpfa_hip.so"
ARCH = os.environ.get("PFA_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # Packed FP32 instructions are disabled for every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; cannot build libpfa_hip.so")
    return exe


def _compile_one(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    obj_dir = ROOT / "_build"
    obj_dir.mkdir(exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        futs = [ex.submit(_compile_one, s, o) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    final = OUT_DIR / LIB_NAME
    os.replace(tmp, final)
    if verbose:
        print(f"built {final}")
    return final


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
