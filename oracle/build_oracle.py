"""Compile the C oracle (oracle/shortlist_oracle.c) with gcc into
oracle/liboracle_shortlist.so.  Test infrastructure only."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "shortlist_oracle.c"
LIB = HERE / "liboracle_shortlist.so"


def build() -> Path:
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-std=c11", str(SRC), "-o", str(LIB)]
    subprocess.run(cmd, check=True)
    return LIB


if __name__ == "__main__":
    print(build())
