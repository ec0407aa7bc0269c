"""Build recipe of the native library (hipcc --offload-arch=gfx950, in-tree)."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"


def build_library(jobs: int | None = None, verbose: bool = False, force: bool = False) -> Path:
    """Compiles malaga_amd/_build/libmalaga_hip.so (make; force: every source again)."""
    jobs = jobs or min(16, os.cpu_count() or 8)
    cmd = ["make", "-C", str(CSRC), f"-j{jobs}"] + (["-B"] if force else [])
    res = subprocess.run(cmd, capture_output=not verbose, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building libmalaga_hip.so failed:\n{res.stdout}\n{res.stderr}")
    out = PKG / "_build" / "libmalaga_hip.so"
    if not out.exists():
        raise RuntimeError(f"build finished but {out} is missing")
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))
