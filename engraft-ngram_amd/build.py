"""Builds the gfx950 HIP library ``libengraft_ngram.so`` in-tree.

``python engraft-ngram_amd/build.py`` or ``build()``: one ``hipcc`` invocation
over every ``csrc/*.hip`` file.  The packed-fp32 target feature is switched off
for all device code (``-Xclang -target-feature -Xclang -packed-fp32-ops``):
hipcc then never emits v_pk_{add,mul,fma}_f32.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB_NAME = "libengraft_ngram.so"
LIB_PATH = PKG / LIB_NAME
ARCH = os.environ.get("EG_OFFLOAD_ARCH", "gfx950")


def sources() -> list[Path]:
    return sorted((PKG / "csrc").glob("*.hip"))


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    return "hipcc"


def build(verbose: bool = False) -> Path:
    """Compiles every HIP source into ``LIB_PATH`` (always rebuilds)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [
        hipcc(), "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        "-I", str(ROOT / "include"), "-I", str(PKG / "csrc"),
        "-o", str(tmp), *[str(s) for s in sources()],
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    if verbose and res.stderr.strip():
        sys.stderr.write(res.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
