"""Builds the gfx950 HIP library ``libengraft_ngram.so`` in-tree, and beside
it the host-only C++ autograd module ``_eg_autograd.so``.

``python engraft-ngram_amd/build.py`` or ``build()``: one ``hipcc`` invocation
over every ``csrc/*.hip`` file.  The packed-fp32 target feature is switched off
for all device code (``-Xclang -target-feature -Xclang -packed-fp32-ops``):
hipcc then never emits v_pk_{add,mul,fma}_f32.  ``csrc/eg_autograd.cpp`` is
compiled by ``g++`` against torch's headers and libraries at the same time.
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


EXT_PATH = PKG / "_eg_autograd.so"
EXT_SOURCE = PKG / "csrc" / "eg_autograd.cpp"


def ext_command(out: Path) -> list[str]:
    """g++ over ``csrc/eg_autograd.cpp``: a CPython module linked to torch."""
    import sysconfig

    from torch.utils import cpp_extension

    import torch

    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-DTORCH_EXTENSION_NAME=_eg_autograd"]
    for inc in [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(ROOT / "include")]:
        cmd += ["-I", inc]
    cmd += ["-o", str(out), str(EXT_SOURCE)]
    for lib_dir in cpp_extension.library_paths():
        cmd += ["-L", lib_dir, f"-Wl,-rpath,{lib_dir}"]
    return cmd + ["-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]


def build(verbose: bool = False) -> Path:
    """Compiles every HIP source into ``LIB_PATH`` and the autograd module into
    ``EXT_PATH``, the two compilers side by side (always rebuilds)."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    ext_tmp = EXT_PATH.with_suffix(".so.tmp")
    cmd = [
        hipcc(), "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-shared",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        "-I", str(ROOT / "include"), "-I", str(PKG / "csrc"),
        "-o", str(tmp), *[str(s) for s in sources()],
    ]
    ext_cmd = ext_command(ext_tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
        print(" ".join(ext_cmd), flush=True)
    procs = [(name, c, subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
             for name, c in (("hipcc", cmd), ("g++", ext_cmd))]
    failed = []
    for name, _, proc in procs:
        out, err = proc.communicate()
        if proc.returncode != 0:
            sys.stderr.write(out + err)
            failed.append(f"{name} failed with exit code {proc.returncode}")
        elif verbose and err.strip():
            sys.stderr.write(err)
    if failed:
        raise RuntimeError("; ".join(failed))
    os.replace(tmp, LIB_PATH)
    os.replace(ext_tmp, EXT_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
