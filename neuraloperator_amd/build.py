"""Build libfnohip.so in-tree with hipcc for gfx950.

    python -m neuraloperator_amd.build        (everything)
    python -m neuraloperator_amd.build -i     (only objects older than their sources)

Every HIP source under ``csrc/`` is compiled to an object in parallel and the
objects are linked into ``neuraloperator_amd/libfnohip.so``.  All device code
is built with packed-FP32 instruction selection disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libfnohip.so"
ARCH = os.environ.get("FNO_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the FNO HIP library cannot be built")


def sources():
    return sorted(CSRC.glob("*.hip"))


def _headers_mtime() -> float:
    heads = list(CSRC.glob("*.h")) + list((PKG.parent / "include").glob("*.h"))
    return max((h.stat().st_mtime for h in heads), default=0.0)


def build(verbose: bool = False, jobs: int = 8, incremental: bool = False) -> Path:
    """Compile every source and link the library.  incremental=True keeps an
    object that is newer than its source and every header."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    objs = []
    heads = _headers_mtime()

    def compile_one(src: Path) -> Path:
        obj = BUILD / (src.stem + ".o")
        if incremental and obj.exists() and obj.stat().st_mtime > max(src.stat().st_mtime, heads):
            return obj
        cmd = [hipcc, *HIPCC_FLAGS, "-I", str(CSRC), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, sources()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, incremental="-i" in sys.argv)
    print(f"built {path}")
