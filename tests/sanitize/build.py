"""Build the C-ABI validation driver (capi_validation.cpp) against a host-only
build of the library's sources, with AddressSanitizer and
UndefinedBehaviorSanitizer on the host code (-Xarch_host: no device code is
built or instrumented; the objects are relocatable device code without any,
so they link without a GPU binary).  Objects and the driver go to
tests/sanitize/_build; a source newer than its object is rebuilt.

    python tests/sanitize/build.py      # prints the driver's path
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
CSRC = ROOT / "neuraloperator_amd" / "csrc"
OUT = HERE / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-Xarch_host", "-fno-sanitize-recover=all"]
COMPILE = ["--offload-arch=gfx950", "-fgpu-rdc", "--cuda-host-only", "-O1", "-g", "-std=c++17",
           "-fno-omit-frame-pointer", *SAN, "-I", str(ROOT / "include")]


def _stale(obj: Path, deps) -> bool:
    return not obj.exists() or obj.stat().st_mtime < max(d.stat().st_mtime for d in deps)


def build() -> Path:
    OUT.mkdir(exist_ok=True)
    headers = list(CSRC.glob("*.h")) + [ROOT / "include" / "fno_hip.h"]
    jobs = [(src, OUT / (src.stem + ".o"), []) for src in sorted(CSRC.glob("*.hip"))]
    jobs.append((HERE / "capi_validation.cpp", OUT / "capi_validation.o", ["-x", "c++"]))

    def one(job):
        src, obj, extra = job
        if _stale(obj, [src, *headers]):
            r = subprocess.run([HIPCC, *COMPILE, *extra, "-c", str(src), "-o", str(obj)],
                               capture_output=True, text=True)
            if r.returncode:
                raise RuntimeError(f"compiling {src.name} failed:\n{r.stderr[-4000:]}")
        return obj

    with ThreadPoolExecutor(min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(one, jobs))
    exe = OUT / "capi_validation"
    if _stale(exe, objs):
        r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-fgpu-rdc", "--hip-link",
                            "-Xarch_host", "-fsanitize=address", "-Xarch_host",
                            "-fsanitize=undefined", "-o", str(exe), *map(str, objs),
                            "-L", str(ROCM / "lib"), "-lamdhip64", "-lpthread"],
                           capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(f"linking the driver failed:\n{r.stderr[-4000:]}")
    return exe


if __name__ == "__main__":
    print(build())
    sys.exit(0)
