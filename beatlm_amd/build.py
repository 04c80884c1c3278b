"""Builds the backend library (beatlm_amd/libbeatlm_hip.so) for gfx950 with
hipcc, one object per source in parallel, and the oracle's C restatement
(oracle/build/liboracle.so) with gcc.

Run as `python -m beatlm_amd.build` or through `__graft_entry__.build()`.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent
REPO = ROOT.parent
CSRC = ROOT / "csrc"
OBJ = ROOT / "_build"
LIB = ROOT / "libbeatlm_hip.so"
ARCH = "gfx950"

# Every HIP translation unit. Packed-FP32 instructions are disabled: only
# hipcc's own scalar/float2 code generation is used for f32 arithmetic.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-value",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

SOURCES = [
    "k_gemm_f32.hip",
    "k_gemm_split.hip",
    "k_gemm_f16.hip",
    "k_flash.hip",
    "k_misc.hip",
    "static_attention.hip",
    "backend.cpp",
    "timer.cpp",
    "ring.cpp",
    "ir.cpp",
    "cost.cpp",
    "schedule.cpp",
    "step.cpp",
    "load.cpp",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the backend needs ROCm's hipcc")


def _compile(src: str) -> pathlib.Path:
    out = OBJ / (src + ".o")
    lang = [] if src.endswith(".hip") else ["-x", "hip"]
    cmd = [hipcc(), *HIP_FLAGS, *lang, "-c", str(CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in r.stderr.splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return out


def _stale(src: str) -> bool:
    """Whether src's object is older than src or any header it may include."""
    out = OBJ / (src + ".o")
    if not out.exists():
        return True
    deps = [CSRC / src, *CSRC.glob("*.hpp"), *CSRC.glob("*.inc"), *(REPO / "include").glob("*.h")]
    return any(d.stat().st_mtime > out.stat().st_mtime for d in deps)


def build_library(jobs: int | None = None, incremental: bool = False) -> pathlib.Path:
    """Compiles every source (incremental: only those whose object is stale)
    and links the library."""
    OBJ.mkdir(exist_ok=True)
    sources = [s for s in SOURCES if (CSRC / s).exists()]
    todo = [s for s in sources if _stale(s)] if incremental else sources
    jobs = jobs or min(max(1, len(todo)), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        list(pool.map(_compile, todo))
    objects = [OBJ / (s + ".o") for s in sources]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> pathlib.Path:
    r = subprocess.run(["make", "-s", "-C", str(REPO / "oracle")], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    return REPO / "oracle" / "build" / "liboracle.so"


def build() -> None:
    build_oracle()
    build_library()


if __name__ == "__main__":
    if "--incremental" in sys.argv:
        build_oracle()
        build_library(incremental=True)
    else:
        build()
    print(LIB)
