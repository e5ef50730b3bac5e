"""Build step for the gfx950 HIP library (libainfer_moe.so, in-tree).

hipcc cross-compiles for gfx950 without a GPU present.  All HIP code is
compiled with packed-fp32 instruction selection disabled.
"""
import os
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libainfer_moe.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["moe_api.hip", "moe_route.hip", "moe_router.hip", "moe_expert.hip", "moe_gemm.hip",
           "moe_decode.hip", "moe_w4a8.hip", "moe_stack.hip", "moe_probe.hip", "moe_binfer.cpp"]
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-gpu-rdc", "-Wall", "-Wno-unused-function",
]


def build_library(verbose: bool = False, out: Path = None) -> Path:
    """Compile every HIP source into ainfer_amd/libainfer_moe.so (or `out`).
    AINFER_HIPFLAGS adds compiler flags, e.g. "-DAINFER_GEMM_TRACE" for the
    prefill GEMM's per-item timestamps (a diagnostic build)."""
    from concurrent.futures import ThreadPoolExecutor
    objs = [str(CSRC / (src + ".o")) for src in SOURCES]
    extra = os.environ.get("AINFER_HIPFLAGS", "").split()
    cmds = [[HIPCC, *[f for f in FLAGS if f != "-shared"], *extra, "-c", str(CSRC / src), "-o", obj]
            for src, obj in zip(SOURCES, objs)]
    jobs = max(1, min(len(cmds), (os.cpu_count() or 1) // 2, 8))
    with ThreadPoolExecutor(jobs) as pool:
        list(pool.map(lambda c: _run(c, verbose), cmds))
    lib = Path(out) if out else LIB
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(lib), *objs], verbose)
    return lib


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


if __name__ == "__main__":
    import sys
    print(build_library(verbose=True, out=Path(sys.argv[1]).resolve() if len(sys.argv) > 1 else None))
