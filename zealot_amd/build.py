"""Builds libzealot_kv.so (HIP kernels + C ABI) for gfx950 with hipcc.

Usage: python -m zealot_amd.build    (or zealot_amd.build.build() from Python)
The library lands in zealot_amd/libzealot_kv.so; objects in zealot_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(HERE, "libzealot_kv.so")
SOURCES = ["status.cpp", "timing.cpp", "block_manager.cpp", "kv_ops.hip", "paged_decode.hip", "paged_prefill.hip", "kv_cache.cpp", "scheduler.cpp",
           "dense_ops.hip", "gemm.cpp", "skinny_gemm.hip", "noalloc_scratch.hip"]
ARCH = "gfx950"
HIPFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall",
    # packed-fp32 VALU ops stay off: hipcc must not emit v_pk_{add,mul,fma}_f32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the decode kernels keep one wave per SIMD,
    # so registers are plentiful, and loop-carried accumulators otherwise get
    # copied between AGPRs and VGPRs on every page
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # the decode kernels claim work with a lane-0 atomic whose result is used
    # one work item later; the wave-aggregating rewrite would wait for it at
    # once and stall the page pipeline
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


# per-file additions: the prefill softmax computes on finite scores and -inf
# only, so its maxima need no NaN quieting (IEEE-mode v_max_f32 otherwise
# gets two canonicalizing moves per compare)
FILE_FLAGS = {"paged_prefill.hip": ["-fno-honor-nans"]}


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), "-x", "hip", *HIPFLAGS, *FILE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP/C++ source and link the shared library (always rebuilds)."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    # hipBLASLt carries the dense projections (gemm.cpp)
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-L/opt/rocm/lib", "-lhipblaslt",
           "-Wl,-rpath,/opt/rocm/lib", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
