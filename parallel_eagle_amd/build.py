"""Build libpe_hip.so (gfx950) in-tree with hipcc.

Each source compiles to an object in parallel, then one link produces
``parallel_eagle_amd/libpe_hip.so``. Packed-FP32 instructions are disabled for
every device compile.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB = PKG / "libpe_hip.so"
BUILD_DIR = PKG / "_build"

SOURCES = [
    "pe_format.hip",
    "pe_gemm.hip",
    "pe_elem.hip",
    "pe_attn.hip",
    "pe_tree.hip",
    "pe_loop.hip",
    "pe_model.cpp",
]

ARCH = os.environ.get("PE_OFFLOAD_ARCH", "gfx950")
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # buffers are reinterpreted between element types throughout (tables
    # written as dwords and read as halves, bf16 rows moved as 16-byte vectors)
    "-fno-strict-aliasing",
    f"-I{INCLUDE}",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


# Per-file code generation options. attn_pair_kernel holds two row tiles' O
# accumulators per wave (more than the 256 architectural VGPRs); with the
# MFMA results in VGPR form the compiler spills 88 values to the accumulation
# registers instead of 254, and copies far fewer of them per round (the other
# kernels of the file compile to the same code either way).
FILE_FLAGS = {
    "pe_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: str) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    extra = FILE_FLAGS.get(src, [])
    cmd = [hipcc(), *COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd = [hipcc(), *COMMON, *extra, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
