"""Build libfastdms_amd.so from the HIP sources in this directory.

Every ``*.hip`` file is compiled for gfx950 with hipcc into an object under
``fastdms_amd/_build`` (in parallel), then linked into
``fastdms_amd/_lib/libfastdms_amd.so``.  Packed-FP32 instruction selection is
disabled for all device code (``-packed-fp32-ops``); FILE_FLAGS adds
per-file code-generation options.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
BUILD_DIR = PKG / "_build"
LIB_DIR = PKG / "_lib"
LIB_PATH = LIB_DIR / "libfastdms_amd.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]
# Per-file flags.  The prefill attention kernel feeds its MFMA results straight
# into VALU softmax / masking: with the results in AGPRs (the compiler's
# default there) every block copies them out and back.
FILE_FLAGS = {
    "prefill_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    # The decode attention kernels take the arguments their first loads need
    # first (the plan of the planned launch, the live counts, append rows and
    # positions of the others); preloading them into SGPRs at
    # wave launch takes one scalar memory round trip off each workgroup's start (code objects carry a fallback
    # prologue that loads them for firmware without preload support).
    "compact_attention.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=10"],
}


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    # the compiler's per-kernel resource report (registers, scratch, spills,
    # LDS, occupancy) is kept beside the object: tests/test_codegen.py reads it
    cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(src.name, []), "-I", str(HERE), "-c", str(src), "-o", str(obj),
           "-Rpass-analysis=kernel-resource-usage"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    (BUILD_DIR / (src.stem + ".resources.txt")).write_text(res.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(HERE.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {HERE}")
    jobs = jobs or min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} HIP sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
