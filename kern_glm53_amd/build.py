"""Builds `kern_glm53_amd/libkg.so` (the C-ABI library of include/kg.h) from csrc/*.hip with hipcc for gfx950,
and `libkg_probe.so`, the benchmark's measurement kernels (csrc/kg_probe.hip: the MFMA-only ceiling).

    python -m kern_glm53_amd.build          # or kern_glm53_amd.build.build()

Every source compiles separately (in parallel) into _build/, then one shared object is linked in-tree.
All HIP code is compiled with packed-fp32 instruction generation turned off; the glue kernels, whose
results are compared bit for bit, additionally with floating-point contraction off (their fused
multiply-adds are explicit).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libkg.so"
PROBE_LIB = PKG / "libkg_probe.so"          # the benchmark's measurement kernels (not the op library)
PROBE_SOURCE = "kg_probe.hip"
INCLUDE = PKG.parent / "include"
ARCH = "gfx950"

SOURCES = {
    "kg_glue.hip": ["-ffp-contract=off"],
    "kg_prep.hip": ["-ffp-contract=off"],
    "kg_norm_rope.hip": ["-ffp-contract=off"],
    "kg_indexer.hip": ["-ffp-contract=off"],
    "kg_fp8_gemm.hip": [],
    "kg_fp8_wfrag.hip": [],
    "kg_bf16_batched.hip": [],
    "kg_mqa_logits.hip": ["-fno-honor-nans"],
}

COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-Wall", "-Wno-unused-command-line-argument", f"-I{CSRC}", f"-I{INCLUDE}"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the kern_glm53_amd kernels need ROCm's hipcc to build")


def _compile(src: str, extra: list[str]) -> pathlib.Path:
    obj = BUILD / (pathlib.Path(src).stem + ".o")
    cmd = [hipcc(), *COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every kernel source and link libkg.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda kv: _compile(*kv), SOURCES.items()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *COMMON, "-shared", str(CSRC / PROBE_SOURCE), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {PROBE_SOURCE}:\n{r.stderr}")
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print(f"built {LIB} and {PROBE_LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
