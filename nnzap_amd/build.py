"""Build libnnzap_amd.so (gfx950) in-tree with explicit hipcc invocations.

Usage: python -m nnzap_amd.build [--jobs N]

Every source under nnzap_amd/csrc/*.hip is compiled for gfx950 only, with
packed-FP32 instruction selection disabled, then linked into
nnzap_amd/libnnzap_amd.so next to this file.  Object files go to
nnzap_amd/_build/ (git-ignored).
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libnnzap_amd.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-but-set-variable",
    # Packed FP32 forms are not emitted (explicit project rule for gfx950).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{HERE.parent / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP toolchain is required to build nnzap_amd")


# Per-source additions.  gemm.hip: MFMA accumulators in VGPRs rather than
# AGPRs (the gate/up GEMM otherwise moves its 64 accumulator registers
# through v_accvgpr_read/mov around the k-phase reduction and the epilogue:
# ~300 instructions per wave; same total register count).
EXTRA_FLAGS = {
    "gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources found")
    jobs = jobs or min(len(sources), max(1, os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    build(ap.parse_args().jobs)
