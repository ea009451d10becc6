"""Compiles tests/c/abi_check.c with gcc against include/nnz.h into
tests/c/libnnz_abi_check.so, linked to nnzap_amd/libnnzap_amd.so (rpath
relative to this directory).  Called by __graft_entry__.build() after the
library is built, and by the ABI tests when the check library is missing."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
SRC = HERE / "abi_check.c"
OUT = HERE / "libnnz_abi_check.so"


def build() -> Path:
    lib_dir = ROOT / "nnzap_amd"
    cmd = ["gcc", "-std=c11", "-O2", "-Wall", "-Wextra", "-Werror", "-shared", "-fPIC",
           f"-I{ROOT / 'include'}", str(SRC), f"-L{lib_dir}", "-lnnzap_amd",
           "-Wl,-rpath,$ORIGIN/../../nnzap_amd", "-o", str(OUT)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed for {SRC.name}:\n{res.stdout}\n{res.stderr}")
    return OUT


if __name__ == "__main__":
    print(build())
