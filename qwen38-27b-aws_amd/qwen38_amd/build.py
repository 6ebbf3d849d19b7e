"""Build libq38.so, the HIP library behind the verify path, in-tree for gfx950.

    python -m qwen38_amd.build        (from qwen38-27b-aws_amd/)

Every source in csrc/ is compiled by hipcc for gfx950 only (objects under csrc/_build/), then linked into
qwen38_amd/libq38.so, which `ext.py` loads. Packed-fp32 instructions are switched off for all device code.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
OBJ = CSRC / "_build"
LIB = PACKAGE / "libq38.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
SOURCES = ["gemm.hip", "norm.hip", "gdn.hip", "attn.hip", "prefill.hip", "pick.hip", "pack.hip", "spec.hip", "noalloc.hip",
           "engine.cpp"]


def _compile(src: str) -> Path:
    out = OBJ / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that line is expected.
    noise = "is not a recognized feature for this target"
    errors = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    if proc.returncode:
        raise RuntimeError(f"hipcc failed on {src}:\n{errors}")
    if errors.strip():
        print(errors, file=sys.stderr)
    return out


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as pool:
        objects = list(pool.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
