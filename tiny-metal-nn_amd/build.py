"""Build libtmnn_hip.so (the gfx950 C-ABI library) in-tree with hipcc.

Usage: python tiny-metal-nn_amd/build.py [--jobs N]

Every HIP translation unit is compiled for gfx950 only, with FMA contraction
off (the encoding, loss and Adam arithmetic round each multiply and add as the
reference's MSL is written) and the packed-FP32 target feature disabled.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "libtmnn_hip.so"
BUILD_DIR = HERE / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["tmnn_hip.hip", "sort.hip"]

COMMON = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{HERE.parent / 'include'}",
]


def _compile(src: str) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    cmd = [HIPCC, *COMMON, "-c", str(CSRC / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(jobs: int = 4) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUT)
    return OUT


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    args = ap.parse_args()
    print(build(args.jobs))
    return 0


if __name__ == "__main__":
    sys.exit(main())
