"""Compile the HIP sources into the in-tree shared library.

The library is the C-ABI declared in include/kvcompress_mi355x.h, built for
gfx950 only.  Usage: python build.py [--jobs N]
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PACKAGE_ROOT = CSRC.parent
REPO = PACKAGE_ROOT.parent
INCLUDE = REPO / "include"
OUTPUT = PACKAGE_ROOT / "kvcompress_mi355x" / "libkvcompress_mi355x.so"
BUILD_DIR = CSRC / "_build"
SOURCES = ("capi.hip", "score.hip", "score_mfma.hip", "score_max.hip", "select.hip", "compact.hip", "decode.hip", "calib.hip", "noalloc.hip")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 instructions are kept out of generated code on this target.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    return str(candidate) if candidate.exists() else "hipcc"


def _compile(source: str) -> Path:
    obj = BUILD_DIR / (Path(source).stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source}:\n{result.stdout}\n{result.stderr}")
    return obj


def build(jobs: int = 4, verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objects = list(pool.map(_compile, SOURCES))
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, OUTPUT)
    if verbose:
        print(f"built {OUTPUT}")
    return OUTPUT


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=4)
    args = parser.parse_args()
    build(args.jobs, verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
