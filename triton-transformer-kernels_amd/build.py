"""Build libttk_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: python triton-transformer-kernels_amd/build.py [--jobs N]

Each csrc/*.hip file is compiled to an object under _build/ (in parallel),
then linked into lib/libttk_hip.so next to this file.  The build always runs
(no staleness check): callers that only load the library never build.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PKG_ROOT / "_build"
LIB_DIR = PKG_ROOT / "lib"
LIB_PATH = LIB_DIR / "libttk_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libttk_hip.so")
    return found


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature; that
    # warning is expected and is filtered from the log.
    lines = [
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in line
    ]
    if proc.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + "\n".join(lines))
    if lines:
        print("\n".join(lines), file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    hipcc = _hipcc()
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    objects = [BUILD_DIR / (src.stem + ".o") for src in sources]
    cmds = [[hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)] for src, obj in zip(sources, objects)]
    workers = jobs or min(len(cmds), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for cmd in cmds:
            if verbose:
                print(" ".join(cmd))
        list(pool.map(_run, cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    if verbose:
        print(" ".join(link))
    _run(link)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--jobs", type=int, default=None)
    parser.add_argument("-v", "--verbose", action="store_true")
    args = parser.parse_args()
    path = build(args.jobs, args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
