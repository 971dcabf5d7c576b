"""Build recipe for libdsk_moe.so (gfx950) -- run from anywhere.

    python deepseeker-v4.1_amd/build.py [--jobs N] [--verbose]

Compiles every ``csrc/*.hip`` with hipcc for gfx950 into ``_build/`` and links
``dsk_moe/libdsk_moe.so`` in-tree (the shared library travels with the source
tree; nothing is installed).  Packed-FP32 instruction selection is disabled
for all device code.  The router and format kernels are compiled without
floating-point contraction, because their results are compared bit for bit
with the CPU oracle.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
BUILD = PKG_ROOT / "_build"
LIB = PKG_ROOT / "dsk_moe" / "libdsk_moe.so"
ARCH = "gfx950"

COMMON = ["--offload-arch=" + ARCH, "-O3", "-fPIC", "-std=c++17",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-command-line-argument", "-munsafe-fp-atomics"]
NO_CONTRACT = {"route.hip", "formats.hip"}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build libdsk_moe)")
    return path


def compile_one(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, "-c", str(src), "-o", str(obj)]
    if src.name in NO_CONTRACT:
        cmd.insert(-4, "-ffp-contract=off")
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: compile_one(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=" + ARCH, "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    lib = build(args.jobs, args.verbose)
    print(f"built {lib}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
