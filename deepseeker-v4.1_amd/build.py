"""Build recipe for libdsk_moe.so (gfx950) -- run from anywhere.

    python deepseeker-v4.1_amd/build.py [--jobs N] [--verbose] [--sanitize]

Compiles every ``csrc/*.hip`` with hipcc for gfx950 into ``_build/`` and links
``dsk_moe/libdsk_moe.so`` in-tree (the shared library travels with the source
tree; nothing is installed).  Packed-FP32 instruction selection is disabled
for all device code.  The router and format kernels are compiled without
floating-point contraction, because their results are compared bit for bit
with the CPU oracle.

``--sanitize`` builds ``dsk_moe/libdsk_moe_san.so`` (objects in
``_build_san/``) whose host code -- the C ABI's argument checks, workspace
layout and launch set-up -- carries AddressSanitizer and UndefinedBehavior-
Sanitizer checks; device code is compiled as usual.  It is loaded with the ASan
runtime preloaded (``DSK_MOE_LIBRARY`` names the library to load) by the CPU
tests of the ABI.
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
# host-only sanitizers: each -fsanitize= applies to the host compilation alone
SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-fno-sanitize-recover=all"]
LIB_SAN = PKG_ROOT / "dsk_moe" / "libdsk_moe_san.so"
BUILD_SAN = PKG_ROOT / "_build_san"


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build libdsk_moe)")
    return path


def compile_one(src: Path, verbose: bool, sanitize: bool = False) -> Path:
    obj = (BUILD_SAN if sanitize else BUILD) / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, *(SANITIZE if sanitize else []), "-c", str(src), "-o", str(obj)]
    if src.name in NO_CONTRACT:
        cmd.insert(-4, "-ffp-contract=off")
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False, sanitize: bool = False) -> Path:
    out_dir, lib = (BUILD_SAN, LIB_SAN) if sanitize else (BUILD, LIB)
    out_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: compile_one(s, verbose, sanitize), sources))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=" + ARCH, "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if sanitize:
        cmd += ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-shared-libsan"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)
    return lib


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--sanitize", action="store_true", help="host ASan/UBSan build (libdsk_moe_san.so)")
    args = ap.parse_args()
    lib = build(args.jobs, args.verbose, args.sanitize)
    print(f"built {lib}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
