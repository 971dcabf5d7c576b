"""Build recipe for the oracle's C restatements (test infrastructure).

    python oracle/build_c.py

Compiles ``oracle/gate_fma.c`` with gcc into ``oracle/_build/libdsk_oracle.so``
(no contraction; the fused multiply-adds are the explicit ones).  The oracle
builds it on first use when it is missing, so tests run from a fresh tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCES = [HERE / "gate_fma.c"]
LIB = HERE / "_build" / "libdsk_oracle.so"


def build() -> Path:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("gcc is needed to build the oracle's C restatement")
    LIB.parent.mkdir(exist_ok=True)
    tmp = LIB.with_name(f"{LIB.name}.{os.getpid()}.tmp")
    cmd = [cc, "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", *map(str, SOURCES),
           "-o", str(tmp), "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle C build failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
    sys.exit(0)
