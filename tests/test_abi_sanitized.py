"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

``test_abi.py`` runs in a child process against ``libdsk_moe_san.so`` (host
code built with ``-fsanitize=address,undefined``, device code as usual; see
``deepseeker-v4.1_amd/build.py --sanitize``) with the ASan runtime preloaded
and both sanitizers set to stop at the first report.  Every check there fails
before any launch, so no GPU is needed.  Skipped where hipcc or the clang ASan
runtime is missing.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "deepseeker-v4.1_amd"


def _asan_runtime() -> str | None:
    clang = shutil.which("clang", path="/opt/rocm/llvm/bin") or shutil.which("clang")
    if clang is None:
        return None
    out = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if out.returncode == 0 and os.path.isabs(path) and os.path.exists(path) else None


def test_abi_checks_under_host_sanitizers():
    rt = _asan_runtime()
    if rt is None or (shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists()):
        pytest.skip("hipcc or the clang ASan runtime is not available")
    sys.path.insert(0, str(PKG))
    import build as B
    lib = B.LIB_SAN
    sources = list(B.CSRC.glob("*")) + [ROOT / "include" / "dsk_moe.h"]
    if not lib.exists() or lib.stat().st_mtime < max(f.stat().st_mtime for f in sources):
        B.build(sanitize=True)
    env = dict(os.environ, LD_PRELOAD=rt, DSK_MOE_LIBRARY=str(lib),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([sys.executable, "-m", "pytest", str(ROOT / "tests" / "test_abi.py"), "-q",
                          "-p", "no:cacheprovider", "-m", "not gpu"],
                         cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    tail = (res.stdout + res.stderr)[-3000:]
    assert res.returncode == 0, tail
    assert "ERROR: AddressSanitizer" not in tail and "runtime error:" not in tail, tail
    assert " passed" in res.stdout, tail
