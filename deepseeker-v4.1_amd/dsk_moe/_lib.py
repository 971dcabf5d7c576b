"""ctypes binding of libdsk_moe.so (the C ABI declared in include/dsk_moe.h).

The library is loaded from this package directory (``DSK_MOE_LIBRARY`` may
name another build of it, e.g. the host-sanitizer build
``libdsk_moe_san.so``).  Loading never falls back to anything else: if the
shared library is missing, or no HIP device is visible when a compute entry
point is called, the call raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(os.environ.get("DSK_MOE_LIBRARY") or Path(__file__).resolve().parent / "libdsk_moe.so")

ABI_VERSION = 1

DSK_OK = 0
ERRORS = {-1: "DSK_EINVAL", -2: "DSK_EALIGN", -3: "DSK_EUNSUPPORTED", -4: "DSK_EHIP",
          -5: "DSK_ESPACE"}

SCORE_SIGMOID = 0
SCORE_SQRTSOFTPLUS = 1
QUANT_FP4 = 0
QUANT_Q3 = 1
DTYPE_BF16 = 0
DTYPE_F32 = 1
STAGE_EVENTS = 10
SCRATCH_BYTES = 32 << 20

# Every function the header declares: name -> (restype, argtypes).
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t


class Desc(ctypes.Structure):
    """Mirror of ``dsk_moe_desc``."""

    _fields_ = [("tokens", _i32), ("hidden", _i32), ("n_experts", _i32), ("top_k", _i32),
                ("inter", _i32), ("inter_shared", _i32), ("score_func", _i32),
                ("quant", _i32), ("x_dtype", _i32), ("gate_dtype", _i32),
                ("route_scale", ctypes.c_float), ("limit", ctypes.c_float)]


class ExpertPtrs(ctypes.Structure):
    """Mirror of ``dsk_expert_ptrs`` (72 bytes)."""

    _fields_ = [(n, _vp) for n in ("w1", "s1", "b1", "w3", "s3", "b3", "w2", "s2", "b2")]


class Residual(ctypes.Structure):
    """Mirror of ``dsk_residual``."""

    _fields_ = [("h", _vp), ("d", _vp), ("gamma", _vp), ("eps", ctypes.c_float), ("h_out", _vp), ("x_out", _vp)]


PDesc = ctypes.POINTER(Desc)

SIGNATURES = {
    "dsk_abi_version": (ctypes.c_int, []),
    "dsk_last_error": (ctypes.c_char_p, []),
    "dsk_workspace_size": (ctypes.c_int, [PDesc, ctypes.POINTER(_sz)]),
    "dsk_route": (ctypes.c_int, [PDesc, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "dsk_dispatch": (ctypes.c_int, [PDesc, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "dsk_dispatch_workspace_size": (ctypes.c_int, [PDesc, ctypes.POINTER(_sz)]),
    "dsk_dispatch_ws": (ctypes.c_int, [PDesc, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "dsk_cap_union": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "dsk_experts": (ctypes.c_int, [PDesc, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "dsk_expert_rows": (ctypes.c_int, [PDesc, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "dsk_moe_forward": (ctypes.c_int, [PDesc, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _vp, _vp, _sz, _vp]),
    "dsk_moe_forward_residual": (ctypes.c_int, [PDesc, ctypes.POINTER(Residual), _vp, _vp, _vp, _vp, _vp, _vp,
                                                _vp, _vp, _vp, _vp, _sz, _vp]),
    "dsk_moe_forward_timed": (ctypes.c_int, [PDesc, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _vp, _vp, _vp, _sz, _vp, _vp, _i32]),
    "dsk_moe_forward_noalloc": (ctypes.c_int, [PDesc, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                               _vp, _vp, _vp]),
    "dsk_workspace_init": (ctypes.c_int, [_vp, _sz, _vp]),
    "dsk_fp4_dequant": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, _i32, _vp]),
    "dsk_fp4_quantize": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "dsk_q3_quantize": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "dsk_q3_dequant": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _vp, _i32, _vp]),
    "dsk_q3_repack": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp]),
    "dsk_fp8_block_dequant": (ctypes.c_int, [_vp, _vp, _i64, _i64, _vp, _i32, _vp]),
    "dsk_rmsnorm": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, ctypes.c_float, _i32, _vp, _vp, _vp]),
}


class DskError(RuntimeError):
    """A libdsk_moe call returned a negative status."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed with {ERRORS.get(code, code)}: {msg}")
        self.code = code


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load and type the shared library once (raises if it is missing)."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is not built; run `python deepseeker-v4.1_amd/build.py`")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.dsk_abi_version() != ABI_VERSION:
                raise ImportError(f"libdsk_moe ABI {lib.dsk_abi_version()} != {ABI_VERSION}")
            _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and raise DskError on a negative status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != DSK_OK:
        msg = lib.dsk_last_error().decode(errors="replace")
        raise DskError(name, rc, msg)
