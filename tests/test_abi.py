"""CPU checks of the C ABI boundary: the library loads, exports what the
header declares, its structs match, and host-side validation rejects bad
requests before any launch (these paths need no GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from dsk_moe import _lib, ops
from oracle import router as R

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dsk_moe.h"
ROUTE_SRC = ROOT / "deepseeker-v4.1_amd" / "csrc" / "gate.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(dsk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 11
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"


def test_abi_version_and_struct_sizes():
    lib = _lib.load()
    assert lib.dsk_abi_version() == _lib.ABI_VERSION == 1
    assert ctypes.sizeof(_lib.Desc) == 48
    assert ctypes.sizeof(_lib.ExpertPtrs) == 72


def _desc(**kw):
    base = dict(tokens=4, hidden=1024, n_experts=64, top_k=6, inter=512, inter_shared=512)
    base.update(kw)
    return ops.make_desc(**base)


@pytest.mark.parametrize("field,value", [("tokens", 0), ("n_experts", 0), ("n_experts", 2048),
                                         ("top_k", 0), ("top_k", 17), ("hidden", 48),
                                         ("score_func", 7), ("x_dtype", 9)])
def test_host_validation_rejects(field, value):
    d = _desc()
    setattr(d, field, value)
    with pytest.raises(_lib.DskError) as ei:
        ops.workspace_size(d)
    assert ei.value.code == -1


def test_workspace_size_is_host_only_and_monotone():
    small = ops.workspace_size(_desc(tokens=1))
    big = ops.workspace_size(_desc(tokens=64))
    assert 0 < small < big
    assert small % 256 == 0


def test_null_and_alignment_errors_before_launch():
    d = _desc()
    lib = _lib.load()
    assert lib.dsk_workspace_size(ctypes.byref(d), None) == -1
    rc = lib.dsk_route(ctypes.byref(d), None, None, None, None, None, None, None)
    assert rc == -1 and b"NULL" in lib.dsk_last_error()
    rc = lib.dsk_fp4_dequant(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 48, ctypes.c_void_p(16), 1, None)
    assert rc == -1                                   # cols % 32
    rc = lib.dsk_fp4_dequant(ctypes.c_void_p(17), ctypes.c_void_p(16), 1, 64, ctypes.c_void_p(16), 1, None)
    assert rc == -2                                   # misaligned
    rc = lib.dsk_experts(ctypes.byref(_desc(quant="q3", inter=96)), *([ctypes.c_void_p(256)] * 14), 1 << 30, None)
    assert rc == -1 and b"128" in lib.dsk_last_error()   # q3 needs K multiples of 128
    rc = lib.dsk_experts(ctypes.byref(_desc(quant="q3", hidden=1056)), *([ctypes.c_void_p(256)] * 14), 1 << 30, None)
    assert rc == -1                                   # hidden % 128
    rows_args = [ctypes.c_void_p(256)] * 10
    rc = lib.dsk_expert_rows(ctypes.byref(_desc()), *rows_args, 1 << 30, None)
    assert rc == -1 and b"inter_shared" in lib.dsk_last_error()    # routed experts only
    rc = lib.dsk_expert_rows(ctypes.byref(_desc(inter_shared=0)), *rows_args[:8], ctypes.c_void_p(264),
                             ctypes.c_void_p(256), 1 << 30, None)
    assert rc == -2                                   # rows not 16-byte aligned
    rc = lib.dsk_expert_rows(ctypes.byref(_desc(inter_shared=0)), *rows_args, 64, None)
    assert rc == -5                                   # workspace too small


def test_route_constants_match_oracle():
    """The hex constants of the router math (gate.h) equal the oracle's derived ones."""
    src = ROUTE_SRC.read_text()

    def arr(name):
        body = re.search(name + r"\[\d+\]\s*=\s*\{(.*?)\};", src, re.S).group(1)
        return [float.fromhex(v) for v in re.findall(r"0x[0-9a-fp.+-]+", body)]

    def scalar(name):
        return float.fromhex(re.search(name + r"\s*=\s*(0x[0-9a-fp.+-]+);", src).group(1))

    assert scalar("kLn2Hi") == R.LN2_HI and scalar("kLn2Lo") == R.LN2_LO
    assert scalar("kLog2e") == R.LOG2E
    assert arr("kExpCoef") == R.EXP_COEF
    assert arr("kAtanhCoef") == R.ATANH_COEF


def test_roles_normalisation_splits_w13():
    import torch
    from dsk_moe.layer import _roles_of
    w13 = (torch.arange(8).reshape(4, 2), torch.arange(4).reshape(4, 1))
    w1, w3, w2 = _roles_of({"w13": w13, "w2": ("a", "b")})
    assert w1[0].tolist() == [[0, 1], [2, 3]] and w3[0].tolist() == [[4, 5], [6, 7]]
    assert w1[1].tolist() == [[0], [1]] and w2 == ("a", "b")


def test_ops_reject_cpu_tensors():
    import torch
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        ops.route(x, torch.zeros(8, 64), torch.zeros(8), 2)


def test_cap_union_size_limit_is_a_clean_rejection():
    """The union cap keeps a batch's (token, slot) pairs and per-expert sums in one
    block's LDS (T*top_k*4 + E*9 bytes of 160 KB): at 256 experts, top-8, up to
    5048 tokens; beyond that DSK_EUNSUPPORTED before any launch."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    assert lib.dsk_cap_union(5049, 256, 8, 64, 0, p, p, p, None) == -3
    assert b"beyond the one-block cap" in lib.dsk_last_error()
    with pytest.raises(_lib.DskError, match="DSK_EUNSUPPORTED"):
        _lib.call("dsk_cap_union", 8192, 256, 8, 64, 0, p, p, p, None)


def test_forward_residual_validation():
    """dsk_moe_forward_residual rejects a missing residual, misaligned stream
    pointers and an x_out that overlaps the stream, before any launch."""
    lib = _lib.load()
    d = _desc(tokens=1)
    ptrs = [ctypes.c_void_p(1 << 20)] * 10          # gate_w .. workspace, all aligned
    call = lambda r: lib.dsk_moe_forward_residual(ctypes.byref(d), r, *ptrs, 1 << 30, None)
    assert call(None) == -1
    row = 1024 * 2                                    # one bf16 row of hidden 1024
    good = dict(h=1 << 24, d=(1 << 24) + 4 * row, gamma=None, eps=1e-6, h_out=(1 << 24) + 8 * row,
                x_out=(1 << 24) + 12 * row)
    assert call(ctypes.byref(_lib.Residual(**{**good, "h": (1 << 24) + 8}))) == -2
    assert call(ctypes.byref(_lib.Residual(**{**good, "x_out": good["h"]}))) == -1
    assert b"overlap" in lib.dsk_last_error()
    assert call(ctypes.byref(_lib.Residual(**{**good, "eps": -1.0}))) == -1
