"""torch-level wrappers of the libdsk_moe entry points.

Every wrapper checks devices, dtypes, shapes and contiguity on the host,
allocates its outputs with torch on the input's device and launches on the
current HIP stream of that device.  Nothing here computes on the CPU: a
tensor that is not on a HIP device is an error.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

SCORE_FUNCS = {"sigmoid": _lib.SCORE_SIGMOID, "sqrtsoftplus": _lib.SCORE_SQRTSOFTPLUS}
QUANTS = {"fp4": _lib.QUANT_FP4, "q3": _lib.QUANT_Q3}
_DTYPES = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else None)


def stream_of(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All tensors on one HIP device and contiguous; returns that device."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"dsk_moe needs HIP device tensors, got a {t.device} tensor")
        if not t.is_contiguous():
            raise ValueError("dsk_moe needs contiguous tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no device tensor given")
    return dev


def dtype_code(dt: torch.dtype, what: str) -> int:
    if dt not in _DTYPES:
        raise ValueError(f"{what} must be bfloat16 or float32, got {dt}")
    return _DTYPES[dt]


def score_code(score_func: str | int) -> int:
    if isinstance(score_func, int):
        return score_func
    if score_func not in SCORE_FUNCS:
        raise ValueError(f"score_func must be one of {sorted(SCORE_FUNCS)}, got {score_func!r}")
    return SCORE_FUNCS[score_func]


def make_desc(*, tokens: int, hidden: int, n_experts: int, top_k: int, inter: int = 32,
              inter_shared: int = 0, score_func: str | int = "sigmoid", quant: str = "fp4",
              x_dtype: torch.dtype = torch.bfloat16, gate_dtype: torch.dtype = torch.float32,
              route_scale: float = 2.5, limit: float = 10.0) -> _lib.Desc:
    return _lib.Desc(tokens, hidden, n_experts, top_k, inter, inter_shared,
                     score_code(score_func), QUANTS[quant], dtype_code(x_dtype, "x"),
                     dtype_code(gate_dtype, "gate_w"), float(route_scale), float(limit))


def workspace_size(desc: _lib.Desc) -> int:
    n = ctypes.c_size_t(0)
    _lib.call("dsk_workspace_size", ctypes.byref(desc), ctypes.byref(n))
    return int(n.value)


_WS_CACHE: dict[tuple, torch.Tensor] = {}
# Workspaces a HIP graph captured: a graph replays raw pointers, so a captured
# workspace is never handed back to the allocator, even after a larger one
# replaced it in the cache.
_WS_CAPTURED: dict[int, torch.Tensor] = {}


def new_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """A zero-initialised device workspace of ``nbytes`` (at least 256) bytes."""
    ws = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)
    _lib.call("dsk_workspace_init", ptr(ws), ws.numel(), stream_of(device))
    return ws


def workspace(desc: _lib.Desc, device: torch.device) -> torch.Tensor:
    """A cached, zero-initialised device workspace of at least ``workspace_size(desc)`` bytes.

    One workspace per (device, stream): calls on one stream are ordered, so they
    may share it; calls on different streams get different workspaces.  A
    workspace used while the stream is being captured into a HIP graph stays
    allocated for the life of the process.
    """
    need = workspace_size(desc)
    stream = torch.cuda.current_stream(device)
    key = (device.type, device.index, stream.cuda_stream)
    ws = _WS_CACHE.get(key)
    capturing = torch.cuda.is_current_stream_capturing()
    if ws is None or ws.numel() < need:
        if capturing:
            # its zero-fill would only be recorded into the graph, and eager calls
            # that reuse the cached workspace would find its counters undefined
            raise RuntimeError("dsk_moe: no workspace of this size exists for the capturing stream; "
                               "run the call once eagerly on that stream first, or pass a workspace "
                               "made with ops.new_workspace")
        ws = new_workspace(need, device)
        _WS_CACHE[key] = ws
    if capturing:
        _WS_CAPTURED[ws.data_ptr()] = ws
    return ws


def route(x: torch.Tensor, gate_w: torch.Tensor, gate_b: torch.Tensor, top_k: int,
          score_func: str | int = "sigmoid", route_scale: float = 2.5):
    """(weights [T,k] f32, idx [T,k] i32, scores [T,E] f32) -- the router of ``dsk_route``."""
    dev = require_device(x, gate_w, gate_b)
    if gate_b.dtype != torch.float32:
        raise ValueError("gate_b must be float32")
    t, h = x.shape
    e = gate_w.shape[0]
    if gate_w.shape != (e, h) or gate_b.shape != (e,):
        raise ValueError(f"gate shapes {tuple(gate_w.shape)}, {tuple(gate_b.shape)} do not fit x {tuple(x.shape)}")
    desc = make_desc(tokens=t, hidden=h, n_experts=e, top_k=top_k, score_func=score_func,
                     x_dtype=x.dtype, gate_dtype=gate_w.dtype, route_scale=route_scale)
    scores = torch.empty((t, e), dtype=torch.float32, device=dev)
    idx = torch.empty((t, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((t, top_k), dtype=torch.float32, device=dev)
    _lib.call("dsk_route", ctypes.byref(desc), ptr(x), ptr(gate_w), ptr(gate_b), ptr(scores),
              ptr(idx), ptr(w), stream_of(dev))
    return w, idx, scores


def cap_union(scores: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, budget: int,
              strict: bool = False) -> None:
    """``dsk_cap_union`` in place on a lock-step batch's routing (the reference's
    ``cap_union``, ``src/deepseeker/mlx_forward.py:213-254``): scores [T, E] f32
    (un-biased), idx [T, k] int32 and w [T, k] f32 in this library's order."""
    dev = require_device(scores, idx, w)
    if scores.dtype != torch.float32 or idx.dtype != torch.int32 or w.dtype != torch.float32:
        raise ValueError("scores and w must be float32, idx int32")
    t, k = idx.shape
    if w.shape != idx.shape or scores.dim() != 2 or scores.shape[0] != t:
        raise ValueError("scores [T, E], idx and w [T, k] must agree")
    _lib.call("dsk_cap_union", t, scores.shape[1], k, int(budget), 1 if strict else 0, ptr(scores), ptr(idx),
              ptr(w), stream_of(dev))


def dispatch(idx: torch.Tensor, n_experts: int, multi_block: bool = False) -> dict:
    """counts, offsets, perm, rank, active of ``dsk_dispatch`` for idx [T,k] int32;
    ``multi_block``: ``dsk_dispatch_ws`` (the forward call's own dispatch, several
    workgroups from 8192 positions), same outputs."""
    dev = require_device(idx)
    if idx.dtype != torch.int32 or idx.dim() != 2:
        raise ValueError("idx must be a 2-D int32 tensor")
    t, k = idx.shape
    desc = make_desc(tokens=t, hidden=32, n_experts=n_experts, top_k=k)
    n = t * k
    out = {"counts": torch.empty(n_experts, dtype=torch.int32, device=dev),
           "offsets": torch.empty(n_experts + 1, dtype=torch.int32, device=dev),
           "perm": torch.empty(n, dtype=torch.int32, device=dev),
           "rank": torch.empty(n, dtype=torch.int32, device=dev),
           "active": torch.empty(n_experts + 1, dtype=torch.int32, device=dev)}
    if multi_block:
        nb = ctypes.c_size_t()
        _lib.call("dsk_dispatch_workspace_size", ctypes.byref(desc), ctypes.byref(nb))
        ws = torch.empty(max(nb.value, 1), dtype=torch.uint8, device=dev)
        _lib.call("dsk_dispatch_ws", ctypes.byref(desc), ptr(idx), ptr(out["counts"]),
                  ptr(out["offsets"]), ptr(out["perm"]), ptr(out["rank"]), ptr(out["active"]),
                  ptr(ws), nb.value, stream_of(dev))
        return out
    _lib.call("dsk_dispatch", ctypes.byref(desc), ptr(idx), ptr(out["counts"]),
              ptr(out["offsets"]), ptr(out["perm"]), ptr(out["rank"]), ptr(out["active"]),
              stream_of(dev))
    return out


def align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int):
    """The ``moe_align_block_size`` contract (reference ``src/deepseeker/moe_align.py:21-46``)
    built on the GPU dispatch: (sorted_ids, expert_ids, num_tokens_post_pad)."""
    if topk_ids.dim() != 2:
        raise ValueError(f"topk_ids must be 2-D, got shape {tuple(topk_ids.shape)}")
    if block_size < 1 or num_experts < 1:
        raise ValueError("block_size and num_experts must be >= 1")
    ids = topk_ids.to(torch.int32).contiguous()
    n = ids.numel()
    if n and (int(ids.min()) < 0 or int(ids.max()) >= num_experts):
        raise ValueError("expert ids out of range")
    d = dispatch(ids, num_experts)
    counts = d["counts"].to(torch.int64)
    padded = (counts + block_size - 1) // block_size * block_size
    pad_off = torch.zeros(num_experts + 1, dtype=torch.int64, device=ids.device)
    pad_off[1:] = torch.cumsum(padded, 0)
    total = int(pad_off[-1])
    sorted_ids = torch.full((total,), n, dtype=torch.int64, device=ids.device)
    if n:
        rows = torch.arange(n, device=ids.device)
        expert_of_row = torch.repeat_interleave(torch.arange(num_experts, device=ids.device), counts)
        dst = pad_off[:-1][expert_of_row] + (rows - d["offsets"][:-1].to(torch.int64)[expert_of_row])
        sorted_ids[dst] = d["perm"].to(torch.int64)
    expert_ids = torch.repeat_interleave(torch.arange(num_experts, device=ids.device),
                                         padded // block_size)
    return sorted_ids, expert_ids, total


def fp4_dequant(packed: torch.Tensor, scales: torch.Tensor, out_dtype=torch.float32) -> torch.Tensor:
    dev = require_device(packed, scales)
    cols = packed.shape[-1] * 2
    lead = packed.shape[:-1]
    rows = packed.numel() // packed.shape[-1]
    if scales.numel() * 32 != packed.numel() * 2:
        raise ValueError("scales must hold one byte per 32 codes")
    out = torch.empty(lead + (cols,), dtype=out_dtype, device=dev)
    _lib.call("dsk_fp4_dequant", ptr(packed), ptr(scales), rows, cols, ptr(out),
              dtype_code(out_dtype, "out"), stream_of(dev))
    return out


def fp4_quantize(w: torch.Tensor):
    dev = require_device(w)
    if w.dtype != torch.float32:
        raise ValueError("fp4_quantize takes float32 weights")
    cols = w.shape[-1]
    rows = w.numel() // cols
    packed = torch.empty(w.shape[:-1] + (cols // 2,), dtype=torch.uint8, device=dev)
    scales = torch.empty(w.shape[:-1] + (cols // 32,), dtype=torch.uint8, device=dev)
    _lib.call("dsk_fp4_quantize", ptr(w), rows, cols, ptr(packed), ptr(scales), stream_of(dev))
    return packed, scales


def q3_quantize(w: torch.Tensor):
    dev = require_device(w)
    if w.dtype != torch.float32:
        raise ValueError("q3_quantize takes float32 weights")
    cols = w.shape[-1]
    rows = w.numel() // cols
    packed = torch.empty(w.shape[:-1] + (cols * 3 // 8,), dtype=torch.uint8, device=dev)
    scales = torch.empty(w.shape[:-1] + (cols // 64,), dtype=torch.float16, device=dev)
    biases = torch.empty_like(scales)
    _lib.call("dsk_q3_quantize", ptr(w), rows, cols, ptr(packed), ptr(scales), ptr(biases),
              stream_of(dev))
    return packed, scales, biases


def q3_repack(rowmajor: torch.Tensor) -> torch.Tensor:
    """Checkpoint q3 codes (row-major 3-byte packs, ``[..., 3K/8]`` u8 or ``[..., 3K/32]``
    int32 / uint32 words) -> the canonical kernel layout ``[..., 3K/8]`` u8 (``dsk_q3_repack``)."""
    dev = require_device(rowmajor)
    raw = rowmajor.view(torch.uint8) if rowmajor.dtype != torch.uint8 else rowmajor
    raw = raw.reshape(rowmajor.shape[:-1] + (-1,))
    cols = raw.shape[-1] * 8 // 3
    if raw.shape[-1] * 8 != cols * 3 or cols % 128:
        raise ValueError(f"q3 rows of {raw.shape[-1]} bytes do not hold a multiple of 128 codes")
    rows = raw.numel() // raw.shape[-1]
    out = torch.empty_like(raw)
    _lib.call("dsk_q3_repack", ptr(raw), rows, cols, ptr(out), stream_of(dev))
    return out


def q3_dequant(packed: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               out_dtype=torch.float32) -> torch.Tensor:
    dev = require_device(packed, scales, biases)
    cols = scales.shape[-1] * 64
    rows = scales.numel() // scales.shape[-1]
    if packed.numel() != rows * cols * 3 // 8:
        raise ValueError("packed size does not match scales")
    out = torch.empty(scales.shape[:-1] + (cols,), dtype=out_dtype, device=dev)
    _lib.call("dsk_q3_dequant", ptr(packed), ptr(scales), ptr(biases), rows, cols, ptr(out),
              dtype_code(out_dtype, "out"), stream_of(dev))
    return out
