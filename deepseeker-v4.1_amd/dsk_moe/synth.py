"""Seeded synthetic MoE layers generated directly on the GPU.

Full-size layers (256 experts of 4096 x 2048 in three roles, ~3.4 GB of FP4
per layer, ~110 GB for a 40-layer stack) are drawn and quantised on the
device: float32 N(0, 0.02) weights one expert role at a time, quantised in
place into the resident bank by ``dsk_fp4_quantize`` / ``dsk_q3_quantize``.
Draw order per layer (one device ``torch.Generator`` seeded with ``seed``):
gate ``[E, H]`` N(0,1)/sqrt(H); bias ``[E]`` U(-0.1, 0.1) (or the log of a
Zipf(s) popularity, no draw); per expert w1 ``[I, H]``, w3 ``[I, H]``,
w2 ``[H, I]``; shared w1, w3 ``[Is, H]``, w2 ``[H, Is]`` (bf16); the caller
draws x.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import _lib
from .bank import ResidentBank, SharedExpert
from .layer import MoELayer
from .ops import ptr, stream_of


def zipf_bias(n_experts: int, s: float) -> torch.Tensor:
    """log of a Zipf(s) popularity over experts (p_e proportional to (e+1)^-s)."""
    p = np.arange(1, n_experts + 1, dtype=np.float64) ** (-s)
    p /= p.sum()
    return torch.from_numpy(np.log(p).astype(np.float32))


def _alloc_bank(quant: str, E: int, H: int, I: int, device) -> dict:
    def fp4(n, k):
        return (torch.empty((E, n, k // 2), dtype=torch.uint8, device=device),
                torch.empty((E, n, k // 32), dtype=torch.uint8, device=device))

    def q3(n, k):
        return (torch.empty((E, n, k * 3 // 8), dtype=torch.uint8, device=device),
                torch.empty((E, n, k // 64), dtype=torch.float16, device=device),
                torch.empty((E, n, k // 64), dtype=torch.float16, device=device))

    make = fp4 if quant == "fp4" else q3
    return {"w1": make(I, H), "w3": make(I, H), "w2": make(H, I)}


def _quantize_into(w: torch.Tensor, parts: tuple, e: int, quant: str) -> None:
    rows, cols = w.shape
    dev = w.device
    if quant == "fp4":
        _lib.call("dsk_fp4_quantize", ptr(w), rows, cols, ctypes.c_void_p(parts[0][e].data_ptr()),
                  ctypes.c_void_p(parts[1][e].data_ptr()), stream_of(dev))
    else:
        _lib.call("dsk_q3_quantize", ptr(w), rows, cols, ctypes.c_void_p(parts[0][e].data_ptr()),
                  ctypes.c_void_p(parts[1][e].data_ptr()), ctypes.c_void_p(parts[2][e].data_ptr()),
                  stream_of(dev))


def make_layer(*, hidden: int, n_experts: int, top_k: int, inter: int, inter_shared: int,
               quant: str = "fp4", seed: int = 0, device="cuda", zipf_s: float | None = None,
               score_func: str = "sigmoid", route_scale: float = 2.5,
               limit: float = 10.0) -> MoELayer:
    """A resident ``MoELayer`` drawn from ``seed`` on ``device``."""
    device = torch.device(device)
    g = torch.Generator(device=device).manual_seed(seed)
    H, E, I = hidden, n_experts, inter
    gate_w = torch.randn((E, H), generator=g, device=device) * (1.0 / math.sqrt(H))
    if zipf_s is None:
        gate_b = torch.rand((E,), generator=g, device=device) * 0.2 - 0.1
    else:
        gate_b = zipf_bias(E, zipf_s).to(device)
    roles = _alloc_bank(quant, E, H, I, device)
    for e in range(E):
        for role, shape in (("w1", (I, H)), ("w3", (I, H)), ("w2", (H, I))):
            w = torch.randn(shape, generator=g, device=device) * 0.02
            _quantize_into(w, roles[role], e, quant)
    bank = ResidentBank(quant, roles)
    shared = None
    if inter_shared:
        sw = [(torch.randn(shape, generator=g, device=device) * 0.02).to(torch.bfloat16)
              for shape in ((inter_shared, H), (inter_shared, H), (H, inter_shared))]
        shared = SharedExpert(*sw, limit=limit)
    return MoELayer(gate_w.contiguous(), gate_b, bank, shared, top_k, score_func=score_func,
                    route_scale=route_scale, limit=limit)
