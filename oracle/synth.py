"""Seeded synthetic MoE layers on the CPU (small shapes; parity fixtures).

Draw order from one ``torch.Generator`` seeded with ``seed`` (CPU stream):

1. gate weight ``[E, H]`` ~ N(0, 1) * (1 / sqrt(H))   (float32)
2. gate bias ``[E]`` ~ U(-0.1, 0.1)                   (float32), or the
   Zipf(s) log-popularity ``log((e+1)^-s / sum)`` when ``zipf_s`` is given
   (no draw is consumed then)
3. for e in 0..E-1: w1 ``[I, H]``, w3 ``[I, H]``, w2 ``[H, I]`` ~ N(0, 1) * 0.02,
   quantised to FP4 (e2m1/E8M0) or q3 affine g64
4. shared w1 ``[Is, H]``, w3 ``[Is, H]``, w2 ``[H, Is]`` ~ N(0, 1) * 0.02 -> bf16
5. x ``[T, H]`` ~ N(0, 1) -> bf16

This is the workload spec's recipe for the small configuration (hidden 1024,
64 experts, top-6, intermediate 512, one shared expert of 512, seed 0) and
for the tiny test shapes.  Full-size layers are generated on the GPU by the
product package with the same order and distributions (its own RNG stream).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import formats as F
from .layer import QUANT_FP4, ExpertBank, LayerSpec


def zipf_bias(n_experts: int, s: float) -> np.ndarray:
    """log of a Zipf(s) popularity over experts: log(p_e), p_e proportional to (e+1)^-s."""
    ranks = np.arange(1, n_experts + 1, dtype=np.float64)
    p = ranks ** (-s)
    p /= p.sum()
    return np.log(p).astype(np.float32)


def quantize_role(w: np.ndarray, quant: str):
    if quant == QUANT_FP4:
        return F.fp4_quantize(w)
    return F.q3_quantize(w)


def make_layer(spec: LayerSpec, seed: int, tokens: int, zipf_s: float | None = None) -> dict:
    """Returns dict(x, gate_w, gate_b, bank, shared) on the CPU."""
    g = torch.Generator().manual_seed(seed)
    h, e, i = spec.H, spec.E, spec.I
    gate_w = (torch.randn((e, h), generator=g) * (1.0 / math.sqrt(h))).to(torch.float32)
    if zipf_s is None:
        gate_b = (torch.rand((e,), generator=g) * 0.2 - 0.1).to(torch.float32)
    else:
        gate_b = torch.from_numpy(zipf_bias(e, zipf_s))
    per_role: dict[str, list] = {"w1": [], "w3": [], "w2": []}
    for _ in range(e):
        for role, shape in (("w1", (i, h)), ("w3", (i, h)), ("w2", (h, i))):
            w = (torch.randn(shape, generator=g) * 0.02).numpy()
            per_role[role].append(quantize_role(w, spec.quant))
    roles = {r: tuple(np.stack([p[c] for p in parts]) for c in range(len(parts[0])))
             for r, parts in per_role.items()}
    shared = None
    if spec.I_shared:
        si = spec.I_shared
        shared = tuple((torch.randn(shape, generator=g) * 0.02).to(torch.bfloat16)
                       for shape in ((si, h), (si, h), (h, si)))
    x = torch.randn((tokens, h), generator=g).to(torch.bfloat16)
    return {"x": x, "gate_w": gate_w, "gate_b": gate_b,
            "bank": ExpertBank(spec.quant, roles), "shared": shared}


def config0_spec() -> LayerSpec:
    """Small layer: hidden 1024, 64 experts, top-6, intermediate 512, shared 512, FP4, sigmoid, 2.5."""
    return LayerSpec(H=1024, E=64, k=6, I=512, I_shared=512)


def tiny_spec(quant: str = QUANT_FP4) -> LayerSpec:
    """Reference-test-sized layer (``tests/test_mlx_forward.py`` uses dim 64, mid 32, E 8)."""
    if quant == QUANT_FP4:
        return LayerSpec(H=64, E=8, k=2, I=32, I_shared=32)
    return LayerSpec(H=128, E=8, k=2, I=128, I_shared=128, quant=quant)
