"""Resident expert banks: all routed experts of a layer stacked in HBM.

The reference keeps pinned experts as stacked banks ``[E_pinned, N, ...]``
(``src/deepseeker/mlx_weights.py:576-649``) and otherwise streams experts
from SSD through an LRU.  On one MI355X every expert of every layer fits in
HBM, so a layer's routed experts live in one ``ResidentBank`` with the same
per-role layout, stacked over all E experts:

* FP4: ``w1, w3 [E, I, H/2] u8`` + ``s1, s3 [E, I, H/32] u8``,
  ``w2 [E, H, I/2] u8`` + ``s2 [E, H, I/32] u8``
* Q3:  ``w* [E, N, 3K/8] u8`` + ``s*, b* [E, N, K/64] f16``

``table`` is the device array of ``dsk_expert_ptrs`` the kernels index by
expert id, built once.  A bank is also callable as the reference's
``expert_fn(e) -> (w1, w3, w2)`` (``src/deepseeker/mlx_runner.py:681-710``),
returning views.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .ops import require_device


class ResidentBank:
    """All routed experts of one layer, resident on one device."""

    def __init__(self, quant: str, roles: dict):
        if quant not in ("fp4", "q3"):
            raise ValueError(f"quant must be 'fp4' or 'q3', got {quant!r}")
        self.quant = quant
        self.roles = {r: tuple(roles[r]) for r in ("w1", "w3", "w2")}
        arity = 2 if quant == "fp4" else 3
        flat = [t for r in ("w1", "w3", "w2") for t in self.roles[r]]
        if any(len(self.roles[r]) != arity for r in self.roles):
            raise ValueError(f"{quant} roles need {arity} tensors each")
        self.device = require_device(*flat)
        w1 = self.roles["w1"][0]
        w2 = self.roles["w2"][0]
        self.n_experts = w1.shape[0]
        self.inter = w1.shape[1]
        self.hidden = w2.shape[1]
        h, i = self.hidden, self.inter
        if quant == "fp4":
            want = {"w1": ((i, h // 2), (i, h // 32)), "w3": ((i, h // 2), (i, h // 32)),
                    "w2": ((h, i // 2), (h, i // 32))}
            dtypes = (torch.uint8, torch.uint8)
        else:
            want = {"w1": ((i, h * 3 // 8), (i, h // 64), (i, h // 64)),
                    "w3": ((i, h * 3 // 8), (i, h // 64), (i, h // 64)),
                    "w2": ((h, i * 3 // 8), (h, i // 64), (h, i // 64))}
            dtypes = (torch.uint8, torch.float16, torch.float16)
        for r, shapes in want.items():
            for t, shp, dt in zip(self.roles[r], shapes, dtypes):
                if tuple(t.shape) != (self.n_experts,) + shp or t.dtype != dt:
                    raise ValueError(f"role {r}: got {tuple(t.shape)} {t.dtype}, "
                                     f"want {(self.n_experts,) + shp} {dt}")
        self.table = self._build_table()

    @classmethod
    def fp4(cls, w1, s1, w3, s3, w2, s2) -> "ResidentBank":
        return cls("fp4", {"w1": (w1, s1), "w3": (w3, s3), "w2": (w2, s2)})

    @classmethod
    def q3(cls, w1, s1, b1, w3, s3, b3, w2, s2, b2) -> "ResidentBank":
        return cls("q3", {"w1": (w1, s1, b1), "w3": (w3, s3, b3), "w2": (w2, s2, b2)})

    def _build_table(self) -> torch.Tensor:
        entries = (_lib.ExpertPtrs * self.n_experts)()
        for e in range(self.n_experts):
            vals = []
            for r in ("w1", "w3", "w2"):
                parts = self.roles[r]
                for c in range(3):
                    if c < len(parts):
                        t = parts[c]
                        vals.append(t.data_ptr() + e * t.stride(0) * t.element_size())
                    else:
                        vals.append(None)
            entries[e] = _lib.ExpertPtrs(*vals)
        raw = torch.frombuffer(bytearray(bytes(entries)), dtype=torch.uint8)
        return raw.to(self.device)

    def __call__(self, e: int):
        return tuple(tuple(t[e] for t in self.roles[r]) for r in ("w1", "w3", "w2"))

    def nbytes_per_expert(self) -> int:
        return sum(t[0].numel() * t.element_size() for r in self.roles.values() for t in r)


class SharedExpert:
    """The shared expert with bf16 weights ``w1, w3 [Is, H]`` and ``w2 [H, Is]``.

    Passed as ``shared_fn`` it is fused into the expert kernels; called
    directly it evaluates the reference's ``_shared_fn`` semantics
    (``src/deepseeker/mlx_runner.py:765-783``) with torch on the device:
    float32 projections, clamped SwiGLU, output cast to x's dtype.
    """

    def __init__(self, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor, limit: float = 10.0):
        self.device = require_device(w1, w3, w2)
        for t in (w1, w3, w2):
            if t.dtype != torch.bfloat16:
                raise ValueError("shared expert weights must be bfloat16")
        self.inter = w1.shape[0]
        self.hidden = w1.shape[1]
        if w3.shape != w1.shape or tuple(w2.shape) != (self.hidden, self.inter):
            raise ValueError("shared expert shapes must be w1, w3 [Is, H] and w2 [H, Is]")
        self.w1, self.w3, self.w2 = w1, w3, w2
        self.limit = float(limit)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        g = torch.clamp(xf @ self.w1.float().T, max=self.limit)
        u = torch.clamp(xf @ self.w3.float().T, -self.limit, self.limit)
        h = g / (1.0 + torch.exp(-g)) * u
        return (h @ self.w2.float().T).to(x.dtype)
