"""The MoE layer forward restated on the CPU: torch fp32 GEMMs, numpy routing.

Follows the reference's ``moe_layer`` (``src/deepseeker/mlx_forward.py:257-419``)
on the resident-expert path (no prefetch, no pipeline, no union cap):

* route (``:290-291``, see ``oracle.router``), then group per unique expert
  in ascending id (``:294-312, 388-396``, see ``oracle.dispatch``);
* shared expert (``src/deepseeker/mlx_runner.py:765-783``): float32
  ``g = min(x W1^T, L)``, ``u = clip(x W3^T, -L, L)``,
  ``h = g / (1 + exp(-g)) * u``, ``ys = h W2^T``, rounded to x.dtype before
  it is added (``mlx_forward.py:309-310, 409-410``);
* per expert (``:388-406``): the same clamped SwiGLU on the expert's rows,
  the route weight multiplies ``h`` *before* the ``w2`` projection, and the
  result is scatter-added into a float32 accumulator in ascending expert id;
* ``out = (acc + f32(ys))`` cast to x.dtype (``:409-419``).

Expert weights are dequantised lazily, only for selected experts.
Parity: pinned by ``moe_forward_f64`` (float64 brute force written
independently with explicit loops) on small shapes, and by the invariants of
the reference tests (``tests/test_mlx_forward.py:241-353``,
``tests/test_grouped.py:42-59``) restated in ``tests/test_oracle.py``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import dispatch as D
from . import formats as F
from . import router as R

QUANT_FP4 = "fp4"
QUANT_Q3 = "q3"


@dataclass
class LayerSpec:
    H: int
    E: int
    k: int
    I: int
    I_shared: int = 0
    score_func: int = R.SCORE_SIGMOID
    route_scale: float = 2.5
    limit: float = 10.0
    quant: str = QUANT_FP4


@dataclass
class ExpertBank:
    """Routed experts of one layer in the reference's stacked bank layout.

    fp4: ``roles[r] = (packed [E, N, K/2] u8, scales [E, N, K/32] u8)``;
    q3:  ``roles[r] = (codes [E, N, 3K/8] u8, scales [E, N, K/64] f16, biases [E, N, K/64] f16)``;
    r in ("w1", "w3", "w2"), with w1, w3: [I, H] and w2: [H, I] (used as x @ W^T).
    """

    quant: str
    roles: dict
    _cache: dict = field(default_factory=dict, repr=False)

    def dequant(self, e: int, role: str) -> np.ndarray:
        key = (int(e), role)
        hit = self._cache.get(key)
        if hit is None:
            parts = [a[e] for a in self.roles[role]]
            if self.quant == QUANT_FP4:
                hit = F.fp4_dequant(*parts)
            else:
                hit = F.q3_dequant(*parts)
            self._cache[key] = hit
        return hit

    def clear_cache(self) -> None:
        self._cache.clear()


def _as_f32_torch(a) -> torch.Tensor:
    if isinstance(a, torch.Tensor):
        return a.detach().to("cpu", torch.float32)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def swiglu(g: torch.Tensor, u: torch.Tensor, limit: float) -> torch.Tensor:
    """Clamped SwiGLU of the reference: g = min(g, L), u = clip(u, -L, L), g / (1 + e^-g) * u."""
    g = torch.clamp(g, max=limit)
    u = torch.clamp(u, -limit, limit)
    return g / (1.0 + torch.exp(-g)) * u


def shared_forward(x32: torch.Tensor, ws1, ws3, ws2, limit: float) -> torch.Tensor:
    """float32 shared-expert output [T, H] (not yet rounded)."""
    w1 = _as_f32_torch(ws1)
    w3 = _as_f32_torch(ws3)
    w2 = _as_f32_torch(ws2)
    h = swiglu(x32 @ w1.T, x32 @ w3.T, limit)
    return h @ w2.T


def moe_forward(x, gate_w, gate_b, bank: ExpertBank, shared, spec: LayerSpec,
                routing: tuple | None = None, pinned: dict | None = None) -> dict:
    """Whole layer.  ``x``: torch [T, H] bf16 or float32 (CPU); ``shared`` is
    ``(ws1, ws3, ws2)`` bf16 tensors or None.  Returns a dict with ``out``
    (x.dtype), ``y_ref`` (float32 before the final cast), ``idx``, ``w``,
    ``scores``, ``counts``, ``offsets``, ``perm``, ``rank``.
    ``routing``: the ``(idx, w, scores, logits)`` of ``router.route`` on these
    inputs when the caller already has it (it is not recomputed).
    ``pinned``: ``{expert: (rows, contrib)}`` as a pinned-gather callback returns
    it (src/deepseeker/mlx_forward.py:313-321): a selected expert found there
    adds ``contrib`` [len(rows), H] (float32, already weighted) at ``rows`` in
    its place in the ascending-expert sum instead of being computed
    (:388-393); entries of experts that were not selected are ignored.
    """
    xt = x.detach().to("cpu")
    x32 = xt.to(torch.float32)
    if routing is None:
        routing = R.route(x32.numpy(), _as_f32_torch(gate_w).numpy(), _as_f32_torch(gate_b).numpy(),
                          spec.k, spec.score_func, spec.route_scale)
    idx, w, s, _ = routing
    counts, offsets, perm, rank = D.dispatch(idx, spec.E)
    t = x32.shape[0]
    acc = torch.zeros((t, spec.H), dtype=torch.float32)
    wt = torch.from_numpy(w)
    for e in D.active_experts(counts):
        if pinned is not None and int(e) in pinned:
            prow, contrib = pinned[int(e)]
            acc.index_add_(0, torch.as_tensor(np.asarray(prow), dtype=torch.int64),
                           torch.as_tensor(contrib, dtype=torch.float32))
            continue
        pos = perm[offsets[e]:offsets[e + 1]].astype(np.int64)
        rows = torch.from_numpy(pos // spec.k)
        cols = torch.from_numpy(pos % spec.k)
        xr = x32[rows]
        w1 = torch.from_numpy(bank.dequant(e, "w1"))
        w3 = torch.from_numpy(bank.dequant(e, "w3"))
        w2 = torch.from_numpy(bank.dequant(e, "w2"))
        h = swiglu(xr @ w1.T, xr @ w3.T, spec.limit)
        h = h * wt[rows, cols].reshape(-1, 1)
        acc.index_add_(0, rows, h @ w2.T)
    if shared is not None:
        ys = shared_forward(x32, *shared, spec.limit).to(xt.dtype).to(torch.float32)
        y_ref = acc + ys
    else:
        y_ref = acc
    return {"out": y_ref.to(xt.dtype), "y_ref": y_ref, "idx": idx, "w": w,
            "scores": s, "counts": counts, "offsets": offsets, "perm": perm,
            "rank": rank}


def moe_forward_f64(x, idx, w, bank: ExpertBank, shared, spec: LayerSpec) -> np.ndarray:
    """Brute-force float64 layer on given routing, explicit loops (small shapes only).

    Independent restatement used to pin ``moe_forward``'s expert math: every
    (token, slot) pair is evaluated on its own, in float64, and summed in
    ascending expert order; the shared output is rounded to x.dtype first.
    """
    xt = x.detach().to("cpu")
    xd = xt.to(torch.float64).numpy()
    t, hdim = xd.shape
    out = np.zeros((t, hdim), dtype=np.float64)
    lim = spec.limit
    for tok in range(t):
        pairs = sorted((int(idx[tok, j]), j) for j in range(idx.shape[1]) if idx[tok, j] >= 0)
        for e, j in pairs:
            w1 = bank.dequant(e, "w1").astype(np.float64)
            w3 = bank.dequant(e, "w3").astype(np.float64)
            w2 = bank.dequant(e, "w2").astype(np.float64)
            hid = np.zeros(spec.I)
            for i in range(spec.I):
                g = min(float(np.dot(w1[i], xd[tok])), lim)
                u = min(max(float(np.dot(w3[i], xd[tok])), -lim), lim)
                hid[i] = g / (1.0 + np.exp(-g)) * u * float(w[tok, j])
            out[tok] += w2 @ hid
    if shared is not None:
        s1, s3, s2 = (_as_f32_torch(a).numpy().astype(np.float64) for a in shared)
        g = np.minimum(xd @ s1.T, lim)
        u = np.clip(xd @ s3.T, -lim, lim)
        ys = (g / (1.0 + np.exp(-g)) * u) @ s2.T
        ys = torch.from_numpy(ys).to(xt.dtype).to(torch.float64).numpy()
        out = out + ys
    return out
