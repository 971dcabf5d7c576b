"""Pinned-expert contributions on the device.

The reference's runner keeps its pinned experts as stacked banks and computes
their share of a layer with ``gather_pinned_contributions``
(``src/deepseeker/mlx_forward.py:159-210``, called by the runner's
``expert_pin_gather`` hook, ``src/deepseeker/mlx_runner.py:949-960``): every
(row, slot) pair routed to a pinned expert becomes one weighted output row
``w2(silu(min(x w1, L)) * clip(x w3, -L, L) * weight)`` in float32, the pairs
ordered by (expert, row), and the result is ``{expert: (rows, contrib)}``.
``moe_layer(pinned_gather_fn=...)`` then adds those rows in the expert's place
of the ascending-expert sum (``:388-393``).

Here the same products run through ``dsk_expert_rows``: the pairs are
dispatched like any routing (expert ascending, then flat position, which is
the reference's pair order) and the expert kernels write each pair's row
instead of combining them.  The activations enter in float32, as the
reference's ``routed_x = x[rows].astype(float32)``.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .bank import ResidentBank
from .ops import dispatch, make_desc, ptr, require_device, stream_of, workspace

_ENTRY = ctypes.sizeof(_lib.ExpertPtrs)


def expert_rows(x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, table: torch.Tensor,
                n_experts: int, quant: str, inter: int, *, limit: float = 10.0):
    """``dsk_expert_rows``: the weighted output row of every pair of ``idx`` in [0, E).

    ``x [T, H]`` (taken in float32), ``idx [T, k]`` int32 and ``w [T, k]``
    float32 on the device, ``table`` the device ``dsk_expert_ptrs[n_experts]``.
    Returns ``(rows [n, H] float32, counts [E] int32 on the host)`` with the
    pairs in dispatch order: expert ascending, then flat position ascending."""
    dev = require_device(x, idx, w, table)
    t, h = x.shape
    if idx.dtype != torch.int32 or w.dtype != torch.float32 or idx.shape != w.shape or idx.shape[0] != t:
        raise ValueError("idx must be int32 [T, k] and w float32 [T, k], with T = x.shape[0]")
    k = idx.shape[1]
    x32 = x.to(torch.float32).contiguous()
    desc = make_desc(tokens=t, hidden=h, n_experts=n_experts, top_k=k, inter=inter, inter_shared=0,
                     quant=quant, x_dtype=torch.float32, limit=limit)
    d = dispatch(idx.contiguous(), n_experts)
    rows = torch.empty((t * k, h), dtype=torch.float32, device=dev)
    ws = workspace(desc, dev)
    _lib.call("dsk_expert_rows", ctypes.byref(desc), ptr(table), ptr(x32), ptr(w.contiguous()),
              ptr(d["counts"]), ptr(d["offsets"]), ptr(d["perm"]), ptr(d["rank"]), ptr(d["active"]),
              ptr(rows), ptr(ws), ws.numel(), stream_of(dev))
    counts = d["counts"].cpu().numpy()       # synchronises: d's buffers are referenced by raw pointer
    n = int(counts.sum())
    return rows[:n], counts


def _as_bank(banks) -> ResidentBank:
    if isinstance(banks, ResidentBank):
        return banks
    roles = {r: tuple(banks[r]) for r in ("w1", "w3", "w2")}
    quant = "fp4" if len(roles["w1"]) == 2 else "q3"
    return ResidentBank(quant, roles)


def gather_pinned_contributions(x: torch.Tensor, indices, weights, banks, slots: dict,
                                limit: float = 10.0) -> dict:
    """Device twin of the reference's ``gather_pinned_contributions``.

    ``x [T, H]`` on the device; ``indices`` / ``weights`` ``[T, k]`` routing in
    any slot order (host arrays or tensors; the reference passes its ascending-key
    order); ``banks`` a ``ResidentBank`` of the pinned experts stacked by slot,
    or the reference's ``{"w1": parts, "w3": parts, "w2": parts}`` with FP4 pairs
    or q3 triples stacked by slot; ``slots`` ``{expert: bank slot}``.
    Returns ``{expert: (rows int32, contrib [len(rows), H] float32 on the
    device)}`` for the pinned experts that receive a pair, rows ascending."""
    if not slots:
        return {}
    bank = _as_bank(banks)
    dev = require_device(x)
    ind = np.ascontiguousarray(indices.cpu() if isinstance(indices, torch.Tensor) else indices, dtype=np.int64)
    wts = np.ascontiguousarray(weights.cpu() if isinstance(weights, torch.Tensor) else weights, dtype=np.float32)
    if ind.ndim != 2 or wts.shape != ind.shape or ind.shape[0] != x.shape[0]:
        raise ValueError("indices and weights must be [T, k] with T = x.shape[0]")
    experts = sorted(int(e) for e in slots)
    slot_ids = [int(slots[e]) for e in experts]
    if min(slot_ids) < 0 or max(slot_ids) >= bank.n_experts:
        raise ValueError(f"slots must lie in [0, {bank.n_experts})")
    local = np.full(ind.shape, -1, dtype=np.int32)
    for i, e in enumerate(experts):
        local[ind == e] = i
    if (local < 0).all():
        return {}
    # the pinned experts' pointer entries in ascending expert order
    sel = torch.as_tensor(slot_ids, dtype=torch.int64, device=dev)
    table = bank.table.view(bank.n_experts, _ENTRY).index_select(0, sel).contiguous().view(-1)
    rows, counts = expert_rows(x, torch.from_numpy(local).to(dev), torch.from_numpy(wts).to(dev), table,
                               len(experts), bank.quant, bank.inter, limit=limit)
    out, off = {}, 0
    for i, e in enumerate(experts):
        n = int(counts[i])
        if n:
            r = np.nonzero((local == i).any(axis=1))[0].astype(np.int32)
            assert r.size == n
            out[e] = (r, rows[off:off + n])
        off += n
    return out
