"""Drop-in MoE layer forward with the reference's call signature.

``moe_layer`` keeps the signature of the reference's
``moe_layer`` (``src/deepseeker/mlx_forward.py:257-263``) on torch tensors of
a HIP device and runs the whole layer in libdsk_moe: router, dispatch,
expert SwiGLU with fused dequant, shared expert, combine and cast.

Arguments as in the reference:

* ``x [T, H]`` bf16 or float32; ``gate_w [E, H]`` float32 or bf16;
  ``gate_b [E]`` float32 (selection bias).
* ``expert_fn``: a ``ResidentBank`` (every expert resident; no host sync),
  or the reference's callable ``expert_fn(e) -> (w1, w3, w2)`` /
  ``{"w1", "w3", "w2"}`` / ``{"w13", "w2"}`` with FP4 pairs or Q3 triples of
  device tensors; a callable is asked only for the experts the router picked,
  which needs one host synchronisation, as in the reference (``:294-295``).
* ``shared_fn``: a ``SharedExpert`` (fused), any callable ``x -> [T, H]`` in
  x's dtype (its output is added before the final cast, as in ``:409-419``),
  or None.
* ``top_k``, ``limit`` (SwiGLU clamp), ``trace_hook(layer, idx, w)`` (called
  once after routing with host lists; idx in ascending key order like the
  reference's ``argsort`` tail), ``layer_id``, ``prefetch_fn(layer, experts)``
  (called with the unique experts, for callers that track residency).

``union_budget > 0`` on a batch of more than one row caps the batch's
expert union as the reference's ``cap_union`` does (``:213-254, 294-305``),
on the device (``dsk_cap_union``): the ``union_budget`` experts with the
largest summed gate score are kept, dropped slots become -1 (the dispatch
skips them) and each row keeps its weight sum; ``union_strict`` drops the
one-expert rescue of rows that would lose everything; ``route_stats``
(``{"coverage", "calls"}``) accumulates the retained weight share per row.
The cap runs in one block that holds the batch's (token, slot) pairs:
T * top_k * 4 + E * 9 bytes must fit 160 KB of LDS (at 256 experts and
top-8, up to 5048 tokens); a larger batch raises ``DskError``
(DSK_EUNSUPPORTED) before anything runs.

``pinned_gather_fn(layer_id, x, idx, w)`` (``:313-321``), called after routing
with host arrays in the trace hook's order, returns ``{expert: (rows,
contrib)}``: each selected expert found there adds its weighted output rows
``contrib`` at ``rows`` instead of being computed (``:388-393``); the other
experts' weighted rows are computed with x in float32 (``dsk_expert_rows``),
each row's contributions are added in ascending expert order, the pinned
ones in their place, and the sum is cast once.  ``dsk_moe.pinned``'s
``gather_pinned_contributions`` is a device version of the reference's
callback body (``:159-210``).

Options of the reference that only concern SSD paging or MLX scheduling are
accepted and have no effect on the result, which the reference documents as
identical with or without them: ``pipeline``, ``async_submit_fn``,
``async_finalize_fn`` (``:273-285``) and ``stack_gateup`` (``:140-156``).

Extensions (keyword-only): ``score_func`` ("sqrtsoftplus", the reference's
default, or "sigmoid"), ``route_scale`` (reference default 1.5), ``out``.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .bank import ResidentBank, SharedExpert
from .ops import cap_union as _cap_union
from .ops import make_desc, ptr, require_device, stream_of, workspace, workspace_size


def _coverage(w_before: torch.Tensor, idx_capped: torch.Tensor) -> float:
    """Share of the batch's gate weight the cap retained (before rescaling), summed as
    the reference does (numpy float32, its slot order: ascending key)."""
    wb = w_before.cpu().numpy()[:, ::-1]
    kept = idx_capped.cpu().numpy()[:, ::-1] >= 0
    total = float(wb.sum())
    return float(np.where(kept, wb, np.float32(0.0)).sum()) / total if total > 0 else 1.0


def _roles_of(weights) -> tuple:
    """Normalise an expert_fn result to ((w1...), (w3...), (w2...))."""
    if isinstance(weights, dict):
        if "w13" in weights:
            parts = weights["w13"]
            if parts[0].shape[0] % 2:
                raise ValueError("stacked gate/up rows must divide evenly")
            half = [p.shape[0] // 2 for p in parts]
            w1 = tuple(p[:n] for p, n in zip(parts, half))
            w3 = tuple(p[n:] for p, n in zip(parts, half))
            return w1, w3, tuple(weights["w2"])
        return tuple(weights["w1"]), tuple(weights["w3"]), tuple(weights["w2"])
    w1, w3, w2 = weights
    return tuple(w1), tuple(w3), tuple(w2)


def _table_from_weights(fetched: dict, n_experts: int, quant: str, device: torch.device,
                        keep: list) -> torch.Tensor:
    """Device ``dsk_expert_ptrs[E]`` from {expert: expert_fn(expert)} (others NULL)."""
    entries = (_lib.ExpertPtrs * n_experts)()
    arity = 2 if quant == "fp4" else 3
    for e, weights in fetched.items():
        vals = []
        for parts in _roles_of(weights):
            if len(parts) != arity:
                raise ValueError(f"expert {e}: {quant} roles need {arity} tensors, got {len(parts)}")
            for t in parts:
                require_device(t)
                keep.append(t)
            vals.extend([parts[c].data_ptr() if c < arity else None for c in range(3)])
        entries[e] = _lib.ExpertPtrs(*vals)
    return torch.frombuffer(bytearray(bytes(entries)), dtype=torch.uint8).to(device)


def moe_layer(x: torch.Tensor, gate_w: torch.Tensor, gate_b: torch.Tensor,
              expert_fn, shared_fn, top_k: int = 6, limit: float = 10.0,
              trace_hook=None, layer_id: int = 0, prefetch_fn=None,
              union_budget: int = 0, route_stats: dict | None = None,
              union_strict: bool = False, pipeline: bool = False,
              async_submit_fn=None, async_finalize_fn=None,
              pinned_gather_fn=None, stack_gateup: bool = False, *,
              score_func: str = "sqrtsoftplus", route_scale: float = 1.5,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """MoE layer forward on the GPU; returns ``[T, H]`` in x's dtype."""
    del pipeline, async_submit_fn, async_finalize_fn, stack_gateup
    dev = require_device(x, gate_w, gate_b)
    if x.dim() != 2:
        raise ValueError(f"x must be [T, H], got {tuple(x.shape)}")
    t, h = x.shape
    e = gate_w.shape[0]
    gate_b = gate_b.to(torch.float32).contiguous()
    if gate_w.shape != (e, h) or gate_b.shape != (e,):
        raise ValueError("gate_w must be [E, H] and gate_b [E]")

    bank = expert_fn if isinstance(expert_fn, ResidentBank) else None
    shared = shared_fn if isinstance(shared_fn, SharedExpert) else None
    if bank is not None:
        quant, inter = bank.quant, bank.inter
        if bank.n_experts != e or bank.hidden != h:
            raise ValueError("ResidentBank geometry does not match gate_w / x")
    if shared is not None and (shared.hidden != h):
        raise ValueError("SharedExpert hidden size does not match x")

    if out is None:
        out = torch.empty_like(x)
    else:
        require_device(out)
        if out.shape != x.shape or out.dtype != x.dtype:
            raise ValueError("out must match x in shape and dtype")
    stream = stream_of(dev)
    union = union_budget > 0 and t > 1
    need_host = bank is None or trace_hook is not None or prefetch_fn is not None or pinned_gather_fn is not None
    split = need_host or union      # route first, then dispatch + experts

    # Route (+ dispatch) first when the host must see the routing.
    idx = torch.empty((t, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((t, top_k), dtype=torch.float32, device=dev)
    keep: list = []
    if bank is None:
        # Learn the expert geometry from the first routed expert below.
        quant, inter = None, None
    probe_inter = inter if bank is not None else 32
    desc = make_desc(tokens=t, hidden=h, n_experts=e, top_k=top_k,
                     inter=probe_inter, inter_shared=shared.inter if shared else 0,
                     score_func=score_func, quant=quant or "fp4", x_dtype=x.dtype,
                     gate_dtype=gate_w.dtype, route_scale=route_scale, limit=limit)
    if split:
        scores = torch.empty((t, e), dtype=torch.float32, device=dev)
        _lib.call("dsk_route", ctypes.byref(desc), ptr(x), ptr(gate_w), ptr(gate_b), ptr(scores),
                  ptr(idx), ptr(w), stream)
    if union:
        w_before = w.clone() if route_stats is not None else None
        _cap_union(scores, idx, w, union_budget, union_strict)
        if route_stats is not None:
            route_stats["coverage"] += _coverage(w_before, idx) * t
            route_stats["calls"] += float(t)
    if need_host:
        idx_h = idx.cpu()
        uniq = sorted(set(int(v) for v in idx_h.flatten().tolist() if 0 <= v < e))
        if bank is None:
            if not uniq:
                raise ValueError("router selected no expert")
            fetched = {ex: expert_fn(ex) for ex in uniq}
            first = _roles_of(fetched[uniq[0]])
            quant = "fp4" if len(first[0]) == 2 else "q3"
            inter = first[0][0].shape[0]
            desc.quant = 0 if quant == "fp4" else 1
            desc.inter = inter
        if prefetch_fn is not None:
            prefetch_fn(layer_id, uniq)
        if trace_hook is not None:
            trace_hook(layer_id, idx_h.flip(1).tolist(), w.cpu().flip(1).tolist())
    pinned: dict = {}
    if pinned_gather_fn is not None:
        got = pinned_gather_fn(layer_id, x, idx_h.flip(1).numpy(), w.cpu().flip(1).numpy()) or {}
        pinned = {int(ex): v for ex, v in got.items() if int(ex) in uniq}

    shared_out = None
    if shared_fn is not None and shared is None:
        shared_out = shared_fn(x)
        if not isinstance(shared_out, torch.Tensor) or shared_out.shape != x.shape:
            raise ValueError("shared_fn must return a [T, H] tensor")
        shared_out = shared_out.to(x.dtype).contiguous()
        require_device(shared_out)

    table = bank.table if bank is not None else _table_from_weights(fetched, e, quant, dev, keep)
    ws = workspace(desc, dev)
    ws1 = shared.w1 if shared else None
    ws3 = shared.w3 if shared else None
    ws2 = shared.w2 if shared else None
    if pinned:
        _with_pinned(desc, x, idx, w, table, (ws1, ws3, ws2), shared_out, pinned, uniq, out, dev, keep)
    elif split:
        from .ops import dispatch as _dispatch  # local: same device, same stream
        d = _dispatch(idx, e)
        _lib.call("dsk_experts", ctypes.byref(desc), ptr(table), ptr(ws1), ptr(ws3), ptr(ws2),
                  ptr(shared_out), ptr(x), ptr(w), ptr(d["counts"]), ptr(d["offsets"]),
                  ptr(d["perm"]), ptr(d["rank"]), ptr(d["active"]), ptr(out), ptr(ws),
                  ws.numel(), stream)
        keep.append(d)
    else:
        _lib.call("dsk_moe_forward", ctypes.byref(desc), ptr(x), ptr(gate_w), ptr(gate_b),
                  ptr(table), ptr(ws1), ptr(ws3), ptr(ws2), ptr(shared_out), ptr(out),
                  ptr(idx), ptr(w), ptr(ws), ws.numel(), stream)
    if keep:
        # Tensors referenced only through raw pointers must outlive the launches.
        torch.cuda.current_stream(dev).synchronize()
    return out


def _with_pinned(desc, x, idx, w, table, shared_w, shared_out, pinned: dict, uniq: list, out, dev,
                 keep: list) -> None:
    """The layer with some selected experts supplied by a pinned-gather callback
    (src/deepseeker/mlx_forward.py:313-321, 388-393).  The other selected
    experts' weighted rows come from ``dsk_expert_rows`` (x in float32); then,
    as the reference's float32 scatter-add, every row's contributions are added
    from zero expert by expert in ascending id -- an expert of the callback
    adds its ``contrib`` rows at its ``rows`` in its place -- followed by the
    shared output rounded to x's dtype, and the sum is cast once."""
    from .ops import dispatch as _dispatch
    from .pinned import expert_rows
    stream = stream_of(dev)
    t, h = x.shape
    e = desc.n_experts
    idx_m = idx.clone()
    for ex in pinned:
        idx_m[idx_m == ex] = -1
    quant = "fp4" if desc.quant == _lib.QUANT_FP4 else "q3"
    computed, counts = expert_rows(x, idx_m, w, table, e, quant, desc.inter, limit=desc.limit)
    idx_mh = idx_m.cpu().numpy()
    # source rows: 0 = zeros, then the computed rows (dispatch order), then each pinned expert's rows
    parts = [torch.zeros((1, h), dtype=torch.float32, device=dev), computed]
    first = {}
    base = 1 + computed.shape[0]
    for ex in sorted(pinned):
        rows, contrib = pinned[ex]
        rows = [int(r) for r in np.asarray(rows).ravel()]
        contrib = torch.as_tensor(contrib).to(device=dev, dtype=torch.float32)
        if contrib.shape != (len(rows), h) or any(not 0 <= r < t for r in rows):
            raise ValueError(f"pinned expert {ex}: contrib must be [len(rows), {h}] with rows in [0, {t})")
        parts.append(contrib)
        first[ex] = (base, rows)
        base += len(rows)
    # per row, its sources in the order of the ascending-expert sum
    order: list[list[int]] = [[] for _ in range(t)]
    comp_row = 1
    for ex in uniq:
        if ex in first:
            b, rows = first[ex]
            for r, tok in enumerate(rows):
                order[tok].append(b + r)
        elif counts[ex]:
            for tok in np.nonzero((idx_mh == ex).any(axis=1))[0]:
                order[int(tok)].append(comp_row)
                comp_row += 1
    depth = max(1, max(len(o) for o in order))
    src = torch.tensor([o + [0] * (depth - len(o)) for o in order], dtype=torch.int64).to(dev)
    rows_all = torch.cat(parts)
    acc = torch.zeros((t, h), dtype=torch.float32, device=dev)
    for j in range(depth):
        acc += rows_all.index_select(0, src[:, j])
    ws1, ws3, ws2 = shared_w
    if ws1 is not None:
        # the shared expert alone (no routed position), rounded to x's dtype
        none = torch.full_like(idx, -1)
        ds = _dispatch(none, e)
        sh = torch.empty_like(x)
        ws_s = workspace(desc, dev)
        _lib.call("dsk_experts", ctypes.byref(desc), ptr(table), ptr(ws1), ptr(ws3), ptr(ws2), None, ptr(x),
                  ptr(w), ptr(ds["counts"]), ptr(ds["offsets"]), ptr(ds["perm"]), ptr(ds["rank"]),
                  ptr(ds["active"]), ptr(sh), ptr(ws_s), ws_s.numel(), stream)
        keep += [ds, none]
        acc += sh.to(torch.float32)
    elif shared_out is not None:
        acc += shared_out.to(torch.float32)
    out.copy_(acc.to(x.dtype))


def experts_forward(x: torch.Tensor, idx: torch.Tensor, w: torch.Tensor, bank: ResidentBank,
                    shared: SharedExpert | None = None, *, limit: float = 10.0,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Expert products for a given routing (``dsk_dispatch`` + ``dsk_experts``): the
    part of ``moe_layer`` after ``route_topk`` (``src/deepseeker/mlx_forward.py:294-419``)
    with ``idx [T, k]`` int32 expert ids and ``w [T, k]`` float32 route weights
    supplied by the caller -- e.g. a recorded trace replayed.  Entries of ``idx``
    outside [0, E) are dropped."""
    dev = require_device(x, idx, w)
    t, h = x.shape
    if idx.dtype != torch.int32 or w.dtype != torch.float32 or idx.shape != w.shape or idx.shape[0] != t:
        raise ValueError("idx must be int32 [T, k] and w float32 [T, k], with T = x.shape[0]")
    if bank.hidden != h or (shared is not None and shared.hidden != h):
        raise ValueError("bank / shared hidden size does not match x")
    idx, w = idx.contiguous(), w.contiguous()
    k = idx.shape[1]
    desc = make_desc(tokens=t, hidden=h, n_experts=bank.n_experts, top_k=k, inter=bank.inter,
                     inter_shared=shared.inter if shared else 0, quant=bank.quant, x_dtype=x.dtype,
                     limit=limit)
    if out is None:
        out = torch.empty_like(x)
    from .ops import dispatch as _dispatch
    d = _dispatch(idx, bank.n_experts)
    ws = workspace(desc, dev)
    _lib.call("dsk_experts", ctypes.byref(desc), ptr(bank.table), ptr(shared.w1 if shared else None),
              ptr(shared.w3 if shared else None), ptr(shared.w2 if shared else None), ptr(None), ptr(x),
              ptr(w), ptr(d["counts"]), ptr(d["offsets"]), ptr(d["perm"]), ptr(d["rank"]),
              ptr(d["active"]), ptr(out), ptr(ws), ws.numel(), stream_of(dev))
    torch.cuda.current_stream(dev).synchronize()   # d's buffers are referenced by raw pointer
    return out


class MoELayer:
    """One resident layer: gate, bank, shared expert and configuration."""

    def __init__(self, gate_w: torch.Tensor, gate_b: torch.Tensor, bank: ResidentBank,
                 shared: SharedExpert | None, top_k: int, *, score_func: str = "sigmoid",
                 route_scale: float = 2.5, limit: float = 10.0):
        self.gate_w, self.gate_b, self.bank, self.shared = gate_w, gate_b.float().contiguous(), bank, shared
        self.top_k, self.score_func, self.route_scale, self.limit = top_k, score_func, route_scale, limit

    def __call__(self, x: torch.Tensor, out: torch.Tensor | None = None,
                 idx: torch.Tensor | None = None, w: torch.Tensor | None = None,
                 trace=None, layer_id: int = 0, ws: torch.Tensor | None = None) -> torch.Tensor:
        """``trace(layer_id, idx, weights)`` (optional, e.g. a ``TraceSink``) receives the
        routing on the host, in ascending key order like the reference's trace_hook.
        ``ws`` (optional): a caller-owned workspace (``ops.new_workspace``) of at least
        ``workspace_bytes(tokens)`` bytes, used instead of the per-stream cached one."""
        dev = require_device(x, self.gate_w)
        t, h = x.shape
        if trace is not None:
            idx = idx if idx is not None else torch.empty((t, self.top_k), dtype=torch.int32, device=dev)
            w = w if w is not None else torch.empty((t, self.top_k), dtype=torch.float32, device=dev)
        desc = make_desc(tokens=t, hidden=h, n_experts=self.bank.n_experts, top_k=self.top_k,
                         inter=self.bank.inter, inter_shared=self.shared.inter if self.shared else 0,
                         score_func=self.score_func, quant=self.bank.quant, x_dtype=x.dtype,
                         gate_dtype=self.gate_w.dtype, route_scale=self.route_scale,
                         limit=self.limit)
        if out is None:
            out = torch.empty_like(x)
        if ws is None:
            ws = workspace(desc, dev)
        elif ws.numel() < workspace_size(desc) or ws.device != dev:
            raise ValueError(f"workspace of {ws.numel()} bytes on {ws.device} is too small for this call")
        s = self.shared
        _lib.call("dsk_moe_forward", ctypes.byref(desc), ptr(x), ptr(self.gate_w), ptr(self.gate_b),
                  ptr(self.bank.table), ptr(s.w1 if s else None), ptr(s.w3 if s else None),
                  ptr(s.w2 if s else None), ptr(None), ptr(out), ptr(idx), ptr(w), ptr(ws),
                  ws.numel(), stream_of(dev))
        if trace is not None:
            trace(layer_id, idx.flip(1).tolist(), w.flip(1).tolist())
        return out

    def forward_residual(self, h: torch.Tensor, d: torch.Tensor, h_out: torch.Tensor, x_out: torch.Tensor,
                         out: torch.Tensor, gamma: torch.Tensor | None = None, eps: float = 1e-6,
                         idx: torch.Tensor | None = None, w: torch.Tensor | None = None,
                         trace=None, layer_id: int = 0, ws: torch.Tensor | None = None) -> torch.Tensor:
        """One step of a layer stack (``dsk_moe_forward_residual``): ``h_out = h + d``
        (rounded to the stream's dtype), ``x_out = rmsnorm(h_out) * gamma``, then the
        layer on ``x_out`` into ``out`` (which may be ``d``).  With ``h_out`` a buffer
        of its own, at one or two bf16 tokens, the layer's first kernel computes the
        update itself."""
        dev = require_device(h, d, h_out, x_out, out, self.gate_w)
        t, hd = h.shape
        for name, v in (("d", d), ("h_out", h_out), ("x_out", x_out), ("out", out)):
            if v.shape != h.shape or v.dtype != h.dtype:
                raise ValueError(f"{name} must match h in shape and dtype")
        if gamma is not None and (gamma.dtype != torch.float32 or gamma.shape != (hd,)):
            raise ValueError("gamma must be float32 [hidden]")
        if trace is not None:
            idx = idx if idx is not None else torch.empty((t, self.top_k), dtype=torch.int32, device=dev)
            w = w if w is not None else torch.empty((t, self.top_k), dtype=torch.float32, device=dev)
        desc = make_desc(tokens=t, hidden=hd, n_experts=self.bank.n_experts, top_k=self.top_k,
                         inter=self.bank.inter, inter_shared=self.shared.inter if self.shared else 0,
                         score_func=self.score_func, quant=self.bank.quant, x_dtype=h.dtype,
                         gate_dtype=self.gate_w.dtype, route_scale=self.route_scale, limit=self.limit)
        if ws is None:
            ws = workspace(desc, dev)
        elif ws.numel() < workspace_size(desc) or ws.device != dev:
            raise ValueError(f"workspace of {ws.numel()} bytes on {ws.device} is too small for this call")
        r = _lib.Residual(h.data_ptr(), d.data_ptr(), gamma.data_ptr() if gamma is not None else None,
                          float(eps), h_out.data_ptr(), x_out.data_ptr())
        s = self.shared
        _lib.call("dsk_moe_forward_residual", ctypes.byref(desc), ctypes.byref(r), ptr(self.gate_w),
                  ptr(self.gate_b), ptr(self.bank.table), ptr(s.w1 if s else None), ptr(s.w3 if s else None),
                  ptr(s.w2 if s else None), ptr(out), ptr(idx), ptr(w), ptr(ws), ws.numel(), stream_of(dev))
        if trace is not None:
            trace(layer_id, idx.flip(1).tolist(), w.flip(1).tolist())
        return out

    def workspace_bytes(self, tokens: int, x_dtype: torch.dtype = torch.bfloat16) -> int:
        """Workspace bytes a call on ``tokens`` rows of ``x_dtype`` needs."""
        return workspace_size(make_desc(
            tokens=tokens, hidden=self.gate_w.shape[1], n_experts=self.bank.n_experts, top_k=self.top_k,
            inter=self.bank.inter, inter_shared=self.shared.inter if self.shared else 0,
            score_func=self.score_func, quant=self.bank.quant, x_dtype=x_dtype,
            gate_dtype=self.gate_w.dtype, route_scale=self.route_scale, limit=self.limit))
