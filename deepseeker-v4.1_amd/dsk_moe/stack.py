"""A stack of resident MoE layers on a residual stream.

The caller of the layer in the reference is the runner's per-layer loop
(``src/deepseeker/mlx_runner.py:2138-2145``), which normalises the residual
stream (``rmsnorm``, ``src/deepseeker/mlx_forward.py:45-59``), runs the layer
and adds its output back.  ``MoEStack`` is that loop over MoE layers only:

    h_0 = x;  h_{l+1} = h_l + layer_l(rmsnorm(h_l))   (rounded to x's dtype)

with every step on the device: ``dsk_rmsnorm`` of x and ``dsk_moe_forward``
for the first layer, then per layer boundary ``dsk_moe_forward_residual``,
which adds the previous layer's output to the stream, normalises it and runs
the layer -- in the decode pipeline at one or two tokens inside the layer's
first kernel (the stream alternates between two buffers, since that kernel's
blocks all read the stream before one of them writes the update) -- and a
final residual add.  ``capture(tokens)`` records the whole stack as one HIP
graph (after an eager warm-up, so the workspace and buffers exist outside the
graph) and ``replay(x)`` runs it.
"""

from __future__ import annotations

import torch

from . import _lib
from .layer import MoELayer
from .ops import new_workspace, ptr, require_device, stream_of

_DTYPES = {torch.bfloat16: 0, torch.float32: 1}


def rmsnorm(x: torch.Tensor, eps: float = 1e-6, gamma: torch.Tensor | None = None,
            residual: torch.Tensor | None = None, h_out: torch.Tensor | None = None,
            out: torch.Tensor | None = None) -> torch.Tensor | None:
    """``dsk_rmsnorm``: h = x (+ residual); h_out <- h; returns out = rmsnorm(h) * gamma.

    With ``out=False`` only the residual update is made (``h_out`` required)."""
    dev = require_device(x)
    if x.dim() != 2 or not x.is_contiguous() or x.dtype not in _DTYPES:
        raise ValueError("x must be a contiguous [rows, hidden] bf16 or float32 tensor")
    for t in (residual, h_out) + ((out,) if isinstance(out, torch.Tensor) else ()):
        if t is not None and (t.shape != x.shape or t.dtype != x.dtype or not t.is_contiguous()):
            raise ValueError("residual / h_out / out must match x")
    if gamma is not None and (gamma.dtype != torch.float32 or gamma.shape != (x.shape[1],)):
        raise ValueError("gamma must be float32 [hidden]")
    want = out is not False
    if want and out is None:
        out = torch.empty_like(x)
    _lib.call("dsk_rmsnorm", ptr(x), ptr(residual), ptr(gamma), x.shape[0], x.shape[1], float(eps),
              _DTYPES[x.dtype], ptr(h_out), ptr(out if want else None), stream_of(dev))
    return out if want else None


class MoEStack:
    """``len(layers)`` MoE layers on an RMSNorm residual stream (eps, gamma per layer or none)."""

    def __init__(self, layers: list[MoELayer], eps: float = 1e-6, gammas: list[torch.Tensor] | None = None):
        if not layers:
            raise ValueError("a stack needs at least one layer")
        self.layers, self.eps = list(layers), float(eps)
        self.gammas = gammas if gammas is not None else [None] * len(layers)
        self._graph = None

    def _buffers(self, x: torch.Tensor):
        return tuple(torch.empty_like(x) for _ in range(4))   # h (two, alternating), y, d

    def forward(self, x: torch.Tensor, out: torch.Tensor | None = None, bufs=None,
                record: list | None = None, trace=None, ws: torch.Tensor | None = None) -> torch.Tensor:
        """h_L for input rows x [T, H].  ``record`` (optional list) receives, per
        layer, copies of (h_l, rmsnorm(h_l), idx_l, layer output); ``trace``
        (optional, e.g. a ``TraceSink``) receives every layer's routing as
        ``trace(layer, idx, weights)`` on the host."""
        h0, h1, y, d = bufs if bufs is not None else self._buffers(x)
        if out is None:
            out = torch.empty_like(x)
        idx = None
        prev = x
        for l, layer in enumerate(self.layers):
            if record is not None:
                idx = torch.empty((x.shape[0], layer.top_k), dtype=torch.int32, device=x.device)
            if l == 0:
                rmsnorm(x, self.eps, self.gammas[0], out=y)
                layer(y, out=d, idx=idx, trace=trace, layer_id=l, ws=ws)
            else:
                h = h0 if l % 2 else h1
                layer.forward_residual(prev, d, h, y, d, gamma=self.gammas[l], eps=self.eps, idx=idx,
                                       trace=trace, layer_id=l, ws=ws)
                prev = h
            if record is not None:
                record.append((prev.clone(), y.clone(), idx, d.clone()))
        rmsnorm(prev, self.eps, residual=d, h_out=out, out=False)
        return out

    __call__ = forward

    def capture(self, tokens: int, dtype: torch.dtype = torch.bfloat16, warmup: int = 2) -> None:
        """Record the stack for ``tokens`` rows as one HIP graph (static input / output
        buffers).  The graph owns its workspace (sized for the largest layer), so
        later eager calls of any size, or other captures, cannot move it."""
        dev = self.layers[0].gate_w.device
        hidden = self.layers[0].gate_w.shape[1]
        self._x = torch.zeros((tokens, hidden), dtype=dtype, device=dev)
        self._out = torch.empty_like(self._x)
        self._bufs = self._buffers(self._x)
        self._ws = new_workspace(max(l.workspace_bytes(tokens, dtype) for l in self.layers), dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.forward(self._x, out=self._out, bufs=self._bufs, ws=self._ws)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self._graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._graph):
            self.forward(self._x, out=self._out, bufs=self._bufs, ws=self._ws)
        torch.cuda.synchronize(dev)

    def replay(self, x: torch.Tensor | None = None) -> torch.Tensor:
        """Run the captured stack (on ``x`` copied into the static input if given);
        returns the static output buffer."""
        if self._graph is None:
            raise RuntimeError("capture() the stack first")
        if x is not None:
            self._x.copy_(x)
        self._graph.replay()
        return self._out
