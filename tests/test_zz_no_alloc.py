"""dsk_moe_forward_noalloc (the layer on the library's per-GPU scratch, no
allocation) against dsk_moe_forward with a caller workspace, through the C ABI.

Outputs, routing indices and weights must be identical bit for bit: the two
entry points run the same kernels on the same inputs, only the workspace
memory differs.  Each case makes two calls in a row on the shared scratch,
the second with fewer tokens (the scratch keeps the first call's contents).
Cases: the full-size decode layer (16 then 1 token), a mid-size layer on the
prefill GEMM path then the decode pipeline (256 then 5 tokens), top-16
routing at 8 tokens (the fused router with its arrival counters in the
scratch) then 2, a call larger than the scratch (rejected before launch), and
replays of a captured HIP graph of the no-allocation call.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from dsk_moe import _lib
from dsk_moe import synth as gsynth
from dsk_moe.ops import make_desc, ptr, stream_of

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _desc(layer, x):
    return make_desc(tokens=x.shape[0], hidden=x.shape[1], n_experts=layer.bank.n_experts, top_k=layer.top_k,
                     inter=layer.bank.inter, inter_shared=layer.shared.inter if layer.shared else 0,
                     score_func=layer.score_func, quant=layer.bank.quant, x_dtype=x.dtype,
                     gate_dtype=layer.gate_w.dtype, route_scale=layer.route_scale, limit=layer.limit)


def noalloc(layer, x, out, idx, w):
    s = layer.shared
    _lib.call("dsk_moe_forward_noalloc", ctypes.byref(_desc(layer, x)), ptr(x), ptr(layer.gate_w),
              ptr(layer.gate_b), ptr(layer.bank.table), ptr(s.w1 if s else None), ptr(s.w3 if s else None),
              ptr(s.w2 if s else None), ptr(None), ptr(out), ptr(idx), ptr(w), stream_of(x.device))


def both(layer, x):
    T, k = x.shape[0], layer.top_k
    idx_a = torch.empty((T, k), dtype=torch.int32, device=DEV)
    w_a = torch.empty((T, k), dtype=torch.float32, device=DEV)
    ref = layer(x, idx=idx_a, w=w_a)
    out = torch.full_like(x, float("nan"))
    idx_b = torch.full((T, k), -7, dtype=torch.int32, device=DEV)
    w_b = torch.full((T, k), float("nan"), dtype=torch.float32, device=DEV)
    noalloc(layer, x, out, idx_b, w_b)
    torch.cuda.synchronize()
    return (ref, idx_a, w_a), (out, idx_b, w_b)


def assert_same(a, b, label):
    for name, p, q in zip(("out", "idx", "w"), a, b):
        assert torch.equal(p.view(torch.int16) if p.dtype == torch.bfloat16 else p,
                           q.view(torch.int16) if q.dtype == torch.bfloat16 else q), f"{label}: {name} differs"


def _x(T, H, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn((T, H), generator=g, device=DEV).to(dtype)


@pytest.mark.parametrize("case", ["full-size decode", "mid prefill then decode", "top-16 fused router"])
def test_noalloc_matches_workspace_entry_point(case):
    if case == "full-size decode":
        layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048, inter_shared=2048,
                                  seed=700, device=DEV)
        sizes, H = (16, 1), 4096
    elif case == "mid prefill then decode":
        layer = gsynth.make_layer(hidden=1024, n_experts=64, top_k=8, inter=512, inter_shared=512,
                                  seed=701, device=DEV)
        sizes, H = (256, 5), 1024
    else:
        layer = gsynth.make_layer(hidden=1024, n_experts=64, top_k=16, inter=512, inter_shared=512,
                                  seed=702, device=DEV)
        sizes, H = (8, 2), 1024
    for i, T in enumerate(sizes):
        print(f"noalloc {case}: call {i + 1}, T={T}", flush=True)
        a, b = both(layer, _x(T, H, 7000 + T))
        assert_same(a, b, f"{case} T={T}")
        assert torch.isfinite(b[0].float()).all()


def test_noalloc_rejects_calls_larger_than_the_scratch():
    print("noalloc: T=4096 full size must be rejected before launch", flush=True)
    layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048, inter_shared=2048,
                              seed=703, device=DEV)
    x = _x(4096, 4096, 9)
    out = torch.zeros_like(x)
    idx = torch.zeros((4096, 8), dtype=torch.int32, device=DEV)
    w = torch.zeros((4096, 8), dtype=torch.float32, device=DEV)
    with pytest.raises(_lib.DskError) as ei:
        noalloc(layer, x, out, idx, w)
    assert ei.value.code == -5 and "scratch" in str(ei.value)
    torch.cuda.synchronize()
    assert int(out.view(torch.int16).abs().sum()) == 0 and int(idx.abs().sum()) == 0   # nothing ran


def test_noalloc_under_graph_capture():
    print("noalloc: captured HIP graph replays vs eager", flush=True)
    layer = gsynth.make_layer(hidden=1024, n_experts=64, top_k=6, inter=512, inter_shared=512,
                              seed=704, device=DEV)
    T = 2
    xs = torch.zeros((T, 1024), dtype=torch.bfloat16, device=DEV)
    out = torch.empty_like(xs)
    idx = torch.empty((T, 6), dtype=torch.int32, device=DEV)
    w = torch.empty((T, 6), dtype=torch.float32, device=DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        noalloc(layer, xs, out, idx, w)             # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        noalloc(layer, xs, out, idx, w)
    torch.cuda.synchronize()
    for rep in range(3):
        x = _x(T, 1024, 7100 + rep)
        eager_idx = torch.empty_like(idx)
        eager_w = torch.empty_like(w)
        ref = layer(x, idx=eager_idx, w=eager_w)
        torch.cuda.synchronize()
        xs.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert_same((ref, eager_idx, eager_w), (out, idx, w), f"replay {rep}")
