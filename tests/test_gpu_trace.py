"""Routing traces from the device path, and recorded routing replayed.

* A two-layer stack run with a TraceSink: the records validate against a
  deepseeker.trace/v1 header and carry each layer's indices and weights in
  ascending key order (the reference hook's order).
* The reference's recorded routing (head of profiles/traces/mlx-en.jsonl:
  E = 384, top-6, 7 prompt tokens per layer) replayed through the dispatch and
  expert kernels (experts_forward) on a 384-expert layer with synthetic
  weights, against the oracle evaluated in float64 on the same routing.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import dsk_moe
from dsk_moe import synth as gsynth
from dsk_moe.layer import experts_forward
from dsk_moe.stack import MoEStack
from dsk_moe.trace import Geometry, Trace, TraceSink, check
from oracle import layer as L
from conftest import assert_layer_close
from test_gpu_layer import _LazyBank

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"


def test_stack_trace_sink():
    print("trace sink on a 2-layer stack", flush=True)
    layers = [gsynth.make_layer(hidden=1024, n_experts=64, top_k=6, inter=512, inter_shared=512,
                                seed=70 + l, device=DEV) for l in range(2)]
    stack = MoEStack(layers)
    x = torch.randn((3, 1024), generator=torch.Generator(device=DEV).manual_seed(1), device=DEV).to(torch.bfloat16)
    sink = TraceSink("req", token_start=10)
    rec = []
    stack(x, record=rec, trace=sink)
    geo = Geometry(n_layers=2, n_routed_experts=64, top_k=6)
    assert len(sink.records) == 2 * 3
    for r in sink.records:
        assert check(r, geo) == []
    for layer in range(2):
        got = [r for r in sink.records if r["layer"] == layer]
        assert [r["token_pos"] for r in got] == [10, 11, 12]
        idx = rec[layer][2].cpu().numpy()
        np.testing.assert_array_equal(np.asarray([r["experts"] for r in got]), idx[:, ::-1])
        for r in got:
            assert abs(sum(r["scores"]) - layers[layer].route_scale) < 1e-4


@pytest.mark.parametrize("layer_id", [0, 7, 29])
def test_replay_recorded_routing(layer_id):
    print(f"replay recorded routing, layer {layer_id}", flush=True)
    tr = Trace.load(GOLDEN / "trace_mlx_en_head.jsonl")
    h = tr.header
    _, _, experts, scores = tr.batches(layer_id)[0]
    T = experts.shape[0]
    spec = L.LayerSpec(H=1024, E=h["n_routed_experts"], k=h["top_k"], I=512, I_shared=512)
    layer = gsynth.make_layer(hidden=spec.H, n_experts=spec.E, top_k=spec.k, inter=spec.I,
                              inter_shared=spec.I_shared, seed=90 + layer_id, device=DEV)
    x = torch.randn((T, spec.H), generator=torch.Generator().manual_seed(layer_id)).to(torch.bfloat16)
    idx = torch.from_numpy(experts).to(DEV)
    w = torch.from_numpy(scores).to(DEV)
    out = experts_forward(x.to(DEV), idx, w, layer.bank, layer.shared).cpu()
    shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2))
    ref = L.moe_forward_f64(x, experts, scores, _LazyBank(layer.bank), shared, spec)
    c, rel = assert_layer_close(out.float(), torch.from_numpy(np.asarray(ref, dtype=np.float32)))
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)
