"""GPU parity of the grouped expert path (batches between the decode pipeline
and the prefill GEMM, bf16 activations) against the oracle.

Routing indices bit-exact; outputs within the layer tolerance.  Cases: the
full-size FP4 layer at T=20; mid-size layers up to 127 tokens (the shared
expert's wide walk takes 64 tokens a pass: 100 and 127 take two, the second
ragged); mid-size layers with skewed routing (every
token to the same few experts, so each slot spans several column tiles of
dispatch rows), q3 experts, no shared expert, a callable shared expert, the
host-dispatch entry point (dsk_experts) reached through a callable
expert_fn, and the factored q3 gate/up at hidden 4096.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import dsk_moe
from dsk_moe import synth as gsynth
from oracle import layer as L
from oracle import synth
from conftest import assert_layer_close
from test_gpu_layer import _LazyBank, run_layer, to_bank, to_shared

pytestmark = pytest.mark.gpu
DEV = "cuda"
MID = dict(H=1024, E=64, k=8, I=512, I_shared=512)


def _skewed(d, hot: int):
    """Gate bias that sends every token to experts 0 .. hot-1 (scores are in (0, 1))."""
    b = d["gate_b"].clone()
    b[:hot] += 10.0
    return b


@pytest.mark.parametrize("quant,T,hot", [
    ("fp4", 20, 0), ("fp4", 20, 8), ("fp4", 37, 8), ("q3", 24, 0), ("q3", 30, 8), ("fp4", 63, 0),
    ("fp4", 100, 0), ("q3", 127, 0),
])
def test_grouped_mid(quant, T, hot):
    print(f"grouped mid {quant} T={T} hot={hot}", flush=True)
    spec = L.LayerSpec(**MID, quant=L.QUANT_Q3 if quant == "q3" else L.QUANT_FP4)
    d = synth.make_layer(spec, 21 + T, T)
    if hot:
        d["gate_b"] = _skewed(d, hot)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    if hot:
        assert (r["idx"] < hot).all()          # each hot expert holds every token: T rows, several tiles
    idx = torch.empty((T, spec.k), dtype=torch.int32, device=DEV)
    layer = dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                             to_shared(d["shared"]), spec.k)
    out = layer(d["x"].to(DEV), idx=idx).cpu()
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


@pytest.mark.parametrize("T,hot", [(12, 0), (30, 4), (40, 0)])
def test_grouped_q3_factored(T, hot):
    """Hidden 4096: the factored q3 gate/up (one row tile x 8 K ranges per block,
    one 512-code superblock per wave); hot = 4 sends every token to experts
    0..3, so each of their slots spans several column tiles."""
    spec = L.LayerSpec(H=4096, E=16, k=4, I=256, I_shared=256, quant=L.QUANT_Q3)
    print(f"grouped q3 factored H=4096 T={T} hot={hot}", flush=True)
    d = synth.make_layer(spec, 70 + T, T)
    if hot:
        d["gate_b"] = _skewed(d, hot)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    idx = torch.empty((T, spec.k), dtype=torch.int32, device=DEV)
    layer = dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                             to_shared(d["shared"]), spec.k)
    out = layer(d["x"].to(DEV), idx=idx).cpu()
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


def test_grouped_no_shared_and_callables():
    """No shared expert; a callable shared_fn (precomputed shared output); a
    callable expert_fn (route on the device, dispatch through dsk_experts)."""
    spec = L.LayerSpec(**MID)
    T = 24
    d = synth.make_layer(spec, 5, T)
    print("grouped mid no shared", flush=True)
    r0 = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], None, spec)
    assert_layer_close(run_layer(d, spec, shared=False).float(), r0["y_ref"])
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    sh = to_shared(d["shared"])
    print("grouped mid callable shared", flush=True)
    out = run_layer(d, spec, shared_fn=lambda x: sh(x))
    assert_layer_close(out.float(), r["y_ref"])
    bank = to_bank(d["bank"])
    print("grouped mid callable expert_fn", flush=True)
    out = run_layer(d, spec, expert_fn=lambda e: bank(e))
    assert_layer_close(out.float(), r["y_ref"])


def test_grouped_full_size_fp4():
    """hidden 4096, 256 experts, top-8, inter 2048, bf16 shared 2048, T=20 (GPU-generated)."""
    T = 20
    print(f"grouped full-size fp4 T={T}", flush=True)
    layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048,
                              inter_shared=2048, seed=3, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(300 + T)
    x = torch.randn((T, 4096), generator=g, device=DEV).to(torch.bfloat16)
    idx = torch.empty((T, 8), dtype=torch.int32, device=DEV)
    out = layer(x, idx=idx).cpu()
    spec = L.LayerSpec(H=4096, E=256, k=8, I=2048, I_shared=2048)
    shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2))
    r = L.moe_forward(x.cpu(), layer.gate_w.cpu(), layer.gate_b.cpu(), _LazyBank(layer.bank), shared, spec)
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


def test_grouped_deterministic():
    """Two calls give identical bits (fixed reduction orders, no atomics)."""
    spec = L.LayerSpec(**MID)
    d = synth.make_layer(spec, 9, 40)
    a = run_layer(d, spec)
    b = run_layer(d, spec)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
