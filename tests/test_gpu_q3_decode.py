"""GPU parity of the q3 decode kernels (factored affine products: gate/up up
to 8 tokens, down up to 4 tokens with I = 2048) against the oracle, through
the whole layer.

The factored kernels feed the raw 3-bit codes to the MFMA and apply each
64-group's fp16 scale and bias to the MFMA output (x . W = s * sum(q x) +
b * sum(x)); the oracle dequantises W first.  Both are exact up to float32
summation and the final bf16 roundings, so the layer tolerance applies.
Cases: every token count of the gate/up kernel (1..8) with bf16 and float32
activations, the scale/bias-window variant (hidden a multiple of 2048) and the
per-block variant (hidden 1024; windows need hidden 4096), activations with a large common offset (the
MFMA sums carry 128 * sum(x / m), removed afterwards), the down kernel
(intermediate 2048) with a shared expert of 2048 or 1024 rows, none, or a
callable one, and batch invariance (a token's row does not depend on the
other tokens of the batch).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import dsk_moe
from oracle import layer as L
from oracle import synth
from conftest import assert_layer_close
from test_gpu_layer import run_layer, to_bank, to_shared

pytestmark = pytest.mark.gpu
DEV = "cuda"
MID = L.LayerSpec(H=1024, E=64, k=8, I=512, I_shared=512, quant=L.QUANT_Q3)      # per-block scales
WIN = L.LayerSpec(H=4096, E=8, k=4, I=256, I_shared=256, quant=L.QUANT_Q3)       # scale windows
DN = L.LayerSpec(H=512, E=8, k=4, I=2048, I_shared=1024, quant=L.QUANT_Q3)        # factored down


def _case(spec, seed, T, dtype, offset=0.0):
    d = synth.make_layer(spec, seed, T)
    g = torch.Generator().manual_seed(seed + 1000)
    x = torch.randn((T, spec.H), generator=g) + offset
    x = x.to(dtype)
    r = L.moe_forward(x, d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    return d, x, r


@pytest.mark.parametrize("spec_name,T,dtype", [
    ("mid", 1, "bf16"), ("mid", 2, "bf16"), ("mid", 3, "bf16"), ("mid", 5, "bf16"), ("mid", 7, "bf16"),
    ("mid", 1, "f32"), ("mid", 4, "f32"), ("mid", 8, "f32"),
    ("win", 1, "bf16"), ("win", 6, "bf16"), ("win", 3, "f32"), ("win", 8, "f32"),
])
def test_q3_decode_tokens(spec_name, T, dtype):
    spec = MID if spec_name == "mid" else WIN
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    print(f"q3 decode {spec_name} T={T} x={dtype}", flush=True)
    d, x, r = _case(spec, 40 + T, T, dt)
    idx = torch.empty((T, spec.k), dtype=torch.int32, device=DEV)
    layer = dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                             to_shared(d["shared"]), spec.k)
    out = layer(x.to(DEV), idx=idx).cpu()
    assert out.dtype == dt
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_q3_decode_offset_activations(dtype):
    """x = N(0, 1) + 8: the MFMA sums are dominated by 128 * sum(x / m)."""
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    print(f"q3 decode win T=2 offset x={dtype}", flush=True)
    d, x, r = _case(WIN, 77, 2, dt, offset=8.0)
    out = run_layer(d, WIN, x=x)
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


def test_q3_decode_batch_invariant():
    """A token's output row does not depend on the rest of the batch (bitwise)
    among batches that run the same kernels: T = 1 and 2 (staged down), and
    T = 3 and 5 (grouped down and combine)."""
    spec = WIN
    d, x, _ = _case(spec, 91, 5, torch.bfloat16)
    layer = dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                             to_shared(d["shared"]), spec.k)
    xd = x.to(DEV)
    print("q3 decode win batch invariance T=1,2 and T=3,5", flush=True)
    alone = torch.cat([layer(xd[t:t + 1]) for t in range(2)]).cpu()
    pair = layer(xd[:2]).cpu()
    assert torch.equal(pair.view(torch.int16), alone.view(torch.int16))
    three = layer(xd[:3]).cpu()
    five = layer(xd[:5]).cpu()
    assert torch.equal(five[:3].view(torch.int16), three.view(torch.int16))


@pytest.mark.parametrize("T,dtype,shared", [
    (1, "bf16", 1024), (2, "bf16", 1024), (1, "f32", 2048), (3, "f32", 1024), (4, "f32", 0),
    (2, "bf16", 0), (1, "bf16", "fn"),
])
def test_q3_down_factored(T, dtype, shared):
    """Intermediate 2048: the factored down kernel with its shared-expert waves
    (2048 or 1024 rows), no shared expert, or a callable (precomputed output)."""
    spec = L.LayerSpec(H=512, E=8, k=4, I=2048, I_shared=shared if isinstance(shared, int) else 1024,
                       quant=L.QUANT_Q3)
    dt = torch.bfloat16 if dtype == "bf16" else torch.float32
    print(f"q3 down H=512 I=2048 T={T} x={dtype} shared={shared}", flush=True)
    d, x, r = _case(spec, 60 + T, T, dt)
    if shared == 0:
        r = L.moe_forward(x, d["gate_w"], d["gate_b"], d["bank"], None, spec)
        out = run_layer(d, spec, x=x, shared=False)
    elif shared == "fn":
        sh = to_shared(d["shared"])
        out = run_layer(d, spec, x=x, shared_fn=lambda t: sh(t))
    else:
        out = run_layer(d, spec, x=x)
    assert out.dtype == dt
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


def test_q3_down_factored_batch_invariant():
    """T = 2 rows equal the two T = 1 rows bitwise (both through the factored kernels)."""
    d, x, _ = _case(DN, 95, 2, torch.bfloat16)
    layer = dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                             to_shared(d["shared"]), DN.k)
    xd = x.to(DEV)
    print("q3 down H=512 I=2048 batch invariance T=1,2", flush=True)
    alone = torch.cat([layer(xd[t:t + 1]) for t in range(2)]).cpu()
    pair = layer(xd).cpu()
    assert torch.equal(pair.view(torch.int16), alone.view(torch.int16))
