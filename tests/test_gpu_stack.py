"""GPU parity of the RMSNorm residual kernel and the MoE layer stack.

RMSNorm rows bit-exact against the oracle's defined order.  Small mixed FP4 /
q3 stacks are checked layer by layer on the device's own stream values
(normalised rows bit-exact, routing bit-exact, layer outputs within the layer
tolerance).  The full-size 40-layer stack (layers 0-19 FP4, 20-39 q3) is
checked layer by layer against the oracle at one and two tokens (normalised
rows and routing bit-exact, every layer's output within the layer tolerance,
the final residual sum bit-exact) and through properties: a 2-token verify
step equals two 1-token steps bit for bit (at one and two tokens the same
decode kernels run, and each adds a token's terms in an order that does not
depend on the other token), and replays of the captured HIP graph equal the
eager run, with eager work between replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import dsk_moe
from dsk_moe import synth as gsynth
from dsk_moe.stack import MoEStack, rmsnorm
from oracle import layer as L
from oracle import stack as S
from oracle import synth
from conftest import assert_layer_close
from test_gpu_layer import to_bank, to_shared

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rows,hidden", [(1, 4096), (3, 1028), (5, 64)])
@pytest.mark.parametrize("mode", ["norm", "residual", "inplace", "gamma"])
def test_rmsnorm_bit_exact(dtype, rows, hidden, mode):
    print(f"rmsnorm {dtype} {rows}x{hidden} {mode}", flush=True)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    g = torch.Generator().manual_seed(rows * hidden)
    x = (torch.randn((rows, hidden), generator=g) * 2).to(tdt)
    r = torch.randn((rows, hidden), generator=g).to(tdt)
    gamma = torch.rand((hidden,), generator=g) + 0.5 if mode == "gamma" else None
    xd = x.to(DEV)
    res = r.to(DEV) if mode in ("residual", "inplace") else None
    h_out = xd if mode == "inplace" else (torch.empty_like(xd) if mode == "residual" else None)
    y = rmsnorm(xd, 1e-6, gamma.to(DEV) if gamma is not None else None, residual=res, h_out=h_out)
    h_ref, y_ref = S.rmsnorm(x.float().numpy(), 1e-6, gamma.numpy() if gamma is not None else None,
                             r.float().numpy() if res is not None else None, dtype)
    np.testing.assert_array_equal(y.float().cpu().numpy(), y_ref)
    if h_out is not None:
        np.testing.assert_array_equal(h_out.float().cpu().numpy(), h_ref)


def _mixed_specs():
    fp4 = L.LayerSpec(H=1024, E=64, k=6, I=512, I_shared=512)
    q3 = L.LayerSpec(H=1024, E=64, k=6, I=512, I_shared=512, quant=L.QUANT_Q3)
    return [fp4, fp4, q3, q3]


@pytest.mark.parametrize("T", [1, 2, 5])
def test_small_mixed_stack_layerwise(T):
    """4 layers (FP4, FP4, q3, q3), H 1024, E 64, top-6: each layer against the oracle on the device's stream."""
    print(f"stack small mixed T={T}", flush=True)
    specs = _mixed_specs()
    data = [synth.make_layer(sp, 40 + l, T) for l, sp in enumerate(specs)]
    layers = [dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                               to_shared(d["shared"]), sp.k) for d, sp in zip(data, specs)]
    stack = MoEStack(layers, eps=1e-6)
    x = data[0]["x"].to(DEV)
    rec = []
    out = stack(x, record=rec).cpu()
    for l, ((h, y, idx, dl), d, sp) in enumerate(zip(rec, data, specs)):
        hn = h.float().cpu().numpy()
        _, y_ref = S.rmsnorm(hn, 1e-6, dtype="bf16")
        np.testing.assert_array_equal(y.float().cpu().numpy(), y_ref)
        r = L.moe_forward(y.cpu(), d["gate_w"], d["gate_b"], d["bank"], d["shared"], sp)
        np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
        c, rel = assert_layer_close(dl.float().cpu(), r["y_ref"])
        print(f"layer {l}: cos={c:.9f} rel={rel:.2e}", flush=True)
    h_last, d_last = rec[-1][0].float().cpu().numpy(), rec[-1][3].float().cpu().numpy()
    np.testing.assert_array_equal(out.float().numpy(), S.round_to(h_last + d_last, "bf16"))


@pytest.fixture(scope="module")
def stack40():
    layers = [gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048, inter_shared=2048,
                                quant="fp4" if l < 20 else "q3", seed=5000 + l, device=DEV)
              for l in range(40)]
    torch.cuda.synchronize()
    yield MoEStack(layers, eps=1e-6)
    del layers
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 2])
def test_full_stack_layerwise(stack40, T):
    """Every one of the 40 full-size layers against the oracle on the device's own stream values."""
    from conftest import DeviceBankView
    from test_gpu_fullshape import _spec
    print(f"stack 40 layers layer by layer T={T}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(90 + T)
    x = torch.randn((T, 4096), generator=g, device=DEV).to(torch.bfloat16)
    rec = []
    out = stack40(x, record=rec).cpu()
    assert len(rec) == 40
    for l, (h, y, idx, dl) in enumerate(rec):
        layer = stack40.layers[l]
        quant = "fp4" if l < 20 else "q3"
        _, y_ref = S.rmsnorm(h.float().cpu().numpy(), 1e-6, dtype="bf16")
        np.testing.assert_array_equal(y.float().cpu().numpy(), y_ref)
        idx_h = idx.cpu().numpy()
        shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2))
        view = DeviceBankView(layer.bank).prefetch(idx_h.ravel())
        try:
            r = L.moe_forward(y.cpu(), layer.gate_w.cpu(), layer.gate_b.cpu(), view, shared, _spec(layer, quant))
        finally:
            view.close()
        np.testing.assert_array_equal(idx_h, r["idx"])
        c, rel = assert_layer_close(dl.float().cpu(), r["y_ref"])
        print(f"layer {l} {quant}: cos={c:.9f} rel={rel:.2e}", flush=True)
    h_last, d_last = rec[-1][0].float().cpu().numpy(), rec[-1][3].float().cpu().numpy()
    np.testing.assert_array_equal(out.float().numpy(), S.round_to(h_last + d_last, "bf16"))


def test_full_stack_verify_and_graph(stack40):
    """40 full-size layers (0-19 FP4, 20-39 q3): B=2 rows == two B=1 steps; graph replays == eager."""
    print("stack 40 layers: B=2 vs 2 x B=1", flush=True)
    g = torch.Generator(device=DEV).manual_seed(9)
    x = torch.randn((2, 4096), generator=g, device=DEV).to(torch.bfloat16)
    both = stack40(x).clone()
    one0 = stack40(x[0:1].contiguous()).clone()
    one1 = stack40(x[1:2].contiguous()).clone()
    assert torch.isfinite(both.float()).all()
    assert torch.equal(both[0:1].view(torch.int16), one0.view(torch.int16))
    assert torch.equal(both[1:2].view(torch.int16), one1.view(torch.int16))
    print("stack 40 layers: graph capture B=2", flush=True)
    stack40.capture(2)
    for rep in range(3):
        xr = torch.randn((2, 4096), generator=g, device=DEV).to(torch.bfloat16)
        eager = stack40(xr).clone()
        torch.cuda.synchronize()
        got = stack40.replay(xr).clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
    # the stream moved: output differs from input and stays finite
    assert not torch.equal(got, xr) and torch.isfinite(got.float()).all()


def test_captured_stack_keeps_its_workspace():
    """A captured stack owns its workspace: an eager call that needs a larger
    one (T=300, prefill sizes) cannot free memory the graph still writes."""
    print("stack capture(1), eager T=300 layer call, replay", flush=True)
    specs = _mixed_specs()[:2]
    data = [synth.make_layer(sp, 60 + l, 1) for l, sp in enumerate(specs)]
    layers = [dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                               to_shared(d["shared"]), sp.k) for d, sp in zip(data, specs)]
    stack = MoEStack(layers, eps=1e-6)
    stack.capture(1)
    g = torch.Generator(device=DEV).manual_seed(61)
    big = torch.randn((300, 1024), generator=g, device=DEV).to(torch.bfloat16)
    for rep in range(3):
        x = torch.randn((1, 1024), generator=g, device=DEV).to(torch.bfloat16)
        layers[0](big)                  # grows (replaces) the cached per-stream workspace
        torch.cuda.synchronize()
        got = stack.replay(x).clone()
        torch.cuda.synchronize()
        want = stack(x).clone()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {rep}"


@pytest.mark.parametrize("case", ["mx-T1", "mx-T2", "q3-T1", "fp4-small-T2", "inplace-T1", "unfused-T5",
                                  "fp4full-T64", "q3-T40", "unfused-T24", "fp4full-T160"])
def test_forward_residual_equals_rmsnorm_then_layer(case):
    """dsk_moe_forward_residual against dsk_rmsnorm + dsk_moe_forward: h_out, x_out
    and the layer output bit for bit.  The MX pipeline (FP4, inter 2048) and the
    gate kernel of the other decode configurations take the update into their
    first kernel; in place (h_out = h) and from five tokens it runs as its own kernel.
    From 9 tokens the reference call's top-k kernel also writes x's FP8 planes (or
    the q3 form) for the grouped gate/up (from 128 tokens for the prefill GEMM), the
    residual call a kernel of their own."""
    print(f"forward_residual {case}", flush=True)
    kind, T = case.rsplit("-T", 1)
    T = int(T)
    if kind in ("mx", "inplace", "fp4full"):
        layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048, inter_shared=2048,
                                  seed=900 + T, device=DEV)
    elif kind == "q3":
        layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048, inter_shared=2048,
                                  quant="q3", seed=910, device=DEV)
    else:
        layer = gsynth.make_layer(hidden=1024, n_experts=64, top_k=6, inter=512, inter_shared=512,
                                  seed=920 + T, device=DEV)
    H = layer.gate_w.shape[1]
    g = torch.Generator(device=DEV).manual_seed(930 + T)
    h = (torch.randn((T, H), generator=g, device=DEV) * 3).to(torch.bfloat16)
    d = torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)
    gamma = torch.rand((H,), generator=g, device=DEV) + 0.5
    # reference: the two calls
    h_ref, y_ref = torch.empty_like(h), torch.empty_like(h)
    rmsnorm(h, 1e-6, gamma, residual=d, h_out=h_ref, out=y_ref)
    out_ref = layer(y_ref).clone()
    # fused
    x_out, out = torch.empty_like(h), torch.empty_like(h)
    h_in = h.clone()
    h_out = h_in if kind == "inplace" else torch.empty_like(h)
    layer.forward_residual(h_in, d, h_out, x_out, out, gamma=gamma, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(h_out.view(torch.int16), h_ref.view(torch.int16))
    assert torch.equal(x_out.view(torch.int16), y_ref.view(torch.int16))
    assert torch.equal(out.view(torch.int16), out_ref.view(torch.int16))
    # the layer's output may overwrite d (as the stack does)
    d2 = d.clone()
    h_out2 = torch.empty_like(h)
    layer.forward_residual(h, d2, h_out2, x_out, d2, gamma=gamma, eps=1e-6)
    assert torch.equal(d2.view(torch.int16), out_ref.view(torch.int16))
    assert torch.equal(h_out2.view(torch.int16), h_ref.view(torch.int16))
