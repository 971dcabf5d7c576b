"""GPU parity of the whole MoE layer against the oracle.

Routing indices bit-exact; outputs within the layer tolerance
(cosine >= 0.99999 and max|y - y_ref| / max|y_ref| <= 1e-2, y_ref the oracle's
float32 output before the final cast).
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

pytestmark = pytest.mark.gpu
DEV = "cuda"


def to_bank(bank: L.ExpertBank) -> dsk_moe.ResidentBank:
    roles = {r: tuple(torch.from_numpy(np.ascontiguousarray(a)).to(DEV) for a in parts)
             for r, parts in bank.roles.items()}
    return dsk_moe.ResidentBank(bank.quant, roles)


def to_shared(shared) -> dsk_moe.SharedExpert | None:
    return None if shared is None else dsk_moe.SharedExpert(*(t.to(DEV) for t in shared))


def run_layer(d, spec, x=None, shared=True, **kw):
    x = d["x"] if x is None else x
    out = dsk_moe.moe_layer(x.to(DEV), d["gate_w"].to(DEV), d["gate_b"].to(DEV),
                            kw.pop("expert_fn", None) or to_bank(d["bank"]),
                            kw.pop("shared_fn", to_shared(d["shared"]) if shared else None),
                            spec.k, spec.limit, score_func="sigmoid" if spec.score_func == 0 else "sqrtsoftplus",
                            route_scale=spec.route_scale, **kw)
    return out.cpu()


@pytest.fixture(scope="module")
def cfg0():
    spec = synth.config0_spec()
    d = synth.make_layer(spec, 0, 4)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    return spec, d, r


def test_config0_layer(cfg0, golden):
    spec, d, r = cfg0
    print("layer cfg0 T=4 H=1024 E=64 k=6 I=512 Is=512", flush=True)
    layer = dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                             to_shared(d["shared"]), spec.k)
    idx = torch.empty((4, spec.k), dtype=torch.int32, device=DEV)
    w = torch.empty((4, spec.k), dtype=torch.float32, device=DEV)
    out = layer(d["x"].to(DEV), idx=idx, w=w).cpu()
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    np.testing.assert_array_equal(w.cpu().numpy(), r["w"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)
    g = golden("cfg0.npz")
    np.testing.assert_array_equal(idx.cpu().numpy(), g["idx"])
    assert_layer_close(out.float(), g["y_ref"])


def test_tiny_golden(golden):
    g = golden("tiny.npz")
    spec = synth.tiny_spec()
    print("layer tiny H=64 E=8 k=2 I=32", flush=True)
    bank = dsk_moe.ResidentBank.fp4(*(torch.from_numpy(g[f"{r}_{p}"]).to(DEV)
                                      for r in ("w1", "w3", "w2") for p in ("packed", "scales")))
    shared = dsk_moe.SharedExpert(*(torch.from_numpy(g[n]).view(torch.bfloat16).to(DEV)
                                    for n in ("ws1", "ws3", "ws2")))
    x = torch.from_numpy(g["x_bf16"]).view(torch.bfloat16)
    out = dsk_moe.moe_layer(x.to(DEV), torch.from_numpy(g["gate_w"]).to(DEV),
                            torch.from_numpy(g["gate_b"]).to(DEV), bank, shared, spec.k,
                            score_func="sigmoid", route_scale=2.5).cpu()
    assert_layer_close(out.float(), g["y_ref"])


def test_float32_x(cfg0):
    spec, d, _ = cfg0
    g = torch.Generator().manual_seed(3)
    x = torch.randn((6, spec.H), generator=g)
    r = L.moe_forward(x, d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    print("layer cfg0 fp32 x T=6", flush=True)
    out = run_layer(d, spec, x=x)
    assert out.dtype == torch.float32
    assert_layer_close(out, r["y_ref"])


def test_no_shared_and_callable_shared(cfg0):
    spec, d, _ = cfg0
    r0 = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], None, spec)
    print("layer cfg0 no shared", flush=True)
    out0 = run_layer(d, spec, shared=False)
    assert_layer_close(out0.float(), r0["y_ref"])
    # reference tests/test_mlx_forward.py:324-353: a shared callable changes the output
    print("layer cfg0 callable shared", flush=True)
    out1 = run_layer(d, spec, shared_fn=lambda t: torch.ones_like(t) * 0.25)
    assert float((out1.float() - out0.float()).abs().max()) > 1e-3
    want = (r0["y_ref"] + 0.25)
    assert_layer_close(out1.float(), want)


def test_callable_expert_fn_forms(cfg0):
    spec, d, r = cfg0
    bank = to_bank(d["bank"])
    seen = []

    def as_dict(e):
        seen.append(e)
        (w1, s1), (w3, s3), w2 = bank(e)
        return {"w13": (torch.cat([w1, w3]), torch.cat([s1, s3])), "w2": w2}

    hooks = []
    print("layer cfg0 callable expert_fn (w13 dict) + trace hook", flush=True)
    out = run_layer(d, spec, expert_fn=as_dict, layer_id=5,
                    trace_hook=lambda layer, idx, w: hooks.append((layer, idx, w)))
    assert_layer_close(out.float(), r["y_ref"])
    assert sorted(seen) == sorted(set(r["idx"].ravel().tolist()))
    assert len(hooks) == 1 and hooks[0][0] == 5
    assert np.array(hooks[0][1]).shape == (4, spec.k)
    assert np.array_equal(np.array(hooks[0][1])[:, ::-1], r["idx"])
    print("layer cfg0 callable expert_fn (tuple)", flush=True)
    out2 = run_layer(d, spec, expert_fn=lambda e: bank(e))
    assert torch.equal(out2.view(torch.int16), out.view(torch.int16))


def test_sqrtsoftplus_reference_router(cfg0):
    spec, d, _ = cfg0
    spec2 = synth.config0_spec()
    spec2.score_func, spec2.route_scale = 1, 1.5
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec2)
    print("layer cfg0 sqrtsoftplus/1.5", flush=True)
    out = run_layer(d, spec2)
    assert_layer_close(out.float(), r["y_ref"])


def test_deterministic_repeat(cfg0):
    spec, d, _ = cfg0
    a = run_layer(d, spec)
    b = run_layer(d, spec)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


class _LazyBank:
    """Oracle view of a GPU ResidentBank: copies one expert role at a time."""

    def __init__(self, bank: dsk_moe.ResidentBank):
        self.bank, self.quant, self._cache = bank, bank.quant, {}

    def dequant(self, e, role):
        key = (e, role)
        if key not in self._cache:
            from oracle import formats as F
            parts = [t[e].cpu().numpy() for t in self.bank.roles[role]]
            self._cache[key] = F.fp4_dequant(*parts) if self.quant == "fp4" else F.q3_dequant(*parts)
        return self._cache[key]


@pytest.mark.parametrize("T", [1, 2, 8])
def test_full_size_fp4_decode(T):
    """hidden 4096, 256 experts, top-8, inter 2048, bf16 shared 2048 (GPU-generated)."""
    print(f"layer full-size fp4 T={T}", flush=True)
    layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048,
                              inter_shared=2048, seed=1, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(100 + T)
    x = torch.randn((T, 4096), generator=g, device=DEV).to(torch.bfloat16)
    idx = torch.empty((T, 8), dtype=torch.int32, device=DEV)
    out = layer(x, idx=idx).cpu()
    spec = L.LayerSpec(H=4096, E=256, k=8, I=2048, I_shared=2048)
    shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2))
    r = L.moe_forward(x.cpu(), layer.gate_w.cpu(), layer.gate_b.cpu(), _LazyBank(layer.bank), shared, spec)
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


@pytest.mark.parametrize("E,T", [(384, 1), (384, 4), (128, 2)])
def test_decode_expert_table_sizes(E, T):
    """Decode pipeline with 384 experts (top-6): the expert pointer table (72
    bytes per expert) does not fit beside the routing block's state in its
    16 KB of LDS, so the descriptors read the table from global memory; 128
    experts take the LDS copy (up to 152 fit).  Two tokens also take the shared
    tiles' start delay."""
    print(f"layer decode E={E} k=6 T={T}", flush=True)
    layer = gsynth.make_layer(hidden=512, n_experts=E, top_k=6, inter=256,
                              inter_shared=256, seed=30 + E + T, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(300 + E + T)
    x = torch.randn((T, 512), generator=g, device=DEV).to(torch.bfloat16)
    idx = torch.empty((T, 6), dtype=torch.int32, device=DEV)
    out = layer(x, idx=idx).cpu()
    spec = L.LayerSpec(H=512, E=E, k=6, I=256, I_shared=256)
    shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2))
    r = L.moe_forward(x.cpu(), layer.gate_w.cpu(), layer.gate_b.cpu(), _LazyBank(layer.bank), shared, spec)
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


def test_mid_size_batch64():
    """B=64 exercises 4 token tiles per weight tile (hidden 1024, 64 experts, top-8)."""
    spec = L.LayerSpec(H=1024, E=64, k=8, I=512, I_shared=512)
    d = synth.make_layer(spec, 7, 64)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    print("layer mid T=64 H=1024 E=64 k=8", flush=True)
    out = run_layer(d, spec)
    assert_layer_close(out.float(), r["y_ref"])


# ---------------------------------------------------------------- q3 experts
@pytest.mark.parametrize("name,spec,T", [
    ("tiny", synth.tiny_spec(L.QUANT_Q3), 4),
    ("cfg0-shape", L.LayerSpec(H=1024, E=64, k=6, I=512, I_shared=512, quant=L.QUANT_Q3), 4),
    ("mid T=64", L.LayerSpec(H=1024, E=64, k=8, I=512, I_shared=512, quant=L.QUANT_Q3), 64),
])
def test_q3_layer(name, spec, T):
    """q3 affine (g64, fp16 scale/bias) routed experts against the oracle."""
    print(f"layer q3 {name} T={T}", flush=True)
    d = synth.make_layer(spec, 11, T)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    idx = torch.empty((T, spec.k), dtype=torch.int32, device=DEV)
    layer = dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                             to_shared(d["shared"]), spec.k)
    out = layer(d["x"].to(DEV), idx=idx).cpu()
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


@pytest.mark.parametrize("T", [1, 16])
def test_full_size_q3(T):
    """hidden 4096, 256 q3 experts, top-8, inter 2048, bf16 shared 2048 (GPU-generated)."""
    print(f"layer full-size q3 T={T}", flush=True)
    layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048,
                              inter_shared=2048, quant="q3", seed=2, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(200 + T)
    x = torch.randn((T, 4096), generator=g, device=DEV).to(torch.bfloat16)
    idx = torch.empty((T, 8), dtype=torch.int32, device=DEV)
    out = layer(x, idx=idx).cpu()
    spec = L.LayerSpec(H=4096, E=256, k=8, I=2048, I_shared=2048, quant=L.QUANT_Q3)
    shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2))
    r = L.moe_forward(x.cpu(), layer.gate_w.cpu(), layer.gate_b.cpu(), _LazyBank(layer.bank), shared, spec)
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


@pytest.mark.parametrize("T", [4, 40])
def test_pinned_gather_contributions(cfg0, T):
    """moe_layer(pinned_gather_fn=...): the callback's weighted rows replace the
    selected experts it returns (reference mlx_forward.py:313-321, 388-393).
    The callback here doubles the true contribution of every other selected
    expert, so the output must follow the callback, not the bank."""
    spec, _, _ = cfg0
    print(f"layer pinned gather T={T}", flush=True)
    d = synth.make_layer(spec, 7, T)
    seen = {}

    def pinned_fn(layer_id, x, idx_np, w_np):
        seen["idx"] = np.array(idx_np)
        sel = sorted({int(v) for v in np.asarray(idx_np).ravel() if v >= 0})[::2]
        x32 = x.detach().cpu().float()
        res = {}
        for e in sel:
            w1, w3, w2 = (torch.from_numpy(d["bank"].dequant(e, n)) for n in ("w1", "w3", "w2"))
            rows, outs = [], []
            for r in range(idx_np.shape[0]):
                for c in range(idx_np.shape[1]):
                    if int(idx_np[r, c]) == e:
                        h = L.swiglu(x32[r:r + 1] @ w1.T, x32[r:r + 1] @ w3.T, spec.limit) * float(w_np[r, c])
                        rows.append(r)
                        outs.append(2.0 * (h @ w2.T)[0])
            res[e] = (np.asarray(rows, dtype=np.int32), torch.stack(outs))
        seen["res"] = res
        return res

    out = run_layer(d, spec, pinned_gather_fn=pinned_fn, layer_id=3)
    plain = run_layer(d, spec)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec, pinned=seen["res"])
    # the callback sees the routing in the reference's order (the trace hook's)
    np.testing.assert_array_equal(seen["idx"], np.flip(r["idx"], axis=1))
    assert_layer_close(out.float(), r["y_ref"])
    assert float((out.float() - plain.float()).abs().max()) > 1e-3


def test_capture_without_warmup_is_refused():
    """A workspace cannot be created while its stream is captured (its zero-fill
    would only be recorded into the graph): the call raises before any launch,
    and after an eager call on that stream the capture works."""
    spec = synth.tiny_spec()
    d = synth.make_layer(spec, 3, 2)
    layer = dsk_moe.MoELayer(d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                             to_shared(d["shared"]), spec.k)
    x = d["x"].to(DEV)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with pytest.raises(RuntimeError, match="no workspace"):
            with torch.cuda.graph(g, stream=side):
                layer(x)
        want = layer(x).clone()              # eager call: the stream's workspace now exists
        side.synchronize()
        g2 = torch.cuda.CUDAGraph()
        out = torch.empty_like(x)
        with torch.cuda.graph(g2, stream=side):
            layer(x, out=out)
    for _ in range(2):
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
