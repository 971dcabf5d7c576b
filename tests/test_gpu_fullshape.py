"""GPU parity at full shapes, every checked row against the oracle.

* q3 layer of the batch sweep (hidden 4096, 256 experts, top-8, inter 2048,
  bf16 shared 2048) at 64 tokens, with uniform routing (~222 experts, the
  grouped path's factored q3 gate/up and down) and with a Zipf(1.1) gate bias
  (a few hot experts spanning several 8-row column tiles): all 64 rows.
* The reference model's own geometry (DeepSeek-V4.1-Flash: hidden 5120,
  384 experts, top-6, expert and shared intermediate 2304, sqrt-softplus
  scores, route scale 1.5; ``profiles/deepseek-v4.1-flash/*/model-manifest.json``
  ``layers.*.ffn.experts.*.w1.weight [2304, 2560]``): FP4 at 1 and 8 tokens
  (decode pipeline, grouped path) and 300 tokens (prefill GEMM; routing of all
  rows, output of every tenth row), q3 at 1 and 16 tokens (K = 2304 is not a
  multiple of 512: superblock tails and the non-factored q3 down).
* Top-k 12 and 16 (the combine's rows past 8, and the decode pipeline's slot
  map with 16 selections per token).
* The FP4 batch-sweep layer (hidden 4096, 256 experts, top-8, inter 2048) at
  64 tokens, every row: the grouped path with ~160 experts, some of them over
  several 8-row column tiles.
* float32 activations at that shape (the reference's tests call the layer
  with float32 x) at 1, 8 and 64 tokens: the general path's hi/lo bf16
  operand split, routing bit-exact.
* q3 experts through the prefill GEMM (from 128 tokens) at both full shapes:
  hidden 4096 / inter 2048 at 256 tokens and the reference geometry at 160
  tokens (routing of every row, output of every other row).

Routing indices and weights bit-exact; outputs within the layer tolerance
(cosine >= 0.99999 and max|y - y_ref| / max|y_ref| <= 1e-2).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from dsk_moe import synth as gsynth
from oracle import layer as L
from oracle import router as R
from conftest import DeviceBankView, assert_layer_close

pytestmark = pytest.mark.gpu
DEV = "cuda"

REF_GEOMETRY = dict(hidden=5120, n_experts=384, top_k=6, inter=2304, inter_shared=2304,
                    score_func="sqrtsoftplus", route_scale=1.5)


def _spec(layer, quant: str) -> L.LayerSpec:
    return L.LayerSpec(H=layer.gate_w.shape[1], E=layer.bank.n_experts, k=layer.top_k, I=layer.bank.inter,
                       I_shared=layer.shared.inter if layer.shared else 0,
                       score_func=R.SCORE_SQRTSOFTPLUS if layer.score_func == "sqrtsoftplus" else R.SCORE_SIGMOID,
                       route_scale=layer.route_scale, limit=layer.limit, quant=quant)


def check_layer(layer, x: torch.Tensor, quant: str, label: str, rows=None):
    """Run the layer on all of x; compare routing of every row and the output of ``rows``."""
    T, k = x.shape[0], layer.top_k
    print(f"{label}: T={T} checked rows={'all' if rows is None else len(rows)}", flush=True)
    idx = torch.empty((T, k), dtype=torch.int32, device=DEV)
    w = torch.empty((T, k), dtype=torch.float32, device=DEV)
    out = layer(x, idx=idx, w=w).cpu()
    idx_h, w_h = idx.cpu().numpy(), w.cpu().numpy()
    spec = _spec(layer, quant)
    xc = x.cpu()
    r_idx, r_w, _, _ = R.route(xc.float().numpy(), layer.gate_w.cpu().float().numpy(),
                               layer.gate_b.cpu().numpy(), k, spec.score_func, spec.route_scale)
    np.testing.assert_array_equal(idx_h, r_idx)
    np.testing.assert_array_equal(w_h, r_w)
    sel = np.arange(T) if rows is None else np.asarray(rows)
    view = DeviceBankView(layer.bank).prefetch(idx_h[sel].ravel())
    shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2)) if layer.shared else None
    try:
        r = L.moe_forward(xc[torch.from_numpy(sel)], layer.gate_w.cpu(), layer.gate_b.cpu(), view, shared, spec)
    finally:
        view.close()
    np.testing.assert_array_equal(idx_h[sel], r["idx"])
    c, rel = assert_layer_close(out[torch.from_numpy(sel)].float(), r["y_ref"])
    counts = np.bincount(idx_h.ravel(), minlength=layer.bank.n_experts)
    print(f"cos={c:.9f} rel={rel:.2e} active={int((counts > 0).sum())} max_rows={int(counts.max())}",
          flush=True)


def _x(T: int, H: int, seed: int) -> torch.Tensor:
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn((T, H), generator=g, device=DEV).to(torch.bfloat16)


# ---------------------------------------------------------------- q3 sweep layer at 64 tokens
@pytest.mark.parametrize("zipf", [None, 1.1])
def test_q3_batch64_all_rows(zipf):
    layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048, inter_shared=2048,
                              quant="q3", seed=12, device=DEV, zipf_s=zipf)
    check_layer(layer, _x(64, 4096, 640), "q3", f"q3 H4096 E256 k8 I2048 zipf={zipf}")
    del layer
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- the reference model's geometry
@pytest.fixture(scope="module")
def ref_fp4():
    layer = gsynth.make_layer(**REF_GEOMETRY, quant="fp4", seed=51, device=DEV)
    yield layer
    del layer
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 8, 300])
def test_reference_geometry_fp4(ref_fp4, T):
    rows = None if T <= 8 else list(range(0, T, 10))
    check_layer(ref_fp4, _x(T, 5120, 5100 + T), "fp4", "ref geometry fp4 H5120 E384 k6 I2304", rows)


@pytest.mark.parametrize("T", [1, 16])
def test_reference_geometry_q3(T):
    layer = gsynth.make_layer(**REF_GEOMETRY, quant="q3", seed=52, device=DEV)
    check_layer(layer, _x(T, 5120, 5200 + T), "q3", "ref geometry q3 H5120 E384 k6 I2304")
    del layer
    torch.cuda.empty_cache()


# ---------------------------------------------------------------- wide top-k
@pytest.mark.parametrize("k,T", [(16, 2), (12, 3), (16, 8), (16, 40)])
def test_wide_topk(k, T):
    layer = gsynth.make_layer(hidden=1024, n_experts=64, top_k=k, inter=512, inter_shared=512,
                              seed=80 + k + T, device=DEV)
    check_layer(layer, _x(T, 1024, 800 + k + T), "fp4", f"top-{k} H1024 E64 I512")


# ---------------------------------------------------------------- FP4 batch sweep layer, bf16 and float32 x
@pytest.fixture(scope="module")
def sweep_fp4():
    layer = gsynth.make_layer(hidden=4096, n_experts=256, top_k=8, inter=2048, inter_shared=2048,
                              quant="fp4", seed=11, device=DEV)
    yield layer
    del layer
    torch.cuda.empty_cache()


def test_fp4_batch64_all_rows(sweep_fp4):
    check_layer(sweep_fp4, _x(64, 4096, 641), "fp4", "fp4 H4096 E256 k8 I2048 B=64")


@pytest.mark.parametrize("T", [1, 8, 64])
def test_fp32_activations_full_size(sweep_fp4, T):
    """float32 x with values off the bf16 grid (the operand's hi/lo split matters)."""
    g = torch.Generator(device=DEV).manual_seed(900 + T)
    x = torch.randn((T, 4096), generator=g, device=DEV, dtype=torch.float32)
    assert not torch.equal(x, x.to(torch.bfloat16).float())
    check_layer(sweep_fp4, x, "fp4", "fp4 H4096 E256 k8 I2048 float32 x")


# ---------------------------------------------------------------- q3 through the prefill GEMM at full shape
@pytest.mark.parametrize("geometry,T", [("sweep", 256), ("reference", 160)])
def test_q3_prefill_full_shape(geometry, T):
    if geometry == "sweep":
        kw = dict(hidden=4096, n_experts=256, top_k=8, inter=2048, inter_shared=2048)
    else:
        kw = dict(REF_GEOMETRY)
    layer = gsynth.make_layer(**kw, quant="q3", seed=53, device=DEV)
    H = kw["hidden"]
    check_layer(layer, _x(T, H, 5300 + T), "q3", f"q3 prefill {geometry} H{H}", rows=list(range(0, T, 2)))
    del layer
    torch.cuda.empty_cache()
