"""Routing of the decode pipeline (its routing block: top-k, slot map and
dispatch rows in one workgroup) against the oracle router, bit for bit:
indices in selection order and route weights.  Batches whose (token, expert)
pairs fit 1024 words (E rounded up to 16, E <= 512) take the rank form of the
routing block, larger ones the serial form; the cases cover both, expert
counts that are not multiples of 16, exact score ties (lower expert id
first), every expert selected (k = E) and one token per expert set.  The layer
output checks the slot map and dispatch rows the expert kernels read."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from dsk_moe import synth as gsynth
from oracle import layer as L
from oracle import router as R
from conftest import assert_layer_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _LazyBank:
    def __init__(self, bank):
        self.bank, self.quant, self._cache = bank, bank.quant, {}

    def dequant(self, e, role):
        key = (e, role)
        if key not in self._cache:
            from oracle import formats as F
            parts = [t[e].cpu().numpy() for t in self.bank.roles[role]]
            self._cache[key] = F.fp4_dequant(*parts)
        return self._cache[key]


def _run(layer, x, k, check_output):
    T = x.shape[0]
    idx = torch.empty((T, k), dtype=torch.int32, device=DEV)
    w = torch.empty((T, k), dtype=torch.float32, device=DEV)
    out = layer(x, idx=idx, w=w)
    ridx, rw, _, _ = R.route(x.cpu().float().numpy(), layer.gate_w.cpu().float().numpy(),
                             layer.gate_b.cpu().numpy(), k, R.SCORE_SIGMOID, layer.route_scale)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(w.cpu().numpy(), rw)
    if check_output:
        H, E = x.shape[1], layer.gate_w.shape[0]
        spec = L.LayerSpec(H=H, E=E, k=k, I=layer.bank.inter, I_shared=layer.shared.inter)
        shared = tuple(t.cpu() for t in (layer.shared.w1, layer.shared.w3, layer.shared.w2))
        r = L.moe_forward(x.cpu(), layer.gate_w.cpu(), layer.gate_b.cpu(), _LazyBank(layer.bank), shared, spec)
        assert_layer_close(out.cpu().float(), r["y_ref"])
    return ridx


@pytest.mark.parametrize("E,k,T", [(256, 8, 1), (256, 8, 2), (256, 8, 4), (256, 8, 5), (256, 4, 16),
                                   (384, 6, 1), (384, 6, 2), (384, 6, 3), (20, 3, 1), (20, 5, 2),
                                   (20, 4, 16), (8, 8, 2), (8, 1, 1)])
def test_decode_route_bit_exact(E, k, T):
    print(f"decode route E={E} k={k} T={T}", flush=True)
    layer = gsynth.make_layer(hidden=256, n_experts=E, top_k=k, inter=256, inter_shared=256,
                              seed=900 + E + T + k, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(910 + E + T + k)
    x = torch.randn((T, 256), generator=g, device=DEV).to(torch.bfloat16)
    ridx = _run(layer, x, k, check_output=T <= 4)
    if k == E:
        assert all(sorted(r) == list(range(E)) for r in ridx.tolist())


@pytest.mark.parametrize("T", [1, 2, 5])
def test_decode_route_exact_ties(T):
    """Experts e, e + 16, e + 32, ... share gate rows and bias: equal keys, the
    lower id is selected first."""
    print(f"decode route ties T={T}", flush=True)
    layer = gsynth.make_layer(hidden=256, n_experts=128, top_k=8, inter=256, inter_shared=256,
                              seed=950 + T, device=DEV)
    layer.gate_w = layer.gate_w[:16].repeat(8, 1).contiguous()
    layer.gate_b = layer.gate_b[:16].repeat(8).contiguous()
    g = torch.Generator(device=DEV).manual_seed(960 + T)
    x = torch.randn((T, 256), generator=g, device=DEV).to(torch.bfloat16)
    ridx = _run(layer, x, 8, check_output=T <= 2)
    for row in ridx:
        for a, b in zip(row[:-1], row[1:]):
            if a % 16 == b % 16:
                assert a < b
