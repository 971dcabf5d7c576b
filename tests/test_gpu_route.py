"""GPU router parity: scores, indices and weights bit-identical to the oracle."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import dsk_moe
from oracle import router as R
from oracle import synth

pytestmark = pytest.mark.gpu
DEV = "cuda"
SF = {"sigmoid": R.SCORE_SIGMOID, "sqrtsoftplus": R.SCORE_SQRTSOFTPLUS}


def check(x, gate_w, gate_b, k, score_func, route_scale):
    print(f"route T={x.shape[0]} H={x.shape[1]} E={gate_w.shape[0]} k={k} {score_func} "
          f"x={x.dtype} gate={gate_w.dtype}", flush=True)
    w, idx, s = dsk_moe.route(x.to(DEV), gate_w.to(DEV), gate_b.to(DEV), k, score_func, route_scale)
    ridx, rw, rs, _ = R.route(x.float().numpy(), gate_w.float().numpy(), gate_b.numpy(), k,
                              SF[score_func], route_scale)
    np.testing.assert_array_equal(s.cpu().numpy(), rs)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    np.testing.assert_array_equal(w.cpu().numpy(), rw)
    return idx.cpu().numpy(), w.cpu().numpy()


def test_route_config0_bit_exact():
    d = synth.make_layer(synth.config0_spec(), 0, 4)
    check(d["x"], d["gate_w"], d["gate_b"], 6, "sigmoid", 2.5)


@pytest.mark.parametrize("T,H,E,k", [(1, 4096, 256, 8), (8, 4096, 256, 8), (64, 4096, 256, 8),
                                     (20, 1056, 100, 5), (3, 64, 8, 2), (33, 512, 384, 6)])
@pytest.mark.parametrize("score_func", ["sigmoid", "sqrtsoftplus"])
def test_route_random_bit_exact(T, H, E, k, score_func):
    g = torch.Generator().manual_seed(T * 7 + E)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    gate_w = torch.randn((E, H), generator=g) / math.sqrt(H)
    gate_b = torch.rand((E,), generator=g) * 0.2 - 0.1
    idx, w = check(x, gate_w, gate_b, k, score_func, 2.5 if score_func == "sigmoid" else 1.5)
    np.testing.assert_allclose(w.sum(axis=1), 2.5 if score_func == "sigmoid" else 1.5, rtol=1e-5)


def test_route_float32_x_and_bf16_gate():
    g = torch.Generator().manual_seed(9)
    x = torch.randn((5, 2048), generator=g)
    gate_w = (torch.randn((64, 2048), generator=g) / 45).to(torch.bfloat16)
    gate_b = torch.rand((64,), generator=g) * 0.2 - 0.1
    check(x, gate_w, gate_b, 6, "sigmoid", 2.5)


def test_route_exact_ties_prefer_lower_index():
    g = torch.Generator().manual_seed(4)
    x = torch.randn((4, 256), generator=g).to(torch.bfloat16)
    base = torch.randn((8, 256), generator=g) / 16
    gate_w = base.repeat(4, 1)                       # experts e, e+8, e+16, e+24 tie exactly
    gate_b = torch.zeros(32)
    idx, _ = check(x, gate_w, gate_b, 6, "sigmoid", 2.5)
    for row in idx:
        for a, b in zip(row[:-1], row[1:]):
            if a % 8 == b % 8:
                assert a < b


def test_route_k_equals_e_and_k_one():
    g = torch.Generator().manual_seed(2)
    x = torch.randn((7, 128), generator=g).to(torch.bfloat16)
    gate_w = torch.randn((16, 128), generator=g) / 11
    gate_b = torch.zeros(16)
    idx, _ = check(x, gate_w, gate_b, 16, "sqrtsoftplus", 1.5)
    assert all(sorted(r) == list(range(16)) for r in idx.tolist())
    check(x, gate_w, gate_b, 1, "sigmoid", 2.5)


def test_route_zipf_bias_skew():
    g = torch.Generator().manual_seed(1)
    x = torch.randn((256, 1024), generator=g).to(torch.bfloat16)
    gate_w = torch.randn((256, 1024), generator=g) / 32
    gate_b = torch.from_numpy(synth.zipf_bias(256, 1.1))
    idx, _ = check(x, gate_w, gate_b, 8, "sigmoid", 2.5)
    counts = np.bincount(idx.ravel(), minlength=256)
    assert counts[0] > counts[-64:].mean()


@pytest.mark.parametrize("T,H,E,k,score_func", [(128, 4096, 256, 8, "sigmoid"), (300, 1056, 100, 5, "sqrtsoftplus"),
                                                (130, 64, 24, 3, "sigmoid"), (257, 2048, 384, 6, "sqrtsoftplus"),
                                                (129, 256, 40, 4, "sigmoid"), (200, 512, 64, 6, "sigmoid")])
@pytest.mark.parametrize("xdt,gdt", [("bf16", "f32"), ("f32", "f32"), ("bf16", "bf16"), ("f32", "bf16")])
def test_route_wide_gate_bit_exact(T, H, E, k, score_func, xdt, gdt):
    """Batches of >= 128 tokens take the wide gate kernel (32x16 tiles staged through
    LDS, segment sums by reduce-scatter); H = 64 and 1056 leave segments empty and
    stage through registers, the multiples of 256 by LDS DMA (H = 256 and 512: one
    and two steps, shorter than the DMA pipeline)."""
    g = torch.Generator().manual_seed(T + H + E)
    x = torch.randn((T, H), generator=g)
    x = x.to(torch.bfloat16) if xdt == "bf16" else x
    gate_w = torch.randn((E, H), generator=g) / math.sqrt(H)
    gate_w = gate_w.to(torch.bfloat16) if gdt == "bf16" else gate_w
    gate_b = torch.rand((E,), generator=g) * 0.2 - 0.1
    check(x, gate_w, gate_b, k, score_func, 2.5 if score_func == "sigmoid" else 1.5)
