"""dsk_cap_union (the reference's cap_union, src/deepseeker/mlx_forward.py:213-254)
against the oracle, bit for bit in indices and weights, and moe_layer with
union_budget > 0 against the oracle layer evaluated on the oracle's capped routing."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import dsk_moe
from dsk_moe.ops import cap_union
from oracle import layer as L
from oracle import router as R
from oracle import synth
from oracle import union as U
from conftest import assert_layer_close
from test_gpu_layer import to_bank, to_shared

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _routing(rng, T, k, E, ties):
    scores = (rng.random((T, E)) + 0.01).astype(np.float32)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    w = np.take_along_axis(scores, idx, 1).astype(np.float32)
    if ties:                           # equal weights in some rows: the rescue's first maximum
        w[::3] = np.float32(0.25)
    return scores, idx, w


@pytest.mark.parametrize("T,k,E,budget", [(2, 2, 16, 2), (5, 6, 64, 9), (16, 8, 256, 24), (64, 8, 256, 40),
                                          (300, 6, 384, 60), (40, 12, 64, 13), (33, 16, 64, 20), (8, 8, 256, 64)])
@pytest.mark.parametrize("strict", [False, True])
def test_cap_union_kernel_bit_exact(T, k, E, budget, strict):
    print(f"cap_union T={T} k={k} E={E} budget={budget} strict={strict}", flush=True)
    rng = np.random.default_rng(T * 1000 + k * 10 + budget)
    for ties in (False, True):
        scores, idx, w = _routing(rng, T, k, E, ties)
        want_i, want_w, _ = U.cap_union(idx, w, E, budget, scores=scores, strict=strict)
        ti, tw = torch.from_numpy(idx).to(DEV), torch.from_numpy(w).to(DEV)
        cap_union(torch.from_numpy(scores).to(DEV), ti, tw, budget, strict)
        np.testing.assert_array_equal(ti.cpu().numpy(), want_i)
        np.testing.assert_array_equal(tw.cpu().numpy().view(np.uint32), want_w.view(np.uint32))


@pytest.mark.parametrize("T,budget,strict", [(16, 20, False), (32, 12, True), (6, 50, False)])
def test_moe_layer_union_budget(T, budget, strict):
    """cfg0 shape (hidden 1024, 64 experts, top-6): device routing capped on the GPU,
    compared with the oracle router + cap_union + oracle layer on the same inputs."""
    print(f"moe_layer union_budget={budget} T={T} strict={strict}", flush=True)
    spec = synth.config0_spec()
    d = synth.make_layer(spec, 31, T)
    x32 = d["x"].float().numpy()
    r_idx, r_w, r_s, r_z = R.route(x32, d["gate_w"].numpy(), d["gate_b"].numpy(), spec.k, spec.score_func,
                                   spec.route_scale)
    c_idx, c_w, cov = U.cap_union(r_idx, r_w, spec.E, budget, scores=r_s, strict=strict)
    ref = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec,
                        routing=(c_idx, c_w, r_s, r_z))
    hooks, stats = [], {"coverage": 0.0, "calls": 0.0}
    out = dsk_moe.moe_layer(d["x"].to(DEV), d["gate_w"].to(DEV), d["gate_b"].to(DEV), to_bank(d["bank"]),
                            to_shared(d["shared"]), spec.k, spec.limit,
                            trace_hook=lambda layer, i, ww: hooks.append((i, ww)), union_budget=budget,
                            route_stats=stats, union_strict=strict, score_func="sigmoid",
                            route_scale=spec.route_scale).cpu()
    got_i = np.asarray(hooks[0][0], dtype=np.int32)[:, ::-1]
    got_w = np.asarray(hooks[0][1], dtype=np.float32)[:, ::-1]
    np.testing.assert_array_equal(got_i, c_idx)
    np.testing.assert_array_equal(got_w.view(np.uint32), c_w.view(np.uint32))
    assert (c_idx < 0).any() == (np.unique(r_idx).size > budget)
    c, rel = assert_layer_close(out.float(), ref["y_ref"])
    assert stats["calls"] == T and abs(stats["coverage"] / T - cov) < 1e-6
    print(f"cos={c:.9f} rel={rel:.2e} coverage={cov:.4f} union={np.unique(r_idx).size}", flush=True)
