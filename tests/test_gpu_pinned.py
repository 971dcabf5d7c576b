"""GPU parity of the pinned-expert contributions (``dsk_expert_rows``,
``dsk_moe.pinned.gather_pinned_contributions``) and of ``moe_layer`` driven by
them, against the oracle.

The contributions are compared pair by pair with the oracle's own per-pair
products (every (row, slot) routed to a pinned expert, float32 x, the route
weight before w2: the reference's ``gather_pinned_contributions``,
``src/deepseeker/mlx_forward.py:159-210``) within the layer tolerance; rows and
pair order exactly.  The pin bank holds its experts in a shuffled slot order,
so the (expert, row) order of the result cannot come from the bank.  A layer
whose ``pinned_gather_fn`` returns them must match the oracle layer, and
within the float32 sum the pinned rows take their ascending-expert place
(checked against the oracle given the very same contribution tensors).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import dsk_moe
from dsk_moe.pinned import gather_pinned_contributions
from oracle import layer as L
from oracle import synth
from conftest import assert_layer_close
from test_gpu_layer import run_layer, to_bank

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _oracle_pairs(spec, d, idx, w, experts):
    """{expert: (rows, [n, H] float32)}: one (row, slot) pair at a time, float32 x."""
    x32 = d["x"].float()
    out = {}
    for e in experts:
        w1, w3, w2 = (torch.from_numpy(d["bank"].dequant(e, n)) for n in ("w1", "w3", "w2"))
        rows, outs = [], []
        for t in range(idx.shape[0]):
            for j in range(idx.shape[1]):
                if int(idx[t, j]) == e:
                    h = L.swiglu(x32[t:t + 1] @ w1.T, x32[t:t + 1] @ w3.T, spec.limit) * float(w[t, j])
                    rows.append(t)
                    outs.append((h @ w2.T)[0])
        if rows:
            out[e] = (np.asarray(rows, dtype=np.int32), torch.stack(outs))
    return out


def _pin_bank(bank: dsk_moe.ResidentBank, experts, seed: int):
    """The pinned experts stacked in a shuffled slot order, and {expert: slot}."""
    order = np.random.default_rng(seed).permutation(len(experts))
    chosen = [experts[i] for i in order]
    sel = torch.tensor(chosen, dtype=torch.int64, device=DEV)
    roles = {r: tuple(t.index_select(0, sel).contiguous() for t in parts) for r, parts in bank.roles.items()}
    return roles, {e: s for s, e in enumerate(chosen)}


@pytest.mark.parametrize("quant,T", [("fp4", 4), ("fp4", 40), ("q3", 6), ("fp4", 300)])
def test_gather_pinned_contributions_pairs(quant, T):
    spec = synth.config0_spec()
    if quant == "q3":
        spec.quant = L.QUANT_Q3
    print(f"pinned contributions {quant} T={T}", flush=True)
    d = synth.make_layer(spec, 31 + T, T)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], None, spec)
    sel = sorted({int(v) for v in r["idx"].ravel()})
    experts = sel[::3] + [e for e in range(spec.E) if e not in sel][:2]    # two pinned experts get no pair
    roles, slots = _pin_bank(to_bank(d["bank"]), experts, T)
    idx_ref, w_ref = np.flip(r["idx"], axis=1), np.flip(r["w"], axis=1)     # the reference's slot order
    got = gather_pinned_contributions(d["x"].to(DEV), idx_ref, w_ref, roles, slots, spec.limit)
    want = _oracle_pairs(spec, d, r["idx"], r["w"], experts)
    assert sorted(got) == sorted(want)
    for e in want:
        np.testing.assert_array_equal(got[e][0], want[e][0])
        assert got[e][1].dtype == torch.float32 and got[e][1].device.type == "cuda"
    g = torch.cat([got[e][1].cpu() for e in sorted(want)])
    ref = torch.cat([want[e][1] for e in sorted(want)])
    c, rel = assert_layer_close(g, ref)
    print(f"pairs={g.shape[0]} cos={c:.9f} rel={rel:.2e}", flush=True)


@pytest.mark.parametrize("T", [5, 40])
def test_layer_with_device_pinned_gather(T):
    """moe_layer(pinned_gather_fn=...) with the device contributions: the oracle layer."""
    spec = synth.config0_spec()
    print(f"layer with device pinned gather T={T}", flush=True)
    d = synth.make_layer(spec, 51 + T, T)
    bank = to_bank(d["bank"])
    pin = [e for e in range(0, spec.E, 2)]
    roles, slots = _pin_bank(bank, pin, 7)
    seen = {}

    def pinned_fn(layer_id, x, idx_np, w_np):
        res = gather_pinned_contributions(x, idx_np, w_np, roles, slots, spec.limit)
        seen["res"] = {e: (rows, c.cpu()) for e, (rows, c) in res.items()}
        return res

    out = run_layer(d, spec, pinned_gather_fn=pinned_fn)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    assert seen["res"], "no pinned expert was routed"
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    # the oracle given the same pinned rows: only the non-pinned products differ
    rp = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec, pinned=seen["res"])
    c2, rel2 = assert_layer_close(out.float(), rp["y_ref"])
    print(f"pinned={len(seen['res'])} cos={c:.9f} rel={rel:.2e}; same rows cos={c2:.9f}", flush=True)


def test_pinned_rows_take_their_ascending_place():
    """Every selected expert pinned with the oracle's own rows: the device sum is
    the oracle's float32 sum in ascending expert order, bit for bit."""
    spec = synth.config0_spec()
    T = 12
    d = synth.make_layer(spec, 77, T)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    sel = sorted({int(v) for v in r["idx"].ravel()})
    pairs = _oracle_pairs(spec, d, r["idx"], r["w"], sel)
    # rows listed in descending order: their position in the sum must not depend on it
    rev = {e: (rows[::-1].copy(), c.flip(0)) for e, (rows, c) in pairs.items()}
    out = run_layer(d, spec, shared=False,
                    pinned_gather_fn=lambda *_: {e: (rows, c.to(DEV)) for e, (rows, c) in rev.items()})
    rp = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], None, spec, pinned=rev)
    np.testing.assert_array_equal(out.float().numpy(), rp["out"].float().numpy())
