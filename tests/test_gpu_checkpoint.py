"""GPU checks of the checkpoint loader.

* dsk_fp8_block_dequant against the oracle on every E4M3 byte and a range of
  E8M0 scales (including 0 and 0xFF), float32 bit for bit and bf16 (the
  scaled E4M3 values are exact in bf16).
* A synthetic checkpoint in the real layout (FP4 experts, FP8 shared expert,
  BF16 gate, two shards): Checkpoint.load_layer -> MoELayer against the oracle
  evaluated on the written arrays (routing bit-exact, output within the layer
  tolerance), and the loaded banks byte-identical to the files.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from dsk_moe.checkpoint import Checkpoint, fp8_block_dequant
from oracle import formats as F
from oracle import layer as L
from ckpt_synth import make_checkpoint
from conftest import assert_layer_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    return bool(((np.isnan(a) & np.isnan(b)) | (a.view(np.uint32) == b.view(np.uint32))).all())


def test_fp8_block_dequant_kernel():
    print("fp8 block dequant", flush=True)
    rows, cols = 64, 512
    codes = np.tile(np.arange(256, dtype=np.uint8), rows * cols // 256).reshape(rows, cols)
    np.random.default_rng(8).shuffle(codes, axis=1)
    scales = np.array([[0, 1, 100, 120, 127, 134, 200, 254, 255, 126, 127, 128, 129, 130, 131, 132],
                       [127] * 16], dtype=np.uint8)
    want = F.fp8_block_dequant(codes, scales)
    cd, sd = torch.from_numpy(codes).to(DEV), torch.from_numpy(scales).to(DEV)
    got32 = fp8_block_dequant(cd, sd, torch.float32).cpu().numpy()
    assert _same_bits(got32, want)
    got16 = fp8_block_dequant(cd, sd, torch.bfloat16).float().cpu().numpy()
    want16 = torch.from_numpy(want).to(torch.bfloat16).float().numpy()
    assert _same_bits(got16, want16)


@pytest.mark.parametrize("T", [1, 5, 40])
def test_load_layer_from_checkpoint(tmp_path, T):
    print(f"checkpoint layer T={T}", flush=True)
    spec = L.LayerSpec(H=256, E=8, k=2, I=128, I_shared=128)
    d = make_checkpoint(tmp_path, spec, 11)
    ck = Checkpoint(tmp_path, d["manifest"])
    layer = ck.load_layer(0, DEV, score_func="sigmoid", route_scale=spec.route_scale)
    packed, scales = d["bank"].roles["w3"]
    assert torch.equal(layer.bank.roles["w3"][0].cpu(), torch.from_numpy(packed))
    assert torch.equal(layer.bank.roles["w3"][1].cpu(), torch.from_numpy(scales))
    for got, want in zip((layer.shared.w1, layer.shared.w3, layer.shared.w2), d["shared"]):
        assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))
    x = (torch.randn((T, spec.H), generator=torch.Generator().manual_seed(T)) * 1.0).to(torch.bfloat16)
    idx = torch.empty((T, spec.k), dtype=torch.int32, device=DEV)
    out = layer(x.to(DEV), idx=idx).cpu()
    r = L.moe_forward(x, d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)


@pytest.mark.parametrize("T", [1, 40])
def test_load_q3_layer_from_checkpoint(tmp_path, T):
    """A synthetic checkpoint with q3 routed experts as the reference's q3 variant
    stores them (U32_Q3_AFFINE words [N, 3K/32] of row-major 3-byte packs, F16
    scale / bias): the loaded bank holds the canonical layout of the same codes
    (repacked on the device), and the layer matches the oracle."""
    print(f"checkpoint q3 layer T={T}", flush=True)
    spec = L.LayerSpec(H=256, E=8, k=2, I=384, I_shared=128, quant=L.QUANT_Q3)
    d = make_checkpoint(tmp_path, spec, 12)
    ck = Checkpoint(tmp_path, d["manifest"])
    assert ck.expert_format(0) == "q3"
    layer = ck.load_layer(0, DEV, score_func="sigmoid", route_scale=spec.route_scale)
    assert layer.bank.quant == "q3"
    for role in ("w1", "w3", "w2"):
        for got, want in zip(layer.bank.roles[role], d["bank"].roles[role]):
            assert np.array_equal(got.cpu().numpy().view(np.uint8), np.ascontiguousarray(want).view(np.uint8)), role
    x = torch.randn((T, spec.H), generator=torch.Generator().manual_seed(50 + T)).to(torch.bfloat16)
    idx = torch.empty((T, spec.k), dtype=torch.int32, device=DEV)
    out = layer(x.to(DEV), idx=idx).cpu()
    r = L.moe_forward(x, d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    np.testing.assert_array_equal(idx.cpu().numpy(), r["idx"])
    c, rel = assert_layer_close(out.float(), r["y_ref"])
    print(f"cos={c:.9f} rel={rel:.2e}", flush=True)
