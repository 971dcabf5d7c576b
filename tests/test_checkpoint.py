"""CPU checks of the checkpoint loader's host side and the FP8 E4M3 oracle.

* The oracle's E4M3 table against torch's float8_e4m3fn decode of all 256
  bytes and the reference's spot values (tests/test_mlx_weights.py:47-57);
  the FP8 block dequant on the reference's seeded recipe (:64-74).
* expert_ranges on the reference's synthetic manifest
  (tests/test_checkpoint_io.py:23-44).
* The reference's real manifest, as a subset fixture: record layout of the
  FP4 experts, the FP8 shared expert and the gate, offsets, per-expert bytes.
* write_safetensors / build_manifest / Checkpoint.read round trip, with the
  safetensors library reading the same files.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from dsk_moe.checkpoint import Checkpoint, build_manifest, expert_ranges, write_safetensors
from oracle import formats as F
from oracle import layer as L
from ckpt_synth import make_checkpoint

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_e4m3_table_matches_torch_and_reference_spots():
    want = torch.frombuffer(bytearray(range(256)), dtype=torch.float8_e4m3fn).float().numpy()
    t = F.E4M3_TABLE
    assert ((np.isnan(want) & np.isnan(t)) | (want.view(np.uint32) == t.view(np.uint32))).all()
    assert t[0x00] == 0.0 and t[0x40] == 2.0 and t[0x3C] == 1.5 and t[0xC0] == -2.0
    assert t[0x78] == 256.0 and t[0x7E] == 448.0 and np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert np.signbit(t[0x80]) and t[0x80] == 0.0


def test_fp8_block_dequant_reference_recipe():
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, size=(32, 64), dtype=np.uint8)
    scales = rng.integers(120, 135, size=(1, 2), dtype=np.uint8)
    got = F.fp8_block_dequant(packed, scales)
    vals = torch.frombuffer(bytearray(packed.tobytes()), dtype=torch.float8_e4m3fn).float().reshape(32, 64)
    gain = torch.exp2(torch.from_numpy(scales.astype(np.float32)) - 127).repeat_interleave(32, 0).repeat_interleave(32, 1)
    want = (vals * gain).numpy()
    assert ((np.isnan(want) & np.isnan(got)) | (want == got)).all()
    with pytest.raises(ValueError):
        F.fp8_block_dequant(packed[:16], scales)


def test_expert_ranges_reference_kat():
    fake = {"tensors": [
        {"name": "a", "subsystem": "routed-expert", "layer": 5, "expert": 7, "shard": "s1", "file_range": [100, 200]},
        {"name": "b", "subsystem": "routed-expert", "layer": 5, "expert": 7, "shard": "s1", "file_range": [0, 50]},
        {"name": "c", "subsystem": "routed-expert", "layer": 5, "expert": 8, "shard": "s1", "file_range": [300, 350]},
        {"name": "d", "subsystem": "routed-expert", "layer": 6, "expert": 7, "shard": "s2", "file_range": [0, 60]},
        {"name": "e", "subsystem": "engram", "layer": None, "expert": None, "shard": "s1", "file_range": [1000, 2000]},
        {"name": "f", "subsystem": "attention", "layer": 5, "expert": None, "shard": "s1", "file_range": [2000, 2100]},
    ]}
    assert expert_ranges(fake, 5, 7) == {"s1": [(0, 50), (100, 200)]}
    assert expert_ranges(fake, 5, 9) == {}


def test_real_manifest_subset_layout():
    m = json.loads((GOLDEN / "manifest_layer0_subset.json").read_text())
    ck = Checkpoint("/nonexistent", m)
    arch = ck.arch
    H, I, E = arch["hidden_size"], arch["moe_intermediate_size"], arch["n_routed_experts"]
    for e in (0, 383):
        total = 0
        for role, (n, k) in (("w1", (I, H)), ("w3", (I, H)), ("w2", (H, I))):
            w = ck.entry(f"layers.0.ffn.experts.{e}.{role}.weight")
            s = ck.entry(f"layers.0.ffn.experts.{e}.{role}.scale")
            assert (w["dtype"], tuple(w["shape"])) == ("I8", (n, k // 2))          # the kernels' FP4 layout
            assert (s["dtype"], tuple(s["shape"])) == ("F8_E8M0", (n, k // 32))
            total += w["bytes"] + s["bytes"]
        assert total == m["expert_stats"]["median_bytes"]
        assert sum(b - a for _, rs in expert_ranges(m, 0, e).items() for a, b in rs) == total
    for role, (n, k) in (("w1", (I, H)), ("w3", (I, H)), ("w2", (H, I))):
        w = ck.entry(f"layers.0.ffn.shared_experts.{role}.weight")
        s = ck.entry(f"layers.0.ffn.shared_experts.{role}.scale")
        assert (w["dtype"], tuple(w["shape"]), s["dtype"], tuple(s["shape"])) == ("F8_E4M3", (n, k), "F8_E8M0",
                                                                                   (n // 32, k // 32))
    g = ck.entry("layers.0.ffn.gate.weight")
    assert (g["dtype"], tuple(g["shape"])) == ("BF16", (E, H))
    assert ck.entry("layers.0.ffn.gate.bias")["dtype"] == "F32"
    for t in m["tensors"]:
        hb = m["shards"][t["shard"]]["header_bytes"]
        assert t["file_range"][0] - t["data_range"][0] == hb and t["file_range"][1] - t["data_range"][1] == hb


def test_safetensors_roundtrip_and_manifest(tmp_path):
    rng = np.random.default_rng(4)
    a = rng.standard_normal((4, 8)).astype(np.float32)
    b = rng.integers(0, 256, (3, 32), dtype=np.uint8)
    c = rng.integers(-128, 128, (5, 2), dtype=np.int8)
    write_safetensors(tmp_path / "x-1.safetensors", {"layers.2.ffn.gate.bias": ("F32", a.shape, a.tobytes()),
                                                   "layers.2.ffn.experts.3.w1.scale": ("U8", b.shape, b.tobytes())})
    write_safetensors(tmp_path / "x-2.safetensors", {"layers.2.ffn.experts.3.w1.weight": ("I8", c.shape, c.tobytes())})
    m = build_manifest(tmp_path)
    ck = Checkpoint(tmp_path, m)
    assert ck.read("layers.2.ffn.gate.bias") == a.tobytes()
    assert ck.read("layers.2.ffn.experts.3.w1.weight") == c.tobytes()
    rec = ck.entry("layers.2.ffn.experts.3.w1.scale")
    assert (rec["subsystem"], rec["layer"], rec["expert"], rec["routed"]) == ("routed-expert", 2, 3, True)
    assert ck.entry("layers.2.ffn.gate.bias")["subsystem"] == "router"
    assert set(expert_ranges(m, 2, 3)) == {"x-1.safetensors", "x-2.safetensors"}
    from safetensors.numpy import load_file
    got = load_file(str(tmp_path / "x-1.safetensors"))
    np.testing.assert_array_equal(got["layers.2.ffn.gate.bias"], a)
    np.testing.assert_array_equal(got["layers.2.ffn.experts.3.w1.scale"], b)
    with pytest.raises(ValueError):
        Checkpoint(tmp_path, {"schema": "other", "tensors": []})


def test_synthetic_checkpoint_bytes(tmp_path):
    """The synthetic checkpoint's bytes read back through the manifest equal what was written."""
    spec = L.LayerSpec(H=256, E=4, k=2, I=128, I_shared=128)
    d = make_checkpoint(tmp_path, spec, 3)
    ck = Checkpoint(tmp_path, d["manifest"])
    assert ck.n_experts(0) == 4
    packed, scales = d["bank"].roles["w2"]
    assert ck.read("layers.0.ffn.experts.2.w2.weight") == packed[2].tobytes()
    assert ck.read("layers.0.ffn.experts.2.w2.scale") == scales[2].tobytes()


def test_mixed_format_layer_is_refused(tmp_path):
    """A q3 layer with two experts left in FP4 (the reference's requantisation
    script takes an expert subset): the format check names both lists."""
    spec = L.LayerSpec(H=256, E=6, k=2, I=128, I_shared=128, quant=L.QUANT_Q3)
    d = make_checkpoint(tmp_path, spec, 4, fp4_experts=frozenset({1, 4}))
    ck = Checkpoint(tmp_path, d["manifest"])
    with pytest.raises(ValueError, match=r"mixed routed-expert formats \(q3: experts \[0, 2, 3, 5\]; FP4: experts \[1, 4\]\)"):
        ck.expert_format(0)
    whole = tmp_path / "q3"
    d = make_checkpoint(whole, spec, 4)
    assert Checkpoint(whole, d["manifest"]).expert_format(0) == "q3"
