"""A small synthetic checkpoint in the layout of the real one (test helper).

Layer 0 of a model with ``spec``'s shapes: routed experts as packed FP4 (I8)
with E8M0 scales, the shared expert as FP8 E4M3 with 32 x 32 E8M0 block
scales, the gate as BF16 and its bias as F32; the experts in one shard, the
rest in another, tensor names as in the real checkpoint.  Returns what the
oracle needs to evaluate the same layer.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from dsk_moe.checkpoint import build_manifest, write_safetensors
from oracle import formats as F
from oracle import layer as L


def make_checkpoint(root: Path, spec: L.LayerSpec, seed: int, fp4_experts: frozenset = frozenset()) -> dict:
    """``spec.quant`` "fp4": routed experts as I8 codes + F8_E8M0 scales; "q3": as the
    reference's q3 variant stores them, U32_Q3_AFFINE words [N, 3K/32] of row-major
    3-byte packs + F16 scale / bias [N, K/64].  ``fp4_experts``: experts kept in FP4
    in a q3 layer (a partly requantised checkpoint)."""
    rng = np.random.default_rng(seed)
    H, E, I, Is = spec.H, spec.E, spec.I, spec.I_shared
    experts, dense = {}, {}
    roles = {"w1": [], "w3": [], "w2": []}
    for e in range(E):
        q3 = spec.quant == L.QUANT_Q3 and e not in fp4_experts
        for role, (n, k) in (("w1", (I, H)), ("w2", (H, I)), ("w3", (I, H))):
            w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
            base = f"layers.0.ffn.experts.{e}.{role}"
            if q3:
                q, s16, b16 = F.q3_quantize_codes(w)
                rowmajor = F.q3_pack_rowmajor(q)
                experts[base + ".weight"] = ("U32_Q3_AFFINE", (n, 3 * k // 32), rowmajor.tobytes())
                experts[base + ".scale"] = ("F16", s16.shape, s16.astype("<f2").tobytes())
                experts[base + ".bias"] = ("F16", b16.shape, b16.astype("<f2").tobytes())
                roles[role].append((F.q3_pack(q), s16, b16))
            else:
                packed, scales = F.fp4_quantize(w)
                experts[base + ".weight"] = ("I8", packed.shape, packed.tobytes())
                experts[base + ".scale"] = ("F8_E8M0", scales.shape, scales.tobytes())
                roles[role].append((packed, scales))
    bank = None if fp4_experts else L.ExpertBank(
        spec.quant, {r: tuple(np.stack(c) for c in zip(*parts)) for r, parts in roles.items()})
    shared = []
    for role, (n, k) in (("w1", (Is, H)), ("w2", (H, Is)), ("w3", (Is, H))):
        codes = rng.integers(0, 256, size=(n, k), dtype=np.uint8)
        codes[(codes & 0x7F) == 0x7F] = 0x38          # no NaN codes
        scales = rng.integers(118, 122, size=(n // 32, k // 32), dtype=np.uint8)
        base = f"layers.0.ffn.shared_experts.{role}"
        dense[base + ".weight"] = ("F8_E4M3", codes.shape, codes.tobytes())
        dense[base + ".scale"] = ("F8_E8M0", scales.shape, scales.tobytes())
        shared.append((role, F.fp8_block_dequant(codes, scales)))
    gate_w = (torch.randn((E, H), generator=torch.Generator().manual_seed(seed)) / np.sqrt(H)).to(torch.bfloat16)
    gate_b = torch.from_numpy(rng.uniform(-0.1, 0.1, E).astype(np.float32))
    dense["layers.0.ffn.gate.weight"] = ("BF16", (E, H), gate_w.view(torch.int16).numpy().tobytes())
    dense["layers.0.ffn.gate.bias"] = ("F32", (E,), gate_b.numpy().tobytes())
    root.mkdir(parents=True, exist_ok=True)
    write_safetensors(root / "model-00001-of-00002.safetensors", dense)
    write_safetensors(root / "model-00002-of-00002.safetensors", experts)
    manifest = build_manifest(root, {"hidden_size": H, "n_routed_experts": E, "num_experts_per_tok": spec.k,
                                     "moe_intermediate_size": I})
    sh = {r: torch.from_numpy(w).to(torch.bfloat16) for r, w in shared}
    return {"manifest": manifest, "gate_w": gate_w, "gate_b": gate_b, "bank": bank,
            "shared": (sh["w1"], sh["w3"], sh["w2"]), "shared_f32": {r: w for r, w in shared}}
