"""Checkpoint -> resident layer: the routed experts of a layer stacked into HBM banks.

The reference reads its safetensors checkpoint through a manifest
(``deepseeker.model-manifest/v1``, written under ``profiles/<model>/<rev>/``):
one record per tensor with ``shard``, ``shape``, ``dtype`` and the absolute
``file_range`` (8-byte header length + JSON header + the tensor's
``data_range``), see ``src/deepseeker/mlx_weights.py:173-188`` (``read_bytes``),
``:263-304`` (per-expert runs) and ``src/deepseeker/checkpoint_io.py:35-47``
(``expert_ranges``).  Its pinned experts are stacked into per-layer banks
(``mlx_weights.py:576-649``); the dense weights, the shared expert among them,
are FP8 E4M3 with one E8M0 scale per 32 x 32 block, dequantised to bf16 once
at load (``mlx_weights.py:82-89, 694-712``).

On one MI355X every expert of a layer is resident, so ``Checkpoint.load_layer``
reads a layer's tensors by byte range and builds a ``MoELayer``:

* routed experts (``I8`` packed e2m1 codes ``[N, K/2]`` + ``F8_E8M0`` scales
  ``[N, K/32]`` per role): byte-identical to the kernels' FP4 layout, copied
  into ``[E, N, K/2]`` / ``[E, N, K/32]`` device banks without arithmetic;
* or q3 routed experts, as the reference's q3 variant stores them for layers
  20-39 (``src/deepseeker/variant_q3.py:1-8``; ``U32_Q3_AFFINE`` words
  ``[N, 3K/32]`` of row-major 3-byte packs + ``F16`` ``.scale`` / ``.bias``
  ``[N, K/64]``, ``src/deepseeker/mlx_weights.py:119-141``): the codes are
  copied to the device and put into the kernels' canonical layout by
  ``dsk_q3_repack``, scales and biases copied unchanged;
* shared expert (``F8_E4M3`` + block scales, or ``BF16``): dequantised on the
  device by ``dsk_fp8_block_dequant`` into bf16;
* gate (``BF16`` or ``F32`` ``[E, H]``) and its bias (``F32`` ``[E]``).

``build_manifest`` writes the same manifest for any directory of safetensors
shards (the reference generates its manifest from the upstream headers), and
``write_safetensors`` writes shards, e.g. synthetic checkpoints for tests.
"""

from __future__ import annotations

import json
import os
import re
import struct
import threading
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .bank import ResidentBank, SharedExpert
from .layer import MoELayer
from .ops import ptr, q3_repack, require_device, stream_of

SCHEMA = "deepseeker.model-manifest/v1"
OFFSET_CONVENTION = ("data_range is [start, end) relative to the safetensors data-section start; "
                     "file_range is absolute from file byte 0 (8-byte header length + JSON header + "
                     "relative offset).")
_ITEM = {"BF16": 2, "F16": 2, "F32": 4, "I8": 1, "U8": 1, "F8_E4M3": 1, "F8_E8M0": 1, "I32": 4, "U32": 4,
         "U32_Q3_AFFINE": 4}
_EXPERT = re.compile(r"^(layers|mtp)\.(\d+)\.ffn\.experts\.(\d+)\.")
_LAYER = re.compile(r"^layers\.(\d+)\.")


# ------------------------------------------------------------------ safetensors files
def read_safetensors_header(path: str | Path) -> tuple[int, dict]:
    """(header_bytes, header) of one safetensors file; header_bytes = 8 + JSON length."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a safetensors file")
        (n,) = struct.unpack("<Q", raw)
        header = json.loads(f.read(n))
    return 8 + n, header


def write_safetensors(path: str | Path, tensors: dict[str, tuple[str, tuple, bytes]]) -> None:
    """Write ``{name: (dtype, shape, raw bytes)}`` as one safetensors file (in the given order)."""
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, data) in tensors.items():
        want = int(np.prod(shape, dtype=np.int64)) * _ITEM[dtype]
        if len(data) != want:
            raise ValueError(f"{name}: {len(data)} bytes for {dtype} {tuple(shape)} (want {want})")
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        blobs.append(data)
        off += len(data)
    js = json.dumps(header, separators=(",", ":")).encode()
    js += b" " * (-len(js) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(js)))
        f.write(js)
        for b in blobs:
            f.write(b)


def _classify(name: str) -> tuple[str, int | None, int | None, bool]:
    m = _EXPERT.match(name)
    if m:
        return ("routed-expert" if m.group(1) == "layers" else "mtp-expert"), int(m.group(2)), int(m.group(3)), True
    m = _LAYER.match(name)
    layer = int(m.group(1)) if m else None
    if ".shared_experts." in name:
        return "shared-expert", layer, None, False
    if ".ffn.gate." in name:
        return "router", layer, None, False
    return "unknown", layer, None, False


def build_manifest(root: str | Path, architecture: dict | None = None) -> dict:
    """The ``deepseeker.model-manifest/v1`` record of every tensor in ``root/*.safetensors``."""
    root = Path(root)
    shards, tensors = {}, []
    for path in sorted(root.glob("*.safetensors")):
        hb, header = read_safetensors_header(path)
        total = 0
        for name, rec in header.items():
            if name == "__metadata__":
                continue
            start, end = rec["data_offsets"]
            subsystem, layer, expert, routed = _classify(name)
            tensors.append({"name": name, "shape": rec["shape"], "dtype": rec["dtype"],
                            "elements": int(np.prod(rec["shape"], dtype=np.int64)), "bytes": end - start,
                            "shard": path.name, "data_range": [start, end], "file_range": [hb + start, hb + end],
                            "subsystem": subsystem, "layer": layer, "expert": expert, "routed": routed,
                            "detail": name})
            total += end - start
        shards[path.name] = {"file_bytes": path.stat().st_size, "header_bytes": hb,
                             "tensor_count": sum(1 for n in header if n != "__metadata__"),
                             "tensor_bytes": total, "container_overhead_bytes": path.stat().st_size - hb - total}
    tensors.sort(key=lambda t: t["name"])
    return {"schema": SCHEMA, "architecture": architecture or {}, "offset_convention": OFFSET_CONVENTION,
            "shards": shards, "tensors": tensors}


# ------------------------------------------------------------------ reading
def expert_ranges(manifest: dict, layer: int, expert: int) -> dict[str, list[tuple[int, int]]]:
    """{shard: sorted [(start, end)]} of every tensor of one routed expert
    (the contract of the reference's ``checkpoint_io.expert_ranges``)."""
    out: dict[str, list[tuple[int, int]]] = {}
    for t in manifest.get("tensors", []):
        if t.get("subsystem") == "routed-expert" and t.get("layer") == layer and t.get("expert") == expert:
            out.setdefault(t["shard"], []).append(tuple(t["file_range"]))
    for r in out.values():
        r.sort()
    return out


class Checkpoint:
    """A safetensors checkpoint described by a ``deepseeker.model-manifest/v1`` manifest."""

    def __init__(self, root: str | Path, manifest: dict | str | Path | None = None):
        self.root = Path(root)
        if manifest is None:
            mpath = self.root / "model-manifest.json"
            manifest = json.loads(mpath.read_text()) if mpath.exists() else build_manifest(self.root)
        elif not isinstance(manifest, dict):
            manifest = json.loads(Path(manifest).read_text())
        if manifest.get("schema") != SCHEMA:
            raise ValueError(f"manifest schema {manifest.get('schema')!r}, want {SCHEMA!r}")
        self.manifest = manifest
        self.arch = manifest.get("architecture", {})
        self.by_name = {t["name"]: t for t in manifest["tensors"]}
        self._fds: dict[str, int] = {}
        self._lock = threading.Lock()

    def close(self) -> None:
        with self._lock:
            for fd in self._fds.values():
                os.close(fd)
            self._fds.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def entry(self, name: str) -> dict:
        try:
            return self.by_name[name]
        except KeyError:
            raise KeyError(f"tensor {name!r} is not in the manifest") from None

    def read(self, name: str) -> bytes:
        """Raw bytes of one tensor (one pread of its file_range)."""
        e = self.entry(name)
        start, end = e["file_range"]
        with self._lock:
            fd = self._fds.get(e["shard"])
            if fd is None:
                fd = os.open(self.root / e["shard"], os.O_RDONLY)
                self._fds[e["shard"]] = fd
        data = os.pread(fd, end - start, start)
        if len(data) != end - start:
            raise RuntimeError(f"short read of {name} from {e['shard']} at {start}")
        return data

    def _array(self, name: str, dtype) -> np.ndarray:
        return np.frombuffer(self.read(name), dtype=dtype).reshape(self.entry(name)["shape"])

    def n_experts(self, layer: int) -> int:
        ids = {t["expert"] for t in self.manifest["tensors"]
               if t.get("subsystem") == "routed-expert" and t.get("layer") == layer}
        if not ids or ids != set(range(len(ids))):
            raise ValueError(f"layer {layer}: routed experts must be numbered 0 .. E-1, found {len(ids)}")
        return len(ids)

    # -------------------------------------------------------------- device objects
    def _format_of(self, layer: int, e: int) -> str:
        base = f"layers.{layer}.ffn.experts.{e}.w1"
        w = self.entry(base + ".weight")
        if w["dtype"] == "U32_Q3_AFFINE" or (base + ".bias") in self.by_name:
            return "q3"
        return "fp4"

    def expert_format(self, layer: int) -> str:
        """``"fp4"`` or ``"q3"``: the routed-expert format of ``layer``.  Every expert
        is checked: a resident bank (and the kernels reading it) hold one format
        per layer, so a partly requantised layer is refused with its expert lists."""
        fmts = [self._format_of(layer, e) for e in range(self.n_experts(layer))]
        if len(set(fmts)) > 1:
            q3 = [e for e, f in enumerate(fmts) if f == "q3"]
            fp4 = [e for e, f in enumerate(fmts) if f == "fp4"]
            raise ValueError(f"layer {layer}: mixed routed-expert formats (q3: experts {q3[:8]}"
                             f"{'...' if len(q3) > 8 else ''}; FP4: experts {fp4[:8]}{'...' if len(fp4) > 8 else ''}); "
                             f"a resident layer holds one format -- requantise all of its experts")
        return fmts[0]

    def _load_q3_bank(self, layer: int, dev: torch.device, E: int) -> ResidentBank:
        roles = {}
        for role in ("w1", "w3", "w2"):
            base = f"layers.{layer}.ffn.experts.0.{role}"
            w, s, b = self.entry(base + ".weight"), self.entry(base + ".scale"), self.entry(base + ".bias")
            if w["dtype"] not in ("U32_Q3_AFFINE", "U32", "I32") or s["dtype"] != "F16" or b["dtype"] != "F16":
                raise ValueError(f"{base}: expected q3 words + F16 scale / bias, got "
                                 f"{w['dtype']} / {s['dtype']} / {b['dtype']}")
            n, words = w["shape"]
            groups = s["shape"][1]
            k = groups * 64
            if tuple(s["shape"]) != (n, groups) or tuple(b["shape"]) != (n, groups) or words * 32 != 3 * k:
                raise ValueError(f"{base}: q3 words {w['shape']} do not match scales {s['shape']} "
                                 f"(want [N, 3K/32] with K = 64 x groups)")
            if k % 128:
                raise ValueError(f"{base}: K={k} is not a multiple of 128")
            staged = torch.empty((E, n, k * 3 // 8), dtype=torch.uint8, device=dev)
            scales = torch.empty((E, n, groups), dtype=torch.float16, device=dev)
            biases = torch.empty((E, n, groups), dtype=torch.float16, device=dev)
            for e in range(E):
                name = f"layers.{layer}.ffn.experts.{e}.{role}"
                if tuple(self.entry(name + ".weight")["shape"]) != (n, words):
                    raise ValueError(f"{name}: shape differs from expert 0")
                raw = np.frombuffer(self.read(name + ".weight"), dtype=np.uint8).reshape(n, -1)
                staged[e].copy_(torch.from_numpy(raw.copy()))
                scales[e].copy_(torch.from_numpy(self._array(name + ".scale", "<f2").copy()))
                biases[e].copy_(torch.from_numpy(self._array(name + ".bias", "<f2").copy()))
            roles[role] = (q3_repack(staged), scales, biases)
            del staged
        return ResidentBank("q3", roles)

    def load_bank(self, layer: int, device: torch.device | str = "cuda") -> ResidentBank:
        """All routed experts of ``layer`` as a ``ResidentBank``: FP4 bytes copied
        unchanged, or q3 codes repacked into the canonical layout on the device."""
        dev = torch.device(device)
        E = self.n_experts(layer)
        if self.expert_format(layer) == "q3":
            return self._load_q3_bank(layer, dev, E)
        roles = {}
        for role in ("w1", "w3", "w2"):
            base = f"layers.{layer}.ffn.experts.0.{role}"
            w, s = self.entry(base + ".weight"), self.entry(base + ".scale")
            if w["dtype"] not in ("I8", "U8") or s["dtype"] not in ("F8_E8M0", "U8"):
                raise ValueError(f"{base}: expected packed FP4 (I8) + E8M0 scales, got {w['dtype']} / {s['dtype']}")
            n, half = w["shape"]
            if tuple(s["shape"]) != (n, half * 2 // 32):
                raise ValueError(f"{base}: scale shape {s['shape']} does not match codes {w['shape']}")
            codes = torch.empty((E, n, half), dtype=torch.uint8, device=dev)
            scales = torch.empty((E, n, half * 2 // 32), dtype=torch.uint8, device=dev)
            for e in range(E):
                name = f"layers.{layer}.ffn.experts.{e}.{role}"
                if tuple(self.entry(name + ".weight")["shape"]) != (n, half):
                    raise ValueError(f"{name}: shape differs from expert 0")
                codes[e].copy_(torch.from_numpy(self._array(name + ".weight", np.uint8)))
                scales[e].copy_(torch.from_numpy(self._array(name + ".scale", np.uint8)))
            roles[role] = (codes, scales)
        return ResidentBank("fp4", roles)

    def _dense_bf16(self, name: str, dev: torch.device) -> torch.Tensor:
        e = self.entry(name + ".weight")
        if e["dtype"] == "BF16":
            return torch.from_numpy(self._array(name + ".weight", np.uint16).copy()).view(torch.bfloat16).to(dev)
        if e["dtype"] != "F8_E4M3":
            raise ValueError(f"{name}.weight: unsupported dtype {e['dtype']}")
        rows, cols = e["shape"]
        codes = torch.from_numpy(self._array(name + ".weight", np.uint8).copy()).to(dev)
        scales = torch.from_numpy(self._array(name + ".scale", np.uint8).copy()).to(dev)
        if tuple(scales.shape) != (rows // 32, cols // 32):
            raise ValueError(f"{name}.scale: shape {tuple(scales.shape)} for {rows} x {cols} codes")
        return fp8_block_dequant(codes, scales, torch.bfloat16)

    def load_shared(self, layer: int, device: torch.device | str = "cuda") -> SharedExpert:
        dev = torch.device(device)
        p = f"layers.{layer}.ffn.shared_experts"
        return SharedExpert(self._dense_bf16(p + ".w1", dev), self._dense_bf16(p + ".w3", dev),
                            self._dense_bf16(p + ".w2", dev))

    def load_gate(self, layer: int, device: torch.device | str = "cuda") -> tuple[torch.Tensor, torch.Tensor]:
        dev = torch.device(device)
        p = f"layers.{layer}.ffn.gate"
        w = self.entry(p + ".weight")
        if w["dtype"] == "BF16":
            gw = torch.from_numpy(self._array(p + ".weight", np.uint16).copy()).view(torch.bfloat16)
        elif w["dtype"] == "F32":
            gw = torch.from_numpy(self._array(p + ".weight", "<f4").copy())
        else:
            raise ValueError(f"{p}.weight: unsupported dtype {w['dtype']}")
        gb = torch.from_numpy(self._array(p + ".bias", "<f4").copy())
        return gw.to(dev), gb.to(dev)

    def load_layer(self, layer: int, device: torch.device | str = "cuda", *, top_k: int | None = None,
                   score_func: str = "sqrtsoftplus", route_scale: float = 1.5,
                   limit: float = 10.0) -> MoELayer:
        """One resident MoE layer: gate, all routed experts, the shared expert (if any)."""
        gw, gb = self.load_gate(layer, device)
        bank = self.load_bank(layer, device)
        shared = (self.load_shared(layer, device)
                  if f"layers.{layer}.ffn.shared_experts.w1.weight" in self.by_name else None)
        k = int(top_k or self.arch.get("num_experts_per_tok") or 0)
        if k < 1:
            raise ValueError("top_k is not given and the manifest has no num_experts_per_tok")
        return MoELayer(gw, gb, bank, shared, k, score_func=score_func, route_scale=route_scale, limit=limit)


def fp8_block_dequant(codes: torch.Tensor, scales: torch.Tensor,
                      out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """``dsk_fp8_block_dequant``: E4M3 codes [R, C] u8 with E8M0 32 x 32 block scales
    [R/32, C/32] u8 -> [R, C] in ``out_dtype`` (bf16 or float32), on the device."""
    dev = require_device(codes, scales)
    if codes.dtype != torch.uint8 or scales.dtype != torch.uint8 or codes.dim() != 2:
        raise ValueError("codes and scales must be 2-D uint8 tensors")
    codes, scales = codes.contiguous(), scales.contiguous()
    rows, cols = codes.shape
    out = torch.empty((rows, cols), dtype=out_dtype, device=dev)
    code = {torch.bfloat16: 0, torch.float32: 1}[out_dtype]
    _lib.call("dsk_fp8_block_dequant", ptr(codes), ptr(scales), rows, cols, ptr(out), code, stream_of(dev))
    return out
