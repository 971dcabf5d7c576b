"""Writes the golden fixtures under tests/golden/ (run from the repo root).

    python tests/golden/make_golden.py [--reference /root/reference]

* ``cfg0.npz``  -- the small layer (hidden 1024, 64 experts, top-6, inter 512,
  shared 512, seed 0, 4 tokens) through the oracle: routing, dispatch, output,
  and SHA-256 digests of every generated tensor (detects generator drift).
* ``tiny.npz``  -- a reference-test-sized layer (H 64, E 8, k 2, I 32,
  shared 32, seed 1, 3 tokens) with all of its tensors.
* ``trace_routes.npz`` -- expert ids and weights of the reference's recorded
  router traces (``profiles/traces/mlx-*.jsonl``: real DeepSeek routing,
  E = 384, k = 6, weights summing to the route scale 1.5), as data.

The fixtures are produced by this build's oracle (the reference cannot run
here); the traces are data files of the reference.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import layer as L  # noqa: E402
from oracle import synth  # noqa: E402

OUT = Path(__file__).resolve().parent


def digest(a) -> str:
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu()
        if a.dtype == torch.bfloat16:
            a = a.view(torch.int16)
        a = a.numpy()
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def layer_digests(d: dict) -> dict:
    out = {"x": digest(d["x"]), "gate_w": digest(d["gate_w"]), "gate_b": digest(d["gate_b"])}
    for role, parts in d["bank"].roles.items():
        for i, p in enumerate(parts):
            out[f"{role}.{i}"] = digest(p)
    if d["shared"] is not None:
        for name, t in zip(("ws1", "ws3", "ws2"), d["shared"]):
            out[name] = digest(t)
    return out


def run(spec, seed, tokens):
    d = synth.make_layer(spec, seed, tokens)
    r = L.moe_forward(d["x"], d["gate_w"], d["gate_b"], d["bank"], d["shared"], spec)
    return d, r


def write_cfg0() -> None:
    spec = synth.config0_spec()
    d, r = run(spec, 0, 4)
    np.savez_compressed(
        OUT / "cfg0.npz",
        idx=r["idx"], w=r["w"], scores=r["scores"], counts=r["counts"], offsets=r["offsets"],
        perm=r["perm"], rank=r["rank"], y_ref=r["y_ref"].numpy(),
        out_bf16=r["out"].view(torch.int16).numpy(),
        digests=np.array(json.dumps(layer_digests(d), sort_keys=True)))


def write_tiny() -> None:
    spec = synth.tiny_spec()
    d, r = run(spec, 1, 3)
    arrays = {"x_bf16": d["x"].view(torch.int16).numpy(), "gate_w": d["gate_w"].numpy(),
              "gate_b": d["gate_b"].numpy()}
    for role, parts in d["bank"].roles.items():
        arrays[f"{role}_packed"], arrays[f"{role}_scales"] = parts
    for name, t in zip(("ws1", "ws3", "ws2"), d["shared"]):
        arrays[name] = t.view(torch.int16).numpy()
    np.savez_compressed(OUT / "tiny.npz", idx=r["idx"], w=r["w"], scores=r["scores"],
                        perm=r["perm"], counts=r["counts"], y_ref=r["y_ref"].numpy(),
                        out_bf16=r["out"].view(torch.int16).numpy(), **arrays)


def write_traces(reference: Path) -> None:
    experts, weights = [], []
    for path in sorted((reference / "profiles" / "traces").glob("mlx-*.jsonl")):
        with open(path, encoding="utf-8") as f:
            for line in f:
                rec = json.loads(line)
                if rec.get("kind") == "record" and rec.get("scores") is not None:
                    experts.append(rec["experts"])
                    weights.append(rec["scores"])
    np.savez_compressed(OUT / "trace_routes.npz", experts=np.asarray(experts, dtype=np.int32),
                        weights=np.asarray(weights, dtype=np.float32))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", type=Path, default=Path("/root/reference"))
    args = ap.parse_args()
    torch.set_num_threads(8)
    write_cfg0()
    write_tiny()
    if (args.reference / "profiles" / "traces").is_dir():
        write_traces(args.reference)
    for p in sorted(OUT.glob("*.npz")):
        print(p.name, p.stat().st_size)
    return 0


if __name__ == "__main__":
    sys.exit(main())
