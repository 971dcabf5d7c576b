"""Writes tests/golden/manifest_layer0_subset.json (run from the repo root).

    python tests/golden/make_manifest_subset.py [--reference /root/reference]

A few records of the reference's checkpoint manifest
(``profiles/deepseek-v4.1-flash/<rev>/model-manifest.json``, schema
``deepseeker.model-manifest/v1``) kept as data: the header fields, the
architecture, the shard record of layer 0's shard, and every tensor record of
layer 0's routed experts 0 and 383, its shared expert and its gate.  The
checkpoint loader's tests read this subset; the weights themselves are not
available here.
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
REV = "dba1be0a40aa45a94ad051997016db3960a90277"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    src = Path(args.reference) / "profiles" / "deepseek-v4.1-flash" / REV / "model-manifest.json"
    m = json.loads(src.read_text())
    keep = []
    for t in m["tensors"]:
        n = t["name"]
        if (n.startswith("layers.0.ffn.experts.0.") or n.startswith("layers.0.ffn.experts.383.")
                or n.startswith("layers.0.ffn.shared_experts.") or n.startswith("layers.0.ffn.gate.")):
            keep.append(t)
    shards = {t["shard"] for t in keep}
    out = {k: m[k] for k in ("schema", "upstream", "architecture", "offset_convention", "expert_stats")}
    out["shards"] = {s: m["shards"][s] for s in sorted(shards)}
    out["tensors"] = keep
    dst = ROOT / "tests" / "golden" / "manifest_layer0_subset.json"
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(f"{dst}: {len(keep)} tensor records from {len(shards)} shard(s)")


if __name__ == "__main__":
    main()
