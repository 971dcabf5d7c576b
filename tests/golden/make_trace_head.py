"""Writes tests/golden/trace_mlx_en_head.jsonl (run from the repo root).

    python tests/golden/make_trace_head.py [--reference /root/reference] [--lines 241]

The header and the first records (routing records and kv/engram events) of the
reference's recorded router trace ``profiles/traces/mlx-en.jsonl``
(``deepseeker.trace/v1``: real DeepSeek routing, 40 layers, 384 experts,
top-6), kept as data so the trace reader is checked against the reference's
own files.
"""

from __future__ import annotations

import argparse
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--lines", type=int, default=241)
    args = ap.parse_args()
    src = Path(args.reference) / "profiles" / "traces" / "mlx-en.jsonl"
    with open(src, encoding="utf-8") as f:
        lines = [next(f) for _ in range(args.lines)]
    dst = ROOT / "tests" / "golden" / "trace_mlx_en_head.jsonl"
    dst.write_text("".join(lines), encoding="utf-8")
    print(f"{dst}: {len(lines)} lines")


if __name__ == "__main__":
    main()
