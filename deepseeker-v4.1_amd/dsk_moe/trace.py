"""Router traces in the reference's ``deepseeker.trace/v1`` JSONL schema.

The reference records the authoritative top-k of every (request, token, layer)
through ``moe_layer``'s ``trace_hook(layer, idx, weights)``
(``src/deepseeker/mlx_forward.py:380-381, 407-408``), collected by a sink
(``scripts/run_mlx.py:34-50``) and written as JSONL (``src/deepseeker/trace.py``):

* line 1, the header: ``kind = "header"``, ``schema = "deepseeker.trace/v1"``,
  ``repo_id``, ``revision``, ``source``, ``n_layers``, ``n_routed_experts``,
  ``top_k``, ``created_at_utc`` (and optionally ``seed``);
* routing records: ``request_id``, ``token_pos`` (>= 0), ``layer``, ``experts``
  (top_k distinct ids in [0, E)), ``scores`` (optional, aligned with experts;
  the hook passes the route weights), ``timing_ms`` / ``bytes_moved``
  (optional numbers), ``extra`` (optional object);
* subsystem events: ``kind = "event"`` with ``extra.kind`` "engram" or "kv".

This module reads and writes that format (traces written here validate with
the reference's reader and the reference's traces with this one), validates
records with the same rules, summarises traces, and provides ``TraceSink``,
which turns the device routing of ``moe_layer``, ``MoELayer`` and ``MoEStack``
into records.  ``routing_batches`` regroups a trace's records into the token
batches a layer saw, for replaying the recorded routing through the dispatch
and expert kernels.
"""

from __future__ import annotations

import datetime
import json
from pathlib import Path

import numpy as np

SCHEMA = "deepseeker.trace/v1"
HEADER_KIND = "header"


def arch_config(manifest: dict) -> dict:
    """Routing geometry (n_layers, n_routed_experts, top_k) from a model manifest's architecture."""
    a = manifest.get("architecture", {})
    return {"n_layers": a["num_hidden_layers"], "n_routed_experts": a["n_routed_experts"],
            "top_k": a["num_experts_per_tok"]}


def make_header(repo_id: str, revision: str, source: str, cfg: dict, seed: int | None = None) -> dict:
    for key in ("n_layers", "n_routed_experts", "top_k"):
        v = cfg.get(key)
        if not isinstance(v, int) or isinstance(v, bool) or v <= 0:
            raise ValueError(f"routing geometry {key}={v!r} must be a positive integer")
    h = {"kind": HEADER_KIND, "schema": SCHEMA, "repo_id": repo_id, "revision": revision, "source": source,
         "n_layers": cfg["n_layers"], "n_routed_experts": cfg["n_routed_experts"], "top_k": cfg["top_k"],
         "created_at_utc": datetime.datetime.now(datetime.timezone.utc).isoformat()}
    if seed is not None:
        h["seed"] = seed
    return h


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _common_problems(r: dict, header: dict) -> list[str]:
    p = []
    if not isinstance(r.get("request_id"), str) or not r["request_id"]:
        p.append("request_id must be a nonempty string")
    if not _is_int(r.get("token_pos")) or r["token_pos"] < 0:
        p.append(f"token_pos out of range: {r.get('token_pos')!r}")
    if not _is_int(r.get("layer")) or not 0 <= r["layer"] < header["n_layers"]:
        p.append(f"layer out of range: {r.get('layer')!r}")
    return p


def validate_record(r: dict, header: dict) -> list[str]:
    """Problems of one record (an empty list when it is valid)."""
    kind = r.get("kind", "record")
    if kind == "event":
        p = _common_problems(r, header)
        extra = r.get("extra")
        if not isinstance(extra, dict) or extra.get("kind") not in ("engram", "kv"):
            p.append(f"event extra.kind must be engram or kv: {extra!r}")
        return p
    if kind != "record":
        return [f"bad kind: {kind!r}"]
    p = _common_problems(r, header)
    k, E = header["top_k"], header["n_routed_experts"]
    ex = r.get("experts")
    if not isinstance(ex, list) or len(ex) != k or any(not _is_int(e) or not 0 <= e < E for e in ex):
        p.append(f"experts must be {k} ids in [0, {E}): {ex!r}")
    elif len(set(ex)) != len(ex):
        p.append(f"duplicate expert ids: {ex!r}")
    sc = r.get("scores")
    if sc is not None and (not isinstance(sc, list) or len(sc) != k
                           or any(not isinstance(s, (int, float)) or isinstance(s, bool) for s in sc)):
        p.append(f"scores must align with experts: {sc!r}")
    for key in ("timing_ms", "bytes_moved"):
        v = r.get(key)
        if v is not None and (not isinstance(v, (int, float)) or isinstance(v, bool)):
            p.append(f"{key} must be numeric: {v!r}")
    if r.get("extra") is not None and not isinstance(r["extra"], dict):
        p.append(f"extra must be an object: {r['extra']!r}")
    return p


def write_trace(path: str | Path, header: dict, records: list[dict]) -> int:
    """Header line + one line per record (routing records get ``kind: "record"``)."""
    with open(path, "w", encoding="utf-8") as f:
        f.write(json.dumps(header) + "\n")
        for r in records:
            f.write(json.dumps(r if "kind" in r else {"kind": "record", **r}) + "\n")
    return len(records)


def read_trace(path: str | Path) -> tuple[dict, list[dict]]:
    """(header, records); raises ValueError at the first malformed line.  Routing
    records come back without their ``kind`` key, events keep it."""
    with open(path, encoding="utf-8") as f:
        lines = [ln for ln in f if ln.strip()]
    if not lines:
        raise ValueError("empty trace file")
    try:
        header = json.loads(lines[0])
    except ValueError as exc:
        raise ValueError(f"line 1: invalid JSON: {exc}") from exc
    if not isinstance(header, dict) or header.get("kind") != HEADER_KIND or header.get("schema") != SCHEMA:
        raise ValueError(f"line 1: not a {SCHEMA} header: {lines[0][:120]!r}")
    records = []
    for n, ln in enumerate(lines[1:], 2):
        try:
            r = json.loads(ln)
        except ValueError as exc:
            raise ValueError(f"line {n}: invalid JSON: {exc}") from exc
        if not isinstance(r, dict):
            raise ValueError(f"line {n}: a record must be an object")
        problems = validate_record(r, header)
        if problems:
            raise ValueError(f"line {n}: {problems[0]}")
        if r.get("kind", "record") == "record":
            r.pop("kind", None)
        records.append(r)
    return header, records


def expert_records(records: list[dict]) -> list[dict]:
    """Routing records only (subsystem events dropped)."""
    return [r for r in records if r.get("kind", "record") == "record"]


def layer_histogram(records: list[dict], n_layers: int) -> dict[int, dict[int, int]]:
    """Per layer, {expert id: times selected}."""
    hist: dict[int, dict[int, int]] = {layer: {} for layer in range(n_layers)}
    for r in expert_records(records):
        b = hist[r["layer"]]
        for e in r["experts"]:
            b[e] = b.get(e, 0) + 1
    return hist


def trace_stats(header: dict, records: list[dict]) -> dict:
    """Record and request counts, distinct experts per layer, and the share of
    adjacent tokens (same request and layer) that kept the same expert set."""
    recs = expert_records(records)
    hist = layer_histogram(recs, header["n_layers"])
    unique = {layer: len(b) for layer, b in hist.items()}
    sets = {(r["request_id"], r["layer"], r["token_pos"]): set(r["experts"]) for r in recs}
    same = pairs = 0
    for (req, layer, pos), s in sets.items():
        nxt = sets.get((req, layer, pos + 1))
        if nxt is not None:
            pairs += 1
            same += s == nxt
    return {"records": len(recs), "requests": len({r["request_id"] for r in recs}),
            "unique_experts_per_layer": unique,
            "mean_unique": sum(unique.values()) / len(unique) if unique else 0.0,
            "adjacent_same_set_ratio": same / pairs if pairs else None}


class TraceSink:
    """Collects routing as trace records: pass ``sink.router`` as ``trace_hook``
    (``moe_layer``) or ``trace=sink`` (``MoELayer``, ``MoEStack``).  ``idx`` and
    ``weights`` are per token, in ascending key order, like the reference's hook."""

    def __init__(self, request_id: str, token_start: int = 0):
        self.request_id = request_id
        self.token_start = token_start
        self.records: list[dict] = []

    def router(self, layer: int, idx: list, weights: list, token_start: int | None = None) -> None:
        t0 = self.token_start if token_start is None else token_start
        for i, (experts, scores) in enumerate(zip(idx, weights)):
            self.records.append({"request_id": self.request_id, "token_pos": t0 + i, "layer": int(layer),
                                 "experts": [int(e) for e in experts], "scores": [float(s) for s in scores]})

    __call__ = router

    def advance(self, tokens: int) -> None:
        """Move the token position on by a batch (after a stack step)."""
        self.token_start += tokens


def routing_batches(records: list[dict], layer: int) -> list[tuple[str, int, np.ndarray, np.ndarray | None]]:
    """The token batches one layer saw: per request, runs of consecutive token
    positions, as (request_id, first position, experts [T, k] int32, scores [T, k]
    float32 or None)."""
    rows: dict[str, dict[int, dict]] = {}
    for r in expert_records(records):
        if r["layer"] == layer:
            rows.setdefault(r["request_id"], {})[r["token_pos"]] = r
    out = []
    for req, by_pos in rows.items():
        pos = sorted(by_pos)
        start = 0
        for i in range(1, len(pos) + 1):
            if i == len(pos) or pos[i] != pos[i - 1] + 1:
                run = [by_pos[p] for p in pos[start:i]]
                ex = np.asarray([r["experts"] for r in run], dtype=np.int32)
                sc = (np.asarray([r["scores"] for r in run], dtype=np.float32)
                      if all(r.get("scores") is not None for r in run) else None)
                out.append((req, pos[start], ex, sc))
                start = i
    return out
