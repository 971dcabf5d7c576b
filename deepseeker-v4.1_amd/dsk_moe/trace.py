"""Router traces in the ``deepseeker.trace/v1`` JSONL format.

The reference records the top-k of every (request, token, layer) through
``moe_layer``'s ``trace_hook(layer, idx, weights)``
(``src/deepseeker/mlx_forward.py:380-381, 407-408``), collects it in a sink
(``scripts/run_mlx.py:34-50``) and stores it as JSONL; the format is defined
in ``src/deepseeker/trace.py:1-21``.  What the format fixes, and this module
therefore keeps:

* line 1 is a header object: ``kind "header"``, ``schema
  "deepseeker.trace/v1"``, ``repo_id``, ``revision``, ``source``, the routing
  geometry ``n_layers``, ``n_routed_experts``, ``top_k``, ``created_at_utc``
  and optionally ``seed``;
* every further line is a routing record (``kind "record"``, or no kind) with
  ``request_id`` (non-empty string), ``token_pos`` (>= 0), ``layer`` (in
  ``[0, n_layers)``), ``experts`` (``top_k`` distinct ids in ``[0, E)``) and
  the optional ``scores`` (``top_k`` numbers), ``timing_ms``, ``bytes_moved``
  (numbers) and ``extra`` (an object); or a subsystem event (``kind
  "event"``) with ``request_id``, ``token_pos``, ``layer`` and an ``extra``
  object whose ``kind`` is ``"engram"`` or ``"kv"``.

The validity rules live in one table (``FIELDS``: per record kind, the fields
with their presence and value rule) read by one validator (``check``); the
file is handled by ``Trace`` (load / save / histogram / summary / per-layer
token batches).  ``TraceSink`` turns the device routing of ``moe_layer``,
``MoELayer`` and ``MoEStack`` into routing records, and ``Trace.batches``
regroups recorded routing into the token runs a layer saw, for replaying it
through the dispatch and expert kernels.
"""

from __future__ import annotations

import datetime
import json
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Iterator

import numpy as np

SCHEMA = "deepseeker.trace/v1"


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _is_number(v) -> bool:
    return isinstance(v, (int, float)) and not isinstance(v, bool)


@dataclass(frozen=True)
class Geometry:
    """The routing geometry a trace is recorded against."""

    n_layers: int
    n_routed_experts: int
    top_k: int

    def __post_init__(self):
        for name in ("n_layers", "n_routed_experts", "top_k"):
            v = getattr(self, name)
            if not _is_int(v) or v < 1:
                raise ValueError(f"trace geometry: {name} = {v!r} is not a positive integer")

    @classmethod
    def of_header(cls, header: dict) -> "Geometry":
        return cls(header.get("n_layers"), header.get("n_routed_experts"), header.get("top_k"))

    @classmethod
    def of_manifest(cls, manifest: dict) -> "Geometry":
        """From a ``deepseeker.model-manifest/v1`` architecture block."""
        arch = manifest.get("architecture") or {}
        return cls(arch.get("num_hidden_layers"), arch.get("n_routed_experts"),
                   arch.get("num_experts_per_tok"))

    def header(self, *, repo_id: str, revision: str, source: str, seed: int | None = None) -> dict:
        h = {"kind": "header", "schema": SCHEMA, "repo_id": repo_id, "revision": revision,
             "source": source, "n_layers": self.n_layers, "n_routed_experts": self.n_routed_experts,
             "top_k": self.top_k,
             "created_at_utc": datetime.datetime.now(datetime.timezone.utc).isoformat()}
        if seed is not None:
            h["seed"] = seed
        return h


# ------------------------------------------------------------------ field rules
# A rule returns None for an acceptable value, else the reason it is not.
Rule = Callable[[object, Geometry], "str | None"]


def _nonempty_text(v, g: Geometry):
    return None if isinstance(v, str) and v else f"want a non-empty string, got {v!r}"


def _index_below(limit: Callable[[Geometry], "int | None"]) -> Rule:
    def rule(v, g: Geometry):
        hi = limit(g)
        if _is_int(v) and v >= 0 and (hi is None or v < hi):
            return None
        span = "[0, inf)" if hi is None else f"[0, {hi})"
        return f"want an integer in {span}, got {v!r}"
    return rule


def _expert_ids(v, g: Geometry):
    if not isinstance(v, list) or len(v) != g.top_k:
        return f"want a list of {g.top_k} expert ids, got {v!r}"
    if not all(_is_int(e) and 0 <= e < g.n_routed_experts for e in v):
        return f"every id must be an integer in [0, {g.n_routed_experts}), got {v!r}"
    if len(set(v)) != len(v):
        return f"ids must be distinct, got {v!r}"
    return None


def _per_slot_numbers(v, g: Geometry):
    if isinstance(v, list) and len(v) == g.top_k and all(_is_number(s) for s in v):
        return None
    return f"want {g.top_k} numbers (one per expert), got {v!r}"


def _number(v, g: Geometry):
    return None if _is_number(v) else f"want a number, got {v!r}"


def _mapping(v, g: Geometry):
    return None if isinstance(v, dict) else f"want an object, got {v!r}"


def _event_payload(v, g: Geometry):
    if isinstance(v, dict) and v.get("kind") in EVENT_KINDS:
        return None
    return f"want an object whose kind is one of {sorted(EVENT_KINDS)}, got {v!r}"


EVENT_KINDS = frozenset({"engram", "kv"})


@dataclass(frozen=True)
class Field:
    key: str
    required: bool
    rule: Rule


_WHO = (Field("request_id", True, _nonempty_text),
        Field("token_pos", True, _index_below(lambda g: None)),
        Field("layer", True, _index_below(lambda g: g.n_layers)))

# record kind -> the fields it may carry (absent or null optional fields are skipped)
FIELDS: dict[str, tuple[Field, ...]] = {
    "record": _WHO + (Field("experts", True, _expert_ids),
                      Field("scores", False, _per_slot_numbers),
                      Field("timing_ms", False, _number),
                      Field("bytes_moved", False, _number),
                      Field("extra", False, _mapping)),
    "event": _WHO + (Field("extra", True, _event_payload),),
}


def check(record: dict, geometry: Geometry) -> list[str]:
    """Every way ``record`` breaks the format (empty when it is valid)."""
    if not isinstance(record, dict):
        return [f"a line must hold a JSON object, got {type(record).__name__}"]
    kind = record.get("kind", "record")
    fields = FIELDS.get(kind)
    if fields is None:
        return [f"kind {kind!r}: want one of {sorted(FIELDS)}"]
    found = []
    for f in fields:
        v = record.get(f.key)
        if v is None:
            if f.required:
                found.append(f"{f.key}: required")
            continue
        why = f.rule(v, geometry)
        if why:
            found.append(f"{f.key}: {why}")
    return found


# ------------------------------------------------------------------ files
def _is_routing(r: dict) -> bool:
    return r.get("kind", "record") == "record"


@dataclass
class Trace:
    """A header and its records.  Routing records are kept without a ``kind``
    key (as ``TraceSink`` makes them); events keep ``kind: "event"``."""

    header: dict
    records: list = field(default_factory=list)

    @property
    def geometry(self) -> Geometry:
        return Geometry.of_header(self.header)

    @staticmethod
    def _lines(path) -> Iterator[tuple[int, object]]:
        with open(path, encoding="utf-8") as f:
            for n, text in enumerate(f, 1):
                if not text.strip():
                    continue
                try:
                    yield n, json.loads(text)
                except json.JSONDecodeError as exc:
                    raise ValueError(f"{path}:{n}: not JSON ({exc.msg})") from exc

    @classmethod
    def load(cls, path: str | Path) -> "Trace":
        """Read and check a trace; the first broken line raises ValueError."""
        lines = cls._lines(path)
        first = next(lines, None)
        if first is None:
            raise ValueError(f"{path}: no header (the file has no lines)")
        n, head = first
        if not isinstance(head, dict) or head.get("kind") != "header" or head.get("schema") != SCHEMA:
            raise ValueError(f"{path}:{n}: want a {SCHEMA} header object first")
        try:
            geo = Geometry.of_header(head)
        except ValueError as exc:
            raise ValueError(f"{path}:{n}: {exc}") from exc
        out = cls(head)
        for n, rec in lines:
            broken = check(rec, geo)
            if broken:
                raise ValueError(f"{path}:{n}: {broken[0]}")
            if _is_routing(rec):
                rec = {k: v for k, v in rec.items() if k != "kind"}
            out.records.append(rec)
        return out

    def save(self, path: str | Path) -> int:
        """Header, then one line per record (routing records tagged ``kind: "record"``);
        returns the number of records written."""
        with open(path, "w", encoding="utf-8") as f:
            f.write(json.dumps(self.header) + "\n")
            for r in self.records:
                tagged = r if "kind" in r else dict(kind="record", **r)
                f.write(json.dumps(tagged) + "\n")
        return len(self.records)

    def routing(self) -> list[dict]:
        """Routing records only (subsystem events left out)."""
        return [r for r in self.records if _is_routing(r)]

    def histogram(self) -> np.ndarray:
        """``[n_layers, n_routed_experts]`` int64: times each expert was selected per layer."""
        geo = self.geometry
        counts = np.zeros((geo.n_layers, geo.n_routed_experts), dtype=np.int64)
        rows = self.routing()
        if rows:
            layers = np.repeat([r["layer"] for r in rows], geo.top_k)
            experts = np.concatenate([r["experts"] for r in rows])
            np.add.at(counts, (layers, experts), 1)
        return counts

    def summary(self) -> dict:
        """Record and request counts, distinct experts per layer, and the share of
        consecutive token pairs (same request and layer) that kept the same set."""
        rows = self.routing()
        distinct = (self.histogram() > 0).sum(axis=1)
        kept = pairs = 0
        if rows:
            # order by (request, layer, position); a pair is two neighbours one position apart
            req_id = {q: i for i, q in enumerate(sorted({r["request_id"] for r in rows}))}
            key = np.array([(req_id[r["request_id"]], r["layer"], r["token_pos"]) for r in rows])
            sets = np.sort(np.array([r["experts"] for r in rows]), axis=1)
            order = np.lexsort((key[:, 2], key[:, 1], key[:, 0]))
            key, sets = key[order], sets[order]
            adj = (key[1:, 0] == key[:-1, 0]) & (key[1:, 1] == key[:-1, 1]) & (key[1:, 2] == key[:-1, 2] + 1)
            pairs = int(adj.sum())
            kept = int((adj & (sets[1:] == sets[:-1]).all(axis=1)).sum())
        return {"records": len(rows), "requests": len({r["request_id"] for r in rows}),
                "distinct_experts_per_layer": distinct.tolist(),
                "mean_distinct": float(distinct.mean()) if distinct.size else 0.0,
                "adjacent_same_set_ratio": kept / pairs if pairs else None}

    def batches(self, layer: int) -> list[tuple[str, int, np.ndarray, np.ndarray | None]]:
        """The token batches one layer saw: per request, runs of consecutive
        positions, as (request_id, first position, experts [T, k] int32, scores
        [T, k] float32, or None when a record of the run has no scores)."""
        by_req: dict[str, dict[int, dict]] = {}
        for r in self.routing():
            if r["layer"] == layer:
                by_req.setdefault(r["request_id"], {})[r["token_pos"]] = r
        out = []
        for req, at in by_req.items():
            pos = np.array(sorted(at))
            cuts = np.flatnonzero(np.diff(pos) != 1) + 1
            for run in np.split(pos, cuts):
                recs = [at[int(p)] for p in run]
                ex = np.array([r["experts"] for r in recs], dtype=np.int32)
                sc = None
                if all(r.get("scores") is not None for r in recs):
                    sc = np.array([r["scores"] for r in recs], dtype=np.float32)
                out.append((req, int(run[0]), ex, sc))
        return out


class TraceSink:
    """Collects device routing as routing records: pass ``sink.router`` as
    ``trace_hook`` (``moe_layer``) or ``trace=sink`` (``MoELayer``, ``MoEStack``).
    ``idx`` and ``weights`` arrive per token in ascending key order, the order of
    the reference's hook; the weights are stored as ``scores``."""

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

    def to_trace(self, geometry: Geometry, *, repo_id: str, revision: str, source: str,
                 seed: int | None = None) -> Trace:
        return Trace(geometry.header(repo_id=repo_id, revision=revision, source=source, seed=seed),
                     list(self.records))


# ------------------------------------------------------------------ the reference's function names
# Tooling written against the reference's module (``src/deepseeker/trace.py``)
# calls these names; each is a thin call into the classes above and returns
# what the reference's function of that name returns.

def arch_config(manifest: dict) -> dict:
    """``{n_layers, n_routed_experts, top_k}`` of a manifest's architecture block."""
    g = Geometry.of_manifest(manifest)
    return {"n_layers": g.n_layers, "n_routed_experts": g.n_routed_experts, "top_k": g.top_k}


def make_header(repo_id: str, revision: str, source: str, cfg: dict, seed: int | None = None) -> dict:
    """The header line for the geometry ``cfg`` (ValueError on a bad geometry)."""
    g = Geometry(cfg.get("n_layers"), cfg.get("n_routed_experts"), cfg.get("top_k"))
    return g.header(repo_id=repo_id, revision=revision, source=source, seed=seed)


def validate_record(record: dict, header: dict) -> list[str]:
    """The problems of one record against a header's geometry (empty: valid)."""
    return check(record, Geometry.of_header(header))


def write_trace(path, header: dict, records: list[dict]) -> int:
    """Header and records as JSONL; returns the number of records."""
    return Trace(header, list(records)).save(path)


def read_trace(path) -> tuple[dict, list[dict]]:
    """``(header, records)`` of a checked trace file (ValueError at the first broken line)."""
    t = Trace.load(path)
    return t.header, t.records


def expert_records(records: list[dict]) -> list[dict]:
    """Routing records only (subsystem events left out)."""
    return [r for r in records if _is_routing(r)]


def layer_histogram(records: list[dict], n_layers: int) -> dict[int, dict[int, int]]:
    """Per layer, ``{expert: times selected}`` over the routing records."""
    out: dict[int, dict[int, int]] = {layer: {} for layer in range(n_layers)}
    for r in expert_records(records):
        bucket = out[r["layer"]]
        for e in r["experts"]:
            bucket[e] = bucket.get(e, 0) + 1
    return out


def trace_stats(header: dict, records: list[dict]) -> dict:
    """The reference's summary keys: ``records``, ``requests``,
    ``unique_experts_per_layer`` ({layer: distinct experts}), ``mean_unique``
    (their mean over the header's layers) and ``adjacent_same_set_ratio``."""
    rows = expert_records(records)
    s = Trace(header, rows).summary()
    unique = {layer: int(n) for layer, n in enumerate(s["distinct_experts_per_layer"])}
    n_layers = header["n_layers"]
    return {"records": s["records"], "requests": s["requests"], "unique_experts_per_layer": unique,
            "mean_unique": sum(unique.values()) / n_layers if n_layers else 0.0,
            "adjacent_same_set_ratio": s["adjacent_same_set_ratio"]}
