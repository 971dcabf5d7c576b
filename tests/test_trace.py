"""The deepseeker.trace/v1 format: the validity rules (the cases of the
reference's tests/test_trace.py), round trips, the reference's own recorded
trace (head of profiles/traces/mlx-en.jsonl as a fixture), and the routing
geometry of the reference's model manifest."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from dsk_moe.trace import FIELDS, Geometry, Trace, TraceSink, check

GOLDEN = Path(__file__).resolve().parent / "golden"
GEO = Geometry(n_layers=2, n_routed_experts=16, top_k=2)


def test_geometry_and_header():
    h = GEO.header(repo_id="repo", revision="rev", source="synthetic", seed=1)
    assert (h["kind"], h["schema"], h["n_layers"], h["top_k"], h["seed"]) == ("header", "deepseeker.trace/v1", 2, 2, 1)
    assert Geometry.of_header(h) == GEO
    for bad in ((0, 16, 2), (2, 16, -1), (2, 1.5, 2), (True, 16, 2)):
        with pytest.raises(ValueError):
            Geometry(*bad)


def test_validity_rules():
    ok = {"request_id": "r", "token_pos": 0, "layer": 1, "experts": [3, 7]}
    assert check(ok, GEO) == []
    assert check(dict(ok, scores=[0.5, 1], timing_ms=1.5, bytes_moved=10, extra={"a": 1}), GEO) == []
    assert check(dict(ok, scores=None), GEO) == []                     # null optional fields are absent
    broken = {"layer": dict(ok, layer=9), "experts": dict(ok, experts=[1]),
              "distinct": dict(ok, experts=[5, 5]), "range": dict(ok, experts=[1, 99]),
              "scores": dict(ok, scores=[0.5]), "request": dict(ok, request_id=""),
              "position": dict(ok, token_pos=-1), "timing": dict(ok, timing_ms="x"),
              "bool id": dict(ok, experts=[True, 2]), "extra": dict(ok, extra=[1]),
              "kind": dict(ok, kind="bogus"), "missing": {"request_id": "r", "token_pos": 0, "layer": 0}}
    for name, rec in broken.items():
        assert check(rec, GEO), name
    assert check(broken["missing"], GEO) == ["experts: required"]
    engram = {"kind": "event", "request_id": "r", "token_pos": 3, "layer": 1, "extra": {"kind": "engram", "n_hashes": 5}}
    kv = {"kind": "event", "request_id": "r", "token_pos": 3, "layer": 1,
          "extra": {"kind": "kv", "compress_rows": 2, "topk_count": 64}}
    assert check(engram, GEO) == [] and check(kv, GEO) == []
    assert check(dict(engram, token_pos=-1), GEO)
    assert check(dict(kv, extra={"kind": "bogus"}), GEO)
    assert check(dict(kv, extra=None), GEO) == ["extra: required"]
    assert set(FIELDS) == {"record", "event"}


def test_roundtrip_and_broken_files(tmp_path):
    sink = TraceSink("req-0")
    sink.router(0, [[1, 2], [3, 4]], [[0.5, 1.0], [0.75, 0.75]])
    sink.advance(2)
    sink(1, [[5, 6]], [[1.0, 0.5]])
    assert [r["token_pos"] for r in sink.records] == [0, 1, 2]
    tr = sink.to_trace(GEO, repo_id="repo", revision="rev", source="synthetic")
    tr.records.append({"kind": "event", "request_id": "req-0", "token_pos": 0, "layer": 1,
                       "extra": {"kind": "kv", "compress_rows": 1, "topk_count": 4}})
    path = tmp_path / "t.jsonl"
    assert tr.save(path) == 4
    lines = [json.loads(s) for s in path.read_text().splitlines()]
    assert [ln["kind"] for ln in lines] == ["header", "record", "record", "record", "event"]
    back = Trace.load(path)
    assert back.header["schema"] == "deepseeker.trace/v1" and back.records == tr.records
    for text in ('{"kind": "nope"}\n', json.dumps(tr.header) + '\n{"kind": "record"}\n',
                 json.dumps(tr.header) + "\n{not json\n", ""):
        path.write_text(text)
        with pytest.raises(ValueError):
            Trace.load(path)


def test_summary_and_batches():
    sink = TraceSink("a")
    sink(0, [[1, 2], [2, 1], [3, 4], [5, 6]], [[1, 1]] * 4)       # positions 0..3
    sink.token_start = 10
    sink(0, [[5, 6]], [[1, 1]])                                     # a second run at 10
    sink(1, [[7, 8]], [[1, 1]])
    tr = sink.to_trace(GEO, repo_id="r", revision="v", source="s")
    st = tr.summary()
    # pairs (0,1) same set, (1,2) and (2,3) differ; 3 -> 10 is not adjacent
    assert st["records"] == 6 and st["requests"] == 1 and st["adjacent_same_set_ratio"] == pytest.approx(1 / 3)
    assert st["distinct_experts_per_layer"] == [6, 2]
    hist = tr.histogram()
    assert hist.shape == (2, 16) and hist[0, 1] == 2 and hist[0, 5] == 2 and hist[1].sum() == 2
    b = tr.batches(0)
    assert [(q, p0, ex.shape) for q, p0, ex, _ in b] == [("a", 0, (4, 2)), ("a", 10, (1, 2))]


def test_reference_recorded_trace():
    tr = Trace.load(GOLDEN / "trace_mlx_en_head.jsonl")
    h = tr.header
    assert (h["n_layers"], h["n_routed_experts"], h["top_k"], h["source"]) == (40, 384, 6, "reference-mlx")
    routing = tr.routing()
    assert len(routing) == 208 and len(tr.records) - len(routing) == 32
    for r in routing:                       # weights in ascending key order, summing to the route scale 1.5
        assert abs(sum(r["scores"]) - 1.5) < 1e-5
    st = tr.summary()
    assert st["records"] == 208 and st["requests"] == 1
    assert tr.histogram()[0].sum() == 7 * 6
    batches = tr.batches(0)
    assert len(batches) == 1
    req, p0, ex, sc = batches[0]
    assert p0 == 0 and ex.shape == (7, 6) and sc.shape == (7, 6)
    assert (np.diff(np.sort(ex, axis=1), axis=1) > 0).all()


def test_geometry_of_real_manifest():
    m = json.loads((GOLDEN / "manifest_layer0_subset.json").read_text())
    assert Geometry.of_manifest(m) == Geometry(40, 384, 6)


def test_reference_function_names(tmp_path):
    """The reference module's functions (src/deepseeker/trace.py:35-208) under
    their names, with its return shapes: hand-computed on a small trace."""
    from dsk_moe import trace as T
    m = json.loads((GOLDEN / "manifest_layer0_subset.json").read_text())
    assert T.arch_config(m) == {"n_layers": 40, "n_routed_experts": 384, "top_k": 6}
    h = T.make_header("r", "v", "synthetic", {"n_layers": 2, "n_routed_experts": 16, "top_k": 2}, seed=3)
    assert h["schema"] == "deepseeker.trace/v1" and h["seed"] == 3 and h["kind"] == "header"
    with pytest.raises(ValueError):
        T.make_header("r", "v", "s", {"n_layers": 0, "n_routed_experts": 16, "top_k": 2})
    recs = [{"request_id": "a", "token_pos": p, "layer": 0, "experts": e}
            for p, e in enumerate([[1, 2], [2, 1], [3, 4]])]
    recs += [{"request_id": "b", "token_pos": 0, "layer": 1, "experts": [5, 6]},
             {"kind": "event", "request_id": "b", "token_pos": 0, "layer": 1, "extra": {"kind": "kv"}}]
    assert T.validate_record(recs[0], h) == []
    assert T.validate_record({"request_id": "a", "token_pos": 0, "layer": 2, "experts": [1, 2]}, h)
    path = tmp_path / "t.jsonl"
    assert T.write_trace(path, h, recs) == 5
    h2, back = T.read_trace(path)
    assert h2 == h and back == recs
    assert len(T.expert_records(back)) == 4
    assert T.layer_histogram(back, 2) == {0: {1: 2, 2: 2, 3: 1, 4: 1}, 1: {5: 1, 6: 1}}
    st = T.trace_stats(h, back)
    assert st == {"records": 4, "requests": 2, "unique_experts_per_layer": {0: 4, 1: 2},
                  "mean_unique": 3.0, "adjacent_same_set_ratio": 0.5}
