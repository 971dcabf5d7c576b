"""The deepseeker.trace/v1 schema: validation rules (the reference's
tests/test_trace.py cases), round trips, the reference's own recorded trace
(head of profiles/traces/mlx-en.jsonl as a fixture), and the manifest's
routing geometry."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from dsk_moe.trace import (TraceSink, arch_config, layer_histogram, make_header, read_trace,
                           routing_batches, trace_stats, validate_record, write_trace)

GOLDEN = Path(__file__).resolve().parent / "golden"
CFG = {"n_layers": 2, "n_routed_experts": 16, "top_k": 2}


def _header():
    return make_header("repo", "rev", "synthetic", CFG, seed=1)


def test_header_geometry():
    h = _header()
    assert (h["kind"], h["schema"], h["n_layers"], h["top_k"], h["seed"]) == ("header", "deepseeker.trace/v1", 2, 2, 1)
    for bad in ({**CFG, "n_layers": 0}, {**CFG, "top_k": -1}, {**CFG, "n_routed_experts": 1.5}):
        with pytest.raises(ValueError):
            make_header("repo", "rev", "synthetic", bad)


def test_validation_rules():
    h = _header()
    assert validate_record({"request_id": "r", "token_pos": 0, "layer": 1, "experts": [3, 7]}, h) == []
    for bad in ({"request_id": "r", "token_pos": 0, "layer": 9, "experts": [1, 2]},
                {"request_id": "r", "token_pos": 0, "layer": 0, "experts": [1]},
                {"request_id": "r", "token_pos": 0, "layer": 0, "experts": [5, 5]},
                {"request_id": "r", "token_pos": 0, "layer": 0, "experts": [1, 99]},
                {"request_id": "r", "token_pos": 0, "layer": 0, "experts": [1, 2], "scores": [0.5]},
                {"request_id": "", "token_pos": 0, "layer": 0, "experts": [1, 2]},
                {"request_id": "r", "token_pos": -1, "layer": 0, "experts": [1, 2]},
                {"request_id": "r", "token_pos": 0, "layer": 0, "experts": [1, 2], "timing_ms": "x"},
                {"kind": "bogus", "request_id": "r", "token_pos": 0, "layer": 0, "experts": [1, 2]}):
        assert validate_record(bad, h), bad
    engram = {"kind": "event", "request_id": "r", "token_pos": 3, "layer": 1, "extra": {"kind": "engram", "n_hashes": 5}}
    kv = {"kind": "event", "request_id": "r", "token_pos": 3, "layer": 1,
          "extra": {"kind": "kv", "compress_rows": 2, "topk_count": 64}}
    assert validate_record(engram, h) == [] and validate_record(kv, h) == []
    assert validate_record(dict(engram, token_pos=-1), h)
    assert validate_record(dict(kv, extra={"kind": "bogus"}), h)


def test_roundtrip_and_corrupt(tmp_path):
    h = _header()
    sink = TraceSink("req-0")
    sink.router(0, [[1, 2], [3, 4]], [[0.5, 1.0], [0.75, 0.75]])
    sink.advance(2)
    sink(1, [[5, 6]], [[1.0, 0.5]])
    recs = sink.records + [{"kind": "event", "request_id": "req-0", "token_pos": 0, "layer": 1,
                            "extra": {"kind": "kv", "compress_rows": 1, "topk_count": 4}}]
    assert [r["token_pos"] for r in sink.records] == [0, 1, 2]
    path = tmp_path / "t.jsonl"
    assert write_trace(path, h, recs) == 4
    back_h, back = read_trace(path)
    assert back_h["schema"] == "deepseeker.trace/v1" and back == recs
    path.write_text('{"kind": "nope"}\n')
    with pytest.raises(ValueError):
        read_trace(path)
    path.write_text(json.dumps(h) + "\n" + '{"kind": "record"}\n')
    with pytest.raises(ValueError):
        read_trace(path)


def test_reference_recorded_trace():
    h, recs = read_trace(GOLDEN / "trace_mlx_en_head.jsonl")
    assert (h["n_layers"], h["n_routed_experts"], h["top_k"], h["source"]) == (40, 384, 6, "reference-mlx")
    routing = [r for r in recs if "experts" in r]
    assert len(routing) == 208 and len(recs) - len(routing) == 32
    for r in routing:                       # weights in ascending key order, summing to the route scale 1.5
        assert abs(sum(r["scores"]) - 1.5) < 1e-5
    st = trace_stats(h, recs)
    assert st["records"] == 208 and st["requests"] == 1
    hist = layer_histogram(recs, 40)
    assert sum(hist[0].values()) == 7 * 6
    batches = routing_batches(recs, 0)
    assert len(batches) == 1
    req, p0, ex, sc = batches[0]
    assert p0 == 0 and ex.shape == (7, 6) and sc.shape == (7, 6)
    assert (np.diff(np.sort(ex, axis=1), axis=1) > 0).all()


def test_arch_config_from_real_manifest():
    m = json.loads((GOLDEN / "manifest_layer0_subset.json").read_text())
    assert arch_config(m) == {"n_layers": 40, "n_routed_experts": 384, "top_k": 6}
