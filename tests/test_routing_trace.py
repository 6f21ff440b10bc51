"""Routing traces (writer in libvbmoe, reader and replays in vbmoe.routing_trace) and frozen plans.

Pinned by: the reference analyzer's own reader cases (tests/test_routing_analysis.py:37-144 of the
reference, restated below), the reference analyzer's reading of a trace written by this library
(tests/golden/routing_trace_small_report.json, made by tests/golden/make_routing_trace_golden.py),
Python's JSON serializer as an independent rendering of the same compact sorted-key records, the
admission restatement (oracle/admission.py) for replays, and the reference seed study's report of
a trace written here.
"""
import copy
import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
GOLDEN = REPO / "tests" / "golden"
PLAN = REPO / "unified-memory-scheduler_amd" / "plans" / "gpt120-trained-hot944.txt"
sys.path.insert(0, str(GOLDEN))


@pytest.fixture(scope="module")
def rt(vb):
    from vbmoe import routing_trace
    return routing_trace


def small_layers(host=(0, 10)):
    return [{"id": 0, "experts": 3, "active": 1, "bytes_per_expert": 10, "static_host_bytes_per_expert": host[0]},
            {"id": 1, "experts": 3, "active": 1, "bytes_per_expert": 10, "static_host_bytes_per_expert": host[1]}]


def records(layers=None, training=None, testing=None):
    """The reference analyzer tests' trace builder (tests/test_routing_analysis.py:37-61)."""
    layers = layers or small_layers()
    training = training or [(0, 0), (0, 1), (1, 0)]
    testing = testing or [(0, 2), (1, 0), (2, 1)]
    out = [{"type": "metadata", "schema_version": 1, "instrumented": True, "capture_scope": "decode_only",
            "context_tokens": 256, "backend_commit": "test", "architecture": "test-moe", "model": "test.gguf",
            "static_device_expert_bytes": sum((l["bytes_per_expert"] - l["static_host_bytes_per_expert"])
                                              * l["experts"] for l in layers),
            "layers": layers}]
    for split, sequence in (("train", training), ("test", testing)):
        out.append({"type": "request_start", "id": split, "split": split, "category": "reasoning",
                    "prompt_tokens": 4, "max_tokens": len(sequence)})
        for token, selected in enumerate(sequence):
            for layer, expert in zip(layers, selected):
                out.append({"type": "route", "request": split, "phase": "decode", "token": token,
                            "layer": layer["id"], "experts": expert if isinstance(expert, list) else [expert]})
        out.append({"type": "request_end", "id": split, "decode_tokens": len(sequence), "stop_reason": "limit",
                    "token_sequence_equivalent": True})
    out.append({"type": "trace_end", "requests": 2, "complete": True})
    return out


def dump(tmp_path, values, name="trace.jsonl"):
    path = tmp_path / name
    path.write_text("".join(json.dumps(v) + "\n" for v in values), encoding="utf-8")
    return path


def write_small(rt, path, layers=None, training=((0, 0), (0, 1), (1, 0)), testing=((0, 2), (1, 0), (2, 1))):
    with rt.TraceWriter(path, layers or small_layers(), "test-moe", "test", 256, model="test.gguf") as w:
        for split, seq in (("train", training), ("test", testing)):
            w.request_start(split, split, "reasoning", 4, len(seq))
            for pair in seq:
                for lid, e in zip((0, 1), pair):
                    w.route(lid, [e])
            w.request_end("limit", True)
    return path


# ------------------------------------------------------------------------------------------------
# writer format


def test_writer_emits_compact_sorted_records(rt, tmp_path):
    path = write_small(rt, tmp_path / "t.jsonl")
    lines = path.read_text().splitlines()
    assert lines[0] == (
        '{"architecture":"test-moe","backend_commit":"test","capture_scope":"decode_only","context_tokens":256,'
        '"instrumented":true,"layers":[{"active":1,"bytes_per_expert":10,"experts":3,"id":0,'
        '"static_host_bytes_per_expert":0,"tensor_types":[]},{"active":1,"bytes_per_expert":10,"experts":3,"id":1,'
        '"static_host_bytes_per_expert":10,"tensor_types":[]}],"model":"test.gguf","schema_version":1,'
        '"static_device_expert_bytes":30,"type":"metadata"}')
    assert lines[1] == ('{"category":"reasoning","id":"train","max_tokens":3,"prompt_tokens":4,"split":"train",'
                        '"type":"request_start"}')
    assert lines[2] == '{"experts":[0],"layer":0,"phase":"decode","request":"train","token":0,"type":"route"}'
    assert lines[8] == ('{"decode_tokens":3,"id":"train","stop_reason":"limit","token_sequence_equivalent":true,'
                        '"type":"request_end"}')
    assert lines[-1] == '{"complete":true,"requests":2,"type":"trace_end"}'
    # the same records, as the reference test builds them, read back identically
    ours = [json.loads(line) for line in lines]
    theirs = records()
    for mine, ref in zip(ours, theirs):
        if mine["type"] == "metadata":
            for layer in mine["layers"]:
                assert layer.pop("tensor_types") == []
        assert mine == ref
    for line in lines:
        assert line == json.dumps(json.loads(line), sort_keys=True, separators=(",", ":"), ensure_ascii=False)
    assert not Path(str(path) + ".part").exists()


def test_writer_string_escapes_and_utf8(rt, vb, tmp_path):
    tricky = 'a"b\\c\nd\te\x01f\x1f\x7f-é-€-😀'
    path = tmp_path / "s.jsonl"
    with rt.TraceWriter(path, small_layers(), "arch\u2028x", "c0mmit", 256, model="m\x08.gguf",
                        token_equivalence_check="ctl\x0c\r") as w:
        for split in ("train", "test"):
            w.request_start(tricky + split, split, "cat/é", 4, 1)
            w.route(0, [2])
            w.route(1, [1])
            w.request_end("limit")
    lines = path.read_text(encoding="utf-8").split("\n")[:-1]   # U+2028 is data, not a line break
    for line in lines:
        assert line == json.dumps(json.loads(line), sort_keys=True, separators=(",", ":"), ensure_ascii=False)
    assert json.loads(lines[0])["architecture"] == "arch\u2028x"
    first = json.loads(lines[1])
    assert first["id"] == tricky + "train" and first["category"] == "cat/é"
    assert '\\u0001' in path.read_text(encoding="utf-8")          # lower-case hex control escapes
    # invalid UTF-8 is rejected, not written
    w = rt.TraceWriter(tmp_path / "u.jsonl", small_layers(), "a", "b", 256)
    for bad in (b"\xff", b"a\xc3", b"\xc0\xaf", b"\xed\xa0\x80"):
        with pytest.raises(vb.VbmError, match="UTF-8"):
            vb.call("vbm_trace_request_start", w.handle, bad, b"train", b"c", 1, 1)
    w.abort()
    assert not (tmp_path / "u.jsonl").exists() and not (tmp_path / "u.jsonl.part").exists()


def test_writer_rejections(rt, vb, tmp_path):
    path = tmp_path / "r.jsonl"
    w = rt.TraceWriter(path, small_layers(), "a", "b", 16)
    assert Path(str(path) + ".part").exists() and not path.exists()
    with pytest.raises(vb.VbmError, match="outside"):
        w.route(0, [0])                                     # no open request
    with pytest.raises(vb.VbmError, match="context"):
        w.request_start("x", "train", "c", 10, 7)            # 10 + 7 > 16
    with pytest.raises(vb.VbmError, match="split"):
        w.request_start("x", "dev", "c", 1, 1)
    w.request_start("x", "train", "c", 4, 2)
    with pytest.raises(vb.VbmError, match="nested"):
        w.request_start("y", "train", "c", 4, 2)
    with pytest.raises(vb.VbmError, match="out-of-order"):
        w.route(1, [0])                                     # layer 0 comes first
    with pytest.raises(vb.VbmError, match="Out-of-range or duplicate"):
        w.route(0, [3])
    with pytest.raises(vb.VbmError, match="active"):
        w.route(0, [0, 1])
    with pytest.raises(vb.VbmError, match="not a routed layer"):
        w.route(5, [0])
    w.route(0, [1])
    with pytest.raises(vb.VbmError, match="Missing or duplicate routing observations in layer 1"):
        w.request_end("eos")
    w.route(1, [2])
    assert w.position() == (2, 1, 1, 0)
    with pytest.raises(vb.VbmError, match="stop reason"):
        w.request_end("limit")                              # 1 of 2 tokens
    w.token(np.array([[0], [1]]))
    with pytest.raises(vb.VbmError, match="max_tokens"):
        w.route(0, [0])
    with pytest.raises(vb.VbmError, match="stop reason"):
        w.request_end("eos")                                # 2 of 2 tokens is the limit
    w.request_end("limit")
    with pytest.raises(vb.VbmError, match="duplicate request"):
        w.request_start("x", "test", "c", 4, 2)
    w.request_start("z", "test", "c", 4, 2)
    with pytest.raises(vb.VbmError, match="incomplete"):
        w.close()                                           # consumes the handle, drops the partial
    assert not path.exists() and not Path(str(path) + ".part").exists()
    # refuses to overwrite a published trace or a partial
    write_small(rt, tmp_path / "done.jsonl")
    with pytest.raises(vb.VbmError, match="overwrite"):
        rt.TraceWriter(tmp_path / "done.jsonl", small_layers(), "a", "b", 16)
    (tmp_path / "p.jsonl.part").write_text("")
    with pytest.raises(vb.VbmError, match="overwrite"):
        rt.TraceWriter(tmp_path / "p.jsonl", small_layers(), "a", "b", 16)
    bad_layers = small_layers()
    bad_layers[0]["active"] = 4
    with pytest.raises(vb.VbmError, match="expert counts"):
        rt.TraceWriter(tmp_path / "q.jsonl", bad_layers, "a", "b", 16)
    bad_layers = small_layers(host=(11, 0))
    with pytest.raises(vb.VbmError, match="byte accounting"):
        rt.TraceWriter(tmp_path / "q.jsonl", bad_layers, "a", "b", 16)


def test_writer_sorts_layers_and_token_strides(rt, tmp_path):
    layers = [{"id": 7, "experts": 3, "active": 1, "bytes_per_expert": 20, "static_host_bytes_per_expert": 20},
              {"id": 2, "experts": 4, "active": 2, "bytes_per_expert": 12, "static_host_bytes_per_expert": 6,
               "tensor_types": ["q8_0", "f32", "q8_0"]}]
    path = tmp_path / "v.jsonl"
    with rt.TraceWriter(path, layers, "a", "b", 64) as w:
        for split, toks in (("train", [[[0, 1], [0, 9]], [[1, 2], [1, 9]]]), ("test", [[[1, 3], [2, 9]]])):
            w.request_start(split, split, "c", 1, len(toks))
            for ids in toks:
                # layer 2 (two experts) first, then layer 7 (one): rows of stride 2, padding ignored
                w.token(np.array(ids, np.int32))
            w.request_end("limit")
    meta = json.loads(path.read_text().splitlines()[0])
    assert [l["id"] for l in meta["layers"]] == [2, 7]
    assert meta["layers"][0]["tensor_types"] == ["f32", "q8_0"]
    assert meta["static_device_expert_bytes"] == 24
    data = rt.read_trace(path)
    assert data.route_experts == [(0, 1), (0,), (1, 2), (1,), (1, 3), (2,)]
    # the reference analyzer test of the same shape: 3 calls, 32 cold bytes, gpu fraction 12/44
    test_calls = sum(len(e) for _, e in data.routes("test"))
    cold = sum(len(e) * data.layers[l].host_bytes for l, e in data.routes("test"))
    total = sum(len(e) * data.layers[l].bytes for l, e in data.routes("test"))
    assert (test_calls, cold) == (3, 32) and abs(1 - cold / total - 12 / 44) < 1e-12


# ------------------------------------------------------------------------------------------------
# reader: the reference analyzer's own cases


def test_reader_counts(rt, tmp_path):
    data = rt.read_trace(dump(tmp_path, records()))
    assert data.decoded("train") == 3 and data.decoded("test") == 3
    assert len(data.route_layer) == 12 and len(data.sha256) == 64
    assert all(r.equivalence_checked for r in data.requests)
    assert [(r.first_route, r.end_route) for r in data.requests] == [(0, 6), (6, 12)]


def test_reader_rejects_incomplete_or_reordered(rt, tmp_path):
    original = records()
    bad = [original[:-1], original + [original[-1]], original[1:]]
    changed = copy.deepcopy(original)
    del changed[3]
    bad.append(changed)
    changed = copy.deepcopy(original)
    changed[2], changed[3] = changed[3], changed[2]
    bad.append(changed)
    for values in bad:
        with pytest.raises(ValueError):
            rt.read_trace(dump(tmp_path, values))


@pytest.mark.parametrize("changes", [{"experts": [True]}, {"experts": [-1]}, {"experts": [3]}, {"experts": [0, 0]},
                                     {"token": True}, {"phase": "prefill"}, {"request": "unknown"}, {"layer": 99}])
def test_reader_rejects_invalid_route(rt, tmp_path, changes):
    values = records()
    values[2].update(changes)
    with pytest.raises(ValueError):
        rt.read_trace(dump(tmp_path, values))


@pytest.mark.parametrize("case", range(10))
def test_reader_rejects_inconsistent_metadata_and_stops(rt, tmp_path, case):
    values = records()
    [lambda v: v[0].update(schema_version=True),
     lambda v: v[0].update(static_device_expert_bytes=29),
     lambda v: v[0]["layers"][0].update(static_host_bytes_per_expert=11),
     lambda v: v[0]["layers"].append(v[0]["layers"][0]),
     lambda v: v[8].update(decode_tokens=2),
     lambda v: v[8].update(stop_reason="eos"),
     lambda v: v[8].update(token_sequence_equivalent=False),
     lambda v: v[8].update(token_sequence_equivalent="true"),
     lambda v: v[-1].update(complete=False),
     lambda v: [r.update(split="test") for r in v if r["type"] == "request_start"]][case](values)
    with pytest.raises(ValueError):
        rt.read_trace(dump(tmp_path, values))


def test_reader_legacy_trace_is_not_verified(rt, tmp_path):
    values = records()
    for v in values:
        v.pop("token_sequence_equivalent", None)
    data = rt.read_trace(dump(tmp_path, values))
    assert not any(r.equivalence_checked for r in data.requests)


def test_hotset_uses_training_counts_only(rt):
    layers = {0: rt.LayerSpec(3, 1, 10, 10)}
    assert rt.hot_experts(rt.Counter({(0, 0): 10, (0, 1): 2}), layers, 10) == [(0, 0)]
    layers = {0: rt.LayerSpec(3, 1, 10, 10), 1: rt.LayerSpec(3, 1, 25, 25)}
    counts = rt.Counter({(1, 0): 5, (0, 2): 5, (0, 1): 4, (1, 1): 9})
    # budget 40: (1,1) 25 B; then count 5 ties by size: (0,2) 10 B; (1,0) no longer fits; (0,1) does not
    assert rt.hot_experts(counts, layers, 40) == [(1, 1), (0, 2)]


# ------------------------------------------------------------------------------------------------
# golden: the reference analyzer reading a trace written by this library


def test_golden_trace_bytes_and_reference_reading(rt, tmp_path):
    import make_routing_trace_golden as mk
    report = json.loads((GOLDEN / "routing_trace_small_report.json").read_text())
    path = mk.write_trace(tmp_path / "small.jsonl")
    assert path.read_bytes() == (GOLDEN / "routing_trace_small.jsonl").read_bytes()
    assert hashlib.sha256(path.read_bytes()).hexdigest() == report["trace_sha256"]
    data = rt.read_trace(path)
    assert data.sha256 == report["trace_sha256"]
    assert len(data.route_layer) == report["events"]
    assert {"train": data.decoded("train"), "test": data.decoded("test")} == report["tokens"]
    assert report["counts"] == {"layers": len(data.layers), "requests": len(data.requests),
                                "train_tokens": data.decoded("train"), "test_tokens": data.decoded("test")}
    assert report["observation_equivalence"]["all_requests_verified"] is True
    plan = rt.plan_from_trace(data, mk.CAPACITY_EXPERTS)
    assert len(plan) == mk.CAPACITY_EXPERTS
    by_layer = {entry["layer"]: entry["experts"] for entry in report["trained_residency_plan"]["layers"]}
    assert {l: sorted(e for ll, e in plan if ll == l) for l in range(4)} == by_layer
    assert report["trained_residency_plan"]["used_bytes"] == len(plan) * mk.EXPERT_BYTES


# ------------------------------------------------------------------------------------------------
# frozen plans and the admission replay


def test_trained_hot944_plan(rt):
    assert hashlib.sha256(PLAN.read_bytes()).hexdigest() == \
        "6a679bec76f1a410ed65fa79c186d164a388fc76419d96dcad5978782343949c"
    plan = rt.read_plan(PLAN, 36, 128)
    assert len(plan) == 944 and len(set(plan)) == 944
    assert plan[:3] == [(26, 38), (30, 116), (35, 117)]
    assert {l for l, _ in plan} == set(range(36))
    with pytest.raises(ValueError):
        rt.read_plan(PLAN, 35, 128)                         # layer 35 out of range
    with pytest.raises(ValueError):
        rt.read_plan(PLAN, 36, 127)                         # expert 127 out of range


@pytest.mark.parametrize("text", ["0 1\n0 1\n", "0\n", "0 1 2\n", "a b\n", "-1 0\n", "0 8\n", "2 0\n"])
def test_plan_rejections(rt, tmp_path, text):
    p = tmp_path / "plan.txt"
    p.write_text(text)
    with pytest.raises(ValueError, match="frozen hybrid plan"):
        rt.read_plan(p, 2, 8)


def test_plan_comments_and_round_trip(rt, tmp_path):
    p = tmp_path / "plan.txt"
    p.write_text("# trained\n\n1 7\n0 3\n")
    assert rt.read_plan(p, 2, 8) == [(1, 7), (0, 3)]
    q = rt.write_plan(tmp_path / "q.txt", [(1, 7), (0, 3)])
    assert rt.read_plan(q, 2, 8) == [(1, 7), (0, 3)]


@pytest.mark.parametrize("policy", [0, 1, 3, 5])
def test_replay_admission_matches_restatement(rt, tmp_path, policy):
    import admission as ref
    data = rt.read_trace(GOLDEN / "routing_trace_small.jsonl")
    plan = rt.plan_from_trace(data, 6)
    margin = 1 if policy == ref.LRU else 2
    stats = rt.replay_admission(data, 2 + 10, policy, recent_window=8, margin=margin, plan=plan,
                                lfu=(2, 1) if policy == ref.LFU else None)
    py = ref.Admission(4, 16, 2, 12, 8, margin, policy)
    if policy == ref.LFU:
        py.lfu_admit_after, py.lfu_fill_after = 2, 1
    for layer, expert in plan:
        py.seed(layer, expert)
    hits = admissions = evictions = staged = 0
    for layer, experts in data.routes():
        h, adm = py.admit(layer, list(experts))
        hits += sum(h)
        admissions += len(adm)
        evictions += sum(1 for _, _, ev in adm if ev >= 0)
        staged += sum(1 for e in experts if py.slot_map[layer * 16 + e] < 0)
    a = stats["all"]
    assert (a.dispatches, a.hits, a.admissions, a.evictions, a.staged) == \
        (len(data.route_layer), hits, admissions, evictions, staged)
    assert a.lookups == 2 * len(data.route_layer) and a.admissions > 0
    assert stats["train"].dispatches + stats["test"].dispatches == a.dispatches
    assert stats["train"].hits + stats["test"].hits == a.hits


# ------------------------------------------------------------------------------------------------
# residency replays against the reference analyzer's own replays of the same traces


@pytest.mark.parametrize("trace_name", ["small", "mixed"])
def test_residency_replays_match_reference_analyzer(rt, trace_name):
    import make_routing_trace_golden as mk
    report = json.loads((GOLDEN / "routing_trace_small_report.json").read_text())
    golden = report["replays"][trace_name]
    params = report["replay_parameters"]
    path = GOLDEN / f"routing_trace_{trace_name}.jsonl"
    data = rt.read_trace(path)
    assert data.sha256 == golden["trace_sha256"]
    costs = params["costs"]
    checked = 0
    for name, want in golden.items():
        if name == "trace_sha256":
            continue
        cold = name.startswith("cold:")
        policy = name.split(":")[-1]
        got = rt.replay_residency(data, policy, params["capacity"][trace_name], costs["ram_gbps"], costs["pcie_gbps"],
                                  costs["gpu_expert_us"], costs["layer_sync_us"], costs["staging_ram_passes"],
                                  admit_after=params["admit_after"], payback_tokens=params["payback_tokens"],
                                  cold_cache=cold)
        assert got["supported"] == want["supported"], name
        if not want["supported"]:
            continue
        for key in mk.KEEP:
            w, g = want[key], got[key]
            if isinstance(w, float):
                assert g == pytest.approx(w, rel=1e-12, abs=0), (name, key, g, w)
            else:
                assert g == w, (name, key, g, w)
        checked += 1
    assert checked >= 10                                    # belady needs equal sizes (mixed: unsupported)


def test_residency_replay_rejects_bad_parameters(rt, vb):
    data = rt.read_trace(GOLDEN / "routing_trace_small.jsonl")
    with pytest.raises(ValueError, match="Unknown residency"):
        rt.replay_residency(data, "unknown", 10, 1.0, 1.0)
    with pytest.raises(vb.VbmError, match="finite and positive"):
        rt.replay_residency(data, "lru", 10, 0.0, 1.0)
    with pytest.raises(vb.VbmError, match="staging"):
        rt.replay_residency(data, "lru", 10, 1.0, 1.0, staging_ram_passes=1)
    with pytest.raises(vb.VbmError, match=">= 1"):
        rt.replay_residency(data, "cost_aware", 10, 1.0, 1.0, payback_tokens=0)


# ------------------------------------------------------------------------------------------------
# prefill summary (routing_trace.cpp:180-225, 500-519, 570-580, 750-769)

SHA = "0123456789abcdef" * 4


def write_prefill(rt, tmp_path, prefill_batches, name="p"):
    """Two requests over small_layers(); prefill_batches(split) yields (layer, ids) per batch."""
    trace, summary = tmp_path / f"{name}.jsonl", tmp_path / f"{name}.json"
    with rt.TraceWriter(trace, small_layers(), "test-moe", "test", 256, model="test.gguf",
                        collector_source_sha256=SHA) as w:
        w.enable_prefill(summary, 512, 128, cpu_threads=8, batch_threads=16)
        for split, seq in (("train", ((0, 0), (0, 1))), ("test", ((1, 2),))):
            w.request_start(split, split, "code", 4, len(seq))
            for layer, ids in prefill_batches(split):
                w.prefill_route(layer, ids)
            for pair in seq:
                w.token(np.array(pair, np.int32).reshape(2, 1))
            w.request_end("limit", True)
    return trace, summary


def test_prefill_summary_format_and_histograms(rt, tmp_path):
    def batches(split):
        yield 0, [[0], [2], [2]]
        yield 1, [[1], [1], [0]]
        yield 0, [[1]]                              # a second batch: layer 0 sees all 4 prompt rows
        if split == "test":
            yield 1, np.zeros((0, 1), np.int32)     # output-pruned batch: zero rows are recorded
    trace, summary = write_prefill(rt, tmp_path, batches)
    text = summary.read_text(encoding="utf-8")
    doc = json.loads(text)
    # nlohmann dump(2) of sorted keys is Python's indent-2 sorted rendering
    assert text == json.dumps(doc, sort_keys=True, indent=2, ensure_ascii=False) + "\n"
    assert {k: doc[k] for k in ("schema_version", "capture_scope", "instrumented", "performance_measurement",
                                "full_model_acceleration_claim", "complete", "batch_size", "microbatch_size",
                                "cpu_threads", "batch_threads", "context_tokens", "model", "architecture",
                                "backend_commit", "collector_source_sha256")} == {
        "schema_version": 1, "capture_scope": "observed_prefill_expert_rows", "instrumented": True,
        "performance_measurement": False, "full_model_acceleration_claim": False, "complete": True,
        "batch_size": 512, "microbatch_size": 128, "cpu_threads": 8, "batch_threads": 16, "context_tokens": 256,
        "model": "test.gguf", "architecture": "test-moe", "backend_commit": "test", "collector_source_sha256": SHA}
    meta = json.loads(trace.read_text().splitlines()[0])
    assert meta["collector_source_sha256"] == SHA and doc["layers"] == meta["layers"]
    assert doc["coverage_note"].startswith("Observed graph rows only")
    train, test = doc["requests"]
    assert train["id"] == "train" and train["split"] == "train" and train["category"] == "code"
    assert train["prompt_tokens"] == 4 and train["token_sequence_equivalent"] is True
    assert [b["expert_row_counts"] for b in train["batches"]] == [[1, 0, 2], [1, 2, 0], [0, 1, 0]]
    assert [(b["layer"], b["rows"], b["active_experts_per_row"]) for b in test["batches"]] == \
        [(0, 3, 1), (1, 3, 1), (0, 1, 1), (1, 0, 1)]
    assert test["batches"][3]["expert_row_counts"] == [0, 0, 0]
    assert train["coverage"] == [{"covers_all_prompt_rows": True, "layer": 0, "observed_rows": 4},
                                 {"covers_all_prompt_rows": False, "layer": 1, "observed_rows": 3}]
    assert not Path(str(summary) + ".part").exists()
    # the decode trace itself is unchanged by the prefill capture
    data = rt.read_trace(trace)
    assert data.decoded("train") == 2 and data.decoded("test") == 1


def test_prefill_histogram_of_random_batches(rt, tmp_path):
    rng = np.random.default_rng(3)
    layers = [{"id": 5, "experts": 32, "active": 4, "bytes_per_expert": 1, "static_host_bytes_per_expert": 0}]
    ids = np.stack([rng.permutation(32)[:4] for _ in range(300)]).astype(np.int32)
    summary = tmp_path / "r.json"
    with rt.TraceWriter(tmp_path / "r.jsonl", layers, "a", "b", 4096, collector_source_sha256=SHA) as w:
        w.enable_prefill(summary, 1, 1)
        w.request_start("r", "train", "c", 300, 1)
        w.prefill_route(5, ids[:100])
        w.prefill_route(5, ids[100:])
        w.token(np.array([[1, 2, 3, 4]], np.int32))
        w.request_end("limit", True)
    doc = json.loads(summary.read_text())
    hists = [b["expert_row_counts"] for b in doc["requests"][0]["batches"]]
    assert hists == [np.bincount(ids[:100].ravel(), minlength=32).tolist(),
                     np.bincount(ids[100:].ravel(), minlength=32).tolist()]
    assert "model" not in doc                                  # omitted like the trace metadata's


def test_prefill_rejections(rt, vb, tmp_path):
    layers = small_layers()
    with pytest.raises(vb.VbmError, match="collector_source_sha256"):
        with rt.TraceWriter(tmp_path / "a.jsonl", layers, "a", "b", 256) as w:
            w.enable_prefill(tmp_path / "a.json", 1, 1)
    with pytest.raises(vb.VbmError, match="64 lower-case hex"):
        rt.TraceWriter(tmp_path / "h.jsonl", layers, "a", "b", 256, collector_source_sha256=SHA.upper())
    (tmp_path / "exists.json").write_text("{}")
    with pytest.raises(vb.VbmError, match="Refusing to overwrite"):
        with rt.TraceWriter(tmp_path / "b.jsonl", layers, "a", "b", 256, collector_source_sha256=SHA) as w:
            w.enable_prefill(tmp_path / "exists.json", 1, 1)
    with pytest.raises(vb.VbmError, match="must not alias"):
        with rt.TraceWriter(tmp_path / "c.jsonl", layers, "a", "b", 256, collector_source_sha256=SHA) as w:
            w.enable_prefill(tmp_path / "c.jsonl.part", 1, 1)

    def case(body, match, name):
        with pytest.raises((vb.VbmError, ValueError), match=match):
            with rt.TraceWriter(tmp_path / f"{name}.jsonl", layers, "a", "b", 256, collector_source_sha256=SHA) as w:
                w.enable_prefill(tmp_path / f"{name}.json", 1, 1)
                w.request_start("r", "train", "c", 4, 1)
                body(w)
        assert not (tmp_path / f"{name}.json").exists() and not (tmp_path / f"{name}.jsonl").exists()

    case(lambda w: w.prefill_route(0, [[3]]), "Out-of-range", "range")
    case(lambda w: w.prefill_route(0, [[-1]]), "Out-of-range", "negative")
    case(lambda w: w.prefill_route(2, [[0]]), "layer", "unknown")
    case(lambda w: w.prefill_route(0, [[0, 1]]), r"\[rows\]\[1\]", "shape")
    case(lambda w: w.prefill_route(0, np.zeros((32769, 1), np.int32)), "0..32768", "rows")
    # a layer without observed rows, or more rows than the prompt, stops decoding
    case(lambda w: (w.prefill_route(0, [[0]]), w.route(0, [1])), "Missing or duplicate prefill", "missing")
    case(lambda w: (w.prefill_route(0, [[0]] * 5), w.prefill_route(1, [[0]]), w.route(0, [1])),
         "Missing or duplicate prefill", "excess")
    case(lambda w: (w.prefill_route(0, [[0]]), w.prefill_route(1, [[0]]), w.route(0, [1]), w.prefill_route(0, [[1]])),
         "precede", "late")
    case(lambda w: w.request_end("eos", True), "Missing or duplicate prefill", "empty")


def test_prefill_duplicate_expert_in_row(rt, vb, tmp_path):
    layers = [{"id": 0, "experts": 8, "active": 2, "bytes_per_expert": 1, "static_host_bytes_per_expert": 0}]
    with pytest.raises(vb.VbmError, match="duplicate routed expert"):
        with rt.TraceWriter(tmp_path / "d.jsonl", layers, "a", "b", 256, collector_source_sha256=SHA) as w:
            w.enable_prefill(tmp_path / "d.json", 1, 1)
            w.request_start("r", "train", "c", 4, 1)
            w.prefill_route(0, [[1, 2], [3, 3]])


def test_belady_hits_is_optimal_by_exhaustive_search(rt):
    """belady_hits against an exhaustive oracle (as tests/test_routing_analysis.py:271-294 of the
    reference does): over every sequence of end-of-layer cache states (each a subset of at most
    `slots` keys of the previous state and the event's experts), the most hits any schedule gets
    on a tiny trace must equal the replay's."""
    from itertools import combinations
    rng = np.random.default_rng(5)
    size = 10
    for trial in range(40):
        experts, active, slots, n_events = 5, 2, 2 + trial % 2, 7
        layers = {0: rt.LayerSpec(experts, active, size, size)}
        requests = [rt.RequestSpan("t", "test", "c", 1, n_events, n_events, True, 0, n_events)]
        picks = [tuple(int(e) for e in rng.choice(experts, active, replace=False)) for _ in range(n_events)]
        data = rt.RoutingTrace({"static_device_expert_bytes": 0}, layers, requests, np.zeros(n_events, np.int32),
                               np.arange(n_events, dtype=np.int32), np.zeros(n_events, np.int32), picks)
        got = rt.replay_residency(data, "belady_hits", slots * size, 64.0, 50.0)
        best = {frozenset(): 0}
        for ev in picks:
            keys = set(ev)
            nxt = {}
            for state, hits in best.items():
                h = hits + len(keys & state)
                pool = sorted(state | keys)
                for m in range(0, min(slots, len(pool)) + 1):
                    for sub in combinations(pool, m):
                        s = frozenset(sub)
                        if nxt.get(s, -1) < h:
                            nxt[s] = h
            best = nxt
        assert got["full_expert_hits"] == max(best.values()), (trial, picks)
