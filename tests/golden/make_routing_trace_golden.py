"""Writes the routing-trace golden fixtures.

1. `routing_trace_small.jsonl`: a decode routing trace written by libvbmoe's trace writer
   (vbmoe.routing_trace.TraceWriter) from `synthetic_routes()` below: 4 routed layers of 16
   experts, top-2, two training and two held-out requests (one ends on "eos").
2. `routing_trace_mixed.jsonl`: the same writer over three layers of unequal expert sizes, top-k
   and static host placement (`mixed_routes()`).
3. `routing_trace_small_report.json`: what the reference's analyzer,
   tools/benchmark/vrambridge-routing.py, reads from the small trace (digest, counts,
   observation-equivalence flag, the training-derived residency plan at a 20-expert budget) and
   its replays of every residency policy over both traces (warm and cold caches) under the
   fixed costs `REPLAY_COSTS`.
   The analyzer is loaded from the reference checkout given on the command line (it is not
   available where the tests run, so its outputs are committed here as data).

Usage: python tests/golden/make_routing_trace_golden.py /root/reference
"""
from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "unified-memory-scheduler_amd"))

TRACE = HERE / "routing_trace_small.jsonl"
REPORT = HERE / "routing_trace_small_report.json"
EXPERT_BYTES = 13_253_760          # one 120B-shape MXFP4 expert group (weights + fp32 biases)
CAPACITY_EXPERTS = 20
LAYERS = [{"id": i, "experts": 16, "active": 2, "bytes_per_expert": EXPERT_BYTES,
           "static_host_bytes_per_expert": EXPERT_BYTES, "tensor_types": ["f32", "mxfp4"]} for i in (0, 1, 2, 3)]
REQUESTS = [("train-coding", "train", "coding", 11, 12, 12), ("train-prose", "train", "prose", 7, 9, 9),
            ("test-reasoning", "test", "reasoning", 5, 10, 10), ("test-coding", "test", "coding", 9, 12, 8)]


def synthetic_routes(seed: int = 20261201) -> dict[str, np.ndarray]:
    """Per request: [decoded tokens][4 layers][2] expert ids, Zipf(1.1) popularity over a seeded
    permutation per layer, with probability 0.5 of repeating the previous token's pair."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, 17) ** 1.1
    p /= p.sum()
    perms = [rng.permutation(16) for _ in LAYERS]
    out = {}
    for ident, _, _, _, _, decoded in REQUESTS:
        ids = np.zeros((decoded, len(LAYERS), 2), np.int32)
        for t in range(decoded):
            for l in range(len(LAYERS)):
                if t and rng.random() < 0.5:
                    ids[t, l] = ids[t - 1, l]
                else:
                    ids[t, l] = perms[l][rng.choice(16, 2, replace=False, p=p)]
        out[ident] = ids
    return out


MIXED = HERE / "routing_trace_mixed.jsonl"
MIXED_LAYERS = [
    {"id": 9, "experts": 24, "active": 3, "bytes_per_expert": 7_777_777, "static_host_bytes_per_expert": 7_777_777,
     "tensor_types": ["q8_0"]},
    {"id": 0, "experts": 16, "active": 2, "bytes_per_expert": EXPERT_BYTES,
     "static_host_bytes_per_expert": EXPERT_BYTES, "tensor_types": ["f32", "mxfp4"]},
    {"id": 5, "experts": 8, "active": 1, "bytes_per_expert": 4_000_000, "static_host_bytes_per_expert": 1_000_000,
     "tensor_types": ["q8_0"]},
]
MIXED_REQUESTS = [("a", "train", "coding", 4, 20, 20), ("b", "train", "prose", 4, 16, 11),
                  ("c", "test", "reasoning", 4, 18, 18), ("d", "test", "prose", 4, 12, 12)]
# replay parameters: Costs(ram_gbps, pcie_gbps, gpu_expert_us, layer_sync_us, staging_ram_passes),
# admit_after, payback_tokens, cache capacity per trace
REPLAY_COSTS = {"ram_gbps": 64.0, "pcie_gbps": 50.0, "gpu_expert_us": 20.0, "layer_sync_us": 5.0,
                "staging_ram_passes": 2}
REPLAY = {"admit_after": 2, "payback_tokens": 8,
          "capacity": {"small": CAPACITY_EXPERTS * EXPERT_BYTES, "mixed": 5 * EXPERT_BYTES}}
POLICIES = ("measured_static", "train_static", "lru", "lfu", "belady_hits", "cost_aware")
KEEP = ("supported", "expert_calls", "full_expert_hits", "cold_cpu_bytes", "weight_upload_bytes", "evictions",
        "shared_ram_traffic_bytes", "serial_estimated_seconds", "optimistic_overlap_estimated_seconds",
        "warmup_cache_upload_bytes", "initial_resident_upload_bytes", "rejected_cost_admissions",
        "warmup_rejected_cost_admissions")


def mixed_routes(seed: int = 7) -> dict[str, list]:
    """Per request: decoded tokens of per-layer expert lists (metadata order of MIXED_LAYERS, which
    the writer sorts by id), uniform without replacement with a skew toward low expert ids."""
    rng = np.random.default_rng(seed)
    out = {}
    for ident, _, _, _, _, decoded in MIXED_REQUESTS:
        toks = []
        for _ in range(decoded):
            row = {}
            for layer in MIXED_LAYERS:
                p = 1.0 / np.arange(1, layer["experts"] + 1) ** 0.9
                row[layer["id"]] = [int(e) for e in rng.choice(layer["experts"], layer["active"], replace=False, p=p / p.sum())]
            toks.append(row)
        out[ident] = toks
    return out


def write_mixed(path: Path) -> Path:
    from vbmoe.routing_trace import TraceWriter
    routes = mixed_routes()
    with TraceWriter(path, MIXED_LAYERS, "mixed-moe", "vbmoe-synthetic", 64) as w:
        for ident, split, category, prompt, max_tokens, decoded in MIXED_REQUESTS:
            w.request_start(ident, split, category, prompt, max_tokens)
            for row in routes[ident]:
                for lid in sorted(row):
                    w.route(lid, row[lid])
            w.request_end("limit" if decoded == max_tokens else "eos")
    return path


def write_trace(path: Path) -> Path:
    from vbmoe.routing_trace import TraceWriter
    routes = synthetic_routes()
    with TraceWriter(path, LAYERS, "gpt-oss", "vbmoe-synthetic", 64, model="synthetic-120b-shape",
                     token_equivalence_check="routing ids read back from the decode kernels; outputs "
                                             "bit-identical with the read-back off") as w:
        for ident, split, category, prompt, max_tokens, decoded in REQUESTS:
            w.request_start(ident, split, category, prompt, max_tokens)
            for t in range(decoded):
                w.token(routes[ident][t])
            w.request_end("limit" if decoded == max_tokens else "eos", True)
    return path


def main() -> int:
    reference = Path(sys.argv[1])
    for p in (TRACE, MIXED, REPORT):
        p.unlink(missing_ok=True)
    write_trace(TRACE)
    write_mixed(MIXED)
    spec = importlib.util.spec_from_file_location(
        "routing_analysis", reference / "tools" / "benchmark" / "vrambridge-routing.py")
    routing = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = routing
    spec.loader.exec_module(routing)
    data = routing.read_trace(TRACE)
    report = routing.analyze(data, routing.Costs(64.0, 50.0), capacity=CAPACITY_EXPERTS * EXPERT_BYTES)
    keep = {k: report[k] for k in ("trace_sha256", "architecture", "backend_commit", "context_tokens", "counts",
                                   "coverage", "observation_equivalence", "trained_residency_plan")}
    keep["events"] = len(data.events)
    keep["tokens"] = {"train": data.tokens_for("train"), "test": data.tokens_for("test")}
    costs = routing.Costs(REPLAY_COSTS["ram_gbps"], REPLAY_COSTS["pcie_gbps"], REPLAY_COSTS["gpu_expert_us"],
                          REPLAY_COSTS["layer_sync_us"], REPLAY_COSTS["staging_ram_passes"])
    replays = {}
    for name, path in (("small", TRACE), ("mixed", MIXED)):
        trace = routing.read_trace(path)
        replays[name] = {"trace_sha256": trace.sha256}
        for cold in (False, True):
            for policy in POLICIES:
                r = routing.replay(trace, policy, REPLAY["capacity"][name], costs, 0.0, REPLAY["admit_after"], 60.0,
                                   cold_cache=cold, payback_tokens=REPLAY["payback_tokens"])
                replays[name][("cold:" if cold else "") + policy] = {k: r.get(k) for k in KEEP}
    keep["replays"] = replays
    keep["replay_parameters"] = {"costs": REPLAY_COSTS, **REPLAY}
    REPORT.write_text(json.dumps(keep, indent=1, sort_keys=True) + "\n")
    print(TRACE, MIXED, REPORT)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
