"""Writes the routing-trace golden fixtures.

1. `routing_trace_small.jsonl`: a decode routing trace written by libvbmoe's trace writer
   (vbmoe.routing_trace.TraceWriter) from `synthetic_routes()` below: 4 routed layers of 16
   experts, top-2, two training and two held-out requests (one ends on "eos").
2. `routing_trace_small_report.json`: what the reference's analyzer,
   tools/benchmark/vrambridge-routing.py, reads from that file: its digest, counts,
   observation-equivalence flag and the training-derived residency plan at a 20-expert budget.
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
    for p in (TRACE, REPORT):
        p.unlink(missing_ok=True)
    write_trace(TRACE)
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
    REPORT.write_text(json.dumps(keep, indent=1, sort_keys=True) + "\n")
    print(TRACE, REPORT)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
