"""Writes the prompt-conditioned seed study fixtures.

1. `routing_trace_prefill.jsonl` and `routing_trace_prefill_summary.json`: a decode routing trace
   and the prefill summary written with it by libvbmoe's trace writer (TraceWriter with
   enable_prefill / prefill_route) from `prefill_routes()` below: 4 routed layers of 16 experts,
   top-2, two training and two held-out requests; prompts arrive in several batches, one
   held-out request's last layer is observed on part of its prompt only (output pruning) and one
   batch has zero rows.
2. `routing_trace_prefill_plan.txt`: the baseline plan (12 experts) the seeds are measured against.
3. `routing_trace_prefill_report.json`: what the reference's study,
   tools/benchmark/vrambridge-prefill-seed.py, reads from them (`read_prefill`) and reports
   (`analyze`) at the fixed costs `COSTS`.
   The study is loaded from the reference checkout given on the command line (it is not available
   where the tests run, so its outputs are committed here as data).

Usage: python tests/golden/make_prefill_seed_golden.py /root/reference
"""
from __future__ import annotations

import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1] / "unified-memory-scheduler_amd"))

TRACE = HERE / "routing_trace_prefill.jsonl"
SUMMARY = HERE / "routing_trace_prefill_summary.json"
PLAN = HERE / "routing_trace_prefill_plan.txt"
REPORT = HERE / "routing_trace_prefill_report.json"
EXPERT_BYTES = 13_253_760
SHA = "5eed" * 16
LAYERS = [{"id": i, "experts": 16, "active": 2, "bytes_per_expert": EXPERT_BYTES,
           "static_host_bytes_per_expert": EXPERT_BYTES, "tensor_types": ["f32", "mxfp4"]} for i in (0, 1, 2, 3)]
# id, split, category, prompt tokens, max tokens, decoded tokens
REQUESTS = [("train-a", "train", "coding", 24, 30, 30), ("train-b", "train", "prose", 17, 26, 26),
            ("test-a", "test", "coding", 20, 24, 24), ("test-b", "test", "reasoning", 13, 22, 19)]
PLAN_KEYS = [(0, 1), (0, 4), (0, 9), (1, 0), (1, 7), (1, 12), (2, 3), (2, 5), (2, 14), (3, 2), (3, 8), (3, 11)]
COSTS = {"ram_gbps": 64.0, "pcie_gbps": 50.0, "gpu_expert_us": 20.0}


def _pair(rng, perm, p):
    return perm[rng.choice(16, 2, replace=False, p=p)]


def prefill_routes(seed: int = 4242) -> dict:
    """Per request: the prompt batches [(layer id, ids [rows][2])] and the decode ids
    [tokens][4][2]. Each request favours its own permutation of the experts (Zipf 1.2), so the
    prompt's routing predicts its decode routing better than the training prior does."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, 17) ** 1.2
    p /= p.sum()
    out = {}
    for ident, split, _, prompt, _, decoded in REQUESTS:
        perms = [rng.permutation(16) for _ in LAYERS]
        batches = []
        cuts = [0, prompt // 3, prompt]                          # two prompt batches per layer
        for b in range(2):
            for l, layer in enumerate(LAYERS):
                rows = cuts[b + 1] - cuts[b]
                if ident == "test-b" and l == 3 and b == 1:
                    rows = 2                                      # pruned: the last layer sees part of the prompt
                ids = np.array([_pair(rng, perms[l], p) for _ in range(rows)], np.int32).reshape(rows, 2)
                batches.append((layer["id"], ids))
        if ident == "train-b":
            batches.append((2, np.zeros((0, 2), np.int32)))       # a zero-row batch
        dec = np.zeros((decoded, len(LAYERS), 2), np.int32)
        for t in range(decoded):
            for l in range(len(LAYERS)):
                dec[t, l] = dec[t - 1, l] if t and rng.random() < 0.4 else _pair(rng, perms[l], p)
        out[ident] = (batches, dec)
    return out


def write_trace(trace: Path, summary: Path) -> tuple[Path, Path]:
    from vbmoe.routing_trace import TraceWriter
    routes = prefill_routes()
    with TraceWriter(trace, LAYERS, "gpt-oss", "vbmoe-synthetic", 64, model="synthetic-120b-shape",
                     collector_source_sha256=SHA) as w:
        w.enable_prefill(summary, 2048, 512, cpu_threads=16, batch_threads=16)
        for ident, split, category, prompt, max_tokens, decoded in REQUESTS:
            batches, dec = routes[ident]
            w.request_start(ident, split, category, prompt, max_tokens)
            for layer, ids in batches:
                w.prefill_route(layer, ids)
            for t in range(decoded):
                w.token(dec[t])
            w.request_end("limit" if decoded == max_tokens else "eos", True)
    return trace, summary


def write_plan(path: Path) -> Path:
    path.write_text("".join(f"{l} {e}\n" for l, e in PLAN_KEYS))
    return path


def main() -> int:
    reference = Path(sys.argv[1])
    for p in (TRACE, SUMMARY, PLAN, REPORT):
        p.unlink(missing_ok=True)
    write_trace(TRACE, SUMMARY)
    write_plan(PLAN)
    spec = importlib.util.spec_from_file_location(
        "prefill_seed", reference / "tools" / "benchmark" / "vrambridge-prefill-seed.py")
    study = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = study
    spec.loader.exec_module(study)
    routing = study.routing
    data = routing.read_trace(TRACE)
    prefill = study.read_prefill(SUMMARY, data)
    baseline = study.read_plan(PLAN, data)
    costs = routing.Costs(COSTS["ram_gbps"], COSTS["pcie_gbps"], COSTS["gpu_expert_us"], 0, 0)
    report = study.analyze(data, prefill, baseline, costs)
    report.pop("limitations")
    report["prefill_read"] = {
        ident: {"counts": sorted([l, e, c] for (l, e), c in obs["counts"].items() if c),
                "rows": sorted([l, r] for l, r in obs["rows"].items()),
                "coverage": sorted([l, c] for l, c in obs["coverage"].items())}
        for ident, obs in prefill.items()}
    REPORT.write_text(json.dumps(report, indent=1, sort_keys=True, allow_nan=False) + "\n")
    print(TRACE, SUMMARY, PLAN, REPORT)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
