#!/usr/bin/env python3
"""MoE decode throughput on one MI355X: 120B-shape MXFP4 stack (hidden 2880, 128 experts, top-4,
intermediate 2880, 36 layers, ~61 GB of expert weights resident in HBM), batch 1 by default.

One step = one decode token through all 36 routed-expert layers (router top-k + softmax on the
given N(0,1) logits, Q8_0 activation quantization, grouping, gate_up GEMV + biases + SwiGLU-OAI,
Q8_0 requantization, down GEMV + bias, weighted rank-ordered combine), replayed as one HIP graph.
Inputs (weights, biases, logits, hidden state) are synthetic, seeded, and resident before timing.

Prints ONE JSON line (stdout). Progress goes to stderr.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "unified-memory-scheduler_amd"))

import vbmoe as vb  # noqa: E402

METRIC = "MoE decode tok/s (120B-shape, bs1) + expert GEMV HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
MXFP4_ROW_BYTES = 2880 // 32 * 17          # 1530 B per 2880-wide row
SEED = 20260120


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


class Stack:
    """36 seeded 120B-shape layers resident on the device."""

    def __init__(self, layers: int, experts: int, hidden: int, inter: int, top_k: int, tokens: int, seed_base: int = 0):
        self.L, self.E, self.H, self.I, self.K, self.T = layers, experts, hidden, inter, top_k, tokens
        self.gate_up, self.down, self.gu_bias, self.dn_bias, self.descs = [], [], [], [], []
        t0 = time.time()
        for l in range(layers):
            gu = vb.Bank(vb.TYPE_MXFP4, 2 * inter, hidden, experts, True)
            dn = vb.Bank(vb.TYPE_MXFP4, hidden, inter, experts, False)
            sb = seed_base + 16 * l
            gu.generate(0, experts, SEED, sb + 1, 0, -8, -3)
            dn.generate(0, experts, SEED, sb + 2, 0, -8, -3)
            gub = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, sb + 3, 0, experts * 2 * inter, 0.0, 0.02))
            dnb = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, sb + 4, 0, experts * hidden, 0.0, 0.02))
            self.gate_up.append(gu)
            self.down.append(dn)
            self.gu_bias.append(gub)
            self.dn_bias.append(dnb)
            self.descs.append(vb.MoeLayerDesc(gu.handle, dn.handle, gub.ptr, dnb.ptr, None, None, None, hidden, inter,
                                              experts, top_k, vb.ACT_SWIGLU_OAI, vb.ORDER_EXACT))
            if l % 6 == 5:
                log(f"generated layers 0..{l} ({(l + 1) * (gu.slot_bytes + dn.slot_bytes) * experts / 1e9:.1f} GB)")
        vb.call("vbm_device_synchronize")
        self.weight_bytes = layers * experts * (self.gate_up[0].slot_bytes + self.down[0].slot_bytes)
        log(f"stack resident: {self.weight_bytes / 1e9:.2f} GB in {time.time() - t0:.1f} s")
        descs = (vb.MoeLayerDesc * layers)(*self.descs)
        plan = C.c_void_p()
        vb.call("vbm_decode_plan_create", descs, layers, C.byref(plan))
        self.plan = plan.value
        self.x0 = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 6, 0, tokens * hidden))
        self.out = vb.DeviceBuffer(4 * tokens * hidden)
        self.logits_cur = vb.DeviceBuffer(4 * layers * tokens * experts)
        self.ids = vb.DeviceBuffer(4 * layers * tokens * top_k)

    def destroy(self) -> None:
        vb.call("vbm_decode_plan_destroy", self.plan)
        for b in self.gate_up + self.down:
            b.destroy()

    def step_logits_bytes(self) -> int:
        return 4 * self.L * self.T * self.E

    def enqueue_step(self, stream, events=None) -> None:
        """x0 -> 36 layers -> out through the fused decode plan (two kernels per layer), reading
        logits_cur. With `events` ([L][4] event handles) kernels A and B of every layer are
        bracketed."""
        ev = None
        if events is not None:
            flat = [e for row in events for e in row]
            ev = (C.c_void_p * len(flat))(*flat)
        vb.call("vbm_decode_step", self.plan, self.x0.ptr, self.logits_cur.ptr, self.out.ptr, self.ids.ptr, None,
                C.cast(ev, C.c_void_p) if ev is not None else None, stream)


def distinct_experts(ids: np.ndarray) -> int:
    return int(sum(len(np.unique(ids[l].reshape(-1))) for l in range(ids.shape[0])))


def host_cpu() -> dict:
    """The host's CPU model (lscpu, else /proc/cpuinfo), its logical CPU count and this process's
    CPU affinity."""
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if model is None:
        try:
            for line in Path("/proc/cpuinfo").read_text().splitlines():
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    return {"model": model, "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}


def baseline_threads() -> int:
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    return max(1, min(threads, len(os.sched_getaffinity(0))))


def cpu_baseline(args, logits_host: np.ndarray) -> dict:
    """The CPU oracle (a port of the reference's ggml x86 MXFP4 x Q8_0 path) timed on this host on
    a bounded sample: the first `--cpu-layers` layers of the same seeded stack, each with all 128
    experts on the host, for as many tokens as fit in --cpu-seconds (all threads) and
    --cpu-seconds-1core (one thread); per-token time scaled to 36 layers."""
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle_py
    oracle_py.load()
    threads = baseline_threads()
    E, H, I, K = args.experts, 2880, 2880, 4
    layers = []
    t0 = time.time()
    for l in range(args.cpu_layers):
        blocks_gu, blocks_dn = E * 2 * I * (H // 32), E * H * (I // 32)
        gu = vb.synth_mxfp4(SEED, 16 * l + 1, 0, blocks_gu)
        dn = vb.synth_mxfp4(SEED, 16 * l + 2, 0, blocks_dn)
        layers.append((gu, dn, vb.synth_normal(SEED, 16 * l + 3, 0, E * 2 * I, 0.0, 0.02),
                       vb.synth_normal(SEED, 16 * l + 4, 0, E * H, 0.0, 0.02)))
    log(f"cpu baseline: {args.cpu_layers} host layers ready in {time.time() - t0:.1f} s; timing with {threads} threads "
        f"and with 1")
    x0 = vb.synth_normal(SEED, 6, 0, H).reshape(1, H)

    def time_decode(n_threads: int, seconds: float):
        done, elapsed = 0, 0.0
        while True:
            tok = done % logits_host.shape[0]
            x = x0
            t = time.perf_counter()
            for l, (gu, dn, gub, dnb) in enumerate(layers):
                r = oracle_py.moe_layer(39, gu, dn, gub, dnb, x, H, I, E, K, activation=1,
                                        logits=logits_host[tok, l].reshape(1, E), threads=n_threads)
                x = r["out"]
            elapsed += time.perf_counter() - t
            done += 1
            if (elapsed >= seconds and done >= 2) or done >= 1_000_000:
                return done, elapsed

    def line(n_threads: int, done: int, elapsed: float) -> dict:
        per_layer_token = elapsed / (done * args.cpu_layers)
        return {"value": round(1.0 / (per_layer_token * args.layers), 3), "unit": "tok/s", "cores": n_threads,
                "kind": "port",
                "sample": f"{done} decode tokens x first {args.cpu_layers} of {args.layers} layers (all {E} experts "
                          f"on host, bs1) in {elapsed:.1f} s; per-layer time scaled x{args.layers}; oracle fast path "
                          f"(ISA level {oracle_py.load().orc_fast_isa()})"}

    result = line(threads, *time_decode(threads, args.cpu_seconds))
    result["single_core"] = line(1, *time_decode(1, args.cpu_seconds_1core))
    result["host"] = host_cpu()
    return result


def cpu_prefill_baseline(args) -> dict:
    """The CPU oracle's Q8_0 x Q8_0 layer (the reference's vec_dot path, tools/engine/native_cpu.cpp:91-104,
    as restated in the oracle) on the prefill workload's own seeded layer: the full 2048-token
    batch with all threads, and a bounded prefix of it with one thread."""
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle_py
    oracle_py.load()
    Hp, Ip, Ep, Kp, Tp = 2048, 768, 128, 8, 2048
    gu = vb.synth_q8_0(SEED, 901, 0, Ep * 2 * Ip * (Hp // 32), 1e-3, 1e-2)
    dn = vb.synth_q8_0(SEED, 902, 0, Ep * Hp * (Ip // 32), 1e-3, 1e-2)
    x = vb.synth_normal(SEED, 903, 0, Tp * Hp).reshape(Tp, Hp)
    logits = vb.synth_normal(SEED, 904, 0, Tp * Ep).reshape(Tp, Ep)
    threads = baseline_threads()

    def run(n_threads: int, tokens: int) -> float:
        t = time.perf_counter()
        oracle_py.moe_layer(8, gu, dn, None, None, x[:tokens], Hp, Ip, Ep, Kp, activation=0, logits=logits[:tokens],
                            threads=n_threads)
        return time.perf_counter() - t

    elapsed, reps = 0.0, 0
    while reps < 1 or (elapsed < args.cpu_seconds and reps < 8):
        elapsed += run(threads, Tp)
        reps += 1
    one_tokens = max(8, min(Tp, int(args.prefill_cpu_tokens_1core)))
    one = run(1, one_tokens)
    return {
        "value": round(reps * Tp / elapsed, 1), "unit": "tok/s", "cores": threads, "kind": "port",
        "sample": f"{reps} x the full {Tp}-token Q8_0 layer (hidden {Hp}, {Ep} experts top-{Kp}, intermediate {Ip}, "
                  f"SiLU) in {elapsed:.1f} s; oracle fast path (ISA level {oracle_py.load().orc_fast_isa()}), "
                  "exact x86 order",
        "single_core": {"value": round(one_tokens / one, 2), "unit": "tok/s", "cores": 1, "kind": "port",
                        "sample": f"the first {one_tokens} tokens of the same layer on one thread in {one:.1f} s"},
    }


INT8_MFMA_PEAK_TOPS = 5000.0


def prefill_measure(args) -> dict:
    """Q8_0 MoE prefill through the MFMA grouped GEMM: hidden 2048, 128 experts, top-8,
    intermediate 768, separate gate/up/down (fused gate|up bank), SiLU, no biases, 2048 tokens of
    N(0,1) activations and N(0,1) router logits; one layer forward in the fast accumulation order
    (exact integer block dots). The GEMMs are timed with events around them in eager calls; the
    layer with events around replays of the call captured as one HIP graph (and eagerly)."""
    Hp, Ip, Ep, Kp, Tp = 2048, 768, 128, 8, 2048
    gu = vb.Bank(vb.TYPE_Q8_0, 2 * Ip, Hp, Ep, True)
    dn = vb.Bank(vb.TYPE_Q8_0, Hp, Ip, Ep, False)
    gu.generate(0, Ep, SEED, 901, 0, 1e-3, 1e-2)
    dn.generate(0, Ep, SEED, 902, 0, 1e-3, 1e-2)
    desc = vb.MoeLayerDesc(gu.handle, dn.handle, None, None, None, None, None, Hp, Ip, Ep, Kp, vb.ACT_SILU,
                           vb.ORDER_FAST)
    x = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 903, 0, Tp * Hp))
    logits = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 904, 0, Tp * Ep))
    out = vb.DeviceBuffer(4 * Tp * Hp)
    ws = C.c_size_t()
    vb.call("vbm_moe_layer_workspace", C.byref(desc), Tp, C.byref(ws))
    work = vb.DeviceBuffer(ws.value)
    stream = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(stream))
    stream = stream.value
    ev = []
    for _ in range(6):
        e = C.c_void_p()
        vb.call("vbm_event_create", C.byref(e))
        ev.append(e.value)
    kern = (C.c_void_p * 4)(*ev[2:6])
    reps = args.prefill_reps
    totals = np.zeros(3)
    for i in range(2 + reps):
        vb.call("vbm_event_record", ev[0], stream)
        vb.call("vbm_moe_layer_forward_profiled", C.byref(desc), x.ptr, logits.ptr, Tp, out.ptr, None, None, work.ptr,
                ws.value, C.cast(kern, C.c_void_p), stream)
        vb.call("vbm_event_record", ev[1], stream)
        vb.call("vbm_stream_synchronize", stream)
        if i >= 2:
            t = [C.c_float() for _ in range(3)]
            vb.call("vbm_event_elapsed_ms", ev[0], ev[1], C.byref(t[0]))
            vb.call("vbm_event_elapsed_ms", ev[2], ev[3], C.byref(t[1]))
            vb.call("vbm_event_elapsed_ms", ev[4], ev[5], C.byref(t[2]))
            totals += [v.value for v in t]
    eager_ms, gu_ms, dn_ms = totals / reps
    # the same layer call captured as one HIP graph (no host launch gaps between its kernels)
    g = C.c_void_p()
    vb.call("vbm_graph_begin_capture", stream)
    vb.call("vbm_moe_layer_forward", C.byref(desc), x.ptr, logits.ptr, Tp, out.ptr, None, None, work.ptr, ws.value,
            stream)
    vb.call("vbm_graph_end_capture", stream, C.byref(g))
    for _ in range(2):
        vb.call("vbm_graph_launch", g.value, stream)
    vb.call("vbm_event_record", ev[0], stream)
    for _ in range(reps):
        vb.call("vbm_graph_launch", g.value, stream)
    vb.call("vbm_event_record", ev[1], stream)
    vb.call("vbm_stream_synchronize", stream)
    t = C.c_float()
    vb.call("vbm_event_elapsed_ms", ev[0], ev[1], C.byref(t))
    vb.call("vbm_graph_destroy", g.value)
    layer_ms = t.value / reps
    ops_gu = 2.0 * Tp * Kp * (2 * Ip) * Hp
    ops_dn = 2.0 * Tp * Kp * Hp * Ip
    gu_tops = ops_gu / (gu_ms * 1e-3) / 1e12
    dn_tops = ops_dn / (dn_ms * 1e-3) / 1e12
    weight_bytes = Ep * (gu.slot_bytes + dn.slot_bytes)
    gu.destroy()
    dn.destroy()
    log(f"prefill (Q8_0, 2048 tokens, 128 experts top-8): layer {layer_ms:.3f} ms as a graph (eager {eager_ms:.3f}) "
        f"-> {Tp / (layer_ms * 1e-3):.0f} tok/s; "
        f"gate_up GEMM {gu_ms * 1e3:.1f} us ({gu_tops:.1f} TOPS), down GEMM {dn_ms * 1e3:.1f} us ({dn_tops:.1f} TOPS)")
    return {
        "workload": "Q8_0 MoE prefill layer: 2048 tokens, hidden 2048, 128 experts, top-8, intermediate 768, SiLU",
        "value": round(Tp / (layer_ms * 1e-3), 1), "unit": "tok/s", "layer_ms": round(layer_ms, 4),
        "launch": "HIP graph of one layer call", "layer_ms_eager": round(eager_ms, 4),
        "order": "fast (exact int8 block dots, fp32 accumulation across blocks)",
        "gate_up_gemm": {"us": round(gu_ms * 1e3, 2), "int8_tops": round(gu_tops, 2),
                         "frac_of_mfma_peak": round(gu_tops / INT8_MFMA_PEAK_TOPS, 4)},
        "down_gemm": {"us": round(dn_ms * 1e3, 2), "int8_tops": round(dn_tops, 2),
                      "frac_of_mfma_peak": round(dn_tops / INT8_MFMA_PEAK_TOPS, 4)},
        "mfma_peak_tops": INT8_MFMA_PEAK_TOPS,
        "expert_weight_bytes": weight_bytes,
        "weight_stream_gbs": round(weight_bytes / ((gu_ms + dn_ms) * 1e-3) / 1e9, 1),
    }


def mxfp8_experiment(args) -> dict:
    """MXFP4 x MXFP8 on the CDNA4 block-scaled matrix cores (vbm_mul_mat_id_mxfp8) beside the
    f16 MFMA path of vbm_mul_mat_id (fast order) on the gate_up projection of the 120B-shape layer:
    hidden 2880 -> 5760 rows, 128 experts, top-4, 2048 tokens of N(0,1) activations with uniformly
    drawn distinct ids. Times each call (activation quantization + grouping + GEMM) with events and
    reports the MXFP8 result's distance from the Q8_0 result. An experiment beside the product
    path: its activations are not the reference's Q8_0."""
    Hm, Rm, Em, Km, Tm = 2880, 5760, 128, 4, 2048
    bank = vb.Bank(vb.TYPE_MXFP4, Rm, Hm, Em, True)
    bank.generate(0, Em, SEED, 905, 0, -8, -3)
    x = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 906, 0, Tm * Hm))
    rng = np.random.default_rng(SEED)
    ids = np.stack([rng.choice(Em, Km, replace=False) for _ in range(Tm)]).astype(np.int32)
    dids = vb.DeviceBuffer.from_array(ids)
    outs = {"f16": vb.DeviceBuffer(4 * Tm * Km * Rm), "mxfp8": vb.DeviceBuffer(4 * Tm * Km * Rm)}
    stream = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(stream))
    stream = stream.value
    ev = []
    for _ in range(2):
        e = C.c_void_p()
        vb.call("vbm_event_create", C.byref(e))
        ev.append(e.value)

    def run(name):
        if name == "f16":
            vb.call("vbm_mul_mat_id", bank.handle, None, None, Em, vb.TYPE_F32, x.ptr, 1, dids.ptr, Km, Tm, Km, None,
                    outs[name].ptr, vb.ORDER_FAST, stream)
        else:
            vb.call("vbm_mul_mat_id_mxfp8", bank.handle, None, Em, x.ptr, 1, dids.ptr, Km, Tm, Km, outs[name].ptr, stream)

    times = {}
    for name in ("f16", "mxfp8"):
        for _ in range(2):
            run(name)
        vb.call("vbm_event_record", ev[0], stream)
        for _ in range(args.prefill_reps):
            run(name)
        vb.call("vbm_event_record", ev[1], stream)
        vb.call("vbm_stream_synchronize", stream)
        ms = C.c_float()
        vb.call("vbm_event_elapsed_ms", ev[0], ev[1], C.byref(ms))
        times[name] = ms.value / args.prefill_reps * 1e3
    ref = outs["f16"].download(np.float32, (Tm * Km, Rm)).astype(np.float64)
    got = outs["mxfp8"].download(np.float32, (Tm * Km, Rm)).astype(np.float64)
    rel = float(np.abs(got - ref).max() / np.abs(ref).max())
    cos = float(np.dot(got.ravel(), ref.ravel()) / (np.linalg.norm(got) * np.linalg.norm(ref)))
    ops = 2.0 * Tm * Km * Rm * Hm
    wbytes = Em * bank.slot_bytes
    bank.destroy()
    vb.call("vbm_stream_destroy", stream)
    log(f"MXFP8 experiment (gate_up, 2048 tokens, 128 experts top-4): f16 MFMA path {times['f16']:.1f} us, "
        f"block-scaled MXFP8 path {times['mxfp8']:.1f} us; max deviation {rel:.2e} of max |out|, cos {cos:.6f}")
    return {
        "workload": "MXFP4 gate_up projection of the 120B-shape layer: 2048 tokens, hidden 2880 -> 5760 rows, 128 experts, top-4",
        "f16_mfma_us": round(times["f16"], 2),
        "mxfp8_block_scaled_us": round(times["mxfp8"], 2),
        "speedup": round(times["f16"] / times["mxfp8"], 3),
        "f16_tops": round(ops / (times["f16"] * 1e-6) / 1e12, 1),
        "mxfp8_tops": round(ops / (times["mxfp8"] * 1e-6) / 1e12, 1),
        "expert_weight_bytes": wbytes,
        "mxfp8_vs_q8_0_max_rel": rel, "mxfp8_vs_q8_0_cos": round(cos, 8),
        "note": "experiment beside the product path: MXFP8 activations (e4m3 + e8m0 per 32) are not the reference's Q8_0",
    }


def graph_layers(descs, T: int, x0, logits, ids, reps: int) -> float:
    """One step = the layers chained through vbm_moe_layer_forward at T tokens, captured as a HIP
    graph; returns the average step time (ms) over `reps` replays (inputs resident, events on the
    launch stream)."""
    L = len(descs)
    H = descs[0].hidden
    ws = C.c_size_t()
    vb.call("vbm_moe_layer_workspace", C.byref(descs[0]), T, C.byref(ws))
    work = vb.DeviceBuffer(ws.value)
    bufs = [vb.DeviceBuffer(4 * T * H), vb.DeviceBuffer(4 * T * H)]
    stream = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(stream))
    stream = stream.value
    E, K = descs[0].n_expert, descs[0].top_k

    def enqueue():
        x = x0.ptr
        for l, d in enumerate(descs):
            out = bufs[l & 1].ptr
            vb.call("vbm_moe_layer_forward", C.byref(d), x, logits.ptr + 4 * l * T * E, T, out,
                    ids.ptr + 4 * l * T * K, None, work.ptr, ws.value, stream)
            x = out

    g = C.c_void_p()
    vb.call("vbm_graph_begin_capture", stream)
    enqueue()
    vb.call("vbm_graph_end_capture", stream, C.byref(g))
    e0, e1 = C.c_void_p(), C.c_void_p()
    vb.call("vbm_event_create", C.byref(e0))
    vb.call("vbm_event_create", C.byref(e1))
    for _ in range(2):
        vb.call("vbm_graph_launch", g.value, stream)
    vb.call("vbm_event_record", e0.value, stream)
    for _ in range(reps):
        vb.call("vbm_graph_launch", g.value, stream)
    vb.call("vbm_event_record", e1.value, stream)
    vb.call("vbm_stream_synchronize", stream)
    t = C.c_float()
    vb.call("vbm_event_elapsed_ms", e0.value, e1.value, C.byref(t))
    vb.call("vbm_graph_destroy", g.value)
    return t.value / reps


def batch_line(descs, T: int, order: int, reps: int, seed_stream: int, slot_bytes: int) -> dict:
    """Decode of T tokens per step through the stack `descs` in accumulation order `order`:
    tok/s, step time and the expert bytes the step streams (distinct experts per layer x slot
    bytes of gate_up + down)."""
    L = len(descs)
    E, K, H = descs[0].n_expert, descs[0].top_k, descs[0].hidden
    ordered = []
    for d in descs:
        c = vb.MoeLayerDesc()
        C.pointer(c)[0] = d
        c.order = order
        ordered.append(c)
    x0 = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, seed_stream, 0, T * H))
    logits = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, seed_stream + 1, 0, L * T * E))
    ids = vb.DeviceBuffer(4 * L * T * K)
    ms = graph_layers(ordered, T, x0, logits, ids, reps)
    ids_host = ids.download(np.int32, (L, T, K))
    distinct = distinct_experts(ids_host)
    step_bytes = distinct * slot_bytes
    return {"tokens": T, "order": "exact" if order == vb.ORDER_EXACT else "fast",
            "path": "MFMA grouped GEMM" if (order == vb.ORDER_FAST and T >= 16 and T * K >= 12 * E) else "batched GEMV",
            "tok_s": round(T / (ms / 1e3), 1), "ms_per_step": round(ms, 4),
            "distinct_experts_per_layer": round(distinct / L, 2),
            "expert_bytes_per_step": int(step_bytes), "expert_gbs": round(step_bytes / (ms / 1e3) / 1e9, 1)}


def batched_measure(args, stack) -> dict:
    """Config 2 at batch 32 on the resident stack (exact GEMV order and the fast MFMA order)."""
    slot = stack.gate_up[0].slot_bytes + stack.down[0].slot_bytes
    lines = [batch_line(stack.descs, 32, order, args.batch_reps, 910, slot) for order in (vb.ORDER_EXACT, vb.ORDER_FAST)]
    for r in lines:
        log(f"config 2 batch {r['tokens']} ({r['order']}, {r['path']}): {r['tok_s']} tok/s, {r['ms_per_step']} ms/step, "
            f"{r['distinct_experts_per_layer']} experts/layer -> {r['expert_gbs']} GB/s")
    return {"workload": "120B-shape MXFP4 stack (36 layers x 128 experts, top-4), decode batch 32", "lines": lines}


def config1_measure(args) -> dict:
    """Config 1: the 32-expert / top-4 / 2880 MXFP4 layer stacked 24 deep (seeded per layer),
    decode batches 1, 8 and 64; batch 1 through the fused decode plan, 8 and 64 through the
    layer forward (batched GEMV; at 64 also the MFMA grouped GEMM)."""
    L, E, H, I, K = 24, 32, 2880, 2880, 4
    st = Stack(L, E, H, I, K, 1, seed_base=1000)
    slot = st.gate_up[0].slot_bytes + st.down[0].slot_bytes
    # batch 1: the fused decode plan
    logits = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 930, 0, L * E))
    vb.call("vbm_memcpy_d2d", st.logits_cur.ptr, logits.ptr, 4 * L * E, None)
    s = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(s))
    s = s.value
    g = C.c_void_p()
    vb.call("vbm_graph_begin_capture", s)
    st.enqueue_step(s)
    vb.call("vbm_graph_end_capture", s, C.byref(g))
    e0, e1 = C.c_void_p(), C.c_void_p()
    vb.call("vbm_event_create", C.byref(e0))
    vb.call("vbm_event_create", C.byref(e1))
    for _ in range(3):
        vb.call("vbm_graph_launch", g.value, s)
    vb.call("vbm_event_record", e0.value, s)
    for _ in range(args.batch_reps * 4):
        vb.call("vbm_graph_launch", g.value, s)
    vb.call("vbm_event_record", e1.value, s)
    vb.call("vbm_stream_synchronize", s)
    t = C.c_float()
    vb.call("vbm_event_elapsed_ms", e0.value, e1.value, C.byref(t))
    vb.call("vbm_graph_destroy", g.value)
    ms1 = t.value / (args.batch_reps * 4)
    ids1 = st.ids.download(np.int32, (L, 1, K))
    b1 = {"tokens": 1, "order": "exact", "path": "fused decode plan (2 kernels per layer)", "tok_s": round(1 / (ms1 / 1e3), 1),
          "ms_per_step": round(ms1, 4), "distinct_experts_per_layer": K,
          "expert_bytes_per_step": int(L * K * slot), "expert_gbs": round(L * K * slot / (ms1 / 1e3) / 1e9, 1)}
    lines = [b1]
    for T, order in ((8, vb.ORDER_EXACT), (64, vb.ORDER_EXACT), (64, vb.ORDER_FAST)):
        lines.append(batch_line(st.descs, T, order, args.batch_reps, 940 + T, slot))
    for r in lines:
        log(f"config 1 batch {r['tokens']} ({r['order']}, {r['path']}): {r['tok_s']} tok/s, {r['ms_per_step']} ms/step, "
            f"{r['distinct_experts_per_layer']} experts/layer -> {r['expert_gbs']} GB/s")
    st.destroy()
    return {"workload": "MXFP4 MoE stack: 24 layers x 32 experts, top-4, hidden 2880, intermediate 2880", "lines": lines}


def tier_measure(args, stack) -> dict:
    """Host-RAM tiered experts on one GPU: the same 36-layer 120B-shape stack with every expert in
    pinned host memory, an HBM pool of 16 GiB of expert groups under causal (classic) admission,
    misses staged with hipMemcpyAsync on a side stream. The pool is first seeded with the trained
    gpt-oss-120b plan of 944 expert groups (plans/gpt120-trained-hot944.txt, in file order, as the
    frozen-plan loader seeds it), unless --tier-plan none. Trace: 512 decode tokens; per layer a
    seeded permutation of the experts with Zipf(1.1) popularity, and with probability 0.6 the
    previous token's set is reused."""
    L, E, K, H, I = stack.L, stack.E, stack.K, stack.H, stack.I
    group_bytes = stack.gate_up[0].slot_bytes + stack.down[0].slot_bytes
    n_slots = (16 << 30) // group_bytes
    gub = (C.c_void_p * L)(*[b.ptr for b in stack.gu_bias])
    dnb = (C.c_void_p * L)(*[b.ptr for b in stack.dn_bias])
    desc = vb.TierDesc(vb.TYPE_MXFP4, H, I, L, E, K, vb.ACT_SWIGLU_OAI, n_slots, 64, 4, vb.ADMIT_CLASSIC,
                       C.cast(gub, C.POINTER(C.c_void_p)), C.cast(dnb, C.POINTER(C.c_void_p)))
    t0 = time.time()
    tier = C.c_void_p()
    vb.call("vbm_tier_create", C.byref(desc), C.byref(tier))
    vb.call("vbm_tier_generate", tier.value, SEED, 16, 1, 2, -8.0, -3.0, None)
    host = C.c_size_t()
    vb.call("vbm_tier_host_bytes", tier.value, C.byref(host))
    plan = []
    if args.tier_plan != "none":
        from vbmoe.routing_trace import read_plan
        plan = read_plan(args.tier_plan, L, E)
        for layer, expert in plan:
            vb.call("vbm_tier_seed", tier.value, layer, expert)
    log(f"tier: {host.value / 1e9:.1f} GB of experts in pinned host memory, {n_slots} device slots "
        f"({n_slots * group_bytes / 2**30:.1f} GiB), {len(plan)} seeded, ready in {time.time() - t0:.1f} s")
    rng = np.random.default_rng(SEED)
    tokens = args.tier_tokens
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    perms = [rng.permutation(E) for _ in range(L)]
    prev = [None] * L
    logits = np.empty((tokens, L, E), np.float32)
    routes = np.empty((tokens, L, K), np.int32)
    for t in range(tokens):
        for l in range(L):
            sel = prev[l] if prev[l] is not None and rng.random() < 0.6 else \
                [int(perms[l][i]) for i in rng.choice(E, K, replace=False, p=p)]
            prev[l] = sel
            routes[t, l] = sel
            lg = rng.standard_normal(E).astype(np.float32)
            lg[sel] = 10.0 - np.arange(K, dtype=np.float32)
            logits[t, l] = lg
    dl = vb.DeviceBuffer.from_array(logits)
    out = vb.DeviceBuffer(4 * H)
    step = 4 * L * E
    stream = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(stream))
    stream = stream.value
    ev0, ev1 = C.c_void_p(), C.c_void_p()
    vb.call("vbm_event_create", C.byref(ev0))
    vb.call("vbm_event_create", C.byref(ev1))
    wall = time.perf_counter()
    vb.call("vbm_event_record", ev0.value, stream)
    for t in range(tokens):
        vb.call("vbm_tier_step", tier.value, stack.x0.ptr, dl.ptr + t * step, out.ptr, None, stream)
    vb.call("vbm_event_record", ev1.value, stream)
    vb.call("vbm_stream_synchronize", stream)
    wall = time.perf_counter() - wall
    ms = C.c_float()
    vb.call("vbm_event_elapsed_ms", ev0.value, ev1.value, C.byref(ms))
    st = vb.TierStats()
    vb.call("vbm_tier_get_stats", tier.value, C.byref(st))
    prefill = None
    if args.tier_prefill_tokens >= 16:
        # multi-token prefill through the same pool: every layer of one batch, residency frozen
        T = args.tier_prefill_tokens
        px = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 900, 0, T * H))
        plg = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 901, 0, L * T * E))
        pout = vb.DeviceBuffer(4 * T * H)
        vb.call("vbm_tier_prefill", tier.value, 0, px.ptr, plg.ptr, T, pout.ptr, None, None, stream)  # warm-up
        vb.call("vbm_stream_synchronize", stream)
        before = vb.TierStats()
        vb.call("vbm_tier_get_stats", tier.value, C.byref(before))
        vb.call("vbm_event_record", ev0.value, stream)
        for l in range(L):
            vb.call("vbm_tier_prefill", tier.value, l, px.ptr, plg.ptr + l * T * E * 4, T, pout.ptr, None, None, stream)
        vb.call("vbm_event_record", ev1.value, stream)
        vb.call("vbm_stream_synchronize", stream)
        pms = C.c_float()
        vb.call("vbm_event_elapsed_ms", ev0.value, ev1.value, C.byref(pms))
        after = vb.TierStats()
        vb.call("vbm_tier_get_stats", tier.value, C.byref(after))
        up = after.uploaded_bytes - before.uploaded_bytes
        prefill = {
            "tokens": T, "layers": L, "ms": round(pms.value, 2), "value": round(T / (pms.value * 1e-3), 1),
            "unit": "prefill tok/s through all layers",
            "resident_experts": int(after.prefill_resident - before.prefill_resident),
            "streamed_experts": int(after.prefill_streamed - before.prefill_streamed),
            "uploaded_gb": round(up / 1e9, 2), "h2d_gbs_overall": round(up / (pms.value * 1e-3) / 1e9, 1),
        }
        log(f"tier prefill: {T} tokens x {L} layers in {pms.value:.1f} ms ({prefill['value']} tok/s); "
            f"{prefill['streamed_experts']} experts streamed, {prefill['resident_experts']} resident; "
            f"{prefill['h2d_gbs_overall']} GB/s of expert copies overall")
    policies = policy_study(args, routes, n_slots, plan, group_bytes, st) if args.tier_policies else None
    live_policy = None
    if args.tier_live_policy != "none":
        # the same trace through a second pool under another admission policy, live
        names = ("classic", "lru", "ranked", "probation", "anchored", "lfu")
        pol = names.index(args.tier_live_policy)
        tier2 = tier     # the same host copies, a fresh pool and admission
        vb.call("vbm_tier_reset", tier2.value, pol, 64, 1 if args.tier_live_policy == "lru" else 4)
        for layer, expert in plan:
            vb.call("vbm_tier_seed", tier2.value, layer, expert)
        vb.call("vbm_event_record", ev0.value, stream)
        for t in range(tokens):
            vb.call("vbm_tier_step", tier2.value, stack.x0.ptr, dl.ptr + t * step, out.ptr, None, stream)
        vb.call("vbm_event_record", ev1.value, stream)
        vb.call("vbm_stream_synchronize", stream)
        ms2 = C.c_float()
        vb.call("vbm_event_elapsed_ms", ev0.value, ev1.value, C.byref(ms2))
        st2 = vb.TierStats()
        vb.call("vbm_tier_get_stats", tier2.value, C.byref(st2))
        live_policy = {"policy": args.tier_live_policy, "value": round(tokens / (ms2.value * 1e-3), 2), "unit": "tok/s",
                       "hit_rate": round(st2.hits / (tokens * L * K), 4), "uploaded_gb": round(st2.uploaded_bytes / 1e9, 2),
                       "hits": int(st2.hits), "admissions": int(st2.admissions), "evictions": int(st2.evictions)}
        log(f"tier ({args.tier_live_policy} admission, live): {live_policy['value']} tok/s, hit rate "
            f"{live_policy['hit_rate']}, {live_policy['uploaded_gb']} GB uploaded")
    deferred = None
    if args.tier_deferred:
        # deferred mode: no host wait inside a step (misses read once from the pinned host copy by
        # the decode kernels, which keep a device copy; admission at the step boundary copies the
        # admitted experts from there); the same trace under classic and LRU
        deferred = {}
        sync_counters = {"classic": (int(st.hits), int(st.admissions), int(st.evictions))}
        if live_policy is not None and args.tier_live_policy == "lru":
            sync_counters["lru"] = (live_policy["hits"], live_policy["admissions"], live_policy["evictions"])
        for name, pol, margin in (("classic", vb.ADMIT_CLASSIC, 4), ("lru", vb.ADMIT_LRU, 1)):
            tier3 = tier
            vb.call("vbm_tier_reset", tier3.value, pol, 64, margin)
            for layer, expert in plan:
                vb.call("vbm_tier_seed", tier3.value, layer, expert)
            vb.call("vbm_tier_set_deferred", tier3.value, 1)
            wall3 = time.perf_counter()
            vb.call("vbm_event_record", ev0.value, stream)
            for t in range(tokens):
                vb.call("vbm_tier_step", tier3.value, stack.x0.ptr, dl.ptr + t * step, out.ptr, None, stream)
            vb.call("vbm_event_record", ev1.value, stream)
            vb.call("vbm_stream_synchronize", stream)
            wall3 = time.perf_counter() - wall3
            ms3 = C.c_float()
            vb.call("vbm_event_elapsed_ms", ev0.value, ev1.value, C.byref(ms3))
            vb.call("vbm_tier_flush", tier3.value)
            st3 = vb.TierStats()
            vb.call("vbm_tier_get_stats", tier3.value, C.byref(st3))
            vb.call("vbm_tier_set_deferred", tier3.value, 0)
            entry = {"value": round(tokens / (ms3.value * 1e-3), 2),
                     "unit": "tok/s", "host_wall_s": round(wall3, 2), "hit_rate": round(st3.hits / (tokens * L * K), 4),
                     "admissions": int(st3.admissions), "experts_read_from_host": int(st3.host_reads),
                     "uploaded_gb": round(st3.uploaded_bytes / 1e9, 2),
                     "host_read_gb": round(st3.host_reads * group_bytes / 1e9, 2),
                     "admission_copy_gb": round(st3.device_copy_bytes / 1e9, 2)}
            ref_counters = sync_counters.get(name)
            if ref_counters is not None:
                mine = (int(st3.hits), int(st3.admissions), int(st3.evictions))
                entry["counters_match_sync"] = ref_counters == mine
            deferred[name] = entry
            log(f"tier deferred ({name}): {entry['value']} tok/s, hit rate {entry['hit_rate']}, "
                f"{entry['host_read_gb']} GB read from host by the kernels, {entry['uploaded_gb']} GB uploaded, "
                f"{entry['admission_copy_gb']} GB of admissions copied on the device")
    vb.call("vbm_tier_destroy", tier.value)
    lookups = tokens * L * K
    h2d = st.uploaded_bytes / (st.copy_ms * 1e-3) / 1e9 if st.copy_ms > 0 else None
    res = {
        "workload": f"120B-shape MXFP4 stack, {n_slots} x {group_bytes} B HBM expert slots (16 GiB), rest in pinned "
                    f"host RAM; {tokens} decode tokens, Zipf(1.1) routing with 0.6 reuse; classic causal admission"
                    + (f"; seeded with {Path(args.tier_plan).name} ({len(plan)} expert groups)" if plan else ""),
        "value": round(tokens / (ms.value * 1e-3), 2), "unit": "tok/s", "host_wall_s": round(wall, 2),
        "hit_rate": round(st.hits / lookups, 4), "lookups": lookups, "admissions": int(st.admissions),
        "evictions": int(st.evictions), "staged_misses": int(st.staged),
        "uploaded_gb": round(st.uploaded_bytes / 1e9, 2), "h2d_gbs": round(h2d, 1) if h2d else None,
        "copy_busy_ms": round(st.copy_ms, 1), "seeded": len(plan), "prefill": prefill, "policies": policies,
        "live_policy": live_policy, "deferred": deferred,
    }
    log(f"tier: {res['value']} tok/s, hit rate {res['hit_rate']}, {res['uploaded_gb']} GB uploaded at "
        f"{res['h2d_gbs']} GB/s copy-busy")
    return res


def policy_study(args, routes, n_slots, plan, group_bytes, live) -> dict:
    """The tier's decode routing written as a routing trace (reference JSONL schema) and replayed
    offline through every causal admission policy on the same pool and seed plan: hit rate and
    expert groups copied per policy. The classic replay must reproduce the live tier's counters."""
    import tempfile
    from vbmoe import routing_trace as rt
    tokens, L, K = routes.shape
    E = args.experts
    layers = [{"id": l, "experts": E, "active": K, "bytes_per_expert": group_bytes,
               "static_host_bytes_per_expert": group_bytes, "tensor_types": ["f32", "mxfp4"]} for l in range(L)]
    with tempfile.TemporaryDirectory() as tmp:
        path = Path(tmp) / "tier_routing.jsonl"
        half = tokens // 2
        with rt.TraceWriter(path, layers, "gpt-oss", "vbmoe", tokens + 1, model="synthetic-120b-shape") as w:
            for name, split, lo, hi in (("zipf-a", "train", 0, half), ("zipf-b", "test", half, tokens)):
                w.request_start(name, split, "synthetic", 1, hi - lo)
                for t in range(lo, hi):
                    w.token(routes[t])
                w.request_end("limit")
        data = rt.read_trace(path)
    out = {"trace_events": len(data.route_layer)}
    names = ("classic", "lru", "ranked", "probation", "anchored", "lfu")
    for policy, name in enumerate(names):
        r = rt.replay_admission(data, n_slots, policy, 64, 1 if name == "lru" else 4, plan=plan)["all"]
        out[name] = {"hit_rate": round(r.hit_rate, 4), "admissions": r.admissions, "staged": r.staged,
                     "copied_groups": r.admissions + r.staged}
    c = out["classic"]
    out["classic_replay_matches_live"] = (c["admissions"], c["staged"]) == (int(live.admissions), int(live.staged)) \
        and abs(c["hit_rate"] - round(live.hits / (tokens * L * K), 4)) < 1e-9
    log("tier policies (offline replay of the tier's trace): " +
        ", ".join(f"{n} {out[n]['hit_rate']}" for n in names) + f"; classic matches live: {out['classic_replay_matches_live']}")
    return out


def read_traffic(path: Path):
    """Measured HBM bytes per gate_up launch from the committed rocprofv3 PMC summary, if any."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith("traffic_bytes_per_launch:"):
            try:
                return int(float(line.split(":", 1)[1].strip()))
            except ValueError:
                return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=1, help="decode batch (tokens per step)")
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--experts", type=int, default=128)
    ap.add_argument("--mode", choices=("graph", "eager"), default="graph")
    ap.add_argument("--decode-schedule", choices=("linked", "two-kernel"), default="two-kernel",
                    help="linked: one launch per layer boundary (down tiles of layer l-1 + gate_up tiles of "
                         "layer l, joined by device-side flags); two-kernel: kernels A and B per layer")
    ap.add_argument("--kernel-reps", type=int, default=20, help="launches per layer in the isolated kernel timing pass")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-seconds-1core", type=float, default=8.0)
    ap.add_argument("--prefill-cpu-tokens-1core", type=int, default=512,
                    help="tokens of the Q8_0 prefill layer timed on one CPU thread")
    ap.add_argument("--cpu-layers", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the Q8_0 prefill GEMM measurement")
    ap.add_argument("--no-mxfp8-experiment", dest="mxfp8_experiment", action="store_false",
                    help="skip the MXFP4 x MXFP8 block-scaled MFMA experiment beside the prefill GEMM")
    ap.add_argument("--no-batched", action="store_true",
                    help="skip the batched decode lines (config 2 at batch 32, config 1 at batches 1/8/64)")
    ap.add_argument("--batch-reps", type=int, default=5, help="graph replays per batched decode line")
    ap.add_argument("--prefill-reps", type=int, default=5)
    ap.add_argument("--no-tier", action="store_true",
                    help="skip the host-RAM tier workload (it pins 61 GB of host memory)")
    ap.add_argument("--tier-tokens", type=int, default=512)
    ap.add_argument("--no-tier-deferred", dest="tier_deferred", action="store_false",
                    help="skip the deferred-mode tier runs (classic and LRU)")
    ap.add_argument("--tier-live-policy", default="lru",
                    choices=("none", "classic", "lru", "ranked", "probation", "anchored", "lfu"),
                    help="run the tier trace a second time live under this admission policy")
    ap.add_argument("--no-tier-policies", dest="tier_policies", action="store_false",
                    help="skip the offline admission-policy replay of the tier's routing trace")
    ap.add_argument("--tier-prefill-tokens", type=int, default=2048,
                    help="prefill batch through the tier's pool after the decode trace (0: skip)")
    ap.add_argument("--tier-plan", default=str(REPO / "unified-memory-scheduler_amd" / "plans" / "gpt120-trained-hot944.txt"),
                    help="frozen plan seeding the tier's pool ('layer expert' lines), or 'none'")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="after the run, launch a plain device copy of BYTES three times (a known-traffic "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.tokens != 1:
        print("bench.py times the single-token decode path; batched decode is covered by the parity tests.",
              file=sys.stderr)
        return 2
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures the routed-expert path on exactly one GPU; --gpus {args.gpus} "
              f"(WORLD_SIZE {world}) is not supported: this build has no multi-GPU path.", file=sys.stderr)
        return 2

    vb.load()
    assert vb.device_count() >= 1, "no HIP device"
    vb.call("vbm_set_device", 0)
    log(f"device: {vb.device_name(0)}")
    H, I, E, K, L, T = 2880, 2880, args.experts, 4, args.layers, args.tokens
    stack = Stack(L, E, H, I, K, T)
    vb.call("vbm_decode_plan_set_linked", stack.plan, 1 if args.decode_schedule == "linked" else 0)
    n_steps = args.warmup + args.steps
    logits_host = vb.synth_normal(SEED, 7, 0, n_steps * L * T * E).reshape(n_steps, L, T, E)
    logits_all = vb.DeviceBuffer.from_array(logits_host)
    stream = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(stream))
    stream = stream.value
    step_bytes = stack.step_logits_bytes()

    graph = None
    if args.mode == "graph":
        g = C.c_void_p()
        vb.call("vbm_graph_begin_capture", stream)
        stack.enqueue_step(stream)
        vb.call("vbm_graph_end_capture", stream, C.byref(g))
        graph = g.value
        log("captured one decode step (36 layers) as a HIP graph")

    def run_step(i: int) -> None:
        vb.call("vbm_memcpy_d2d", stack.logits_cur.ptr, logits_all.ptr + i * step_bytes, step_bytes, stream)
        if graph is not None:
            vb.call("vbm_graph_launch", graph, stream)
        else:
            stack.enqueue_step(stream)

    for i in range(args.warmup):
        run_step(i)
    vb.call("vbm_stream_synchronize", stream)
    vb.call("vbm_device_synchronize")
    ev0, ev1 = C.c_void_p(), C.c_void_p()
    vb.call("vbm_event_create", C.byref(ev0))
    vb.call("vbm_event_create", C.byref(ev1))
    distinct = 0
    t_wall = time.perf_counter()
    vb.call("vbm_event_record", ev0.value, stream)
    for i in range(args.steps):
        run_step(args.warmup + i)
    vb.call("vbm_event_record", ev1.value, stream)
    vb.call("vbm_stream_synchronize", stream)
    vb.call("vbm_device_synchronize")
    wall = time.perf_counter() - t_wall
    ms = C.c_float()
    vb.call("vbm_event_elapsed_ms", ev0.value, ev1.value, C.byref(ms))
    ms_total = ms.value
    for i in range(args.steps):
        ids = np.stack([np.lexsort((np.arange(E), -logits_host[args.warmup + i, l, t]))[:K]
                        for l in range(L) for t in range(T)]).reshape(L, T * K)
        distinct += distinct_experts(ids)
    tok_s = args.steps * T / (ms_total / 1e3)
    ms_per_step = ms_total / args.steps
    expert_bytes = 2 * I * MXFP4_ROW_BYTES + H * MXFP4_ROW_BYTES + (2 * I + H) * 4
    step_weight_bytes = distinct / args.steps * expert_bytes
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step, {tok_s:.1f} tok/s "
        f"(host wall {wall:.3f} s); step expert bytes {step_weight_bytes / 1e9:.3f} GB -> "
        f"{step_weight_bytes / (ms_per_step / 1e3) / 1e9:.0f} GB/s")

    # Isolated kernel timing: for every layer, a HIP graph of `--kernel-reps` back-to-back launches of
    # kernel A (then of kernel B) on the state the last timed step left, timed with events on the
    # launch stream. Both kernels are idempotent, so each launch streams the same routed experts.
    def time_kernel(layer: int, which: int) -> float:
        g = C.c_void_p()
        vb.call("vbm_graph_begin_capture", stream)
        for _ in range(args.kernel_reps):
            vb.call("vbm_decode_kernel", stack.plan, layer, which, stack.x0.ptr, stack.logits_cur.ptr, stream)
        vb.call("vbm_graph_end_capture", stream, C.byref(g))
        vb.call("vbm_graph_launch", g.value, stream)            # warm
        vb.call("vbm_event_record", ev0.value, stream)
        vb.call("vbm_graph_launch", g.value, stream)
        vb.call("vbm_event_record", ev1.value, stream)
        vb.call("vbm_stream_synchronize", stream)
        vb.call("vbm_graph_destroy", g.value)
        t = C.c_float()
        vb.call("vbm_event_elapsed_ms", ev0.value, ev1.value, C.byref(t))
        return t.value / args.kernel_reps

    # Sweep timing: a HIP graph of two passes over all layers launching only kernel A (then only
    # kernel B), so every launch streams weights that no recent launch has read (36 layers of
    # either kernel exceed the 256 MB memory-side cache), as in the step; per-launch time.
    def time_sweep(which: int, passes: int = 2) -> float:
        g = C.c_void_p()
        vb.call("vbm_graph_begin_capture", stream)
        for _ in range(passes):
            for layer in range(L):
                vb.call("vbm_decode_kernel", stack.plan, layer, which, stack.x0.ptr, stack.logits_cur.ptr, stream)
        vb.call("vbm_graph_end_capture", stream, C.byref(g))
        vb.call("vbm_graph_launch", g.value, stream)            # warm
        vb.call("vbm_event_record", ev0.value, stream)
        vb.call("vbm_graph_launch", g.value, stream)
        vb.call("vbm_event_record", ev1.value, stream)
        vb.call("vbm_stream_synchronize", stream)
        vb.call("vbm_graph_destroy", g.value)
        t = C.c_float()
        vb.call("vbm_event_elapsed_ms", ev0.value, ev1.value, C.byref(t))
        return t.value / (passes * L)

    # The per-step logits copy that precedes every timed graph launch, timed alone (20 copies of the
    # last step's logits, which the buffer already holds).
    def time_step_copy(n: int = 20) -> float:
        vb.call("vbm_event_record", ev0.value, stream)
        for _ in range(n):
            vb.call("vbm_memcpy_d2d", stack.logits_cur.ptr, logits_all.ptr + (n_steps - 1) * step_bytes, step_bytes, stream)
        vb.call("vbm_event_record", ev1.value, stream)
        vb.call("vbm_stream_synchronize", stream)
        t = C.c_float()
        vb.call("vbm_event_elapsed_ms", ev0.value, ev1.value, C.byref(t))
        return t.value / n

    if args.kernel_reps > 0 and args.decode_schedule == "two-kernel":
        gu_avg_us = sum(time_kernel(l, 0) for l in range(L)) / L * 1e3
        dn_avg_us = sum(time_kernel(l, 1) for l in range(L)) / L * 1e3
        gu_sw_us, dn_sw_us = time_sweep(0) * 1e3, time_sweep(1) * 1e3
        copy_us = time_step_copy() * 1e3
    else:   # counter-collection runs (and the linked schedule, whose launches hold both kernels' work)
        gu_avg_us = dn_avg_us = gu_sw_us = dn_sw_us = float("nan")
        copy_us = 0.0
    last_ids = np.stack([np.lexsort((np.arange(E), -logits_host[n_steps - 1, l, 0]))[:K] for l in range(L)])
    # Algorithmic bytes per launch of kernel A: K experts x (5760 rows x 1530 B + 5760 fp32 biases)
    # + logits (E x 4 B) + previous layer outputs (K x 2880 x 4 B) + fp32 GLU outputs (K x 2880 x
    # 4 B). Kernel B: K experts x (2880 x 1530 B + 2880 x 4 B) + GLU outputs in (K x 2880 x 4 B)
    # + outputs (K x 2880 x 4 B).
    mean_distinct = distinct_experts(last_ids.reshape(L, K)) / L
    gu_bytes = mean_distinct * (2 * I * MXFP4_ROW_BYTES + 2 * I * 4) + E * 4 + K * H * 4 + K * I * 4
    dn_bytes = mean_distinct * (H * MXFP4_ROW_BYTES + H * 4) + K * I * 4 + K * H * 4
    gu_gbs = gu_bytes / (gu_avg_us * 1e-6) / 1e9
    dn_gbs = dn_bytes / (dn_avg_us * 1e-6) / 1e9
    # Kernel times inside the timed step. An event record between two kernels of a graph costs
    # about 4 us on this GPU (a step with one around every kernel took 1.25 instead of 0.62 ms),
    # so the step is timed whole: its time less the logits copy before each graph launch, per
    # layer, is split between kernels A and B in the ratio of their sweep launch times (cold
    # weights and back-to-back launches, as in the step). The committed rocprofv3 kernel trace of
    # this command measures the in-step kernel durations directly.
    layer_us = (ms_per_step * 1e3 - copy_us) / L
    gu_in_us = gu_sw_us * layer_us / (gu_sw_us + dn_sw_us)
    dn_in_us = dn_sw_us * layer_us / (gu_sw_us + dn_sw_us)
    gu_in_gbs = gu_bytes / (gu_in_us * 1e-6) / 1e9
    dn_in_gbs = dn_bytes / (dn_in_us * 1e-6) / 1e9
    step_gbs = step_weight_bytes / (ms_per_step / 1e3) / 1e9

    def num(v, nd):
        return round(v, nd) if np.isfinite(v) else None
    log(f"in the step: kernel A {gu_in_us:.2f} us -> {gu_in_gbs:.0f} GB/s, kernel B {dn_in_us:.2f} us -> "
        f"{dn_in_gbs:.0f} GB/s; step {step_gbs:.0f} GB/s = {step_gbs / HBM_PEAK_GBS:.3f} of peak")
    log(f"isolated repeats: kernel A (route + combine + quantize + gate_up GEMV): {gu_avg_us:.2f} us avg over {L} x "
        f"{args.kernel_reps} launches -> {gu_gbs:.0f} GB/s; kernel B (down GEMV): {dn_avg_us:.2f} us -> {dn_gbs:.0f} GB/s")
    log(f"sweeps over all layers: kernel A {gu_sw_us:.2f} us, kernel B {dn_sw_us:.2f} us per launch; "
        f"logits copy {copy_us:.2f} us per step")
    traffic = read_traffic(REPO / "profiles" / "decode_gate_up_120b_bs1_pmc.md")

    batched = None if args.no_batched else batched_measure(args, stack)
    config1 = None if args.no_batched else config1_measure(args)
    prefill = None if args.no_prefill else prefill_measure(args)
    if prefill is not None and args.mxfp8_experiment:
        prefill["mxfp8_experiment"] = mxfp8_experiment(args)
    tier = None if args.no_tier else tier_measure(args, stack)

    cpu = None
    if not args.no_cpu and T == 1:
        cpu = cpu_baseline(args, logits_host[:, :, 0, :])
        log(f"cpu baseline: {cpu['value']} tok/s on {cpu['cores']} threads, {cpu['single_core']['value']} tok/s on 1; "
            f"host {cpu['host']}")
        if prefill is not None:
            prefill["cpu_baseline"] = cpu_prefill_baseline(args)
            log(f"cpu prefill baseline: {prefill['cpu_baseline']['value']} tok/s on {prefill['cpu_baseline']['cores']} "
                f"threads, {prefill['cpu_baseline']['single_core']['value']} tok/s on 1")

    result = {
        "metric": METRIC,
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i32+f32",
        "data": "synthetic (seeded MXFP4 codes, e8m0 in [-8,-3], N(0,0.02) biases, N(0,1) logits and hidden state)",
        "config": {
            "workload": f"120B-shape MXFP4 MoE decode: {L} layers x {E} experts, top-{K}, hidden {H}, "
                        f"intermediate {I}, batch {T}, weights resident in HBM",
            "layers": L, "experts": E, "top_k": K, "hidden": H, "intermediate": I, "batch": T,
            "resident_weight_bytes": stack.weight_bytes, "launch": args.mode,
            "kernels_per_layer": 2 if args.decode_schedule == "two-kernel" else None,
            "schedule": args.decode_schedule,
            "expert_bytes_per_step": round(step_weight_bytes),
            "step_expert_gbs": round(step_weight_bytes / (ms_per_step / 1e3) / 1e9, 1),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_gate_up_kernel<MXFP4> (routing + combine + Q8_0 + gate_up GEMV + bias + SwiGLU-OAI)",
            "achieved": num(gu_in_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": num(gu_in_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/decode_gate_up_120b_bs1_pmc.md (rocprofv3 FETCH_SIZE + WRITE_SIZE)",
            "bytes_per_launch": round(gu_bytes),
            "avg_launch_us": num(gu_in_us, 3),
            "timing": "kernel A's share of the timed step: (ms_per_step - the per-step logits copy) / layers split "
                      "between kernels A and B in the ratio of their launch times in sweeps over all layers (events "
                      "around graphs of back-to-back launches of one kernel, cold weights)",
            "sweep": {"gate_up_us": num(gu_sw_us, 3), "down_us": num(dn_sw_us, 3), "step_copy_us": num(copy_us, 3)},
            "step_frac": num(step_gbs / HBM_PEAK_GBS, 4),
            "step_achieved": num(step_gbs, 1),
            "down_kernel": {"achieved": num(dn_in_gbs, 1), "avg_launch_us": num(dn_in_us, 3),
                            "bytes_per_launch": round(dn_bytes)},
            "isolated": {"timing": f"graphs of {args.kernel_reps} back-to-back launches of one layer's kernel",
                         "gate_up_us": num(gu_avg_us, 3), "gate_up_frac": num(gu_gbs / HBM_PEAK_GBS, 4),
                         "down_us": num(dn_avg_us, 3), "down_frac": num(dn_gbs / HBM_PEAK_GBS, 4)},
        },
        "cpu_baseline": cpu,
        "batched": batched,
        "config1": config1,
        "prefill": prefill,
        "tier": tier,
    }
    print(json.dumps(result), flush=True)
    if args.copy_probe > 0:
        n = args.copy_probe // 16 * 16
        src, dst = vb.DeviceBuffer(n), vb.DeviceBuffer(n)
        for _ in range(3):
            vb.call("vbm_copy_kernel", dst.ptr, src.ptr, n, stream)
        vb.call("vbm_stream_synchronize", stream)
        log(f"copy probe: 3 x {n} B")
    if graph is not None:
        vb.call("vbm_graph_destroy", graph)
    return 0


if __name__ == "__main__":
    sys.exit(main())
