"""Fused single-token decode (vbm_decode_step) against the oracle's chained layers, on the
120B shape (hidden 2880, 128 experts, top-4, intermediate 2880) with given N(0,1) logits.
Expert ids must match exactly per layer; the final output within 1e-3 max relative error and
cosine >= 0.99999 (it is expected to be bit-identical)."""
import ctypes as C

import numpy as np
import pytest

import helpers as H
from test_gpu_layer import Layer

pytestmark = pytest.mark.gpu


def run_decode(gpu, layers, x, logits, graph=False):
    descs = (gpu.MoeLayerDesc * len(layers))(*[l.desc() for l in layers])
    plan = C.c_void_p()
    gpu.call("vbm_decode_plan_create", descs, len(layers), C.byref(plan))
    try:
        L, E, K, Hd = len(layers), layers[0].E, layers[0].K, layers[0].H
        dx, dl = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(logits)
        out, ids, w = gpu.DeviceBuffer(4 * Hd), gpu.DeviceBuffer(4 * L * K), gpu.DeviceBuffer(4 * L * K)
        if graph:
            stream = C.c_void_p()
            gpu.call("vbm_stream_create", C.byref(stream))
            g = C.c_void_p()
            gpu.call("vbm_graph_begin_capture", stream.value)
            gpu.call("vbm_decode_step", plan.value, dx.ptr, dl.ptr, out.ptr, ids.ptr, w.ptr, None, stream.value)
            gpu.call("vbm_graph_end_capture", stream.value, C.byref(g))
            results = []
            for _ in range(3):     # several replays, each checked against the eager result
                gpu.call("vbm_memset", out.ptr, 0, 4 * Hd, stream.value)
                gpu.call("vbm_graph_launch", g.value, stream.value)
                gpu.call("vbm_stream_synchronize", stream.value)
                results.append(out.download(np.float32, Hd))
            gpu.call("vbm_graph_destroy", g.value)
            gpu.call("vbm_stream_destroy", stream.value)
            return results, ids.download(np.int32, (L, K)), w.download(np.float32, (L, K))
        gpu.call("vbm_decode_step", plan.value, dx.ptr, dl.ptr, out.ptr, ids.ptr, w.ptr, None, None)
        gpu.call("vbm_stream_synchronize", None)
        return out.download(np.float32, Hd), ids.download(np.int32, (L, K)), w.download(np.float32, (L, K))
    finally:
        gpu.call("vbm_decode_plan_destroy", plan.value)


def oracle_chain(orc, layers, x, logits):
    ids, ws = [], []
    for l, layer in enumerate(layers):
        r = layer.forward_cpu(orc, x.reshape(1, -1), logits[l].reshape(1, -1))
        ids.append(r["ids"][0])
        ws.append(r["weights"][0])
        x = r["out"][0]
    return x, np.stack(ids), np.stack(ws)


def test_decode_step_matches_oracle_120b_shape(gpu, orc):
    L = 3
    layers = [Layer(gpu, H.MX, 2880, 2880, 128, 4, seed=120, layer=l, router=False) for l in range(L)]
    x = gpu.synth_normal(120, 6, 0, 2880)
    logits = gpu.synth_normal(120, 7, 0, L * 128).reshape(L, 128)
    out, ids, w = run_decode(gpu, layers, x, logits)
    ref, ref_ids, ref_w = oracle_chain(orc, layers, x, logits)
    assert np.array_equal(ids, ref_ids)
    assert np.allclose(w, ref_w, rtol=1e-6, atol=0)
    max_rel, cos = H.rel_err_and_cos(out, ref)
    same = float(np.mean(out.view(np.uint32) == ref.view(np.uint32)))
    print(f"[decode 120b-shape x{L}] max_rel={max_rel:.3e} cos={cos:.9f} bitwise_equal_fraction={same:.6f}", flush=True)
    assert max_rel <= 1e-3 and cos >= 0.99999
    # graph replays give the eager bits every time
    outs, gids, _ = run_decode(gpu, layers, x, logits, graph=True)
    assert np.array_equal(gids, ids)
    for o in outs:
        assert H.bits_equal(o, out)
    for layer in layers:
        layer.destroy()


def test_decode_step_q8_0_silu(gpu, orc):
    """Q8_0 weights, SiLU, no biases (hidden 2048, 128 experts, top-8, intermediate 768). Weight
    scales in [1e-4, 5e-4] (element std ~0.02) keep the chained hidden state finite."""
    L = 3
    layers = [Layer(gpu, H.Q8, 2048, 768, 128, 8, seed=7, layer=l, router=False, biases=False, activation=0,
                    q8_scale=(1e-4, 5e-4)) for l in range(L)]
    x = gpu.synth_normal(7, 6, 0, 2048)
    logits = gpu.synth_normal(7, 7, 0, L * 128).reshape(L, 128)
    out, ids, _ = run_decode(gpu, layers, x, logits)
    ref, ref_ids, _ = oracle_chain(orc, layers, x, logits)
    assert np.array_equal(ids, ref_ids)
    max_rel, cos = H.rel_err_and_cos(out, ref)
    assert np.all(np.isfinite(ref))
    same = float(np.mean(out.view(np.uint32) == ref.view(np.uint32)))
    print(f"[decode q8_0 silu x{L}] max_rel={max_rel:.3e} cos={cos:.9f} bitwise_equal_fraction={same:.6f}", flush=True)
    assert max_rel <= 1e-3 and cos >= 0.99999, (max_rel, cos)
    for layer in layers:
        layer.destroy()


def test_decode_randomized_shapes_bitwise(gpu, orc):
    """8 seeded random single-token decode plans (1..3 layers; both weight types and activations;
    hidden 64..1024, intermediate 64..768, 2..200 experts, top-1..8, with or without biases)
    against the oracle's layer chain: routing and output bit-identical."""
    rng = np.random.default_rng(5150)
    for case in range(8):
        type_id = H.MX if case % 2 == 0 else H.Q8
        hidden, inter = 64 * int(rng.integers(1, 17)), 64 * int(rng.integers(1, 13))
        experts = int(rng.integers(2, 201))
        top_k = int(rng.integers(1, min(8, experts) + 1))
        n_layers = int(rng.integers(1, 4))
        biases = bool(rng.random() < 0.6)
        act = gpu.ACT_SWIGLU_OAI if rng.random() < 0.5 else gpu.ACT_SILU
        label = (f"case {case}: type={type_id} H={hidden} I={inter} E={experts} top{top_k} L={n_layers} "
                 f"biases={biases} act={act}")
        print(f"[random decode] {label}", flush=True)
        layers = [Layer(gpu, type_id, hidden, inter, experts, top_k, seed=800 + case, layer=l, router=False,
                        biases=biases, activation=act) for l in range(n_layers)]
        x = gpu.synth_normal(800 + case, 6, 0, hidden)
        logits = gpu.synth_normal(800 + case, 7, 0, n_layers * experts).reshape(n_layers, experts)
        out, ids, _ = run_decode(gpu, layers, x, logits)
        ref, ref_ids, _ = oracle_chain(orc, layers, x, logits)
        assert np.array_equal(ids, ref_ids), label
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), f"{label}: {H.diff_report(out, ref)}"
        for layer in layers:
            layer.destroy()
