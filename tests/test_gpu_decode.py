"""Fused single-token decode (vbm_decode_step) against the oracle's chained layers, on the
120B shape (hidden 2880, 128 experts, top-4, intermediate 2880) with given N(0,1) logits, in both
step schedules: two kernels per layer, and the linked step (one launch per layer boundary, the
gate_up tiles waiting on device-side flags published by the previous layer's down tiles).
Expert ids must match exactly per layer and the output bit for bit: the step uses the oracle's
arithmetic and order (the BASELINE bound of 1e-3 max relative error / cosine >= 0.99999 is
looser)."""
import ctypes as C

import numpy as np
import pytest

import helpers as H
from test_gpu_layer import Layer

pytestmark = pytest.mark.gpu


def set_mode(gpu, plan, linked):
    if linked is not None:
        gpu.call("vbm_decode_plan_set_linked", plan, 1 if linked else 0)
    got = C.c_int()
    gpu.call("vbm_decode_plan_get_linked", plan, C.byref(got))
    return bool(got.value)


def check_plan(gpu, plan):
    """Every linked wait of the plan's steps so far ended before its time limit."""
    n = C.c_int64(-1)
    gpu.call("vbm_decode_plan_check", plan, C.byref(n))
    assert n.value == 0


def run_decode(gpu, layers, x, logits, graph=False, linked=None, extra_logits=()):
    """One step on `logits` (then one step per array of `extra_logits`, same x) through a fresh
    plan; returns (out, ids, weights) of every step, or for graph=True the outputs of three
    replays of the captured first step."""
    descs = (gpu.MoeLayerDesc * len(layers))(*[l.desc() for l in layers])
    plan = C.c_void_p()
    gpu.call("vbm_decode_plan_create", descs, len(layers), C.byref(plan))
    try:
        mode = set_mode(gpu, plan.value, linked)
        if linked is not None:
            assert mode == linked
        L, E, K, Hd = len(layers), layers[0].E, layers[0].K, layers[0].H
        dx, dl = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(logits)
        out, ids, w = gpu.DeviceBuffer(4 * Hd), gpu.DeviceBuffer(4 * L * K), gpu.DeviceBuffer(4 * L * K)
        print(f"[decode] L={L} E={E} K={K} H={Hd} linked={mode} graph={graph}", flush=True)
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
            check_plan(gpu, plan.value)
            return results, ids.download(np.int32, (L, K)), w.download(np.float32, (L, K))
        steps = []
        for lg in (logits, *extra_logits):
            dl = gpu.DeviceBuffer.from_array(lg)
            gpu.call("vbm_decode_step", plan.value, dx.ptr, dl.ptr, out.ptr, ids.ptr, w.ptr, None, None)
            gpu.call("vbm_stream_synchronize", None)
            steps.append((out.download(np.float32, Hd), ids.download(np.int32, (L, K)), w.download(np.float32, (L, K))))
        check_plan(gpu, plan.value)
        return steps[0] if not extra_logits else steps
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


@pytest.mark.parametrize("linked", [True, False])
def test_decode_step_matches_oracle_120b_shape(gpu, orc, linked):
    L = 3
    layers = [Layer(gpu, H.MX, 2880, 2880, 128, 4, seed=120, layer=l, router=False) for l in range(L)]
    x = gpu.synth_normal(120, 6, 0, 2880)
    logits = gpu.synth_normal(120, 7, 0, L * 128).reshape(L, 128)
    out, ids, w = run_decode(gpu, layers, x, logits, linked=linked)
    ref, ref_ids, ref_w = oracle_chain(orc, layers, x, logits)
    assert np.array_equal(ids, ref_ids)
    assert np.allclose(w, ref_w, rtol=1e-6, atol=0)
    max_rel, cos = H.rel_err_and_cos(out, ref)
    print(f"[decode 120b-shape x{L} linked={linked}] max_rel={max_rel:.3e} cos={cos:.9f}", flush=True)
    assert H.bits_equal(out, ref), H.diff_report(out, ref)
    # graph replays give the eager bits every time (the linked step's epoch advances per replay)
    outs, gids, _ = run_decode(gpu, layers, x, logits, graph=True, linked=linked)
    assert np.array_equal(gids, ids)
    for o in outs:
        assert H.bits_equal(o, out)
    for layer in layers:
        layer.destroy()


def test_decode_schedule_selection(gpu):
    """The two-kernel step is the default; the linked step can be chosen at the 2880 shape and is
    refused (VBM_ERR_INVALID_ARGUMENT) for shapes it is not built for."""
    layer = Layer(gpu, H.MX, 2880, 2880, 128, 4, seed=121, layer=0, router=False)
    small = Layer(gpu, H.MX, 1024, 512, 16, 2, seed=122, layer=0, router=False)
    try:
        for lay, can_link in ((layer, True), (small, False)):
            descs = (gpu.MoeLayerDesc * 1)(lay.desc())
            plan = C.c_void_p()
            gpu.call("vbm_decode_plan_create", descs, 1, C.byref(plan))
            try:
                assert set_mode(gpu, plan.value, None) is False
                if can_link:
                    assert set_mode(gpu, plan.value, True) is True
                else:
                    with pytest.raises(gpu.VbmError):
                        gpu.call("vbm_decode_plan_set_linked", plan.value, 1)
                    assert set_mode(gpu, plan.value, None) is False
            finally:
                gpu.call("vbm_decode_plan_destroy", plan.value)
    finally:
        layer.destroy()
        small.destroy()


@pytest.mark.parametrize("n_layers,experts,top_k", [(1, 128, 4), (2, 32, 4), (4, 128, 1), (2, 64, 8), (3, 128, 2)])
def test_decode_linked_shapes_bitwise(gpu, orc, n_layers, experts, top_k):
    """Linked step at the 2880 shape: one layer (first and last launch only), two layers (no middle
    launch), 32 experts (config 0/1), top-1, top-2 and top-8 (arrival counts per tile other than
    four), each bit-identical to the oracle's chain and to the two-kernel step."""
    layers = [Layer(gpu, H.MX, 2880, 2880, experts, top_k, seed=300 + experts + top_k, layer=l, router=False)
              for l in range(n_layers)]
    x = gpu.synth_normal(300 + experts, 6, 0, 2880)
    logits = gpu.synth_normal(300 + experts, 7, 0, n_layers * experts).reshape(n_layers, experts)
    out, ids, _ = run_decode(gpu, layers, x, logits, linked=True)
    ref, ref_ids, _ = oracle_chain(orc, layers, x, logits)
    assert np.array_equal(ids, ref_ids)
    assert H.bits_equal(out, ref), H.diff_report(out, ref)
    out2, ids2, _ = run_decode(gpu, layers, x, logits, linked=False)
    assert np.array_equal(ids2, ids) and H.bits_equal(out2, out)
    for layer in layers:
        layer.destroy()


def test_decode_linked_consecutive_steps(gpu, orc):
    """Six steps on one plan with fresh logits each (the epoch and the arrival counters carry over
    between steps): every step equals the oracle's chain for its logits."""
    L, E = 3, 128
    layers = [Layer(gpu, H.MX, 2880, 2880, E, 4, seed=410, layer=l, router=False) for l in range(L)]
    x = gpu.synth_normal(410, 6, 0, 2880)
    all_logits = [gpu.synth_normal(410, 20 + s, 0, L * E).reshape(L, E) for s in range(6)]
    steps = run_decode(gpu, layers, x, all_logits[0], linked=True, extra_logits=all_logits[1:])
    for s, (lg, (out, ids, _)) in enumerate(zip(all_logits, steps)):
        ref, ref_ids, _ = oracle_chain(orc, layers, x, lg)
        assert np.array_equal(ids, ref_ids), f"step {s}"
        assert H.bits_equal(out, ref), f"step {s}: {H.diff_report(out, ref)}"
    for layer in layers:
        layer.destroy()


def test_decode_linked_non_resident_expert_is_loud(gpu):
    """An expert whose slot map entry is -1 poisons the output (NaN) in both schedules, as the
    two-kernel step does, and never reads outside the bank."""
    E = 32
    layer = Layer(gpu, H.MX, 2880, 2880, E, 4, seed=77, layer=0, router=False)
    logits = np.full((2, E), -1.0, dtype=np.float32)
    logits[:, 5] = 3.0                      # expert 5 is routed first in both layers
    layers = [layer, layer]
    slot_map = np.arange(E, dtype=np.int32)
    slot_map[5] = -1
    dmap = gpu.DeviceBuffer.from_array(slot_map)
    descs_list = []
    for l in layers:
        d = l.desc()
        d.expert_to_slot = dmap.ptr
        descs_list.append(d)
    descs = (gpu.MoeLayerDesc * 2)(*descs_list)
    x = gpu.synth_normal(77, 6, 0, 2880)
    for linked in (True, False):
        plan = C.c_void_p()
        gpu.call("vbm_decode_plan_create", descs, 2, C.byref(plan))
        try:
            set_mode(gpu, plan.value, linked)
            dx, dl = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(logits)
            out = gpu.DeviceBuffer(4 * 2880)
            gpu.call("vbm_decode_step", plan.value, dx.ptr, dl.ptr, out.ptr, None, None, None, None)
            gpu.call("vbm_stream_synchronize", None)
            check_plan(gpu, plan.value)
            assert np.all(np.isnan(out.download(np.float32, 2880))), f"linked={linked}"
        finally:
            gpu.call("vbm_decode_plan_destroy", plan.value)
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
