"""Host-RAM expert tier (vbm_tier_*) on the GPU: every token's output must be bit-identical to the
fully resident decode plan holding the same experts and to the oracle's layer chain, routing
identical, and the tier's admission counters equal to the Python restatement fed with the same
routes; tier prefill must be bit-identical to the resident fused layer and within the fast order's
tolerance of the oracle."""
import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import admission as ref  # noqa: E402

pytestmark = pytest.mark.gpu

SEED = 515


def routed_logits(rng, L, E, K, tokens):
    """Logits whose top-K per layer follows a Zipf-like trace with reuse (as in the tier config)."""
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    perms = [rng.permutation(E) for _ in range(L)]
    prev = [None] * L
    out = np.empty((tokens, L, E), np.float32)
    chosen = []
    for t in range(tokens):
        row = []
        for l in range(L):
            sel = prev[l] if prev[l] is not None and rng.random() < 0.6 else \
                [int(perms[l][i]) for i in rng.choice(E, K, replace=False, p=p)]
            prev[l] = sel
            lg = rng.standard_normal(E).astype(np.float32)
            for r, e in enumerate(sel):
                lg[e] = 10.0 - r
            out[t, l] = lg
            row.append(sel)
        chosen.append(row)
    return out, chosen


def host_layer(vb, type_id, l, E, H, I, p0, p1):
    """ggml bytes and biases of layer l, regenerated on the host: the bytes vbm_bank_generate and
    vbm_tier_generate (layer stride 16, gate_up stream 1, down stream 2) put on the device."""
    n_gu, n_dn = E * 2 * I * (H // 32), E * H * (I // 32)
    if type_id == 39:
        gu, dn = vb.synth_mxfp4(SEED, 16 * l + 1, 0, n_gu, p0, p1), vb.synth_mxfp4(SEED, 16 * l + 2, 0, n_dn, p0, p1)
    else:
        gu, dn = vb.synth_q8_0(SEED, 16 * l + 1, 0, n_gu, p0, p1), vb.synth_q8_0(SEED, 16 * l + 2, 0, n_dn, p0, p1)
    return (gu, dn, vb.synth_normal(SEED, 16 * l + 3, 0, E * 2 * I, 0.0, 0.02),
            vb.synth_normal(SEED, 16 * l + 4, 0, E * H, 0.0, 0.02))


def oracle_chain(orc, host, type_id, act, x, logits_t, H, I, E, K):
    """The oracle's single-token chain through every layer (ggml x86 CPU path, exact order)."""
    for l, (gu, dn, gb, db) in enumerate(host):
        x = orc.moe_layer(type_id, gu, dn, gb, db, x.reshape(1, H), H, I, E, K, activation=act,
                          logits=logits_t[l].reshape(1, E))["out"][0]
    return x


@pytest.mark.parametrize("type_id,policy,margin,mode", [
    (39, 0, 4, "sync"), (39, 1, 1, "sync"), (8, 2, 2, "sync"),
    (39, 0, 4, "deferred"), (39, 1, 1, "deferred"), (8, 2, 2, "graph"), (39, 1, 1, "graph"),
    (39, 0, 4, "graph_nosync"), (39, 1, 1, "graph_nosync"),
])
def test_tier_matches_resident_plan(gpu, orc, type_id, policy, margin, mode):
    """Synchronous mode (per-layer admission and staging), deferred mode (no host wait inside a
    step: misses read from the pinned host copy into the device staging area, admission at the step
    boundary, admitted experts copied into their slots from their staged copies) and deferred mode
    with the step's device part captured once as a HIP graph and replayed per token: every token
    bit-identical to the resident plan and to the oracle chain, counters equal to the Python
    admission fed the same routes. graph_nosync replays token after token with no host
    synchronization between them (each begin's own wait on the previous replay's hand-off is
    what orders the admissions), copying every token's logits in and outputs out on the stream."""
    vb = gpu
    L, E, K, H, I, slots = 3, 16, 4, 256, 256, 4 + 9
    act = vb.ACT_SWIGLU_OAI if type_id == 39 else vb.ACT_SILU
    p0, p1 = (-8, -3) if type_id == 39 else (1e-4, 5e-4)
    biases = []
    for l in range(L):
        gb = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 16 * l + 3, 0, E * 2 * I, 0.0, 0.02))
        db = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 16 * l + 4, 0, E * H, 0.0, 0.02))
        biases.append((gb, db))
    # resident reference: per-layer banks holding every expert
    banks, descs = [], []
    for l in range(L):
        gu = vb.Bank(type_id, 2 * I, H, E, True)
        dn = vb.Bank(type_id, H, I, E, False)
        gu.generate(0, E, SEED, 16 * l + 1, 0, p0, p1)
        dn.generate(0, E, SEED, 16 * l + 2, 0, p0, p1)
        banks.append((gu, dn))
        descs.append(vb.MoeLayerDesc(gu.handle, dn.handle, biases[l][0].ptr, biases[l][1].ptr, None, None, None, H, I,
                                     E, K, act, vb.ORDER_EXACT))
    plan = C.c_void_p()
    vb.call("vbm_decode_plan_create", (vb.MoeLayerDesc * L)(*descs), L, C.byref(plan))
    # tier over the same experts
    gub = (C.c_void_p * L)(*[b[0].ptr for b in biases])
    dnb = (C.c_void_p * L)(*[b[1].ptr for b in biases])
    desc = vb.TierDesc(type_id, H, I, L, E, K, act, slots, 8, margin, policy,
                       C.cast(gub, C.POINTER(C.c_void_p)), C.cast(dnb, C.POINTER(C.c_void_p)))
    tier = C.c_void_p()
    vb.call("vbm_tier_create", C.byref(desc), C.byref(tier))
    vb.call("vbm_tier_generate", tier.value, SEED, 16, 1, 2, p0, p1, None)
    py = ref.Admission(L, E, K, slots, 8, margin, policy)
    for l, e in ((0, 3), (2, 5)):
        vb.call("vbm_tier_seed", tier.value, l, e)
        py.seed(l, e)
    host = [host_layer(vb, type_id, l, E, H, I, p0, p1) for l in range(L)]
    rng = np.random.default_rng(type_id + policy)
    tokens = 30
    logits, chosen = routed_logits(rng, L, E, K, tokens)
    x_host = vb.synth_normal(SEED, 6, 0, H)
    x = vb.DeviceBuffer.from_array(x_host)
    dl = vb.DeviceBuffer(logits[0].nbytes)
    o1, o2 = vb.DeviceBuffer(4 * H), vb.DeviceBuffer(4 * H)
    i1, i2 = vb.DeviceBuffer(4 * L * K), vb.DeviceBuffer(4 * L * K)
    staged = 0
    stream, graph = None, None
    if mode != "sync":
        vb.call("vbm_tier_set_deferred", tier.value, 1)
    if mode in ("graph", "graph_nosync"):
        st_ = C.c_void_p()
        vb.call("vbm_stream_create", C.byref(st_))
        stream = st_.value
        g = C.c_void_p()
        vb.call("vbm_graph_begin_capture", stream)
        vb.call("vbm_tier_step_enqueue", tier.value, x.ptr, dl.ptr, o2.ptr, i2.ptr, stream)
        vb.call("vbm_graph_end_capture", stream, C.byref(g))
        graph = g.value
    if mode == "graph_nosync":
        tok_bytes, ids_bytes = logits[0].nbytes, 4 * L * K
        dl_all = vb.DeviceBuffer.from_array(np.ascontiguousarray(logits))
        out_all, ids_all = vb.DeviceBuffer(4 * H * tokens), vb.DeviceBuffer(ids_bytes * tokens)
        for t in range(tokens):
            vb.call("vbm_tier_step_begin", tier.value)
            vb.call("vbm_memcpy_d2d", dl.ptr, dl_all.ptr + t * tok_bytes, tok_bytes, stream)
            vb.call("vbm_graph_launch", graph, stream)
            vb.call("vbm_memcpy_d2d", out_all.ptr + t * 4 * H, o2.ptr, 4 * H, stream)
            vb.call("vbm_memcpy_d2d", ids_all.ptr + t * ids_bytes, i2.ptr, ids_bytes, stream)
        vb.call("vbm_stream_synchronize", stream)
        tier_out = out_all.download(np.float32, (tokens, H))
        tier_ids = ids_all.download(np.int32, (tokens, L, K))
    for t in range(tokens):
        dl.upload(logits[t])
        vb.call("vbm_decode_step", plan.value, x.ptr, dl.ptr, o1.ptr, i1.ptr, None, None, None)
        if mode == "graph_nosync":
            vb.call("vbm_stream_synchronize", None)
            o2.upload(tier_out[t])
            i2.upload(tier_ids[t])
        elif mode == "graph":
            vb.call("vbm_tier_step_begin", tier.value)
            vb.call("vbm_graph_launch", graph, stream)
            vb.call("vbm_stream_synchronize", stream)
        else:
            vb.call("vbm_tier_step", tier.value, x.ptr, dl.ptr, o2.ptr, i2.ptr, None)
        vb.call("vbm_stream_synchronize", None)
        a, b = o1.download(np.float32, H), o2.download(np.float32, H)
        ia, ib = i1.download(np.int32, (L, K)), i2.download(np.int32, (L, K))
        assert np.array_equal(ia, ib) and ia.tolist() == chosen[t], t
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), t
        want = oracle_chain(orc, host, type_id, act, x_host, logits[t], H, I, E, K)
        assert np.array_equal(want.view(np.uint32), b.view(np.uint32)), f"token {t} differs from the oracle"
        for l in range(L):
            hits, made = py.admit(l, chosen[t][l])
            admitted = {e for _, e, _ in made}
            staged += sum(1 for r, e in enumerate(chosen[t][l]) if not hits[r] and e not in admitted)
    if mode != "sync":
        vb.call("vbm_tier_flush", tier.value)            # the last step's admissions
    st = vb.TierStats()
    vb.call("vbm_tier_get_stats", tier.value, C.byref(st))
    print(f"[tier type={type_id} policy={policy} mode={mode}] hits={st.hits}/{tokens * L * K} admissions={st.admissions} "
          f"evictions={st.evictions} staged={st.staged} uploaded={st.uploaded_bytes}", flush=True)
    assert (st.dispatches, st.hits, st.admissions, st.evictions) == (tokens * L, py.hits, py.admissions, py.evictions)
    assert st.staged == staged and st.admissions > 0
    assert st.staged > 0 or policy == ref.LRU          # lru with margin 1 admits every miss
    group_bytes = (2 * I * (H // 32) + H * (I // 32)) * (17 if type_id == 39 else 34)
    if mode == "sync":
        assert st.host_reads == 0 and st.device_copy_bytes == 0
    else:
        # every pick read from the host copy was a miss (admissions are visible from the next step
        # on; a miss can also be a pick that sat in a slot during the step and was evicted by an
        # earlier rank's admission of its layer); every admission copied into its slot on the
        # device; the only host uploads are the two seeds
        assert 0 < st.host_reads <= tokens * L * K - st.hits
        assert st.admissions * group_bytes <= st.device_copy_bytes <= 2 * st.admissions * group_bytes
        assert st.uploaded_bytes == 2 * group_bytes
    if graph is not None:
        vb.call("vbm_graph_destroy", graph)
        vb.call("vbm_stream_destroy", stream)
    vb.call("vbm_tier_destroy", tier.value)
    vb.call("vbm_decode_plan_destroy", plan.value)
    for gu, dn in banks:
        gu.destroy()
        dn.destroy()


def test_tier_routing_trace_replays_to_the_same_decisions(gpu, tmp_path):
    """A routing trace recorded by the tier (vbm_tier_set_trace) holds exactly the routed experts,
    the tier's outputs are bit-identical with and without it attached, and replaying the trace
    through the admission alone reproduces the tier's counters."""
    from vbmoe import routing_trace as rt
    vb = gpu
    L, E, K, H, I, slots, policy, margin = 3, 16, 4, 256, 256, 4 + 9, vb.ADMIT_LFU, 4
    biases = [(vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 16 * l + 3, 0, E * 2 * I, 0.0, 0.02)),
               vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 16 * l + 4, 0, E * H, 0.0, 0.02))) for l in range(L)]
    gub = (C.c_void_p * L)(*[b[0].ptr for b in biases])
    dnb = (C.c_void_p * L)(*[b[1].ptr for b in biases])
    desc = vb.TierDesc(39, H, I, L, E, K, vb.ACT_SWIGLU_OAI, slots, 8, margin, policy,
                       C.cast(gub, C.POINTER(C.c_void_p)), C.cast(dnb, C.POINTER(C.c_void_p)))
    tiers = []
    for _ in range(2):
        tier = C.c_void_p()
        vb.call("vbm_tier_create", C.byref(desc), C.byref(tier))
        vb.call("vbm_tier_generate", tier.value, SEED, 16, 1, 2, -8.0, -3.0, None)
        for l, e in ((0, 3), (2, 5)):
            vb.call("vbm_tier_seed", tier.value, l, e)
        tiers.append(tier.value)
    ids = [3, 7, 11]
    expert_bytes = 2 * I * (H // 32) * 17 + H * (I // 32) * 17 + 4 * (2 * I + H)   # MXFP4 weights + fp32 biases
    layers = [{"id": i, "experts": E, "active": K, "bytes_per_expert": expert_bytes,
               "static_host_bytes_per_expert": expert_bytes, "tensor_types": ["f32", "mxfp4"]} for i in ids]
    path = tmp_path / "tier.jsonl"
    writer = rt.TraceWriter(path, layers, "gpt-oss", "vbmoe-test", 64, model="synthetic",
                            token_equivalence_check="tier outputs with and without the trace attached")
    rng = np.random.default_rng(77)
    x = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 6, 0, H))
    dl = vb.DeviceBuffer(4 * L * E)
    outs = [vb.DeviceBuffer(4 * H), vb.DeviceBuffer(4 * H)]
    vb.call("vbm_tier_set_trace", tiers[0], writer.handle)
    with pytest.raises(vb.VbmError, match="no open request"):
        vb.call("vbm_tier_step", tiers[0], x.ptr, dl.ptr, outs[0].ptr, None, None)   # rejected before any work
    routed = []
    for name, split, tokens in (("warm", "train", 14), ("held-out", "test", 9)):
        logits, chosen = routed_logits(rng, L, E, K, tokens)
        routed += chosen
        writer.request_start(name, split, "coding", 3, tokens)
        for t in range(tokens):
            dl.upload(logits[t])
            for tier, o in zip(tiers, outs):
                vb.call("vbm_tier_step", tier, x.ptr, dl.ptr, o.ptr, None, None)
            vb.call("vbm_stream_synchronize", None)
            a, b = (o.download(np.float32, H) for o in outs)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (name, t)
        writer.request_end("limit", True)
    vb.call("vbm_tier_set_trace", tiers[0], None)
    writer.close()
    data = rt.read_trace(path)
    assert [list(e) for e in data.route_experts] == [sel for row in routed for sel in row]
    assert data.route_layer.tolist() == ids * len(routed)
    stats = rt.replay_admission(data, slots, policy, recent_window=8, margin=margin, plan=[(0, 3), (2, 5)])
    for tier in tiers:
        st = vb.TierStats()
        vb.call("vbm_tier_get_stats", tier, C.byref(st))
        a = stats["all"]
        assert (st.dispatches, st.hits, st.admissions, st.evictions, st.staged) == \
            (a.dispatches, a.hits, a.admissions, a.evictions, a.staged)
        vb.call("vbm_tier_destroy", tier)
    print(f"[tier trace] {len(data.route_layer)} routes, hit rate {stats['all'].hit_rate:.3f} "
          f"(train {stats['train'].hit_rate:.3f}, test {stats['test'].hit_rate:.3f})", flush=True)


@pytest.mark.parametrize("type_id", [39, 8])
def test_tier_prefill_matches_resident_layer(gpu, orc, type_id):
    """Multi-token prefill through the tier (resident experts in one pass, the others streamed
    through the reserved slots in chunks) is bit-identical to the fused layer forward over banks
    holding every expert (both in the fast accumulation order), before and after decode steps
    have changed the pool."""
    vb = gpu
    L, E, K, H, I, slots, T = 2, 16, 4, 256, 256, 4 + 6, 48
    act = vb.ACT_SWIGLU_OAI if type_id == 39 else vb.ACT_SILU
    p0, p1 = (-8, -3) if type_id == 39 else (1e-4, 5e-4)
    biases = [(vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 16 * l + 3, 0, E * 2 * I, 0.0, 0.02)),
               vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 16 * l + 4, 0, E * H, 0.0, 0.02))) for l in range(L)]
    banks, descs = [], []
    for l in range(L):
        gu, dn = vb.Bank(type_id, 2 * I, H, E, True), vb.Bank(type_id, H, I, E, False)
        gu.generate(0, E, SEED, 16 * l + 1, 0, p0, p1)
        dn.generate(0, E, SEED, 16 * l + 2, 0, p0, p1)
        banks.append((gu, dn))
        descs.append(vb.MoeLayerDesc(gu.handle, dn.handle, biases[l][0].ptr, biases[l][1].ptr, None, None, None,
                                     H, I, E, K, act, vb.ORDER_FAST))
    gub = (C.c_void_p * L)(*[b[0].ptr for b in biases])
    dnb = (C.c_void_p * L)(*[b[1].ptr for b in biases])
    desc = vb.TierDesc(type_id, H, I, L, E, K, act, slots, 8, 2, vb.ADMIT_CLASSIC,
                       C.cast(gub, C.POINTER(C.c_void_p)), C.cast(dnb, C.POINTER(C.c_void_p)))
    tier = C.c_void_p()
    vb.call("vbm_tier_create", C.byref(desc), C.byref(tier))
    vb.call("vbm_tier_generate", tier.value, SEED, 16, 1, 2, p0, p1, None)
    for l, e in ((0, 3), (0, 5), (0, 7), (1, 2)):
        vb.call("vbm_tier_seed", tier.value, l, e)
    host = [host_layer(vb, type_id, l, E, H, I, p0, p1) for l in range(L)]
    rng = np.random.default_rng(type_id)
    out1, out2 = vb.DeviceBuffer(4 * T * H), vb.DeviceBuffer(4 * T * H)
    i1, i2 = vb.DeviceBuffer(4 * T * K), vb.DeviceBuffer(4 * T * K)
    w1, w2 = vb.DeviceBuffer(4 * T * K), vb.DeviceBuffer(4 * T * K)

    def compare(tag):
        for l in range(L):
            x_host = rng.standard_normal((T, H)).astype(np.float32)
            lg_host = rng.standard_normal((T, E)).astype(np.float32)
            x = vb.DeviceBuffer.from_array(x_host)
            lg = vb.DeviceBuffer.from_array(lg_host)
            ws = C.c_size_t()
            vb.call("vbm_moe_layer_workspace", C.byref(descs[l]), T, C.byref(ws))
            work = vb.DeviceBuffer(ws.value)
            vb.call("vbm_moe_layer_forward", C.byref(descs[l]), x.ptr, lg.ptr, T, out1.ptr, i1.ptr, w1.ptr, work.ptr,
                    ws.value, None)
            vb.call("vbm_tier_prefill", tier.value, l, x.ptr, lg.ptr, T, out2.ptr, i2.ptr, w2.ptr, None)
            vb.call("vbm_stream_synchronize", None)
            assert np.array_equal(i1.download(np.int32, (T, K)), i2.download(np.int32, (T, K))), (tag, l)
            assert np.array_equal(w1.download(np.uint32, (T, K)), w2.download(np.uint32, (T, K))), (tag, l)
            a, b = out1.download(np.uint32, (T, H)), out2.download(np.uint32, (T, H))
            assert np.array_equal(a, b), (tag, l, int(np.count_nonzero(a != b)))
            gu, dn, gb, db = host[l]
            want = orc.moe_layer(type_id, gu, dn, gb, db, x_host, H, I, E, K, activation=act, logits=lg_host,
                                 threads=8)
            assert np.array_equal(want["ids"], i2.download(np.int32, (T, K))), (tag, l)
            got = b.view(np.float32)
            g, r = got.astype(np.float64).ravel(), want["out"].astype(np.float64).ravel()
            max_rel = float(np.abs(g - r).max() / np.abs(r).max())
            cos = float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r)))
            assert max_rel <= 1e-3 and cos >= 0.99999, (tag, l, max_rel, cos)

    compare("seeded")
    # decode steps admit experts into the pool and stage misses in the reserved slots
    logits, _ = routed_logits(np.random.default_rng(4), L, E, K, 8)
    x1 = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 6, 0, H))
    dl, o = vb.DeviceBuffer(logits[0].nbytes), vb.DeviceBuffer(4 * H)
    for t in range(8):
        dl.upload(logits[t])
        vb.call("vbm_tier_step", tier.value, x1.ptr, dl.ptr, o.ptr, None, None)
    compare("after decode")
    with pytest.raises(vb.VbmError, match="16"):
        vb.call("vbm_tier_prefill", tier.value, 0, x1.ptr, dl.ptr, 8, out2.ptr, None, None, None)
    st = vb.TierStats()
    vb.call("vbm_tier_get_stats", tier.value, C.byref(st))
    print(f"[tier prefill type={type_id}] tokens={st.prefill_tokens} resident={st.prefill_resident} "
          f"streamed={st.prefill_streamed} admissions={st.admissions}", flush=True)
    assert st.prefill_tokens == 4 * T and st.prefill_resident > 0 and st.prefill_streamed > 0
    vb.call("vbm_tier_destroy", tier.value)
    for gu, dn in banks:
        gu.destroy()
        dn.destroy()


def test_tier_prefill_records_the_prefill_summary(gpu, tmp_path):
    """With a trace that writes the prefill summary attached, each vbm_tier_prefill records its
    routed ids as one prompt batch (rows per expert), and the following decode steps record routes
    as before; the summary's histograms equal the counts of the ids the prefill returned."""
    from vbmoe import routing_trace as rt
    vb = gpu
    L, E, K, H, I, slots, T = 2, 16, 4, 256, 256, 4 + 6, 40
    desc = vb.TierDesc(39, H, I, L, E, K, vb.ACT_SWIGLU_OAI, slots, 8, 2, vb.ADMIT_CLASSIC, None, None)
    tier = C.c_void_p()
    vb.call("vbm_tier_create", C.byref(desc), C.byref(tier))
    vb.call("vbm_tier_generate", tier.value, SEED, 16, 1, 2, -8.0, -3.0, None)
    layers = [{"id": i, "experts": E, "active": K, "bytes_per_expert": 1000, "static_host_bytes_per_expert": 1000}
              for i in (4, 9)]
    path, summary = tmp_path / "p.jsonl", tmp_path / "p.json"
    writer = rt.TraceWriter(path, layers, "gpt-oss", "vbmoe-test", 128, collector_source_sha256="ab" * 32)
    writer.enable_prefill(summary, T, T)
    vb.call("vbm_tier_set_trace", tier.value, writer.handle)
    rng = np.random.default_rng(9)
    out, ids = vb.DeviceBuffer(4 * T * H), vb.DeviceBuffer(4 * T * K)
    expected = []
    writer.request_start("r0", "test", "chat", T, 3)
    for l in range(L):
        x = vb.DeviceBuffer.from_array(rng.standard_normal((T, H)).astype(np.float32))
        lg = vb.DeviceBuffer.from_array(rng.standard_normal((T, E)).astype(np.float32))
        vb.call("vbm_tier_prefill", tier.value, l, x.ptr, lg.ptr, T, out.ptr, ids.ptr, None, None)
        vb.call("vbm_stream_synchronize", None)
        expected.append(np.bincount(ids.download(np.int32, (T, K)).ravel(), minlength=E).tolist())
    logits, chosen = routed_logits(rng, L, E, K, 3)
    x1 = vb.DeviceBuffer.from_array(vb.synth_normal(SEED, 6, 0, H))
    dl, o = vb.DeviceBuffer(logits[0].nbytes), vb.DeviceBuffer(4 * H)
    for t in range(3):
        dl.upload(logits[t])
        vb.call("vbm_tier_step", tier.value, x1.ptr, dl.ptr, o.ptr, None, None)
    vb.call("vbm_stream_synchronize", None)
    writer.request_end("limit", True)
    vb.call("vbm_tier_set_trace", tier.value, None)
    writer.close()
    vb.call("vbm_tier_destroy", tier.value)
    doc = json.loads(summary.read_text())
    req = doc["requests"][0]
    assert [(b["layer"], b["rows"]) for b in req["batches"]] == [(4, T), (9, T)]
    assert [b["expert_row_counts"] for b in req["batches"]] == expected
    assert all(c["covers_all_prompt_rows"] for c in req["coverage"])
    routes = [r for r in map(json.loads, path.read_text().splitlines()) if r["type"] == "route"]
    assert [r["experts"] for r in routes] == [sel for row in chosen for sel in row]
