"""Config 4 at its own size: the 120B-shape stack (36 layers x 128 MXFP4 experts, hidden and
intermediate 2880, top-4, SwiGLU-OAI, biases) with every expert in pinned host memory and a 16 GiB
device pool (1299 expert groups) under the reference's default (classic) causal admission, seeded
with the trained gpt-oss-120b plan of 944 expert groups, decoding a 64-token Zipf(1.1) trace that
reuses the previous token's experts with probability 0.6.

Checked for every token: the routed ids equal the oracle router's, the tier's output is
bit-identical to the fully resident decode plan over the same experts, and after the trace the
tier's dispatch / hit / admission / eviction / staging counters equal the plain-Python admission
restatement (oracle/admission.py) fed the same routes. Three tokens also go through the oracle's
36-layer chain (the ggml x86 CPU path), which must match bit for bit."""
import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import admission as ref  # noqa: E402

pytestmark = pytest.mark.gpu

SEED = 4242
L, E, K, HID, INTER = 36, 128, 4, 2880, 2880
PLAN = Path(__file__).resolve().parents[1] / "unified-memory-scheduler_amd" / "plans" / "gpt120-trained-hot944.txt"


def zipf_trace(rng, tokens):
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    perms = [rng.permutation(E) for _ in range(L)]
    prev = [None] * L
    logits = np.empty((tokens, L, E), np.float32)
    routes = []
    for t in range(tokens):
        row = []
        for l in range(L):
            sel = prev[l] if prev[l] is not None and rng.random() < 0.6 else \
                [int(perms[l][i]) for i in rng.choice(E, K, replace=False, p=p)]
            prev[l] = sel
            lg = rng.standard_normal(E).astype(np.float32)
            lg[sel] = 10.0 - np.arange(K, dtype=np.float32)
            logits[t, l] = lg
            row.append(sel)
        routes.append(row)
    return logits, routes


class HostExperts:
    """ggml bytes of single experts regenerated on the host from the counter-based generator (the
    same bytes vbm_bank_generate and vbm_tier_generate put on the device), cached by key."""

    def __init__(self, vb):
        self.vb, self.cache = vb, {}
        self.gu_blocks, self.dn_blocks = 2 * INTER * (HID // 32), HID * (INTER // 32)

    def get(self, layer, expert):
        key = (layer, expert)
        if key not in self.cache:
            gu = self.vb.synth_mxfp4(SEED, 16 * layer + 1, expert * self.gu_blocks, self.gu_blocks)
            dn = self.vb.synth_mxfp4(SEED, 16 * layer + 2, expert * self.dn_blocks, self.dn_blocks)
            self.cache[key] = (gu, dn)
        return self.cache[key]


def oracle_token(orc, experts, biases, x, logits_t, ids_t):
    """The oracle's decode chain for one token over the 36 layers. Routing is the oracle router on
    the full logits (checked against ids_t); the expert math uses compact arrays of the K routed
    experts, whose own top-k over their logits picks them in the same rank order with the same
    softmax weights."""
    for l in range(L):
        _, rid, _ = orc.router(logits=logits_t[l:l + 1], top_k=K)
        assert rid[0].tolist() == ids_t[l].tolist(), l
        sel = rid[0]
        gu = np.concatenate([experts.get(l, int(e))[0] for e in sel])
        dn = np.concatenate([experts.get(l, int(e))[1] for e in sel])
        gub = np.concatenate([biases[l][0][e] for e in sel])
        dnb = np.concatenate([biases[l][1][e] for e in sel])
        compact_logits = logits_t[l][sel].reshape(1, K)
        r = orc.moe_layer(39, gu, dn, gub, dnb, x.reshape(1, HID), HID, INTER, K, K, activation=1,
                          logits=compact_logits, threads=16)
        assert r["ids"][0].tolist() == list(range(K))
        x = r["out"][0]
    return x


def test_tier_config4_full_shape_matches_resident_plan_and_oracle(gpu, orc):
    vb = gpu
    from vbmoe.routing_trace import read_plan
    host_biases = [(vb.synth_normal(SEED, 16 * l + 3, 0, E * 2 * INTER, 0.0, 0.02).reshape(E, 2 * INTER),
                    vb.synth_normal(SEED, 16 * l + 4, 0, E * HID, 0.0, 0.02).reshape(E, HID)) for l in range(L)]
    dev_biases = [(vb.DeviceBuffer.from_array(g), vb.DeviceBuffer.from_array(d)) for g, d in host_biases]
    banks, descs = [], []
    for l in range(L):
        gu = vb.Bank(39, 2 * INTER, HID, E, True)
        dn = vb.Bank(39, HID, INTER, E, False)
        gu.generate(0, E, SEED, 16 * l + 1, 0, -8, -3)
        dn.generate(0, E, SEED, 16 * l + 2, 0, -8, -3)
        banks.append((gu, dn))
        descs.append(vb.MoeLayerDesc(gu.handle, dn.handle, dev_biases[l][0].ptr, dev_biases[l][1].ptr, None, None,
                                     None, HID, INTER, E, K, vb.ACT_SWIGLU_OAI, vb.ORDER_EXACT))
    group_bytes = banks[0][0].slot_bytes + banks[0][1].slot_bytes
    n_slots = (16 << 30) // group_bytes
    assert n_slots == 1299
    plan = C.c_void_p()
    vb.call("vbm_decode_plan_create", (vb.MoeLayerDesc * L)(*descs), L, C.byref(plan))
    gub = (C.c_void_p * L)(*[b[0].ptr for b in dev_biases])
    dnb = (C.c_void_p * L)(*[b[1].ptr for b in dev_biases])
    desc = vb.TierDesc(39, HID, INTER, L, E, K, vb.ACT_SWIGLU_OAI, n_slots, 64, 4, vb.ADMIT_CLASSIC,
                       C.cast(gub, C.POINTER(C.c_void_p)), C.cast(dnb, C.POINTER(C.c_void_p)))
    tier = C.c_void_p()
    vb.call("vbm_tier_create", C.byref(desc), C.byref(tier))
    try:
        vb.call("vbm_tier_generate", tier.value, SEED, 16, 1, 2, -8.0, -3.0, None)
        py = ref.Admission(L, E, K, n_slots, 64, 4, ref.CLASSIC)
        seeds = read_plan(PLAN, L, E)
        assert len(seeds) == 944
        for layer, expert in seeds:
            vb.call("vbm_tier_seed", tier.value, layer, expert)
            py.seed(layer, expert)
        print(f"[config4] stack and tier ready: {n_slots} slots, {len(seeds)} seeded", flush=True)
        tokens = 64
        logits, routes = zipf_trace(np.random.default_rng(SEED), tokens)
        x = vb.synth_normal(SEED, 6, 0, HID)
        dx = vb.DeviceBuffer.from_array(x)
        dl = vb.DeviceBuffer(logits[0].nbytes)
        o1, o2 = vb.DeviceBuffer(4 * HID), vb.DeviceBuffer(4 * HID)
        i1, i2 = vb.DeviceBuffer(4 * L * K), vb.DeviceBuffer(4 * L * K)
        experts = HostExperts(vb)
        staged = 0
        for t in range(tokens):
            dl.upload(logits[t])
            vb.call("vbm_decode_step", plan.value, dx.ptr, dl.ptr, o1.ptr, i1.ptr, None, None, None)
            vb.call("vbm_tier_step", tier.value, dx.ptr, dl.ptr, o2.ptr, i2.ptr, None)
            vb.call("vbm_stream_synchronize", None)
            a, b = o1.download(np.float32, HID), o2.download(np.float32, HID)
            ia, ib = i1.download(np.int32, (L, K)), i2.download(np.int32, (L, K))
            assert ia.tolist() == routes[t] and np.array_equal(ia, ib), t
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), t
            assert np.all(np.isfinite(b)), t
            for l in range(L):
                hits, made = py.admit(l, routes[t][l])
                admitted = {e for _, e, _ in made}
                staged += sum(1 for r, e in enumerate(routes[t][l]) if not hits[r] and e not in admitted)
            if t in (0, 1, tokens - 1):
                want = oracle_token(orc, experts, host_biases, x, logits[t], ia)
                assert np.array_equal(want.view(np.uint32), b.view(np.uint32)), f"token {t} differs from the oracle"
                print(f"[config4] token {t}: tier == resident plan == oracle (bitwise)", flush=True)
        st = vb.TierStats()
        vb.call("vbm_tier_get_stats", tier.value, C.byref(st))
        print(f"[config4] {tokens} tokens: hit rate {st.hits / (tokens * L * K):.4f}, admissions {st.admissions}, "
              f"evictions {st.evictions}, staged {st.staged}, uploaded {st.uploaded_bytes / 1e9:.2f} GB", flush=True)
        assert (st.dispatches, st.hits, st.admissions, st.evictions) == (tokens * L, py.hits, py.admissions,
                                                                          py.evictions)
        assert st.staged == staged and st.admissions > 0 and st.staged > 0
    finally:
        vb.call("vbm_tier_destroy", tier.value)
        vb.call("vbm_decode_plan_destroy", plan.value)
        for gu, dn in banks:
            gu.destroy()
            dn.destroy()
