"""GPU parity: libvbmoe.so (through its C ABI) against the CPU oracle on identical seeded inputs.

Bar: bit-exact for bank bytes, quantizer output, grouping, expert ids, integer block dots and the
x86-contract GEMV (whose fp32 order is reproduced); fp32 layer outputs within 1e-3 max relative
error (max|gpu - cpu| / max|cpu|) and cosine >= 0.99999.
"""
import ctypes as C

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def test_bank_upload_export_is_lossless(gpu):
    for type_id, rows, k, inter in [(H.MX, 5760, 2880, True), (H.MX, 2880, 2880, False), (H.Q8, 1536, 2048, True),
                                    (H.Q8, 2048, 768, False), (H.MX, 64, 448, False)]:
        w = H.synth_weights(type_id, 1234, 7, 2, rows, k)
        bank = H.make_bank(type_id, w, 2, rows, k, inter)
        per = w.size // 2
        for e in range(2):
            assert np.array_equal(bank.export(e), w[e * per:(e + 1) * per]), (type_id, rows, k, inter, e)
        bank.destroy()


def test_device_generator_matches_host_generator(gpu):
    rows, k, experts = 5760, 2880, 3
    bank = gpu.Bank(H.MX, rows, k, experts, True)
    bank.generate(0, experts, 99, 11, 5, -8, -3)
    per_blocks = rows * (k // 32)
    for s in range(experts):
        host = gpu.synth_mxfp4(99, 11, (5 + s) * per_blocks, per_blocks)
        assert np.array_equal(bank.export(s), host), s
    qb = gpu.Bank(H.Q8, 768, 2048, 2, False)
    qb.generate(0, 2, 7, 3, 0, 1e-3, 1e-2)
    per_blocks = 768 * 64
    for s in range(2):
        assert np.array_equal(qb.export(s), gpu.synth_q8_0(7, 3, s * per_blocks, per_blocks)), s


def activation_patterns(k: int, rows: int):
    """tools/trace/hybrid_layer.cpp:593-605 patterns plus N(0,1)."""
    i = np.arange(k * rows)
    yield "normal", np.random.default_rng(8).standard_normal(k * rows).astype(np.float32)
    for sample, mag in enumerate((0.2, 50.0, 500.0)):
        yield f"sine{mag}", (mag * np.sin(((i + 1) * (sample + 3)) * 0.017)).astype(np.float32)
    yield "zero", np.zeros(k * rows, np.float32)
    yield "q8-ties", np.where(i % 32 == 0, 127.0, np.where(i % 32 == 1, -127.0,
                              np.where(i % 2 == 1, -1.0, 1.0) * (0.5 + ((i + 7) % 31)))).astype(np.float32)


def test_quantize_q8_0_bitwise(gpu, orc):
    k, rows = 2880, 5
    for name, x in activation_patterns(k, rows):
        dx = gpu.DeviceBuffer.from_array(x)
        dq = gpu.DeviceBuffer(rows * (k // 32) * 34)
        gpu.call("vbm_quantize_q8_0", dx.ptr, rows, k, k, dq.ptr, None)
        got = dq.download(np.uint8, (rows, k // 32 * 34))
        assert np.array_equal(got, orc.quantize_q8_0(x.reshape(rows, k))), name


@pytest.mark.parametrize("experts,active,tokens,strided,mask", [
    (4, 1, 1, False, "none"), (7, 3, 2, True, "partial"), (8, 4, 3, False, "all"), (16, 8, 3, True, "partial"),
    (8, 8, 2, False, "none"), (32, 4, 1, False, "none"),
])
def test_mul_mat_id_mxfp4_bitwise_small(gpu, orc, experts, active, tokens, strided, mask):
    """tests/test_masked_matmul.cpp:76-105 cases: ids (token + 3 rank) % experts, -1 masks, strided ids."""
    k, rows = 256, 64
    w = H.synth_weights(H.MX, 3, experts, experts, rows, k)
    bank = H.make_bank(H.MX, w, experts, rows, k)
    x = gpu.synth_normal(3, 100 + experts, 0, tokens * k).reshape(tokens, 1, k) * np.float32(0.1)
    ids = np.array([[(t + r * 3) % experts for r in range(active)] for t in range(tokens)], np.int32)
    if mask == "partial":
        ids.reshape(-1)[::2] = -1
    elif mask == "all":
        ids[:] = -1
    stride_ids = np.concatenate([ids, np.zeros((tokens, 1), np.int32)], axis=1) if strided else ids
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, stride_ids, active)
    ref = orc.mul_mat_id(39, w, k, rows, experts, 0, x, 1, stride_ids, active, tokens, stride_ids.shape[1])
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    bank.destroy()


def adversarial_mxfp4(experts: int, rows: int, k: int) -> np.ndarray:
    """tools/trace/hybrid_layer.cpp:964-979 fixture: exponents {0,1,2,120,126,127,128,130}."""
    nb = k // 32
    exps = np.array([0, 1, 2, 120, 126, 127, 128, 130], np.uint8)
    out = np.empty((experts * rows * nb, 17), np.uint8)
    blocks = np.arange(experts * rows * nb)
    out[:, 0] = exps[(blocks // nb) % 8]
    j = np.arange(16)
    out[:, 1:] = (((blocks[:, None] + j) % 16) | (((blocks[:, None] * 7 + j * 3) % 16) << 4)).astype(np.uint8)
    return out.reshape(-1)


def test_mul_mat_id_mxfp4_adversarial_and_neg128(gpu, orc):
    """Adversarial exponents and activation code -128 (tests/test_quantized_cuda.cpp:31-53)."""
    k, rows, experts, tokens = 128, 64, 4, 2
    w = adversarial_mxfp4(experts, rows, k)
    bank = H.make_bank(H.MX, w, experts, rows, k)
    ids = np.array([[0, 2, 1], [3, 0, 2]], np.int32)
    for sample in range(12):
        x = np.array([0.0 if sample == 0 else np.sin((i * 13 + sample * 31) * 0.07) * sample
                      for i in range(tokens * 3 * k)], np.float32).reshape(tokens, 3, k)
        q = orc.quantize_q8_0(x.reshape(-1, k)).reshape(tokens, 3, -1)
        if sample == 11:
            q.reshape(-1, 34)[:, 2] = 128                   # inject -128 codes
        if sample == 10:
            q.reshape(-1, 34)[:, 2:] = 128                  # every code -128
        got = H.mul_mat_id(bank, experts, q, gpu.TYPE_Q8_0, 3, ids, 3)
        ref = orc.mul_mat_id(39, w, k, rows, experts, 8, q, 3, ids, 3, tokens, 3)
        assert H.bits_equal(got, ref), (sample, H.diff_report(got, ref))
    bank.destroy()


def test_mul_mat_id_mxfp4_matches_repacked_8x8_contract(gpu, orc):
    """Row a8: the GPU's exact-order GEMV against the oracle's restatement of the repacked 8x8 CPU
    contract (tools/trace/exact_packed_cpu.h:52-88) on block_mxfp4x8-packed copies of the same
    experts (the packing the expert export at HP:751-762 inverts): bit-identical per row, with
    the recipe of tests/test_exact_packed_cpu.cpp:55-72 (exponents 96 + r % 40, two rows at 0/1,
    one activation code -128), for one and for several tokens."""
    rng = np.random.default_rng(417)
    experts, rows, n = 4, 64, 2880
    blocks = n // 32
    w = np.zeros((experts, rows, blocks, 17), np.uint8)
    w[..., 0] = 96 + rng.integers(0, 40, (experts, rows, blocks))
    w[..., 1:] = rng.integers(0, 256, (experts, rows, blocks, 16))
    w[:, 0, 0, 0], w[:, 0, 1, 0] = 0, 1
    bank = H.make_bank(H.MX, w.reshape(-1), experts, rows, n)
    for tokens in (1, 3):
        x = rng.uniform(-8, 8, (tokens, n)).astype(np.float32)
        q = orc.quantize_q8_0(x).reshape(tokens, 1, -1)
        q.reshape(-1)[2] = 0x80                                   # one activation code -128
        ids = np.stack([rng.choice(experts, 2, replace=False) for _ in range(tokens)]).astype(np.int32)
        got = H.mul_mat_id(bank, experts, q, gpu.TYPE_Q8_0, 1, ids, 2)
        for t in range(tokens):
            for r, e in enumerate(ids[t]):
                packed = orc.pack_mxfp4x8(w[e].reshape(-1), rows, blocks)
                ref = orc.gemv_mxfp4x8(packed, q[t, 0], n, rows)
                assert H.bits_equal(got[t, r], ref), (tokens, t, r, H.diff_report(got[t, r], ref))
    bank.destroy()


@pytest.mark.parametrize("tokens", [1, 8, 64])
def test_mul_mat_id_mxfp4_bitwise_config_shapes(gpu, orc, tokens):
    """Config 0/1 shapes: E=32, top-4, H=I=2880, down (2880 x 2880) and fused gate_up (5760 x 2880)."""
    k, experts, active = 2880, 32, 4
    rng = np.random.default_rng(tokens)
    ids = np.stack([rng.choice(experts, active, replace=False) for _ in range(tokens)]).astype(np.int32)
    for rows, inter, name in [(2880, False, "down"), (5760, True, "gate_up")]:
        w = H.synth_weights(H.MX, 17, 1 if inter else 2, experts, rows, k)
        bank = H.make_bank(H.MX, w, experts, rows, k, inter)
        bias = gpu.synth_normal(17, 3, 0, experts * rows, 0.0, 0.02)
        x = gpu.synth_normal(17, 4 + tokens, 0, tokens * k).reshape(tokens, 1, k)
        got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, active, bias=bias)
        ref = orc.mul_mat_id(39, w, k, rows, experts, 0, x, 1, ids, active, tokens, active, bias=bias, threads=8)
        assert H.bits_equal(got, ref), (name, H.diff_report(got, ref))
        bank.destroy()


def test_mul_mat_id_q8_0_bitwise(gpu, orc):
    """Config 3 shapes: H=2048, I=768, gate (768 x 2048) and down (2048 x 768)."""
    experts, active, tokens = 16, 8, 6
    rng = np.random.default_rng(33)
    ids = np.stack([rng.choice(experts, active, replace=False) for _ in range(tokens)]).astype(np.int32)
    for rows, k in [(768, 2048), (2048, 768)]:
        w = H.synth_weights(H.Q8, 21, rows, experts, rows, k)
        bank = H.make_bank(H.Q8, w, experts, rows, k)
        x = gpu.synth_normal(21, 5, 0, tokens * k).reshape(tokens, 1, k)
        got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, active)
        ref = orc.mul_mat_id(8, w, k, rows, experts, 0, x, 1, ids, active, tokens, active, threads=8)
        assert H.bits_equal(got, ref), (rows, k, H.diff_report(got, ref))
        bank.destroy()


def test_mul_mat_id_slot_map_and_residency_errors(gpu, orc):
    k, rows, experts = 256, 32, 6
    w = H.synth_weights(H.MX, 9, 9, experts, rows, k)
    resident = [4, 1, 5]
    bank = gpu.Bank(H.MX, rows, k, len(resident))
    per = w.size // experts
    for slot, e in enumerate(resident):
        bank.upload(slot, w[e * per:(e + 1) * per])
    slot_map = np.full(experts, -1, np.int32)
    slot_map[resident] = np.arange(len(resident))
    ids = np.array([[4, 1], [5, 4]], np.int32)
    x = gpu.synth_normal(9, 1, 0, 2 * k).reshape(2, 1, k)
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, 2, slot_map=slot_map, slot_map_host=slot_map)
    ref = orc.mul_mat_id(39, w, k, rows, experts, 0, x, 1, ids, 2, 2, 2)
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    with pytest.raises(gpu.VbmError) as err:       # non-resident expert (quantized_cuda.cu:224-227)
        H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, np.array([[0, 1]], np.int32), 2, slot_map=slot_map,
                     slot_map_host=slot_map)
    assert err.value.status == 1
    bank.destroy()


def _group_on_gpu(gpu, ids, n_ids, tokens, stride, n_as):
    d_ids = gpu.DeviceBuffer.from_array(np.ascontiguousarray(ids, np.int32))
    counts, offsets, rows = (gpu.DeviceBuffer(4 * n) for n in (n_as, n_as + 1, n_ids * tokens))
    err = gpu.DeviceBuffer(4)
    gpu.call("vbm_group_by_expert", d_ids.ptr, n_ids, tokens, stride, n_as, counts.ptr, offsets.ptr, rows.ptr,
             err.ptr, None)
    o = offsets.download(np.int32, n_as + 1)
    return (counts.download(np.int32, n_as), o, rows.download(np.int32, n_ids * tokens)[: o[-1]],
            int(err.download(np.int32, 1)[0]))


def test_grouping_exact(gpu, orc):
    rng = np.random.default_rng(12)
    for n_as, n_ids, tokens in [(32, 4, 1), (32, 4, 64), (128, 4, 32), (128, 8, 2048), (7, 3, 5), (1024, 6, 700)]:
        ids = np.stack([rng.choice(n_as, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
        ids[rng.random(ids.shape) < 0.05] = -1
        c, o, r, err = _group_on_gpu(gpu, ids, n_ids, tokens, n_ids, n_as)
        rc, ro, rr = orc.group_by_expert(ids, n_ids, tokens, n_ids, n_as)
        assert np.array_equal(c, rc) and np.array_equal(o, ro) and np.array_equal(r, rr) and err == 0


def test_grouping_duplicates_strides_single_expert_and_bad_ids(gpu, orc):
    """Entries in (token, rank) order whatever the ids hold: repeated experts within a token, a
    token stride wider than n_ids, one expert only, chunk boundaries (1024 entries) cut inside
    a token; ids outside [-1, n_as) set the error flag and are skipped."""
    rng = np.random.default_rng(13)
    for n_as, n_ids, tokens, stride in [(16, 5, 999, 7), (1, 3, 1500, 3), (300, 8, 1029, 8), (2, 1, 4099, 1)]:
        full = rng.integers(-1, n_as, size=(tokens, stride)).astype(np.int32)
        full[:, n_ids:] = 10**6                   # columns beyond n_ids are never read
        c, o, r, err = _group_on_gpu(gpu, full, n_ids, tokens, stride, n_as)
        rc, ro, rr = orc.group_by_expert(full, n_ids, tokens, stride, n_as)
        assert np.array_equal(c, rc) and np.array_equal(o, ro) and np.array_equal(r, rr) and err == 0
    ids = rng.integers(0, 64, size=(3000, 4)).astype(np.int32)
    bad = rng.random(ids.shape) < 0.01
    ids[bad] = np.where(rng.random(bad.sum()) < 0.5, 64, -5)
    c, o, r, err = _group_on_gpu(gpu, ids, 4, 3000, 4, 64)
    clean = np.where(bad, -1, ids).astype(np.int32)
    rc, ro, rr = orc.group_by_expert(clean, 4, 3000, 4, 64)
    assert err == 1 and np.array_equal(c, rc) and np.array_equal(o, ro) and np.array_equal(r, rr)


def test_grouping_single_workgroup_edges(gpu, orc):
    """Groupings of at most 1024 entries take the one-workgroup kernel (count, scan and place in
    LDS): exactly 1024 entries over 1024 experts, a token stride wider than n_ids with -1 ids, one
    expert, 1023 entries, and ids outside [-1, n_as) (error flag set, entries skipped)."""
    rng = np.random.default_rng(14)
    for n_as, n_ids, tokens, stride in [(1024, 4, 256, 4), (16, 5, 204, 7), (1, 3, 341, 3), (300, 8, 128, 8),
                                        (1024, 1, 1, 1)]:
        full = rng.integers(-1, n_as, size=(tokens, stride)).astype(np.int32)
        full[:, n_ids:] = 10**6                   # columns beyond n_ids are never read
        c, o, r, err = _group_on_gpu(gpu, full, n_ids, tokens, stride, n_as)
        rc, ro, rr = orc.group_by_expert(full, n_ids, tokens, stride, n_as)
        assert np.array_equal(c, rc) and np.array_equal(o, ro) and np.array_equal(r, rr) and err == 0, (n_as, tokens)
    ids = rng.integers(0, 64, size=(200, 4)).astype(np.int32)
    bad = rng.random(ids.shape) < 0.03
    ids[bad] = np.where(rng.random(bad.sum()) < 0.5, 64, -5)
    c, o, r, err = _group_on_gpu(gpu, ids, 4, 200, 4, 64)
    clean = np.where(bad, -1, ids).astype(np.int32)
    rc, ro, rr = orc.group_by_expert(clean, 4, 200, 4, 64)
    assert err == 1 and np.array_equal(c, rc) and np.array_equal(o, ro) and np.array_equal(r, rr)


def test_router_ids_exact(gpu, orc):
    for n_expert, hidden, tokens, top_k in [(32, 2880, 8, 4), (128, 2880, 32, 4), (128, 2048, 16, 8)]:
        w = gpu.synth_normal(5, 1, 0, n_expert * hidden, 0.0, 0.02).reshape(n_expert, hidden)
        x = gpu.synth_normal(5, 2, 0, tokens * hidden).reshape(tokens, hidden)
        dw, dx = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x)
        dl = gpu.DeviceBuffer(4 * tokens * n_expert)
        di, dwt = gpu.DeviceBuffer(4 * tokens * top_k), gpu.DeviceBuffer(4 * tokens * top_k)
        gpu.call("vbm_router_topk_softmax", dw.ptr, None, dx.ptr, hidden, dl.ptr, n_expert, tokens, top_k, di.ptr,
                 dwt.ptr, None)
        logits, ids, wts = orc.router(router_w=w, x=x, n_expert=n_expert, n_tokens=tokens, top_k=top_k, hidden=hidden)
        assert H.bits_equal(dl.download(np.float32, (tokens, n_expert)), logits)
        assert np.array_equal(di.download(np.int32, (tokens, top_k)), ids)
        assert np.allclose(dwt.download(np.float32, (tokens, top_k)), wts, rtol=4e-7, atol=0)
    # Given logits with exact ties: lower index first (topk-tie-probe.cpp:111-113).
    logits = np.array([[1, 3, 3, 0, 3, 2, 2, 3]], np.float32)
    dl = gpu.DeviceBuffer.from_array(logits)
    di, dwt = gpu.DeviceBuffer(16), gpu.DeviceBuffer(16)
    gpu.call("vbm_router_topk_softmax", None, None, None, 0, dl.ptr, 8, 1, 4, di.ptr, dwt.ptr, None)
    assert di.download(np.int32, 4).tolist() == [1, 2, 4, 7]


@pytest.mark.parametrize("n_expert", [100, 128, 200, 256, 257, 300, 1024])
def test_router_topk_given_logits_canonical_order(gpu, n_expert):
    """Top-k of given logits (the router takes up to 1024 experts and refuses more): ids in the
    canonical order (value descending, lower index first on ties), including rows full of ties and
    a row whose winners sit in the last lanes; weights are the softmax of the picks within 1e-6.
    The expert counts cover each register width of the kernel (2, 4 and 16 logits per lane) at
    and around its limits."""
    rng = np.random.default_rng(300 + n_expert)
    tokens, top_k = 24, 8
    logits = rng.standard_normal((tokens, n_expert)).astype(np.float32)
    logits[1] = np.round(logits[1])                                  # many exact ties
    logits[2] = 1.0                                                  # all tied: indices 0..k-1
    logits[3, -top_k:] = 10.0                                        # winners at the end
    dl = gpu.DeviceBuffer.from_array(logits)
    di, dwt = gpu.DeviceBuffer(4 * tokens * top_k), gpu.DeviceBuffer(4 * tokens * top_k)
    gpu.call("vbm_router_topk_softmax", None, None, None, 0, dl.ptr, n_expert, tokens, top_k, di.ptr, dwt.ptr, None)
    ids = di.download(np.int32, (tokens, top_k))
    wts = dwt.download(np.float32, (tokens, top_k))
    idx = np.arange(n_expert)
    for t in range(tokens):
        want = np.lexsort((idx, -logits[t].astype(np.float64)))[:top_k]
        assert ids[t].tolist() == want.tolist(), t
        v = logits[t, want].astype(np.float64)
        e = np.exp(v - v.max())
        assert np.allclose(wts[t], e / e.sum(), rtol=1e-6, atol=0), t
    with pytest.raises(gpu.VbmError):
        gpu.call("vbm_router_topk_softmax", None, None, None, 0, dl.ptr, 1025, 1, top_k, di.ptr, dwt.ptr, None)


@pytest.mark.parametrize("n_expert,hidden,top_k", [(32, 2880, 4), (128, 2048, 8)])
def test_router_ids_equal_float64_topk_where_determined(gpu, orc, n_expert, hidden, top_k):
    """The reference's router fp32 order (upstream ggml_mul_mat) is parity-unpinned; wherever the
    float64 logits separate the top k + 1 by more than twice the worst-case error of any fp32
    summation order, the device's ids must equal the float64 top-k (so they equal the reference's
    whatever its order), and they equal the oracle's everywhere."""
    from test_oracle import router_near_ties
    rng = np.random.default_rng(190 + n_expert)
    tokens = 256
    w = (rng.standard_normal((n_expert, hidden)) * 0.02).astype(np.float32)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    dw, dx = gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer.from_array(x)
    dl = gpu.DeviceBuffer(4 * tokens * n_expert)
    di, dwt = gpu.DeviceBuffer(4 * tokens * top_k), gpu.DeviceBuffer(4 * tokens * top_k)
    gpu.call("vbm_router_topk_softmax", dw.ptr, None, dx.ptr, hidden, dl.ptr, n_expert, tokens, top_k, di.ptr,
             dwt.ptr, None)
    ids = di.download(np.int32, (tokens, top_k))
    want, determined = router_near_ties(w, x, top_k)
    _, oids, _ = orc.router(router_w=w, x=x, n_expert=n_expert, n_tokens=tokens, top_k=top_k, hidden=hidden)
    print(f"[router {n_expert}x{hidden}] near-tie fraction {1 - determined.mean():.4f}", flush=True)
    assert np.array_equal(ids[determined], want[determined])
    assert np.array_equal(ids, oids)


def test_combine_bitwise_and_order(gpu, orc):
    y = gpu.synth_normal(4, 1, 0, 3 * 4 * 2880).reshape(3, 4, 2880) * np.float32(1e3)
    w = gpu.synth_normal(4, 2, 0, 12).reshape(3, 4)
    dy, dw, do = gpu.DeviceBuffer.from_array(y), gpu.DeviceBuffer.from_array(w), gpu.DeviceBuffer(3 * 2880 * 4)
    gpu.call("vbm_weighted_combine", dy.ptr, dw.ptr, 2880, 4, 3, do.ptr, None)
    ref = np.empty((3, 2880), np.float32)
    orc.load().orc_weighted_combine(y.ctypes.data, w.ctypes.data, 2880, 4, 3, ref.ctypes.data)
    assert H.bits_equal(do.download(np.float32, (3, 2880)), ref)
    probe = np.array([1e20, -1e20, 1.0], np.float32).reshape(1, 3, 1)
    dy, dw, do = gpu.DeviceBuffer.from_array(probe), gpu.DeviceBuffer.from_array(np.ones((1, 3), np.float32)), gpu.DeviceBuffer(4)
    gpu.call("vbm_weighted_combine", dy.ptr, dw.ptr, 1, 3, 1, do.ptr, None)
    assert do.download(np.float32, 1)[0] == 1.0


@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
def test_mul_mat_id_every_chunk_width_bitwise(gpu, orc, type_id):
    """The batched GEMV runs each expert's jobs in chunks of up to 8 tokens at the narrowest width
    in {1, 2, 4, 8} that holds the chunk: per-expert counts 1, 2, 3, 4, 5, 8, 9 and 17 reach every
    width, partial chunks of widths 4 and 8 and several chunks per expert (top-1 ids, so each
    count is exact), with biases, a half-live last tile pair (rows 96) and per-token activations."""
    counts = [1, 2, 3, 4, 5, 8, 9, 17, 0]
    experts, k, rows = len(counts), 512, 96
    rng = np.random.default_rng(91)
    ids = rng.permutation(np.repeat(np.arange(experts), counts)).astype(np.int32).reshape(-1, 1)
    tokens = ids.shape[0]
    w = H.synth_weights(type_id, 91, 1, experts, rows, k)
    bank = H.make_bank(type_id, w, experts, rows, k)
    bias = gpu.synth_normal(91, 2, 0, experts * rows, 0.0, 0.02)
    x = gpu.synth_normal(91, 3, 0, tokens * k).reshape(tokens, 1, k)
    print(f"[chunk widths type={type_id}] tokens={tokens} counts={counts}", flush=True)
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, 1, bias=bias)
    ref = orc.mul_mat_id(type_id, w, k, rows, experts, 0, x, 1, ids, 1, tokens, 1, bias=bias)
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    bank.destroy()


def test_mul_mat_id_mxfp4_matrix_path_exponent_ranges_bitwise(gpu, orc):
    """The MXFP4 batched GEMV runs chunks of 3..8 tokens on the matrix cores and folds the block
    exponents into the weight conversion only when every exponent of a tile pair's rows lies in
    [-14, 12] (ggml e8m0 bytes 114..140); other tile pairs take ldexp per output. Per expert:
    all in range (the generator's), both boundaries (114 and 140) in range, one byte just outside
    (113 or 141) in one tile pair only, a tail block outside (K = 576: two groups of eight blocks
    and a two-block tail), and every byte far outside (90..180, finite results); top-1 ids with
    counts 3, 4, 5, 8 and 12 reach widths 4 and 8 (12 = 8 + 4), rows 96 (a half-live pair)."""
    k, rows = 576, 96
    nb = k // 32
    counts = [4, 8, 3, 5, 12, 8]
    experts = len(counts)
    w = H.synth_weights(H.MX, 77, 1, experts, rows, k).reshape(experts, rows, nb, 17)
    w[1, 0, 0, 0], w[1, 95, nb - 1, 0] = 114, 140              # boundaries: still folded
    w[2, 5, 3, 0] = 113                                        # pair 0 unfolded, pair 1 folded
    w[3, 70, 9, 0] = 141                                       # pair 1 unfolded, pair 0 folded
    w[4, 33, nb - 1, 0] = 100                                  # a tail block of pair 0
    rng = np.random.default_rng(77)
    w[5, :, :, 0] = rng.integers(90, 181, size=(rows, nb)).astype(np.uint8)
    w = w.reshape(-1)
    bank = H.make_bank(H.MX, w, experts, rows, k)
    ids = rng.permutation(np.repeat(np.arange(experts), counts)).astype(np.int32).reshape(-1, 1)
    tokens = ids.shape[0]
    bias = gpu.synth_normal(77, 2, 0, experts * rows, 0.0, 0.02)
    x = gpu.synth_normal(77, 3, 0, tokens * k).reshape(tokens, 1, k)
    print(f"[matrix path exponents] tokens={tokens} counts={counts}", flush=True)
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, 1, bias=bias)
    ref = orc.mul_mat_id(39, w, k, rows, experts, 0, x, 1, ids, 1, tokens, 1, bias=bias)
    assert np.all(np.isfinite(ref))
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    bank.destroy()


def test_mul_mat_id_randomized_shapes_bitwise(gpu, orc):
    """24 seeded random MUL_MAT_ID cases in the exact order against the oracle, bit for bit:
    MXFP4 or Q8_0 weights, 1..40 experts, top-k 1..8 (distinct per token, some -1 masks), 1..48
    tokens, rows 32..320 (half-live last tile pairs included), k 64..1024, fp32 or ggml Q8_0
    activations (the latter with injected -128 codes), broadcast or per-rank activation rows,
    with and without biases."""
    rng = np.random.default_rng(20261202)
    for case in range(24):
        type_id = H.MX if case % 2 == 0 else H.Q8
        experts = int(rng.integers(1, 41))
        active = int(rng.integers(1, min(8, experts) + 1))
        tokens = int(rng.integers(1, 49))
        rows = 32 * int(rng.integers(1, 11))
        k = 64 * int(rng.integers(1, 17))
        b_ne1 = 1 if rng.random() < 0.5 else active
        q8_input = rng.random() < 0.4
        ids = np.stack([rng.choice(experts, active, replace=False) for _ in range(tokens)]).astype(np.int32)
        if rng.random() < 0.3:
            ids.reshape(-1)[rng.random(ids.size) < 0.2] = -1
        w = H.synth_weights(type_id, 500 + case, 1, experts, rows, k)
        bank = H.make_bank(type_id, w, experts, rows, k)
        bias = gpu.synth_normal(500 + case, 2, 0, experts * rows, 0.0, 0.02) if rng.random() < 0.5 else None
        x = gpu.synth_normal(500 + case, 3, 0, tokens * b_ne1 * k).reshape(tokens, b_ne1, k)
        label = (f"case {case}: type={type_id} experts={experts} top{active} tokens={tokens} rows={rows} k={k} "
                 f"b_ne1={b_ne1} q8={q8_input} bias={bias is not None}")
        print(f"[random mul_mat_id] {label}", flush=True)
        if q8_input:
            q = orc.quantize_q8_0(x.reshape(tokens * b_ne1, k)).reshape(-1, 34)
            q[rng.random(q.shape[0]) < 0.25, 2 + int(rng.integers(0, 32))] = 128      # -128 codes
            b, b_type, orc_type = q.reshape(tokens, b_ne1, -1), gpu.TYPE_Q8_0, 8
        else:
            b, b_type, orc_type = x, gpu.TYPE_F32, 0
        got = H.mul_mat_id(bank, experts, b, b_type, b_ne1, ids, active, bias=bias)
        ref = orc.mul_mat_id(type_id, w, k, rows, experts, orc_type, b, b_ne1, ids, active, tokens, active, bias=bias)
        assert H.bits_equal(got, ref), f"{label}: {H.diff_report(got, ref)}"
        bank.destroy()


@pytest.mark.parametrize("order,tokens", [(0, 6), (1, 64)])
def test_mul_mat_id_unmapped_expert_and_invalid_ids_are_nan(gpu, orc, order, tokens):
    """Without a host copy of the map to check against, a routed expert whose expert->slot entry is
    -1 gives NaN output rows (exact order: the batched GEMV; fast order at 64 tokens: the grouped
    GEMM), and so do ids outside [-1, n_as), which the grouping skips; -1 ids stay zero rows and
    every other row equals the oracle (bitwise in the exact order, within tolerance in the fast)."""
    k, rows, experts, n_ids = 256, 128, 4, 2
    rng = np.random.default_rng(31 + order)
    w = H.synth_weights(H.MX, 31, 1, experts, rows, k)
    bank = H.make_bank(H.MX, w, experts, rows, k)
    slot_map = np.arange(experts, dtype=np.int32)
    slot_map[2] = -1
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
    ids[0] = [2, 0]
    ids[1] = [-1, 1]
    ids[2] = [experts, 3]      # invalid: one past the last expert
    ids[3] = [1, -7]           # invalid: below -1
    x = gpu.synth_normal(31, 2, 0, tokens * k).reshape(tokens, 1, k)
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, n_ids, order=order, slot_map=slot_map)
    safe = np.where((ids >= 0) & (ids < experts) & (ids != 2), ids, -1).astype(np.int32)
    ref = orc.mul_mat_id(39, w, k, rows, experts, 0, x, 1, safe, n_ids, tokens, n_ids, threads=8)
    poisoned = ((ids == 2) | (ids >= experts) | (ids < -1))
    assert poisoned.sum() >= 3
    assert np.all(np.isnan(got[poisoned])), "unmapped / invalid rows must be NaN"
    assert np.all(got[ids == -1] == 0.0)
    keep = ~poisoned
    if order == 0:
        assert H.bits_equal(got[keep], ref[keep]), H.diff_report(got[keep], ref[keep])
    else:
        max_rel, cos = H.rel_err_and_cos(got[keep], ref[keep])
        assert max_rel <= 1e-3 and cos >= 0.99999
    bank.destroy()


@pytest.mark.parametrize("order,tokens", [(0, 4), (1, 96)])
def test_layer_unmapped_expert_gives_nan_rows(gpu, orc, order, tokens):
    """The fused layer over banks whose expert->slot map holds -1 for a routed expert: the tokens
    routed to it come out NaN (never stale workspace data from an earlier call), the others equal
    the oracle (bitwise in the exact order, within tolerance in the fast)."""
    from test_gpu_layer import Layer
    E, K, Hd = 8, 2, 256
    layer = Layer(gpu, H.MX, Hd, Hd, E, K, seed=57, router=False, order=order)
    x = gpu.synth_normal(57, 6, 0, tokens * Hd).reshape(tokens, Hd)
    logits = gpu.synth_normal(57, 7, 0, tokens * E).reshape(tokens, E)
    ref = layer.forward_cpu(orc, x, logits)
    # fill the workspace with a correct earlier result first, then unmap one routed expert
    layer.forward_gpu(x, logits)
    bad = int(ref["ids"][0, 0])
    slot_map = np.arange(E, dtype=np.int32)
    slot_map[bad] = -1
    dmap = gpu.DeviceBuffer.from_array(slot_map)
    d = layer.desc()
    d.expert_to_slot = dmap.ptr
    ws = C.c_size_t()
    gpu.call("vbm_moe_layer_workspace", C.byref(d), tokens, C.byref(ws))
    work = gpu.DeviceBuffer(ws.value)
    dx, dl = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(logits)
    out = gpu.DeviceBuffer(4 * tokens * Hd)
    gpu.call("vbm_moe_layer_forward", C.byref(d), dx.ptr, dl.ptr, tokens, out.ptr, None, None, work.ptr, ws.value, None)
    gpu.call("vbm_stream_synchronize", None)
    got = out.download(np.float32, (tokens, Hd))
    hit = np.any(ref["ids"] == bad, axis=1)
    assert hit[0] and not hit.all()
    assert np.all(np.isnan(got[hit]))
    if order == 0:
        assert H.bits_equal(got[~hit], ref["out"][~hit])
    else:
        max_rel, cos = H.rel_err_and_cos(got[~hit], ref["out"][~hit])
        assert max_rel <= 1e-3 and cos >= 0.99999
    layer.destroy()


def test_add_id_matches_oracle(gpu, orc):
    """GGML_OP_ADD_ID (hybrid-experts.patch:1464-1480): y[:, r, t] += bias[:, ids[r, t]], -1 ids
    untouched, with a token stride on the ids (a top-k view of a wider argsort)."""
    rng = np.random.default_rng(44)
    rows, n_ids, tokens, n_as, stride = 96, 3, 17, 9, 5
    y = rng.standard_normal((tokens, n_ids, rows)).astype(np.float32)
    bias = rng.standard_normal((n_as, rows)).astype(np.float32)
    ids_full = rng.integers(-1, n_as, (tokens, stride)).astype(np.int32)
    ids = ids_full[:, :n_ids]
    ref = y.copy()
    for t in range(tokens):
        for r in range(n_ids):
            if ids[t, r] >= 0:
                ref[t, r] = ref[t, r] + bias[ids[t, r]]
    dy, db, di = (gpu.DeviceBuffer.from_array(a) for a in (y, bias, ids_full))
    gpu.call("vbm_add_id", dy.ptr, db.ptr, n_as, di.ptr, rows, n_ids, tokens, stride, None)
    got = dy.download(np.float32, y.shape)
    assert H.bits_equal(got, ref)


@pytest.mark.parametrize("activation", [0, 1])
def test_glu_matches_oracle(gpu, orc, activation):
    """GGML_OP_GLU swiglu / swiglu_oai (alpha 1.702, limit 7) on strided gate / up views of one
    fused [2I] row per (rank, token), as ggml splits the fused gate_up output, against the oracle's
    activation: within 2 ulp (expf bits are unpinned upstream), values past the clamp included."""
    rng = np.random.default_rng(45 + activation)
    n_rows, width = 37, 200
    gu = (rng.standard_normal((n_rows, 2 * width)) * 6).astype(np.float32)
    gu[0, :8] = [-30, -7.5, -7, 0, 7, 7.5, 30, np.float32(1e-30)]
    out = gpu.DeviceBuffer(4 * n_rows * width)
    dgu = gpu.DeviceBuffer.from_array(gu)
    gpu.call("vbm_glu", activation, dgu.ptr, dgu.ptr + 4 * width, out.ptr, n_rows, width, 2 * width, 2 * width,
             width, C.c_float(1.702), C.c_float(7.0), None)
    got = out.download(np.float32, (n_rows, width))
    ref = np.empty_like(got)
    for i in range(n_rows):
        ref[i] = orc.glu(activation, gu[i, :width], gu[i, width:])
    ulp = np.abs(got.astype(np.float64) - ref.astype(np.float64)) / np.spacing(np.abs(ref)).astype(np.float64)
    print(f"[glu act={activation}] max ulp {float(ulp.max()):.1f}, exact fraction {float(np.mean(got == ref)):.4f}",
          flush=True)
    assert ulp.max() <= 2


@pytest.mark.parametrize("order,tokens", [(0, 12), (1, 96)])
def test_mul_mat_id_caller_workspace_matches(gpu, orc, order, tokens):
    """vbm_mul_mat_id_ws over a caller workspace of the size vbm_mul_mat_id_workspace reports is
    bit-identical to vbm_mul_mat_id (library scratch) and to the oracle in the exact order; a
    workspace one byte short is rejected before any work is enqueued."""
    k, rows, experts, n_ids = 512, 128, 6, 2
    rng = np.random.default_rng(61 + order)
    w = H.synth_weights(H.Q8, 61, 1, experts, rows, k)
    bank = H.make_bank(H.Q8, w, experts, rows, k)
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = gpu.synth_normal(61, 2, 0, tokens * k).reshape(tokens, 1, k)
    ref = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, n_ids, order=order)
    need = C.c_size_t()
    gpu.call("vbm_mul_mat_id_workspace", bank.handle, experts, 1, n_ids, tokens, order, C.byref(need))
    assert need.value > 0
    ws = gpu.DeviceBuffer(need.value)
    dx, di = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(ids)
    dst = gpu.DeviceBuffer(tokens * n_ids * rows * 4)
    gpu.call("vbm_mul_mat_id_ws", bank.handle, None, None, experts, gpu.TYPE_F32, dx.ptr, 1, di.ptr, n_ids, tokens,
             n_ids, None, dst.ptr, order, ws.ptr, need.value, None)
    gpu.call("vbm_stream_synchronize", None)
    got = dst.download(np.float32, (tokens, n_ids, rows))
    assert H.bits_equal(got, ref)
    if order == 0:
        want = orc.mul_mat_id(8, w, k, rows, experts, 0, x, 1, ids, n_ids, tokens, n_ids, threads=8)
        assert H.bits_equal(got, want)
    with pytest.raises(gpu.VbmError, match="workspace too small"):
        gpu.call("vbm_mul_mat_id_ws", bank.handle, None, None, experts, gpu.TYPE_F32, dx.ptr, 1, di.ptr, n_ids, tokens,
                 n_ids, None, dst.ptr, order, ws.ptr, need.value - 1, None)
    bank.destroy()
