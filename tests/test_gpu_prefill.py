"""Prefill-sized token groups through the MFMA grouped GEMM (fast accumulation order).

Every 32-element integer block dot is exact; only the fp32 accumulation across blocks follows a
different order than the CPU's 8-lane chains. With unit scales all fp32 sums are exact integers,
so there the GEMM must reproduce the oracle bit for bit (including the x86 VPSIGNB correction for
activation code -128); with the benchmark's value distributions the outputs must be within 1e-3
max relative error and cosine >= 0.99999 of the oracle, with expert ids identical."""
import ctypes as C

import numpy as np
import pytest

import helpers as H
from test_gpu_layer import Layer

pytestmark = pytest.mark.gpu


def unit_scale_q8(experts, rows, k, rng):
    """Q8_0 weights with codes in [-3, 3] and fp16 scale 1.0."""
    blk = np.zeros((experts * rows * (k // 32), 34), np.uint8)
    blk[:, 0], blk[:, 1] = 0x00, 0x3C
    blk[:, 2:] = rng.integers(-3, 4, (blk.shape[0], 32)).astype(np.int8).view(np.uint8)
    return blk.reshape(-1)


def unit_scale_mxfp4(experts, rows, k, rng):
    """MXFP4 weights with e8m0 byte 127 (E8M0_HALF = 0.5, i.e. the true e2m1 values)."""
    blk = np.zeros((experts * rows * (k // 32), 17), np.uint8)
    blk[:, 0] = 127
    blk[:, 1:] = rng.integers(0, 256, (blk.shape[0], 16)).astype(np.uint8)
    return blk.reshape(-1)


def unit_scale_activations(n, k, rng):
    """fp32 rows whose Q8_0 quantization has d = 1: integers in [-8, 8] plus one 127 per block."""
    x = rng.integers(-8, 9, (n, k)).astype(np.float32)
    x[:, ::32] = 127.0
    return x


@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
@pytest.mark.parametrize("rows,k", [(256, 512), (96, 320), (160, 448), (64, 384), (128, 64)])
def test_gemm_integer_block_dots_exact(gpu, orc, type_id, rows, k):
    """Unit-scale weights and activations: bit-identical to the oracle. The shapes cover bank
    groups with and without tail blocks (k = 320, 448: MXFP4 tails of 2 and 6 blocks, Q8_0 tails
    of 2), rows of tail blocks only (k = 64: no full group, so no staged chunk at all) and tile
    pairs whose second 32-row tile is past the last row (rows = 96, 160)."""
    rng = np.random.default_rng(71 + k)
    experts, n_ids, tokens = 8, 4, 64
    w = (unit_scale_mxfp4 if type_id == H.MX else unit_scale_q8)(experts, rows, k, rng)
    bank = H.make_bank(type_id, w, experts, rows, k)
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = unit_scale_activations(tokens, k, rng).reshape(tokens, 1, k)
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, n_ids, order=gpu.ORDER_FAST)
    ref = orc.mul_mat_id(type_id, w, k, rows, experts, 0, x, 1, ids, n_ids, tokens, n_ids, threads=8)
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    # the same with ggml Q8_0 activations carrying -128 codes (x86 VPSIGNB contract)
    q = orc.quantize_q8_0(x.reshape(tokens, k)).reshape(tokens, 1, -1)
    qb = q.reshape(-1, 34)
    qb[::3, 2 + 5] = 128
    qb[::7, 2:10] = 128
    got = H.mul_mat_id(bank, experts, q, gpu.TYPE_Q8_0, 1, ids, n_ids, order=gpu.ORDER_FAST)
    ref = orc.mul_mat_id(type_id, w, k, rows, experts, 8, q, 1, ids, n_ids, tokens, n_ids, threads=8)
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    bank.destroy()


@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
def test_gemm_power_of_two_scales_exact(gpu, orc, type_id):
    """Per-block power-of-two scales: Q8_0 weight scales 2^-22 .. 2^-20 (fp16 subnormals), MXFP4
    exponents 2^-2 .. 1, activation scales 2^-2 .. 1. Every product and every fp32 sum is exact,
    so the fast order must equal the oracle bit for bit; a kernel that flushed subnormal fp16
    scales, or paired one block's scale with another block's dot, fails it."""
    rng = np.random.default_rng(7200 + type_id)
    experts, n_ids, tokens, rows, k = 4, 2, 160, 128, 256
    if type_id == H.Q8:
        w = unit_scale_q8(experts, rows, k, rng).reshape(-1, 34)
        bits = np.array([0x0004, 0x0008, 0x0010], np.uint16)[rng.integers(0, 3, w.shape[0])]
        w[:, 0:2] = bits.astype("<u2").view(np.uint8).reshape(-1, 2)
    else:
        w = unit_scale_mxfp4(experts, rows, k, rng).reshape(-1, 17)
        w[:, 0] = rng.integers(125, 128, w.shape[0])
    w = w.reshape(-1)
    bank = H.make_bank(type_id, w, experts, rows, k)
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = unit_scale_activations(tokens, k, rng)
    x *= np.repeat(np.exp2(-rng.integers(0, 3, (tokens, k // 32))), 32, axis=1).astype(np.float32)
    x = x.reshape(tokens, 1, k)
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, n_ids, order=gpu.ORDER_FAST)
    ref = orc.mul_mat_id(type_id, w, k, rows, experts, 0, x, 1, ids, n_ids, tokens, n_ids, threads=8)
    assert np.any(ref != 0)
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    bank.destroy()


@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
@pytest.mark.parametrize("experts,n_ids,tokens", [(2, 2, 190), (3, 2, 257), (4, 2, 300), (2, 2, 300), (2, 2, 192),
                                                   (2, 2, 193), (2, 2, 385)])
def test_gemm_multi_tile_experts_exact(gpu, orc, type_id, experts, n_ids, tokens):
    """Experts with 150..385 routed jobs run the grouped GEMM over one to three job tiles (128 jobs
    for MXFP4, 192 for Q8_0: full ones and a partial last one, down to a single job), each tile's
    live jobs split between its two wave halves. With unit scales every fp32 sum is an exact
    integer, so the GEMM must match the oracle bit for bit, for fp32 inputs and for ggml Q8_0
    inputs carrying -128 codes (the flagged kernel)."""
    rng = np.random.default_rng(7000 + experts)
    rows, k = 128, 256
    w = (unit_scale_mxfp4 if type_id == H.MX else unit_scale_q8)(experts, rows, k, rng)
    bank = H.make_bank(type_id, w, experts, rows, k)
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
    per_expert = np.bincount(ids.ravel(), minlength=experts)
    print(f"[multi-tile gemm type={type_id}] jobs per expert {per_expert.tolist()}", flush=True)
    assert per_expert.max() > 128 and np.any(per_expert % 128 != 0)
    x = unit_scale_activations(tokens, k, rng).reshape(tokens, 1, k)
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, n_ids, order=gpu.ORDER_FAST)
    ref = orc.mul_mat_id(type_id, w, k, rows, experts, 0, x, 1, ids, n_ids, tokens, n_ids, threads=8)
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    q = orc.quantize_q8_0(x.reshape(tokens, k)).reshape(tokens, 1, -1)
    qb = q.reshape(-1, 34)
    qb[::5, 2 + 9] = 128
    qb[::11, 2:8] = 128
    got = H.mul_mat_id(bank, experts, q, gpu.TYPE_Q8_0, 1, ids, n_ids, order=gpu.ORDER_FAST)
    ref = orc.mul_mat_id(type_id, w, k, rows, experts, 8, q, 1, ids, n_ids, tokens, n_ids, threads=8)
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    bank.destroy()


@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
def test_gemm_unaligned_destination_exact(gpu, orc, type_id):
    """A destination 4 bytes past a 16-byte boundary takes the per-element stores of the fp32
    epilogue (aligned ones leave through the LDS tile as 16-byte stores), and fp32 activations 4
    bytes past one take the scalar loads of the row quantizer: bit-identical to the oracle with
    unit scales, biases included, over a bank whose last tile pair is half live."""
    rng = np.random.default_rng(7100 + type_id)
    experts, n_ids, tokens, rows, k = 3, 2, 150, 96, 256
    w = (unit_scale_mxfp4 if type_id == H.MX else unit_scale_q8)(experts, rows, k, rng)
    bank = H.make_bank(type_id, w, experts, rows, k)
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = unit_scale_activations(tokens, k, rng).reshape(tokens, 1, k)
    bias = rng.integers(-4, 5, experts * rows).astype(np.float32)
    ref = orc.mul_mat_id(type_id, w, k, rows, experts, 0, x, 1, ids, n_ids, tokens, n_ids, bias=bias, threads=8)
    for off, boff in ((0, 0), (4, 0), (0, 4), (4, 4)):
        got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, n_ids, bias=bias, order=gpu.ORDER_FAST,
                           dst_offset=off, b_offset=boff)
        assert H.bits_equal(got, ref), (off, boff, H.diff_report(got, ref))
    bank.destroy()


@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
def test_prefill_layer_multi_tile_experts(gpu, orc, type_id):
    """The fused layer (gate_up GEMM with the GLU + requantization epilogue, then the down GEMM)
    with 4 experts top-2 at T = 300, so every expert holds 110..190 jobs over 2..3 job tiles:
    ids exact, output within the fast order's tolerance of the oracle."""
    layer = Layer(gpu, type_id, 256, 256, 4, 2, seed=4400 + type_id, router=False,
                  activation=1 if type_id == H.MX else 0, order=gpu.ORDER_FAST)
    T = 300
    x = gpu.synth_normal(4400 + type_id, 6, 0, T * 256).reshape(T, 256)
    logits = gpu.synth_normal(4400 + type_id, 7, 0, T * 4).reshape(T, 4)
    out, ids, _ = layer.forward_gpu(x, logits)
    ref = layer.forward_cpu(orc, x, logits)
    assert np.array_equal(ids, ref["ids"])
    per_expert = np.bincount(ids.ravel(), minlength=4)
    assert per_expert.min() > 64, per_expert
    max_rel, cos = H.rel_err_and_cos(out, ref["out"])
    print(f"[prefill multi-tile type={type_id}] jobs {per_expert.tolist()} max_rel={max_rel:.3e} cos={cos:.9f}",
          flush=True)
    assert max_rel <= 1e-3 and cos >= 0.99999
    layer.destroy()


def test_gemm_mxfp4_exponent_ranges_exact(gpu, orc):
    """Row tiles whose block exponents sit inside the range folded into the f16 weight operand
    (e in [-14, 12]: bytes 114, 127, 140) and outside it (bytes 141 and 113, the ldexp path),
    mixed within one workgroup's tile pair; every fp32 sum stays an exact multiple of its block
    scale, so the result must match the oracle bit for bit."""
    rng = np.random.default_rng(73)
    experts, rows, k, n_ids, tokens = 4, 320, 512, 2, 48
    blk = unit_scale_mxfp4(experts, rows, k, rng).reshape(experts, rows, k // 32, 17)
    pattern = np.array([141, 127, 114, 140, 113], np.uint8)
    blk[:, :, :, 0] = pattern[(np.arange(rows) // 32) % len(pattern)][None, :, None]
    blk[:, 224:256, :, 0] = 140          # one out-of-range block inside an otherwise folded tile
    blk[:, 224:256, 3, 0] = 141          # (scales 2^12 and 2^13 keep every sum exact)
    w = blk.reshape(-1)
    bank = H.make_bank(H.MX, w, experts, rows, k)
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = unit_scale_activations(tokens, k, rng).reshape(tokens, 1, k)
    got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, n_ids, order=gpu.ORDER_FAST)
    ref = orc.mul_mat_id(H.MX, w, k, rows, experts, 0, x, 1, ids, n_ids, tokens, n_ids, threads=8)
    assert H.bits_equal(got, ref), H.diff_report(got, ref)
    bank.destroy()


def test_gemm_mul_mat_id_fast_within_tolerance_and_broadcast(gpu, orc):
    """Config 0/1 gate_up shape (5760 x 2880, interleaved) with biases, T = 96 (12 routed rows per
    expert: the grouped GEMM), broadcast and per-rank activations."""
    rng = np.random.default_rng(72)
    experts, k, rows, n_ids, tokens = 32, 2880, 5760, 4, 96
    w = H.synth_weights(H.MX, 72, 1, experts, rows, k)
    bank = H.make_bank(H.MX, w, experts, rows, k, True)
    bias = gpu.synth_normal(72, 3, 0, experts * rows, 0.0, 0.02)
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(tokens)]).astype(np.int32)
    for b_ne1 in (1, n_ids):
        x = gpu.synth_normal(72, 4 + b_ne1, 0, tokens * b_ne1 * k).reshape(tokens, b_ne1, k)
        got = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, b_ne1, ids, n_ids, bias=bias, order=gpu.ORDER_FAST)
        ref = orc.mul_mat_id(39, w, k, rows, experts, 0, x, b_ne1, ids, n_ids, tokens, n_ids, bias=bias, threads=8)
        max_rel, cos = H.rel_err_and_cos(got, ref)
        print(f"[gemm gate_up b_ne1={b_ne1}] max_rel={max_rel:.3e} cos={cos:.9f}", flush=True)
        assert max_rel <= 1e-3 and cos >= 0.99999
    bank.destroy()


def test_prefill_layer_q8_0_config3_shape(gpu, orc):
    """Config 3 shape (hidden 2048, 128 experts, top-8, intermediate 768, Q8_0, SiLU, no biases)
    at T = 256 tokens through the fused layer in the fast order."""
    layer = Layer(gpu, H.Q8, 2048, 768, 128, 8, seed=303, router=False, biases=False, activation=0,
                  order=gpu.ORDER_FAST)
    T = 256
    x = gpu.synth_normal(303, 6, 0, T * 2048).reshape(T, 2048)
    logits = gpu.synth_normal(303, 7, 0, T * 128).reshape(T, 128)
    out, ids, w = layer.forward_gpu(x, logits)
    ref = layer.forward_cpu(orc, x, logits)
    assert np.array_equal(ids, ref["ids"])
    max_rel, cos = H.rel_err_and_cos(out, ref["out"])
    print(f"[prefill config3 T={T}] max_rel={max_rel:.3e} cos={cos:.9f}", flush=True)
    assert max_rel <= 1e-3 and cos >= 0.99999
    layer.destroy()


def test_prefill_layer_q8_0_config3_full_2048_tokens(gpu, orc):
    """Config 3 at its own size: 2048 tokens, hidden 2048, 128 experts top-8, intermediate 768,
    Q8_0, SiLU, no biases, fast order (about 128 jobs per expert, so most experts span two or three
    64-job tiles of the grouped GEMM). Ids exact; max |out - ref| / max |ref| <= 1e-3 and cosine
    >= 0.99999 against the oracle's layer."""
    layer = Layer(gpu, H.Q8, 2048, 768, 128, 8, seed=3030, router=False, biases=False, activation=0,
                  order=gpu.ORDER_FAST)
    T = 2048
    x = gpu.synth_normal(3030, 6, 0, T * 2048).reshape(T, 2048)
    logits = gpu.synth_normal(3030, 7, 0, T * 128).reshape(T, 128)
    out, ids, _ = layer.forward_gpu(x, logits)
    ref = layer.forward_cpu(orc, x, logits, threads=16)
    assert np.array_equal(ids, ref["ids"])
    per_expert = np.bincount(ids.ravel(), minlength=128)
    max_rel, cos = H.rel_err_and_cos(out, ref["out"])
    print(f"[prefill config3 T={T}] jobs per expert {per_expert.min()}..{per_expert.max()} "
          f"max_rel={max_rel:.3e} cos={cos:.9f}", flush=True)
    assert per_expert.max() > 128
    assert max_rel <= 1e-3 and cos >= 0.99999
    layer.destroy()


def test_prefill_layer_graph_replays_match_eager(gpu):
    """The fast-order layer (top-k, grouping, both grouped GEMMs, combine) captured as one HIP
    graph: every replay gives the eager call's ids and output bits, with the output cleared before
    it and an eager layer call on other inputs through the same workspace after it."""
    layer = Layer(gpu, H.Q8, 2048, 768, 128, 8, seed=3131, router=False, biases=False, activation=0,
                  order=gpu.ORDER_FAST)
    T, Hd, K = 512, 2048, 8
    x = gpu.synth_normal(3131, 6, 0, T * Hd).reshape(T, Hd)
    logits = gpu.synth_normal(3131, 7, 0, T * 128).reshape(T, 128)
    ref, ref_ids, _ = layer.forward_gpu(x, logits)
    d = layer.desc()
    ws = C.c_size_t()
    gpu.call("vbm_moe_layer_workspace", C.byref(d), T, C.byref(ws))
    work = gpu.DeviceBuffer(ws.value)
    dx, dl = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(logits)
    dx2 = gpu.DeviceBuffer.from_array(gpu.synth_normal(3131, 8, 0, T * Hd))
    dl2 = gpu.DeviceBuffer.from_array(gpu.synth_normal(3131, 9, 0, T * 128))
    out, ids, out2 = gpu.DeviceBuffer(4 * T * Hd), gpu.DeviceBuffer(4 * T * K), gpu.DeviceBuffer(4 * T * Hd)
    stream = C.c_void_p()
    gpu.call("vbm_stream_create", C.byref(stream))
    s = stream.value
    g = C.c_void_p()
    gpu.call("vbm_graph_begin_capture", s)
    gpu.call("vbm_moe_layer_forward", C.byref(d), dx.ptr, dl.ptr, T, out.ptr, ids.ptr, None, work.ptr, ws.value, s)
    gpu.call("vbm_graph_end_capture", s, C.byref(g))
    try:
        for rep in range(3):
            gpu.call("vbm_memset", out.ptr, 0, 4 * T * Hd, s)
            gpu.call("vbm_graph_launch", g.value, s)
            gpu.call("vbm_stream_synchronize", s)
            print(f"[prefill graph replay {rep}]", flush=True)
            assert np.array_equal(ids.download(np.int32, (T, K)), ref_ids)
            got = out.download(np.float32, (T, Hd))
            assert H.bits_equal(got, ref), H.diff_report(got, ref)
            gpu.call("vbm_moe_layer_forward", C.byref(d), dx2.ptr, dl2.ptr, T, out2.ptr, None, None, work.ptr,
                     ws.value, s)
            gpu.call("vbm_stream_synchronize", s)
    finally:
        gpu.call("vbm_graph_destroy", g.value)
        gpu.call("vbm_stream_destroy", s)
        layer.destroy()


def test_prefill_layer_mxfp4_config1_shape(gpu, orc):
    """Config 1 layer (MXFP4, 32 experts, top-4, 2880, SwiGLU-OAI, biases) at T = 96 (12 routed rows
    per expert, the grouped GEMM's threshold), fast order."""
    layer = Layer(gpu, H.MX, 2880, 2880, 32, 4, seed=78, order=gpu.ORDER_FAST)
    T = 96
    x = gpu.synth_normal(78, 6, 0, T * 2880).reshape(T, 2880)
    out, ids, w = layer.forward_gpu(x)
    ref = layer.forward_cpu(orc, x)
    assert np.array_equal(ids, ref["ids"])
    max_rel, cos = H.rel_err_and_cos(out, ref["out"])
    print(f"[prefill config1 T={T}] max_rel={max_rel:.3e} cos={cos:.9f}", flush=True)
    assert max_rel <= 1e-3 and cos >= 0.99999
    layer.destroy()


@pytest.mark.parametrize("experts,tokens", [(128, 32), (32, 24), (32, 64)])
def test_fast_order_small_groups_take_the_exact_gemv(gpu, orc, experts, tokens):
    """Below 12 routed rows per expert on average a fast-order call runs the exact-order GEMV
    (faster there than the grouped GEMM): the layer output is bit-identical to the exact order's
    and to the oracle's."""
    assert tokens * 4 < 12 * experts and tokens >= 16
    fast = Layer(gpu, H.MX, 2880, 2880, experts, 4, seed=91, router=False, order=gpu.ORDER_FAST)
    x = gpu.synth_normal(91, 6, 0, tokens * 2880).reshape(tokens, 2880)
    logits = gpu.synth_normal(91, 7, 0, tokens * experts).reshape(tokens, experts)
    out, ids, _ = fast.forward_gpu(x, logits)
    fast.order = gpu.ORDER_EXACT
    exact, ids_e, _ = fast.forward_gpu(x, logits)
    ref = fast.forward_cpu(orc, x, logits)
    assert np.array_equal(ids, ids_e) and np.array_equal(ids, ref["ids"])
    assert np.array_equal(out.view(np.uint32), exact.view(np.uint32))
    assert np.array_equal(out.view(np.uint32), ref["out"].view(np.uint32)), H.diff_report(out, ref["out"])
    fast.destroy()


def test_gemm_randomized_shapes_within_tolerance(gpu, orc):
    """8 seeded random fast-order MUL_MAT_ID calls large enough for the MFMA grouped GEMM
    (>= 16 tokens, 12..200 routed rows per expert on average): both weight types, 2..16 experts, top-1..4,
    rows 64..320, k 64..1024, fp32 or ggml Q8_0 (with -128 codes) inputs, with or without biases,
    against the oracle within the fast order's tolerance (max error / max |ref| <= 1e-3, cosine >=
    0.99999)."""
    rng = np.random.default_rng(6060)
    for case in range(8):
        type_id = H.MX if case % 2 == 0 else H.Q8
        experts = int(rng.integers(2, 17))
        active = int(rng.integers(1, min(4, experts) + 1))
        # 12..200 routed jobs per expert on average: one or two 128-job tiles per expert
        tokens = max(16, -(-int(rng.integers(12, 201)) * experts // active))
        rows, k = 64 * int(rng.integers(1, 6)), 64 * int(rng.integers(1, 17))
        q8_input = rng.random() < 0.4
        ids = np.stack([rng.choice(experts, active, replace=False) for _ in range(tokens)]).astype(np.int32)
        w = H.synth_weights(type_id, 900 + case, 1, experts, rows, k)
        bank = H.make_bank(type_id, w, experts, rows, k)
        bias = gpu.synth_normal(900 + case, 2, 0, experts * rows, 0.0, 0.02) if rng.random() < 0.5 else None
        x = gpu.synth_normal(900 + case, 3, 0, tokens * k).reshape(tokens, 1, k)
        label = (f"case {case}: type={type_id} experts={experts} top{active} tokens={tokens} rows={rows} k={k} "
                 f"q8={q8_input} bias={bias is not None}")
        print(f"[random gemm] {label}", flush=True)
        if q8_input:
            q = orc.quantize_q8_0(x.reshape(tokens, k)).reshape(-1, 34)
            q[rng.random(q.shape[0]) < 0.25, 2 + int(rng.integers(0, 32))] = 128
            b, b_type, orc_type = q.reshape(tokens, 1, -1), gpu.TYPE_Q8_0, 8
        else:
            b, b_type, orc_type = x, gpu.TYPE_F32, 0
        got = H.mul_mat_id(bank, experts, b, b_type, 1, ids, active, bias=bias, order=gpu.ORDER_FAST)
        ref = orc.mul_mat_id(type_id, w, k, rows, experts, orc_type, b, 1, ids, active, tokens, active, bias=bias)
        max_rel, cos = H.rel_err_and_cos(got, ref)
        assert max_rel <= 1e-3 and cos >= 0.99999, f"{label}: max_rel={max_rel:.3e} cos={cos:.9f}"
        bank.destroy()


@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
def test_prefill_layer_unmapped_expert_poisons_its_tokens(gpu, type_id):
    """Fast-order layer on the grouped GEMMs with one expert mapped to no slot: its workgroups
    poison their GLU blocks and down rows, so exactly the tokens routed to it come out NaN after
    the rank-ordered combine, every other token is bit-identical to the run with every expert
    mapped, and repeated calls through the same workspace give the same bits."""
    E, K, Hd, I, T = 8, 2, 256, 256, 256
    layer = Layer(gpu, type_id, Hd, I, E, K, seed=5150 + type_id, router=False,
                  activation=1 if type_id == H.MX else 0, order=gpu.ORDER_FAST)
    x = gpu.synth_normal(5150 + type_id, 6, 0, T * Hd).reshape(T, Hd)
    logits = gpu.synth_normal(5150 + type_id, 7, 0, T * E).reshape(T, E)
    full, ids, _ = layer.forward_gpu(x, logits)
    assert np.all(np.isfinite(full))
    again, _, _ = layer.forward_gpu(x, logits)
    assert H.bits_equal(again, full)
    dead = 3
    slot_map = np.arange(E, dtype=np.int32)
    slot_map[dead] = -1
    dmap = gpu.DeviceBuffer.from_array(slot_map)
    d = layer.desc()
    d.expert_to_slot = dmap.ptr
    ws = C.c_size_t()
    gpu.call("vbm_moe_layer_workspace", C.byref(d), T, C.byref(ws))
    work = gpu.DeviceBuffer(ws.value)
    dx, dl = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(logits)
    out = gpu.DeviceBuffer(4 * T * Hd)
    for rep in range(2):
        gpu.call("vbm_memset", out.ptr, 0, 4 * T * Hd, None)
        gpu.call("vbm_moe_layer_forward", C.byref(d), dx.ptr, dl.ptr, T, out.ptr, None, None, work.ptr, ws.value, None)
        gpu.call("vbm_stream_synchronize", None)
        got = out.download(np.float32, (T, Hd))
        hit = np.any(ids == dead, axis=1)
        print(f"[prefill unmapped expert type={type_id} rep={rep}] tokens on expert {dead}: {int(hit.sum())}", flush=True)
        assert 0 < hit.sum() < T
        assert np.all(np.isnan(got[hit]))
        assert H.bits_equal(got[~hit], full[~hit]), H.diff_report(got[~hit], full[~hit])
    layer.destroy()
