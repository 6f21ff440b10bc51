"""Pins the CPU oracle (oracle/vbm_oracle.c) before it is trusted as the GPU path's checker.

Each check is chosen so that a plausible restatement mistake (lane map, nibble order, VPSIGNB
corner, e8m0 subnormal encoding, reduction tree, rounding mode, grouping order) fails it:
  - the reference's own compiled restatement tools/trace/cpu_mxfp4_vnni.cpp (oracle/_ref) on the
    vector recipe of tests/test_cpu_research.py:27-46 (seed 4217, adversarial exponents/scales);
  - brute-force integer dots in int64 and float64 dequantization;
  - closed forms (e8m0 = 2^(e-128), fp16 RNE = numpy float16, Q8_0 ties, softmax, SwiGLU clamps);
  - known answers of tests/test_expert_dispatch.cpp:65-73 (reduction order) and the reference's
    own dispatch test compiled against this repository's ExpertPlan.
"""
import ctypes as C
import math
import random
import struct
import subprocess

import numpy as np
import pytest

MX_TABLE = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], dtype=np.int64)


def cpu_has_avx512vnni() -> bool:
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    return "avx512_vnni" in flags and "avx512vl" in flags


def mx_values(block: bytes) -> np.ndarray:
    qs = np.frombuffer(block[1:17], dtype=np.uint8)
    nib = np.concatenate([qs & 15, qs >> 4])
    return MX_TABLE[nib]


def contract_lanes(w: np.ndarray, a: np.ndarray) -> np.ndarray:
    """|w| * VPSIGNB(a, w) summed per 4-element lane (independent numpy form)."""
    a = a.astype(np.int64)
    signed = np.where(w > 0, a, np.where(w == 0, 0, np.where(a == -128, -128, -a)))
    return (np.abs(w) * signed).reshape(8, 4).sum(axis=1)


# ---------------------------------------------------------------------------------- fp16 / e8m0
def test_fp16_conversions_match_ieee(orc):
    lib = orc.load()
    halves = np.arange(65536, dtype=np.uint16)
    ref = halves.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_fp16_to_fp32(int(h)) for h in halves[::7]], dtype=np.float32)
    sel = ref[::7]
    finite = np.isfinite(sel)
    assert np.array_equal(got[finite].view(np.uint32), sel[finite].view(np.uint32))
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 5, 4000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.9802322e-08, 1.0009766,
                  2049.0, 2051.0, -3.0517578e-05], dtype=np.float32)])
    with np.errstate(over="ignore"):                     # 65520 and the 1e4-scaled draws round to inf
        expected = vals.astype(np.float16).view(np.uint16)
    got = np.array([lib.orc_fp32_to_fp16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, expected)


def test_e8m0_half_is_power_of_two(orc):
    lib = orc.load()
    for e in range(255):
        assert lib.orc_e8m0_half(e) == math.ldexp(1.0, e - 128), e
    # encoding of the two subnormal cases (quantized_cuda.cu:161): 0x00200000 << e
    assert struct.pack("<f", lib.orc_e8m0_half(0)) == struct.pack("<I", 0x00200000)
    assert struct.pack("<f", lib.orc_e8m0_half(1)) == struct.pack("<I", 0x00400000)


# ---------------------------------------------------------------------------------- MXFP4 dot
def research_vectors(width: int, sample: int, rng: random.Random):
    """tests/test_cpu_research.py:30-38 recipe."""
    weights, activation = bytearray(), bytearray()
    for _ in range(width // 32):
        weights += bytes([rng.choice([0, 1, 2, 110, 120, 126, 127, 128, 130])])
        weights += rng.randbytes(16)
        scale = rng.choice([0, 1, 0x0400, 0x1000, 0x3C00, 0x3C01, 0x5000, 0x8000])
        activation += struct.pack("<H", scale)
        activation += bytes(rng.randrange(256) for _ in range(32)) if sample else bytes(32)
    return bytes(weights), bytes(activation)


@pytest.mark.skipif(not cpu_has_avx512vnni(), reason="oracle/_ref VNNI restatement needs AVX512VL+VNNI")
def test_mxfp4_dot_matches_reference_restatement_bits(orc):
    if not orc.REF_VNNI.exists():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    ref = C.CDLL(str(orc.REF_VNNI))
    fn = ref.ggml_vec_dot_mxfp4_q8_0
    fn.argtypes = [C.c_int, C.POINTER(C.c_float), C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_int]
    fn.restype = None
    lib = orc.load()
    rng = random.Random(4217)
    compared = 0
    for width in (64, 128, 2880):
        for sample in range(80):
            w, a = research_vectors(width, sample, rng)
            x, y = C.create_string_buffer(w), C.create_string_buffer(a)
            out = C.c_float()
            fn(width, C.byref(out), 0, x, 0, y, 0, 1)
            mine = lib.orc_vec_dot_mxfp4_q8_0(width, x, y)
            assert struct.pack("<f", mine) == struct.pack("<f", out.value), (width, sample)
            compared += 1
    assert compared == 240


def test_repacked_8x8_contract_equals_standard_bits(orc):
    """Row a8. The reference's own tests/test_exact_packed_cpu.cpp:55-85 asserts that the repacked
    8x8 GEMV (tools/trace/exact_packed_cpu.h:52-88) reproduces ggml_vec_dot_mxfp4_q8_0 bit for bit;
    the same recipe here (n in {64, 256, 2880}, 8/16/64 rows, exponents 96 + r % 40 with rows 0/1
    at exponents 0/1, Q8_0 activations of U(-8, 8) with one code -128) checks the oracle's
    restatement of the repacked layout and tile against the reference's standard contract compiled
    from cpu_mxfp4_vnni.cpp (oracle/_ref), or against the oracle's restatement of it when the
    reference sources are absent. A lane-map, chunk or tree mistake in the repacked restatement
    changes bits here."""
    lib = orc.load()
    native = None
    if orc.REF_VNNI.exists():
        ref = C.CDLL(str(orc.REF_VNNI))
        native = ref.ggml_vec_dot_mxfp4_q8_0
        native.argtypes = [C.c_int, C.POINTER(C.c_float), C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p,
                           C.c_size_t, C.c_int]
        native.restype = None
    rng = np.random.default_rng(417)
    checks = 0
    for n in (64, 256, 2880):
        blocks = n // 32
        for columns in (8, 16, 64):
            w = np.zeros((columns, blocks, 17), np.uint8)
            w[:, :, 0] = 96 + rng.integers(0, 40, (columns, blocks))
            w[:, :, 1:] = rng.integers(0, 256, (columns, blocks, 16))
            w[0, 0, 0], w[0, 1, 0] = 0, 1
            x = rng.uniform(-8, 8, n).astype(np.float32)
            act = orc.quantize_q8_0(x.reshape(1, n)).reshape(-1).copy()
            act[2] = 0x80                                       # activations[0].qs[0] = -128
            packed = orc.pack_mxfp4x8(w.reshape(-1), columns, blocks)
            actual = orc.gemv_mxfp4x8(packed, act, n, columns)
            expected = np.empty(columns, np.float32)
            for c in range(columns):
                row = np.ascontiguousarray(w[c].reshape(-1))
                if native is not None:
                    out = C.c_float()
                    native(n, C.byref(out), 0, row.ctypes.data, 0, act.ctypes.data, 0, 1)
                    expected[c] = out.value
                else:
                    expected[c] = lib.orc_vec_dot_mxfp4_q8_0(n, row.ctypes.data, act.ctypes.data)
            assert expected.tobytes() == actual.tobytes(), (n, columns)
            checks += 1
    assert checks == 9


def test_repacked_layout_round_trip_and_shapes(orc):
    """orc_unpack_mxfp4x8 restates the expert export of HP:751-762; packing then exporting is the
    identity on raw block_mxfp4 rows, and the GEMV rejects what exact_packed_cpu.h:80 rejects."""
    rng = np.random.default_rng(5)
    raw = rng.integers(0, 256, 24 * 7 * 17).astype(np.uint8)
    packed = orc.pack_mxfp4x8(raw, 24, 7)
    assert packed.size == 3 * 7 * 136
    assert np.array_equal(orc.unpack_mxfp4x8(packed, 24, 7), raw)
    group = packed[:136]                                    # rows 0..7, block 0
    assert list(group[:8]) == [raw[r * 7 * 17] for r in range(8)]
    assert bytes(group[8 + (1 * 8 + 3) * 8: 8 + (1 * 8 + 3) * 8 + 8]) == bytes(raw[3 * 7 * 17 + 1 + 8: 3 * 7 * 17 + 17])
    act = np.zeros(2 * 34, np.uint8)
    for n, rows in ((32, 8), (64, 12)):
        with pytest.raises(ValueError):
            orc.gemv_mxfp4x8(np.zeros(136 * 4, np.uint8), act, n, rows)


def test_mxfp4_block_lanes_brute_force(orc):
    lib = orc.load()
    rng = np.random.default_rng(5)
    lanes = np.zeros(8, np.int32)
    for trial in range(400):
        blk = bytes([int(rng.integers(0, 256))]) + rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
        act = rng.integers(-128, 128, 32).astype(np.int8)
        if trial % 3 == 0:
            act[rng.integers(0, 32, 4)] = -128          # VPSIGNB corner (test_quantized_cuda.cpp:36-38)
        y = b"\x00\x3c" + act.tobytes()
        total = lib.orc_mxfp4_block_lanes(blk, y, lanes.ctypes.data)
        expected = contract_lanes(mx_values(blk), act)
        assert np.array_equal(lanes, expected), trial
        assert total == expected.sum()
        if not (act == -128).any():   # without -128 the contract is the true product
            assert total == int((mx_values(blk) * act.astype(np.int64)).sum())


def test_mxfp4_dot_float64_bound(orc):
    """The fp32 dot equals the exact float64 sum up to fp32 accumulation error."""
    lib = orc.load()
    rng = np.random.default_rng(11)
    for _ in range(50):
        nb = 90
        w = bytearray()
        exact = 0.0
        act = bytearray()
        for b in range(nb):
            e = int(rng.integers(119, 125))
            blk = bytes([e]) + rng.integers(0, 256, 16, dtype=np.uint8).tobytes()
            q = rng.integers(-127, 128, 32).astype(np.int8)
            d = np.float16(rng.uniform(1e-3, 1e-2))
            w += blk
            act += d.tobytes() + q.tobytes()
            exact += float(d) * math.ldexp(1.0, e - 128) * float((mx_values(blk) * q.astype(np.int64)).sum())
        got = lib.orc_vec_dot_mxfp4_q8_0(nb * 32, bytes(w), bytes(act))
        assert abs(got - exact) <= 1e-5 * max(1.0, abs(exact))


# ---------------------------------------------------------------------------------- Q8_0
def test_q8_block_lanes_brute_force(orc):
    lib = orc.load()
    rng = np.random.default_rng(6)
    lanes = np.zeros(8, np.int32)
    for _ in range(300):
        w = rng.integers(-127, 128, 32).astype(np.int8)
        a = rng.integers(-127, 128, 32).astype(np.int8)
        total = lib.orc_q8_block_lanes(b"\0\0" + w.tobytes(), b"\0\0" + a.tobytes(), lanes.ctypes.data)
        prod = (w.astype(np.int64) * a.astype(np.int64)).reshape(8, 4).sum(axis=1)
        assert np.array_equal(lanes, prod)
        assert total == prod.sum()


@pytest.mark.skipif(not cpu_has_avx512vnni(), reason="oracle/_ref VNNI restatement needs AVX512VL+VNNI")
def test_q8_0_dot_lane_arithmetic_equals_reference_mxfp4_restatement(orc):
    """The Q8_0 x Q8_0 dot's per-lane arithmetic (block scale product, int -> fp32, FMA into the
    lane) and final hsum8 tree against the reference's compiled MXFP4 restatement
    (cpu_mxfp4_vnni.cpp:49-68): Q8_0 weights that hold the doubled e2m1 integers of an MXFP4 block
    with scale 2^(e-128) (an exact fp16), and zero weights in the odd blocks (so the MXFP4 odd chain
    adds exact zeros), make both dots the same arithmetic, so the results must agree bit for bit.
    This does NOT pin the chain structure across blocks: with every odd block zero, one FMA chain
    per lane and the MXFP4 dot's even/odd chains give the same bits. The structure the oracle uses
    (one chain per lane, upstream AVX2 ggml_vec_dot_q8_0_q8_0) is parity-unpinned: upstream ggml is
    not in the reference; the float64 bound test below checks its arithmetic."""
    if not orc.REF_VNNI.exists():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    ref = C.CDLL(str(orc.REF_VNNI))
    fn = ref.ggml_vec_dot_mxfp4_q8_0
    fn.argtypes = [C.c_int, C.POINTER(C.c_float), C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_int]
    fn.restype = None
    lib = orc.load()
    rng = np.random.default_rng(2880)
    for n in (64, 640, 2880):
        for _ in range(40):
            mx, q8, act = b"", b"", b""
            for b in range(n // 32):
                e = int(rng.integers(114, 144)) if b % 2 == 0 else int(rng.integers(0, 256))
                qs = rng.integers(0, 256, 16).astype(np.uint8) if b % 2 == 0 else np.zeros(16, np.uint8)
                blk = bytes([e]) + qs.tobytes()
                mx += blk
                d = np.float16(math.ldexp(1.0, e - 128)) if b % 2 == 0 else np.float16(1.0)
                q8 += d.tobytes() + mx_values(blk).astype(np.int8).tobytes()
                da = np.float16(rng.uniform(1e-3, 1e-1))
                act += da.tobytes() + rng.integers(-127, 128, 32).astype(np.int8).tobytes()
            out = C.c_float()
            fn(n, C.byref(out), 0, C.create_string_buffer(mx), 0, C.create_string_buffer(act), 0, 1)
            mine = lib.orc_vec_dot_q8_0_q8_0(n, q8, act)
            assert struct.pack("<f", mine) == struct.pack("<f", out.value), n


@pytest.mark.parametrize("y_entries,expected,ruled_out", [
    # accumulators reduce as (s0 + s2) + (s1 + s3): big + (-big) first, then + 1
    ({0: 2.0 ** 25, 8: 1.0, 16: -(2.0 ** 25)}, 1.0, "sequential"),
    # the 4-wide horizontal adds: (t0 + t1) + (t2 + t3), each pair rounding 2^25 + 1 to 2^25
    ({0: 2.0 ** 25, 1: 1.0, 2: -(2.0 ** 25), 3: 1.0}, 0.0, "sequential"),
    # the 256-bit fold lo + hi comes first: (2^25 + 1) rounds before -2^25 joins
    ({0: 2.0 ** 25, 4: 1.0, 1: -(2.0 ** 25)}, 0.0, "sequential"),
    # one fp32 FMA chain per lane across 32-element steps (no wider accumulator)
    ({0: 2.0 ** 25, 32: 1.0, 64: -(2.0 ** 25)}, 0.0, "exact"),
])
def test_f32_dot_reduction_order_probes(orc, y_entries, expected, ruled_out):
    """ggml_vec_dot_f32 with GGML_SIMD on AVX2 (upstream ggml, not vendored: four 8-wide FMA
    accumulators, GGML_F32x8_REDUCE, then (lo128 + hi128) and two hadds): each probe's answer,
    derived by hand from that order, differs from a sequential fp32 sum or from the exact sum
    (2^25 has an fp32 spacing of 4)."""
    n = 96
    x = np.ones(n, np.float32)
    y = np.zeros(n, np.float32)
    for i, v in y_entries.items():
        y[i] = v
    got = orc.load().orc_vec_dot_f32(n, x.ctypes.data, y.ctypes.data)
    assert got == expected
    if ruled_out == "sequential":
        seq = np.float32(0.0)
        for v in y:
            seq = np.float32(seq + v)
        assert seq != expected
    else:
        assert float(np.sum(y.astype(np.float64))) != expected


def test_quantize_q8_0_closed_forms(orc):
    # q8-ties pattern of tools/trace/hybrid_layer.cpp:599-601: amax = 127 so codes are RNE(x).
    n = 32 * 6
    for sample in range(3):
        i = np.arange(n)
        x = np.where(i % 32 == 0, 127.0, np.where(i % 32 == 1, -127.0,
                     np.where(i % 2 == 1, -1.0, 1.0) * (0.5 + ((i + 7 * sample) % 31)))).astype(np.float32)
        q = orc.quantize_q8_0(x)[0].reshape(-1, 34)
        assert (q[:, :2].copy().view(np.uint16) == np.float16(1.0).view(np.uint16)).all()
        codes = q[:, 2:].view(np.int8).reshape(-1)
        assert np.array_equal(codes, np.rint(x).astype(np.int8))      # numpy rint = half to even
    zero = orc.quantize_q8_0(np.zeros(64, np.float32))[0]
    assert not zero.any()
    # Random rows: scale = fp16(amax/127) and codes = RNE(x * (127/amax)) in float32.
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 40) * 10.0 ** rng.integers(-3, 3, 32 * 40)).astype(np.float32)
    q = orc.quantize_q8_0(x)[0].reshape(-1, 34)
    for b in range(40):
        v = x[b * 32:(b + 1) * 32]
        amax = np.float32(np.abs(v).max())
        assert q[b, :2].copy().view(np.uint16)[0] == np.float16(amax / np.float32(127)).view(np.uint16)
        idv = np.float32(127) / amax
        assert np.array_equal(q[b, 2:].view(np.int8), np.rint(v * idv).astype(np.int8))
    # Idempotence: requantizing the dequantized row returns the same bytes.
    deq = (q[:, 2:].view(np.int8).astype(np.float32) * q[:, :2].copy().view(np.float16).astype(np.float32)).reshape(-1)
    assert np.array_equal(orc.quantize_q8_0(deq)[0].reshape(-1, 34), q)


# ---------------------------------------------------------------------------------- routing
def test_topk_canonical_order(orc):
    lib = orc.load()
    rng = np.random.default_rng(9)
    cases = [np.arange(32, 0, -1, dtype=np.float32), (np.arange(128) < 4).astype(np.float32),
             np.array([(c * 37 + 17) % 31 for c in range(128)], dtype=np.float32),
             np.zeros(64, np.float32), rng.standard_normal(128).astype(np.float32)]
    for logits in cases:
        for k in (1, 2, 4, 8):
            out = np.empty(k, np.int32)
            lib.orc_topk(logits.ctypes.data, len(logits), k, out.ctypes.data)
            expected = np.lexsort((np.arange(len(logits)), -logits))[:k]
            assert np.array_equal(out, expected)


def test_softmax_selected_closed_form(orc):
    rng = np.random.default_rng(4)
    for k in (1, 4, 8):
        v = rng.standard_normal(k).astype(np.float32) * 3
        out = np.empty(k, np.float32)
        orc.load().orc_softmax_selected(v.ctypes.data, k, out.ctypes.data)
        e = np.exp((v - v.max()).astype(np.float64))          # ggml subtracts the max in float32
        assert np.allclose(out, e / e.sum(), rtol=3e-7, atol=0)
        assert abs(float(out.astype(np.float64).sum()) - 1.0) < 1e-6


def test_grouping_is_stable_counting_sort(orc):
    rng = np.random.default_rng(2)
    for experts, active, tokens in [(4, 1, 1), (7, 3, 3), (8, 8, 2), (16, 4, 64), (128, 8, 300), (32, 4, 1)]:
        ids = np.array([[(t + r * 3) % experts for r in range(active)] for t in range(tokens)], np.int32)
        if tokens > 3:
            ids = rng.integers(0, experts, (tokens, active)).astype(np.int32)
            ids[rng.random((tokens, active)) < 0.1] = -1
        counts, offsets, rows = orc.group_by_expert(ids, active, tokens, active, experts)
        flat = ids.reshape(-1)
        valid = np.nonzero(flat >= 0)[0]
        expected = valid[np.argsort(flat[valid], kind="stable")]
        assert np.array_equal(rows, expected)
        assert np.array_equal(counts, np.bincount(flat[valid], minlength=experts))
        assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    with pytest.raises(ValueError):
        orc.group_by_expert(np.array([[5]], np.int32), 1, 1, 1, 4)


# ---------------------------------------------------------------------------------- GLU, combine
def test_swiglu_oai_and_silu_closed_forms(orc):
    g = np.array([9.0, 7.0, 0.0, -3.0, 1.5, -20.0, 6.99], np.float32)
    u = np.array([-9.0, 8.0, 2.0, 0.5, -7.5, 3.0, 7.01], np.float32)
    out = np.empty_like(g)
    orc.load().orc_glu(1, g.ctypes.data, u.ctypes.data, out.ctypes.data, len(g), 1.702, 7.0)
    gc, uc = np.minimum(g, 7).astype(np.float64), np.clip(u, -7, 7).astype(np.float64)
    ref = gc / (1 + np.exp(-1.702 * gc)) * (uc + 1)
    assert np.allclose(out, ref, rtol=2e-6, atol=1e-7)
    assert out[2] == 0.0 and out[0] == out[0]
    orc.load().orc_glu(0, g.ctypes.data, u.ctypes.data, out.ctypes.data, len(g), 1.702, 7.0)
    gd = g.astype(np.float64)
    assert np.allclose(out, gd / (1 + np.exp(-gd)) * u, rtol=2e-6, atol=1e-7)


def test_combine_reduction_order(orc):
    # tests/test_expert_dispatch.cpp:65-73: (1e20 + -1e20) + 1 == 1 only in rank order.
    y = np.array([1e20, -1e20, 1.0], np.float32).reshape(1, 3, 1)
    w = np.ones((1, 3), np.float32)
    out = np.empty((1, 1), np.float32)
    orc.load().orc_weighted_combine(y.ctypes.data, w.ctypes.data, 1, 3, 1, out.ctypes.data)
    assert out[0, 0] == 1.0


# ---------------------------------------------------------------------------------- mul_mat_id
def test_mul_mat_id_masks_and_matches_float64(orc, vb):
    k, rows, experts = 256, 32, 8
    nb = k // 32
    w = vb.synth_mxfp4(42, 1, 0, experts * rows * nb)
    tokens, active = 3, 4
    x = vb.synth_normal(42, 2, 0, tokens * k).reshape(tokens, 1, k)
    ids = np.array([[(t + r * 3) % experts for r in range(active)] for t in range(tokens)], np.int32)
    ids[0, 1] = -1
    out = orc.mul_mat_id(39, w, k, rows, experts, 0, x, 1, ids, active, tokens, active)
    assert not out[0, 1].any()
    q = orc.quantize_q8_0(x.reshape(tokens, k))
    wb = w.reshape(experts, rows, nb, 17)
    for t in range(tokens):
        qa = q[t].reshape(nb, 34)
        a = qa[:, 2:].view(np.int8).astype(np.float64)
        da = qa[:, :2].copy().view(np.float16).astype(np.float64).reshape(-1)
        for r in range(active):
            e = ids[t, r]
            if e < 0:
                continue
            for i in range(rows):
                exact = 0.0
                for b in range(nb):
                    blk = bytes(wb[e, i, b])
                    exact += da[b] * math.ldexp(1.0, blk[0] - 128) * float((mx_values(blk) * a[b]).sum())
                assert abs(out[t, r, i] - exact) <= 1e-5 * max(1.0, abs(exact))
    # The multithreaded fast path is bit-identical to the scalar path.
    fast = orc.mul_mat_id(39, w, k, rows, experts, 0, x, 1, ids, active, tokens, active, threads=4)
    assert np.array_equal(fast.view(np.uint32), out.view(np.uint32))


def test_q8_mul_mat_id_fast_equals_scalar(orc, vb):
    k, rows, experts = 768, 64, 4
    w = vb.synth_q8_0(5, 3, 0, experts * rows * (k // 32))
    x = vb.synth_normal(5, 4, 0, 2 * k).reshape(2, 1, k)
    ids = np.array([[0, 3], [2, 1]], np.int32)
    a = orc.mul_mat_id(8, w, k, rows, experts, 0, x, 1, ids, 2, 2, 2)
    b = orc.mul_mat_id(8, w, k, rows, experts, 0, x, 1, ids, 2, 2, 2, threads=3)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---------------------------------------------------------------------------------- dispatch
def test_reference_dispatch_test_passes_against_expert_plan(orc):
    if not orc.REF_DISPATCH_TEST.exists():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    proc = subprocess.run([str(orc.REF_DISPATCH_TEST)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stderr
    assert "passed" in proc.stdout
    asan = orc.REF_DISPATCH_TEST.with_name("test_expert_dispatch_asan")
    if asan.exists():   # the same test with AddressSanitizer + UBSan over ExpertPlan
        proc = subprocess.run([str(asan)], capture_output=True, text=True, timeout=120,
                              env={"ASAN_OPTIONS": "detect_leaks=1", "UBSAN_OPTIONS": "halt_on_error=1"})
        assert proc.returncode == 0, proc.stderr
        assert "passed" in proc.stdout and "runtime error" not in proc.stderr


U32 = 2.0 ** -24


def gamma(n: int) -> float:
    """Higham's gamma_n = n u / (1 - n u) for fp32 (u = 2^-24): |computed - exact| <= gamma_n *
    sum |terms| for any sum of the terms evaluated with at most n roundings along each term's path."""
    return n * U32 / (1.0 - n * U32)


def test_q8_0_dot_within_float64_bound(orc):
    """orc_vec_dot_q8_0_q8_0 against the exact value sum_b fp16(dx_b) fp16(dy_b) sum_i x_i y_i'
    (float64; y_i' = the VPSIGNB-contract activation), within the rigorous bound of the oracle's
    structure: per block one rounding of the scale product, one FMA per block along each of the 8
    lane chains, then 3 tree levels, so every term meets at most nb + 4 roundings. A dropped block,
    a wrong sign or a transposed scale moves the result far outside it."""
    lib = orc.load()
    rng = np.random.default_rng(88)
    worst = 0.0
    for n in (64, 768, 2048, 2880):
        nb = n // 32
        for _ in range(30):
            w = np.empty((nb, 34), np.uint8)
            a = np.empty((nb, 34), np.uint8)
            w[:, :2] = np.float16(rng.uniform(1e-3, 1e-2, nb)).view(np.uint8).reshape(nb, 2)
            a[:, :2] = np.float16(rng.uniform(1e-3, 1e-1, nb)).view(np.uint8).reshape(nb, 2)
            wq = rng.integers(-128, 128, (nb, 32)).astype(np.int8)
            aq = rng.integers(-128, 128, (nb, 32)).astype(np.int8)
            w[:, 2:], a[:, 2:] = wq.view(np.uint8), aq.view(np.uint8)
            dw = w[:, :2].copy().view(np.float16).astype(np.float64).ravel()
            da = a[:, :2].copy().view(np.float16).astype(np.float64).ravel()
            # VPSIGNB contract: |w| (w = -128 reads as 128) times a negated where w < 0 (-128 stays)
            mag = np.where(wq == -128, 128, np.abs(wq.astype(np.int64)))
            neg = np.where(aq == -128, -128, -aq.astype(np.int64))
            signed = np.where(wq < 0, neg, np.where(wq == 0, 0, aq.astype(np.int64)))
            lanes = (mag * signed).reshape(nb, 8, 4).sum(axis=2)
            terms = (dw * da)[:, None] * lanes
            exact = float(terms.sum())
            got = lib.orc_vec_dot_q8_0_q8_0(n, w.ctypes.data, a.ctypes.data)
            bound = gamma(nb + 4) * float(np.abs(terms).sum())
            assert abs(got - exact) <= bound, (n, got, exact, bound)
            worst = max(worst, abs(got - exact) / bound)
    print(f"[q8 dot] worst error / bound = {worst:.3f}")


def test_f32_dot_within_float64_bound(orc):
    """orc_vec_dot_f32 (router logits) against the exact float64 dot, within the rigorous bound of
    its structure (an FMA chain of n/32 steps per accumulator, 5 reduction levels)."""
    lib = orc.load()
    rng = np.random.default_rng(89)
    for n in (32, 2048, 2880):
        for _ in range(50):
            x = rng.standard_normal(n).astype(np.float32)
            y = (rng.standard_normal(n) * 0.02).astype(np.float32)
            terms = x.astype(np.float64) * y.astype(np.float64)
            got = lib.orc_vec_dot_f32(n, x.ctypes.data, y.ctypes.data)
            bound = gamma(n // 32 + 5) * float(np.abs(terms).sum())
            assert abs(got - float(terms.sum())) <= bound, (n, got)


def router_near_ties(w, x, top_k):
    """Float64 router logits and, per token, whether its top-k (ids and order) is determined for
    every fp32 evaluation order: all gaps between consecutive logits among the top k + 1 exceed
    twice gamma_H * sum |w_ij x_j| (the largest error any fp32 summation order can make)."""
    prod = np.abs(w.astype(np.float64))[None, :, :] * np.abs(x.astype(np.float64))[:, None, :]
    bound = gamma(w.shape[1]) * prod.sum(axis=2)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    order = np.argsort(-exact, axis=1, kind="stable")
    top = np.take_along_axis(exact, order[:, : top_k + 1], axis=1)
    margin = 2 * bound.max(axis=1)
    determined = np.all(top[:, :-1] - top[:, 1:] > margin[:, None], axis=1)
    return order[:, :top_k].astype(np.int32), determined


@pytest.mark.parametrize("n_expert,hidden,top_k", [(32, 2880, 4), (128, 2880, 4), (128, 2048, 8)])
def test_router_ids_equal_float64_topk_where_determined(orc, n_expert, hidden, top_k):
    """The reference computes router logits with upstream ggml_mul_mat (build_lora_mm,
    llama-b11669-hybrid-experts.patch:1357-1385), whose fp32 order is parity-unpinned (upstream
    ggml is not in the reference). What the mathematics fixes: wherever the top-k + 1 float64
    logits are separated by more than twice the worst-case fp32 error of ANY summation order, every
    order, the reference's included, picks the float64 top-k; the oracle's ids must equal it there.
    Router weights N(0, 0.02) and hidden states N(0, 1) as in configs 0 and 1; the near-tie
    fraction (tokens whose ids the bound cannot fix) is reported."""
    rng = np.random.default_rng(90 + n_expert + top_k)
    tokens = 512
    w = (rng.standard_normal((n_expert, hidden)) * 0.02).astype(np.float32)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    _, ids, _ = orc.router(router_w=w, x=x, n_expert=n_expert, n_tokens=tokens, top_k=top_k, hidden=hidden)
    want, determined = router_near_ties(w, x, top_k)
    print(f"[router {n_expert}x{hidden} top{top_k}] near-tie fraction {1 - determined.mean():.4f}")
    assert determined.mean() > 0.5
    assert np.array_equal(ids[determined], want[determined])


def test_glu_bitwise_equals_reference_f32_experts(orc):
    """orc_glu against the reference executor's own activation stage (tools/engine/f32_experts.cpp:
    68-73, compiled in oracle/_ref with the host libm), bit for bit, for SwiGLU-OAI (alpha 1.702,
    limit 7: values on both sides of the clamps) and SiLU."""
    path = orc.HERE / "_ref" / "libref_f32_experts.so"
    if not path.exists():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    ref = C.CDLL(str(path))
    ref.ref_glu.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64]
    ref.ref_glu.restype = C.c_int
    rng = np.random.default_rng(91)
    n = 20000
    g = (rng.standard_normal(n) * 6).astype(np.float32)
    u = (rng.standard_normal(n) * 6).astype(np.float32)
    edges = np.array([7.0, -7.0, 6.9999995, 7.0000005, -7.0000005, 30.0, -30.0, 88.0, -88.0, 1e-30, -1e-30, 1.0,
                      -1.0], np.float32)
    g[: edges.size], u[: edges.size] = edges, edges[::-1]
    g[g == 0] = 1.0
    u[u == 0] = 1.0
    for activation in (0, 1):
        want = np.empty(n, np.float32)
        assert ref.ref_glu(activation, g.ctypes.data, u.ctypes.data, want.ctypes.data, n) == 0
        got = orc.glu(activation, g, u)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), activation
        if activation == 1:   # the clamps are active on this data (a dropped clamp fails above)
            assert np.any(g > 7) and np.any(np.abs(u) > 7)
