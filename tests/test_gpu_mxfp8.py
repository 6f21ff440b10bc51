"""The MXFP4 x MXFP8 experiment on the block-scaled matrix cores (vbm_quantize_mxfp8,
vbm_mul_mat_id_mxfp8). It has no counterpart in the reference, whose activations are Q8_0, so
its checks are against the arithmetic it implements: the quantizer against a brute-force nearest
e4m3 search (OCP MX rules), the GEMM against float64 sums of the dequantized MXFP4 weights times
the dequantized MXFP8 activations, and its distance from the reference's Q8_0 path is reported."""
import numpy as np
import pytest

import helpers as H
import vbmoe as vb

pytestmark = pytest.mark.gpu

E2M1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6], np.float64)


def e4m3_table():
    codes = np.arange(256)
    s, e, m = codes >> 7, (codes >> 3) & 15, codes & 7
    v = np.where(e > 0, (1 + m / 8.0) * np.exp2(e - 7.0), m / 8.0 * 2.0 ** -6)
    v = np.where(s == 1, -v, v)
    v[(codes & 0x7F) == 0x7F] = np.nan                      # e4m3fn NaN codes
    return v


E4M3 = e4m3_table()


def quantize_mxfp8_ref(x):
    """MXFP8 block quantization by brute force: X the smallest power of two with amax / X <= 448,
    each value the nearest finite e4m3 of v / X (ties to the even code)."""
    rows, k = x.shape
    nb = k // 32
    codes = np.zeros((rows, k), np.uint8)
    scales = np.zeros((rows, nb), np.uint8)
    finite = np.where(np.isfinite(E4M3))[0]
    vals = E4M3[finite]
    for r in range(rows):
        for b in range(nb):
            blk = x[r, b * 32:(b + 1) * 32].astype(np.float64)
            amax = np.abs(blk).max()
            sx = -127
            while amax * 2.0 ** -sx > 448:
                sx += 1
            scales[r, b] = sx + 127
            y = np.clip(blk * 2.0 ** -sx, -448, 448)
            d = np.abs(y[:, None] - vals[None, :])
            tie = d == d.min(axis=1, keepdims=True)
            even = tie & ((finite[None, :] & 1) == 0)             # ties go to the even mantissa
            pick = np.where(even.any(axis=1), finite[np.argmax(even, axis=1)], finite[np.argmax(tie, axis=1)])
            codes[r, b * 32:(b + 1) * 32] = pick
    return codes, scales


def dequant_mxfp4(ggml, rows, k):
    """ggml block_mxfp4 rows (e8m0 byte + 16 code bytes; element i < 16 the low nibble of qs[i],
    i >= 16 the high nibble of qs[i - 16]) -> float64 [rows][k]."""
    nb = k // 32
    blocks = ggml.reshape(rows, nb, 17)
    e = blocks[:, :, 0].astype(np.int64)
    qs = blocks[:, :, 1:]
    codes = np.concatenate([qs & 15, qs >> 4], axis=2)
    return (E2M1[codes] * np.exp2(e - 127.0)[:, :, None]).reshape(rows, k)


def test_mxfp4_dequant_matches_the_oracle():
    """The numpy MXFP4 reading used below against the oracle's MXFP4 dot on one-hot activations."""
    import oracle_py as orc
    k, rows = 256, 8
    w = H.synth_weights(H.MX, 31, 1, 1, rows, k)
    ref = dequant_mxfp4(w, rows, k)
    for j in (0, 5, 15, 16, 31, 32, 100, 255):
        b = np.zeros((1, k), np.float32)
        b[0, j] = 1.0
        got = orc.mul_mat_id(H.MX, w, k, rows, 1, 0, b, 1, np.zeros((1, 1), np.int32), 1, 1, 1)[0, 0]
        expect = ref[:, j] * 127 * float(np.float16(1 / 127))
        assert np.allclose(got, expect, rtol=1e-6, atol=0), j


@pytest.fixture(scope="module")
def gpu_mx():
    vb.call("vbm_set_device", 0)
    return vb


def test_quantize_mxfp8_matches_brute_force(gpu_mx):
    rng = np.random.default_rng(41)
    k = 256
    x = rng.standard_normal((6, k)).astype(np.float32)
    x[1, :32] = 0.0                                          # an all-zero block
    x[2, 32:64] *= 1e-40                                     # a subnormal block
    x[3, 64:96] = np.float32(447.9)                          # saturation neighbourhood
    x[3, 64] = 1.0e6
    x[4, :] = np.round(x[4, :] * 16) / 16                    # ties at the coarse e4m3 steps
    x[5, 96:128] = rng.choice([-1, 1], 32) * np.exp2(rng.integers(-20, 20, 32)).astype(np.float32)
    dx = vb.DeviceBuffer.from_array(x)
    dc, ds = vb.DeviceBuffer(x.size), vb.DeviceBuffer(x.size // 32)
    vb.call("vbm_quantize_mxfp8", dx.ptr, x.shape[0], k, k, dc.ptr, ds.ptr, None)
    vb.call("vbm_stream_synchronize", None)
    codes = dc.download(np.uint8, x.shape)
    scales = ds.download(np.uint8, (x.shape[0], k // 32))
    rc, rs = quantize_mxfp8_ref(x)
    assert np.array_equal(scales, rs)
    got = E4M3[codes] * np.exp2(scales.astype(np.float64) - 127).repeat(32, axis=1)
    ref = E4M3[rc] * np.exp2(rs.astype(np.float64) - 127).repeat(32, axis=1)
    assert np.array_equal(got, ref), np.argwhere(got != ref)[:5]


@pytest.mark.parametrize("case", ["broadcast", "per-rank-interleaved-map"])
def test_mxfp8_mul_mat_id_matches_float64(gpu_mx, case):
    """Every output against float64 sums over the dequantized operands, within 2e-4 of the sum of
    |products| (the matrix core's internal accumulation is not an fp32 chain); -1 ids give zero
    rows; experts with 75 jobs run two 64-job tiles; K = 2880 has a two-block tail."""
    import oracle_py as orc
    rng = np.random.default_rng(43)
    k, rows, E, K, T = 2880, 192, 8, 2, 300
    w = H.synth_weights(H.MX, 44, 1, E, rows, k)
    per_rank = case != "broadcast"
    bank = H.make_bank(H.MX, w, E, rows, k, interleave=per_rank)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ids[7, 1] = -1
    b_ne1 = K if per_rank else 1
    x = rng.standard_normal((T, b_ne1, k)).astype(np.float32)
    slot_map = None
    if per_rank:                                              # a permuted expert -> slot map
        perm = rng.permutation(E).astype(np.int32)
        wp = w.reshape(E, -1)[np.argsort(perm)].reshape(-1)
        bank.destroy()
        bank = H.make_bank(H.MX, wp, E, rows, k, interleave=True)
        slot_map = vb.DeviceBuffer.from_array(perm)
    dx, dids = vb.DeviceBuffer.from_array(x), vb.DeviceBuffer.from_array(ids)
    dst = vb.DeviceBuffer(4 * T * K * rows)
    vb.call("vbm_mul_mat_id_mxfp8", bank.handle, vb.ptr(slot_map), E, dx.ptr, b_ne1, dids.ptr, K, T, K, dst.ptr, None)
    vb.call("vbm_stream_synchronize", None)
    got = dst.download(np.float32, (T, K, rows)).astype(np.float64)
    dc, ds = vb.DeviceBuffer(x.size), vb.DeviceBuffer(x.size // 32)
    vb.call("vbm_quantize_mxfp8", dx.ptr, T * b_ne1, k, k, dc.ptr, ds.ptr, None)
    vb.call("vbm_stream_synchronize", None)
    xq = (E4M3[dc.download(np.uint8, (T * b_ne1, k))] *
          np.exp2(ds.download(np.uint8, (T * b_ne1, k // 32)).astype(np.float64) - 127).repeat(32, axis=1))
    xq = xq.reshape(T, b_ne1, k)
    wd = dequant_mxfp4(w, E * rows, k).reshape(E, rows, k)
    ref = np.zeros((T, K, rows))
    mag = np.zeros((T, K, rows))
    for t in range(T):
        for r in range(K):
            e = ids[t, r]
            if e < 0:
                continue
            xv = xq[t, r if per_rank else 0]
            ref[t, r] = wd[e] @ xv
            mag[t, r] = np.abs(wd[e]) @ np.abs(xv)
    assert np.all(got[7, 1] == 0.0)
    err = np.abs(got - ref) / np.maximum(mag, 1e-30)
    print(f"[mxfp8 {case}] max |err| / sum|p| = {err.max():.3e}", flush=True)
    assert err.max() <= 2e-4
    # distance from the reference's Q8_0 arithmetic (oracle), for the record
    q = orc.mul_mat_id(H.MX, w, k, rows, E, 0, x.reshape(T * b_ne1, k), b_ne1, ids, K, T, K).astype(np.float64)
    live = ids >= 0
    rel = np.abs(got - q)[live].max() / np.abs(q[live]).max()
    print(f"[mxfp8 {case}] max deviation from the Q8_0 oracle, relative to max |out| = {rel:.3e}", flush=True)
    assert rel < 0.1
    bank.destroy()
