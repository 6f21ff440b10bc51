"""vbm_mul_mat_id_noalloc (fixed device scratch, no allocation) against vbm_mul_mat_id on the same
inputs: bit-identical outputs on two calls in a row, the second smaller than the first, in both
accumulation orders (the batched GEMV and the MFMA grouped GEMM) and with caller-quantized Q8_0
input carrying -128 codes; a shape needing more than the fixed scratch is rejected before
anything is enqueued."""
import ctypes as C

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


def noalloc(gpu, bank, n_as, b, b_type, ids, n_ids, order, bias=None):
    tokens = ids.shape[0]
    db, di = gpu.DeviceBuffer.from_array(np.ascontiguousarray(b)), gpu.DeviceBuffer.from_array(ids)
    dbias = gpu.DeviceBuffer.from_array(bias) if bias is not None else None
    dst = gpu.DeviceBuffer(tokens * n_ids * bank.rows * 4)
    gpu.call("vbm_mul_mat_id_noalloc", bank.handle, None, n_as, b_type, db.ptr, 1, di.ptr, n_ids, tokens, n_ids,
             gpu.ptr(dbias), dst.ptr, order, None)
    gpu.call("vbm_stream_synchronize", None)
    return dst.download(np.float32, (tokens, n_ids, bank.rows))


@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
@pytest.mark.parametrize("order,tokens", [(0, (40, 9)), (1, (160, 64))])
def test_noalloc_matches_mul_mat_id_twice(gpu, type_id, order, tokens):
    k, rows, experts, n_ids = 1024, 192, 6, 2
    rng = np.random.default_rng(900 + type_id + order)
    w = H.synth_weights(type_id, 900 + order, 1, experts, rows, k)
    bank = H.make_bank(type_id, w, experts, rows, k)
    bias = gpu.synth_normal(901, 2, 0, experts * rows, 0.0, 0.02)
    for call, T in enumerate(tokens):
        ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(T)]).astype(np.int32)
        ids[0, 1] = -1
        x = gpu.synth_normal(902 + call, 3, 0, T * k).reshape(T, 1, k)
        want = H.mul_mat_id(bank, experts, x, gpu.TYPE_F32, 1, ids, n_ids, bias=bias, order=order)
        got = noalloc(gpu, bank, experts, x, gpu.TYPE_F32, ids, n_ids, order, bias)
        print(f"[noalloc type={type_id} order={order} call {call}] T={T}", flush=True)
        assert H.bits_equal(got, want), H.diff_report(got, want)
        assert np.all(got[0, 1] == 0.0)
    # ggml Q8_0 activations with -128 codes (the flagged kernels)
    T = tokens[1]
    ids = np.stack([rng.choice(experts, n_ids, replace=False) for _ in range(T)]).astype(np.int32)
    import oracle_py
    oracle_py.load()
    q = oracle_py.quantize_q8_0(gpu.synth_normal(903, 3, 0, T * k).reshape(T, k)).reshape(-1, 34)
    q[::3, 2 + 7] = 128
    q = q.reshape(T, 1, -1)
    want = H.mul_mat_id(bank, experts, q, gpu.TYPE_Q8_0, 1, ids, n_ids, order=order)
    got = noalloc(gpu, bank, experts, q, gpu.TYPE_Q8_0, ids, n_ids, order)
    assert H.bits_equal(got, want), H.diff_report(got, want)
    bank.destroy()


def test_noalloc_rejects_shapes_beyond_its_scratch(gpu):
    k, rows, experts, n_ids, T = 4096, 64, 4, 2, 2048
    bank = gpu.Bank(H.MX, rows, k, experts)
    need = C.c_size_t()
    gpu.call("vbm_mul_mat_id_workspace", bank.handle, experts, 1, n_ids, T, gpu.ORDER_FAST, C.byref(need))
    assert need.value > 16 << 20
    db = gpu.DeviceBuffer(T * k * 4)
    di = gpu.DeviceBuffer.from_array(np.zeros((T, n_ids), np.int32))
    dst = gpu.DeviceBuffer(T * n_ids * rows * 4)
    with pytest.raises(gpu.VbmError, match="fixed") as err:
        gpu.call("vbm_mul_mat_id_noalloc", bank.handle, None, experts, gpu.TYPE_F32, db.ptr, 1, di.ptr, n_ids, T,
                 n_ids, None, dst.ptr, gpu.ORDER_FAST, None)
    assert err.value.status == 1
    bank.destroy()
