"""GGUF expert tensors on the GPU: experts loaded from a GGUF file into banks export back to the
file's bytes (lossless, as tests/test_masked_matmul.cpp:59-72 of the reference checks the repack
round trip); a layer over GGUF-loaded banks matches the oracle on the same bytes; and the
host-RAM tier filled from the same file (vbm_tier_load_gguf) reproduces the resident decode plan
bit for bit."""
import ctypes as C

import numpy as np
import pytest

import gguf_writer as W
import helpers as Hlp

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 256, 16, 4


def write_model(tmp_path, gtype, seed):
    rng = np.random.default_rng(seed)
    tensors, arrays = [], {}
    for layer in (0, 1):
        t, a = W.expert_layer_tensors(layer, gtype, H, I, E, rng)
        tensors += t
        arrays[layer] = a
    path = W.write_gguf(tmp_path / f"m{gtype}-00001-of-00001.gguf", [("general.architecture", W.STRING, "gpt-oss")],
                        tensors)
    return path, arrays


@pytest.mark.parametrize("gtype", [39, 8])
def test_gguf_layer_lossless_and_matches_oracle(gpu, orc, tmp_path, gtype):
    vb = gpu
    from vbmoe.gguf import GgufFile
    path, arrays = write_model(tmp_path, gtype, 11 + gtype)
    act = vb.ACT_SWIGLU_OAI if gtype == 39 else vb.ACT_SILU
    with GgufFile(path) as f:
        for layer in (0, 1):
            a = arrays[layer]
            gu, dn = vb.Bank(gtype, 2 * I, H, E, True), vb.Bank(gtype, H, I, E, False)
            bgu, bdn = vb.DeviceBuffer(4 * E * 2 * I), vb.DeviceBuffer(4 * E * H)
            slots = np.arange(E)[::-1].copy()                  # expert e in slot E-1-e
            f.load_layer(layer, np.arange(E), gu, dn, slots=slots, gate_up_bias=bgu.ptr, down_bias=bdn.ptr)
            for e in range(E):
                assert np.array_equal(gu.export(int(slots[e])), a["gate_up"][e]), (layer, e)
                assert np.array_equal(dn.export(int(slots[e])), a["down"][e]), (layer, e)
            assert np.array_equal(bgu.download(np.float32, (E, 2 * I)), a["gate_up_bias"])
            assert np.array_equal(bdn.download(np.float32, (E, H)), a["down_bias"])
            # layer forward over the slot-mapped banks vs the oracle on the file's bytes
            smap = vb.DeviceBuffer.from_array(slots.astype(np.int32))
            desc = vb.MoeLayerDesc(gu.handle, dn.handle, bgu.ptr, bdn.ptr, smap.ptr, None, None, H, I, E, K, act,
                                   vb.ORDER_EXACT)
            T = 3
            x = vb.synth_normal(77, layer, 0, T * H).reshape(T, H)
            logits = vb.synth_normal(78, layer, 0, T * E).reshape(T, E)
            ws = C.c_size_t()
            vb.call("vbm_moe_layer_workspace", C.byref(desc), T, C.byref(ws))
            work = vb.DeviceBuffer(ws.value)
            dx, dl = vb.DeviceBuffer.from_array(x), vb.DeviceBuffer.from_array(logits)
            out, ids, w = vb.DeviceBuffer(4 * T * H), vb.DeviceBuffer(4 * T * K), vb.DeviceBuffer(4 * T * K)
            vb.call("vbm_moe_layer_forward", C.byref(desc), dx.ptr, dl.ptr, T, out.ptr, ids.ptr, w.ptr, work.ptr,
                    ws.value, None)
            vb.call("vbm_stream_synchronize", None)
            ref = orc.moe_layer(gtype, a["gate_up"].reshape(-1), a["down"].reshape(-1), a["gate_up_bias"].reshape(-1),
                                a["down_bias"].reshape(-1), x, H, I, E, K, activation=act, logits=logits)
            got = out.download(np.float32, (T, H))
            assert np.array_equal(ids.download(np.int32, (T, K)), ref["ids"])
            max_rel, cos = Hlp.rel_err_and_cos(got, ref["out"])
            same = float(np.mean(got.view(np.uint32) == ref["out"].view(np.uint32)))
            print(f"[gguf type={gtype} layer={layer}] max_rel={max_rel:.3e} cos={cos:.9f} "
                  f"bitwise_equal_fraction={same:.6f}", flush=True)
            assert max_rel <= 1e-3 and cos >= 0.99999
            gu.destroy()
            dn.destroy()


def test_tier_from_gguf_matches_resident_plan(gpu, tmp_path):
    vb = gpu
    from vbmoe.gguf import GgufFile
    path, _ = write_model(tmp_path, 39, 5)
    L, slots = 2, K + 7
    with GgufFile(path) as f:
        banks, biases, descs = [], [], []
        for l in range(L):
            gu, dn = vb.Bank(39, 2 * I, H, E, True), vb.Bank(39, H, I, E, False)
            bgu, bdn = vb.DeviceBuffer(4 * E * 2 * I), vb.DeviceBuffer(4 * E * H)
            f.load_layer(l, np.arange(E), gu, dn, gate_up_bias=bgu.ptr, down_bias=bdn.ptr)
            banks.append((gu, dn))
            biases.append((bgu, bdn))
            descs.append(vb.MoeLayerDesc(gu.handle, dn.handle, bgu.ptr, bdn.ptr, None, None, None, H, I, E, K,
                                         vb.ACT_SWIGLU_OAI, vb.ORDER_EXACT))
        plan = C.c_void_p()
        vb.call("vbm_decode_plan_create", (vb.MoeLayerDesc * L)(*descs), L, C.byref(plan))
        tb = [(vb.DeviceBuffer(4 * E * 2 * I), vb.DeviceBuffer(4 * E * H)) for _ in range(L)]
        for l in range(L):
            vb.call("vbm_gguf_load_biases", f.handle, l, tb[l][0].ptr, tb[l][1].ptr, None)
        gub = (C.c_void_p * L)(*[b[0].ptr for b in tb])
        dnb = (C.c_void_p * L)(*[b[1].ptr for b in tb])
        desc = vb.TierDesc(39, H, I, L, E, K, vb.ACT_SWIGLU_OAI, slots, 8, 4, vb.ADMIT_CLASSIC,
                           C.cast(gub, C.POINTER(C.c_void_p)), C.cast(dnb, C.POINTER(C.c_void_p)))
        tier = C.c_void_p()
        vb.call("vbm_tier_create", C.byref(desc), C.byref(tier))
        bad = (C.c_int64 * L)(0, 7)
        with pytest.raises(vb.VbmError, match="missing"):
            vb.call("vbm_tier_load_gguf", tier.value, f.handle, bad, None)
        vb.call("vbm_tier_load_gguf", tier.value, f.handle, (C.c_int64 * L)(0, 1), None)
    x = vb.DeviceBuffer.from_array(vb.synth_normal(5, 6, 0, H))
    dl = vb.DeviceBuffer(4 * L * E)
    o1, o2 = vb.DeviceBuffer(4 * H), vb.DeviceBuffer(4 * H)
    rng = np.random.default_rng(3)
    for t in range(12):
        dl.upload(rng.standard_normal(L * E).astype(np.float32))
        vb.call("vbm_decode_step", plan.value, x.ptr, dl.ptr, o1.ptr, None, None, None, None)
        vb.call("vbm_tier_step", tier.value, x.ptr, dl.ptr, o2.ptr, None, None)
        vb.call("vbm_stream_synchronize", None)
        a, b = o1.download(np.float32, H), o2.download(np.float32, H)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), t
    st = vb.TierStats()
    vb.call("vbm_tier_get_stats", tier.value, C.byref(st))
    print(f"[gguf tier] hits={st.hits}/{12 * L * K} staged={st.staged} admissions={st.admissions}", flush=True)
    vb.call("vbm_tier_destroy", tier.value)
    vb.call("vbm_decode_plan_destroy", plan.value)
    for gu, dn in banks:
        gu.destroy()
        dn.destroy()
