"""Fused routed-expert layer (vbm_moe_layer_forward) against the oracle's restatement of the
reference expert_branch graph, on the seeded configs. Expert ids and routing order must match
exactly; fp32 outputs within 1e-3 max relative error and cosine >= 0.99999."""
import ctypes as C

import numpy as np
import pytest

import helpers as H

pytestmark = pytest.mark.gpu


class Layer:
    """Seeded synthetic layer: tensors are pure functions of (seed, layer, tensor id)."""

    def __init__(self, vb, type_id, hidden, inter, experts, top_k, seed, layer=0, router=True, biases=True,
                 activation=1, q8_scale=(1e-3, 1e-2), order=None):
        self.vb, self.type_id = vb, type_id
        self.H, self.I, self.E, self.K = hidden, inter, experts, top_k
        self.activation = activation
        self.order = vb.ORDER_EXACT if order is None else order
        base = 16 * layer
        self.gu = H.synth_weights(type_id, seed, base + 1, experts, 2 * inter, hidden, q8_scale)
        self.dn = H.synth_weights(type_id, seed, base + 2, experts, hidden, inter, q8_scale)
        self.gu_b = vb.synth_normal(seed, base + 3, 0, experts * 2 * inter, 0.0, 0.02) if biases else None
        self.dn_b = vb.synth_normal(seed, base + 4, 0, experts * hidden, 0.0, 0.02) if biases else None
        self.rw = vb.synth_normal(seed, base + 5, 0, experts * hidden, 0.0, 0.02).reshape(experts, hidden) if router else None
        self.gu_bank = H.make_bank(type_id, self.gu, experts, 2 * inter, hidden, interleave=True)
        self.dn_bank = H.make_bank(type_id, self.dn, experts, hidden, inter)
        self.d_gu_b = vb.DeviceBuffer.from_array(self.gu_b) if biases else None
        self.d_dn_b = vb.DeviceBuffer.from_array(self.dn_b) if biases else None
        self.d_rw = vb.DeviceBuffer.from_array(self.rw) if router else None

    def desc(self):
        vb = self.vb
        return vb.MoeLayerDesc(self.gu_bank.handle, self.dn_bank.handle, vb.ptr(self.d_gu_b), vb.ptr(self.d_dn_b),
                               None, vb.ptr(self.d_rw), None, self.H, self.I, self.E, self.K, self.activation,
                               self.order)

    def forward_gpu(self, x, logits=None):
        vb = self.vb
        T = x.shape[0]
        d = self.desc()
        ws = C.c_size_t()
        vb.call("vbm_moe_layer_workspace", C.byref(d), T, C.byref(ws))
        work = vb.DeviceBuffer(ws.value)
        dx = vb.DeviceBuffer.from_array(x)
        dl = vb.DeviceBuffer.from_array(logits) if logits is not None else vb.DeviceBuffer(4 * T * self.E)
        out, ids, w = vb.DeviceBuffer(4 * T * self.H), vb.DeviceBuffer(4 * T * self.K), vb.DeviceBuffer(4 * T * self.K)
        vb.call("vbm_moe_layer_forward", C.byref(d), dx.ptr, dl.ptr, T, out.ptr, ids.ptr, w.ptr, work.ptr, ws.value, None)
        vb.call("vbm_stream_synchronize", None)
        return (out.download(np.float32, (T, self.H)), ids.download(np.int32, (T, self.K)),
                w.download(np.float32, (T, self.K)))

    def forward_cpu(self, orc, x, logits=None, threads=8):
        return orc.moe_layer(self.type_id, self.gu, self.dn, self.gu_b, self.dn_b, x, self.H, self.I, self.E, self.K,
                             activation=self.activation, logits=logits, router_w=self.rw, threads=threads)

    def destroy(self):
        self.gu_bank.destroy()
        self.dn_bank.destroy()


def check(got, ref, label):
    out, ids, w = got
    assert np.array_equal(ids, ref["ids"]), f"{label}: expert ids differ"
    assert np.allclose(w, ref["weights"], rtol=1e-6, atol=0), f"{label}: routing weights"
    max_rel, cos = H.rel_err_and_cos(out, ref["out"])
    same = float(np.mean(out.view(np.uint32) == ref["out"].view(np.uint32)))
    print(f"[{label}] max_rel={max_rel:.3e} cos={cos:.9f} bitwise_equal_fraction={same:.6f}", flush=True)
    assert max_rel <= 1e-3 and cos >= 0.99999, label


@pytest.mark.parametrize("tokens", [1, 8])
def test_layer_config0_mxfp4_swiglu_oai(gpu, orc, tokens):
    """Config 0: hidden 2880, 32 experts, top-4, intermediate 2880, router weight N(0,0.02)."""
    layer = Layer(gpu, H.MX, 2880, 2880, 32, 4, seed=2024)
    x = gpu.synth_normal(2024, 6, 0, tokens * 2880).reshape(tokens, 2880)
    check(layer.forward_gpu(x), layer.forward_cpu(orc, x), f"config0 T={tokens}")
    layer.destroy()


def test_layer_config1_chained_layers(gpu, orc):
    """Config 1 shape (32 experts, top-4, 2880), several independently seeded layers chained at T=8."""
    x = gpu.synth_normal(77, 6, 0, 8 * 2880).reshape(8, 2880)
    x_gpu, x_cpu = x, x
    for l in range(3):
        layer = Layer(gpu, H.MX, 2880, 2880, 32, 4, seed=77, layer=l)
        got = layer.forward_gpu(x_gpu)
        ref = layer.forward_cpu(orc, x_gpu)          # same input as the GPU for a per-layer check
        check(got, ref, f"config1 layer={l}")
        x_gpu = got[0]
        layer.destroy()


def test_layer_q8_0_silu_given_logits(gpu, orc):
    """Config 3 shape (hidden 2048, 128 experts, top-8, intermediate 768, SiLU, no biases)."""
    layer = Layer(gpu, H.Q8, 2048, 768, 128, 8, seed=303, router=False, biases=False, activation=0)
    T = 16
    x = gpu.synth_normal(303, 6, 0, T * 2048).reshape(T, 2048)
    logits = gpu.synth_normal(303, 7, 0, T * 128).reshape(T, 128)
    check(layer.forward_gpu(x, logits), layer.forward_cpu(orc, x, logits), "config3-shape T=16")
    layer.destroy()


def test_layer_glu_epilogue_many_tokens_per_expert(gpu, orc):
    """The fused gate_up GEMV's GLU + requantize epilogue over multi-chunk experts: 8 experts,
    top-4, 40 tokens (20 jobs per expert on average: chunks of 8 and partial chunks), exact order."""
    layer = Layer(gpu, H.MX, 1024, 512, 8, 4, seed=404)
    T = 40
    x = gpu.synth_normal(404, 6, 0, T * 1024).reshape(T, 1024)
    out, ids, w = layer.forward_gpu(x)
    ref = layer.forward_cpu(orc, x)
    assert np.array_equal(ids, ref["ids"])
    assert np.array_equal(out.view(np.uint32), ref["out"].view(np.uint32)), H.diff_report(out, ref["out"])
    layer.destroy()


@pytest.mark.parametrize("tokens,experts,hidden,inter", [(16, 64, 1024, 512), (17, 64, 1024, 512), (1, 1024, 256, 128),
                                                         (3, 1024, 256, 128)])
def test_layer_one_launch_routing_boundary(gpu, orc, tokens, experts, hidden, inter):
    """Up to 16 tokens the batched layer routes, groups and quantizes its input in one launch;
    from 17 tokens the top-k runs beside the quantization and the grouping follows. Both sides of
    the boundary, and 1024 experts (16 logits per lane), bitwise against the oracle in the exact
    order."""
    layer = Layer(gpu, H.MX, hidden, inter, experts, 4, seed=505 + tokens, router=False)
    x = gpu.synth_normal(505, 6, tokens, tokens * hidden).reshape(tokens, hidden)
    logits = gpu.synth_normal(505, 7, tokens, tokens * experts).reshape(tokens, experts)
    out, ids, w = layer.forward_gpu(x, logits)
    ref = layer.forward_cpu(orc, x, logits)
    assert np.array_equal(ids, ref["ids"])
    assert np.allclose(w, ref["weights"], rtol=1e-6, atol=0)
    assert np.array_equal(out.view(np.uint32), ref["out"].view(np.uint32)), H.diff_report(out, ref["out"])
    layer.destroy()


def test_layer_randomized_shapes_bitwise(gpu, orc):
    """10 seeded random fused layers in the exact order against the oracle's layer: both weight
    types and activations, hidden 64..1024, intermediate 64..768, 2..48 experts, top-1..6, 1..24
    tokens, given logits or the fp32 router, with or without biases. Expert ids and outputs must be
    bit-identical."""
    rng = np.random.default_rng(4040)
    for case in range(10):
        type_id = H.MX if case % 2 == 0 else H.Q8
        hidden, inter = 64 * int(rng.integers(1, 17)), 64 * int(rng.integers(1, 13))
        experts = int(rng.integers(2, 49))
        top_k = int(rng.integers(1, min(6, experts) + 1))
        tokens = int(rng.integers(1, 25))
        router, biases = bool(rng.random() < 0.5), bool(rng.random() < 0.6)
        act = gpu.ACT_SWIGLU_OAI if rng.random() < 0.5 else gpu.ACT_SILU
        label = (f"case {case}: type={type_id} H={hidden} I={inter} E={experts} top{top_k} T={tokens} "
                 f"router={router} biases={biases} act={act}")
        print(f"[random layer] {label}", flush=True)
        layer = Layer(gpu, type_id, hidden, inter, experts, top_k, seed=700 + case, router=router, biases=biases,
                      activation=act)
        x = gpu.synth_normal(700 + case, 6, 0, tokens * hidden).reshape(tokens, hidden)
        logits = None if router else gpu.synth_normal(700 + case, 7, 0, tokens * experts).reshape(tokens, experts)
        out, ids, w = layer.forward_gpu(x, logits)
        ref = layer.forward_cpu(orc, x, logits)
        assert np.array_equal(ids, ref["ids"]), label
        assert np.array_equal(out.view(np.uint32), ref["out"].view(np.uint32)), f"{label}: {H.diff_report(out, ref['out'])}"
        layer.destroy()
