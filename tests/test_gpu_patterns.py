"""The reference's activation patterns for its operator self-tests (tools/trace/hybrid_layer.cpp:
593-604: "zero", "q8-ties" with Q8_0 rounding ties and +/-127 block maxima, and "sine" at
magnitudes 0.2 / 50 / 500 by sample) through the fused layer (exact order, 3 tokens) and the
single-token decode step, against the oracle. Expert ids must match and the fp32 outputs must be
bit-identical (the exact order reproduces the CPU arithmetic)."""
import numpy as np
import pytest

import helpers as H
from test_gpu_decode import oracle_chain, run_decode
from test_gpu_layer import Layer

pytestmark = pytest.mark.gpu

CASES = [("zero", 0), ("q8-ties", 0), ("q8-ties", 1), ("sine", 0), ("sine", 1), ("sine", 2)]


def activation_input(hidden: int, rows: int, sample: int, pattern: str) -> np.ndarray:
    """hybrid_layer.cpp:593-604 with self_test = true."""
    n = hidden * rows
    i = np.arange(n)
    if pattern == "zero":
        x = np.zeros(n, np.float32)
    elif pattern == "q8-ties":
        x = np.where(i % 2 == 1, -1.0, 1.0) * (0.5 + ((i + 7 * sample) % 31))
        x = np.where(i % 32 == 0, 127.0, np.where(i % 32 == 1, -127.0, x))
    else:
        magnitude = np.float32(0.2 if sample % 3 == 0 else 50.0 if sample % 3 == 1 else 500.0)
        angle = ((i + 1) * (sample + 3)).astype(np.float32) * np.float32(0.017)
        x = magnitude * np.sin(angle, dtype=np.float32)
    return np.asarray(x, np.float32).reshape(rows, hidden)


def test_q8_ties_pattern_has_ties():
    x = activation_input(2880, 1, 0, "q8-ties")
    assert x[0, 0] == 127.0 and x[0, 1] == -127.0 and x[0, 2] == 2.5
    # every block's maximum is 127, so codes are the values themselves: half-integers round to even
    assert np.all(np.abs(x.reshape(-1, 32)).max(axis=1) == 127.0)


@pytest.mark.parametrize("pattern,sample", CASES)
@pytest.mark.parametrize("type_id", [H.MX, H.Q8])
def test_layer_patterns_bit_identical(gpu, orc, type_id, pattern, sample):
    act = gpu.ACT_SWIGLU_OAI if type_id == H.MX else gpu.ACT_SILU
    layer = Layer(gpu, type_id, 2880, 2880, 32, 4, seed=593 + sample, router=False, activation=act)
    x = activation_input(2880, 3, sample, pattern)
    logits = gpu.synth_normal(593, 9 + sample, 0, 3 * 32).reshape(3, 32)
    out, ids, w = layer.forward_gpu(x, logits)
    ref = layer.forward_cpu(orc, x, logits)
    assert np.array_equal(ids, ref["ids"])
    assert np.array_equal(out.view(np.uint32), ref["out"].view(np.uint32)), \
        f"{pattern}/{sample}: {H.diff_report(out, ref['out'])}"
    layer.destroy()


@pytest.mark.parametrize("pattern,sample", CASES)
def test_decode_patterns_bit_identical(gpu, orc, pattern, sample):
    L = 2
    layers = [Layer(gpu, H.MX, 2880, 2880, 32, 4, seed=601, layer=l, router=False) for l in range(L)]
    x = activation_input(2880, 1, sample, pattern)[0]
    logits = gpu.synth_normal(601, 20 + sample, 0, L * 32).reshape(L, 32)
    out, ids, _ = run_decode(gpu, layers, x, logits)
    ref, ref_ids, _ = oracle_chain(orc, layers, x, logits)
    assert np.array_equal(ids, ref_ids)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)), f"{pattern}/{sample}: {H.diff_report(out, ref)}"
    for layer in layers:
        layer.destroy()
