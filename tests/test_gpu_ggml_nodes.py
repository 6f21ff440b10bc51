"""The ggml backend boundary on the GPU: vbm_graph_compute over the node list the reference builds
for one routed-expert layer (third_party/patches/llama-b11669-hybrid-experts.patch:1394-1683, joined
at :1905-1916), checked bit for bit against the oracle's layer in the exact order; strided views
through every node kind against numpy or the flat entry points."""
import ctypes as C

import numpy as np
import pytest

import helpers as H
from ggml_graph import Graph, f32_bits

pytestmark = pytest.mark.gpu

F32, I32 = 0, 26


def download(vb, ptr, shape, dtype=np.float32):
    out = np.empty(shape, dtype)
    vb.call("vbm_memcpy_d2h", out.ctypes.data, ptr, out.nbytes, None)
    return out


def split_rows(ggml_bytes, experts, rows, k, type_id, first, count):
    """Rows [first, first + count) of every expert of a ggml expert tensor, as a new tensor."""
    per_row = (k // 32) * H.block_bytes(type_id)
    w = ggml_bytes.reshape(experts, rows, per_row)
    return np.ascontiguousarray(w[:, first:first + count]).reshape(-1)


def build_expert_branch(vb, g, layer, dx, ids_buf, ids_stride, dw, T, fused):
    """The resident expert_branch of the reference as ggml nodes (weights applied after the FFN)."""
    Hd, I, E, K = layer.H, layer.I, layer.E, layer.K
    x = g.leaf(F32, (Hd, 1, T), dx.ptr)
    ids = g.leaf(I32, (K, T), ids_buf.ptr, nb=[4, 4 * ids_stride, 4 * ids_stride * T, 4 * ids_stride * T])
    weights = g.leaf(F32, (1, K, T), dw.ptr)
    out_bufs = []

    def new(ne, type_id=F32):
        n = int(np.prod(ne))
        buf = vb.DeviceBuffer(4 * n)
        out_bufs.append(buf)
        return buf.ptr

    if fused:
        as_gu = g.expert_tensor(layer.gu_bank, layer.type_id, Hd, 2 * I, E)
        gate_up = g.tensor(F32, (2 * I, K, T), new((2 * I, K, T)), op=vb.NODE_MUL_MAT_ID, srcs=(as_gu, x, ids))
        if layer.d_gu_b is not None:
            bias = g.leaf(F32, (2 * I, E), layer.d_gu_b.ptr)
            gate_up = g.tensor(F32, (2 * I, K, T), new((2 * I, K, T)), op=vb.NODE_ADD_ID, srcs=(gate_up, bias, ids))
        nb = list(gate_up.nb)
        gate = g.view(gate_up, (I, K, T), nb, 0)
        up = g.view(gate_up, (I, K, T), nb, I * 4)
    else:
        as_up = g.expert_tensor(layer.up_bank, layer.type_id, Hd, I, E)
        as_gate = g.expert_tensor(layer.gate_bank, layer.type_id, Hd, I, E)
        up = g.tensor(F32, (I, K, T), new((I, K, T)), op=vb.NODE_MUL_MAT_ID, srcs=(as_up, x, ids))
        gate = g.tensor(F32, (I, K, T), new((I, K, T)), op=vb.NODE_MUL_MAT_ID, srcs=(as_gate, x, ids))
    if layer.activation == vb.ACT_SWIGLU_OAI:
        params = (vb.GLU_OP_SWIGLU_OAI, 0, f32_bits(1.702), f32_bits(7.0))
    else:
        params = (vb.GLU_OP_SWIGLU, 0)
    act = g.tensor(F32, (I, K, T), new((I, K, T)), op=vb.NODE_GLU, srcs=(gate, up), params=params)
    as_dn = g.expert_tensor(layer.dn_bank, layer.type_id, I, Hd, E)
    experts = g.tensor(F32, (Hd, K, T), new((Hd, K, T)), op=vb.NODE_MUL_MAT_ID, srcs=(as_dn, act, ids))
    if layer.d_dn_b is not None:
        bias = g.leaf(F32, (Hd, E), layer.d_dn_b.ptr)
        experts = g.tensor(F32, (Hd, K, T), new((Hd, K, T)), op=vb.NODE_ADD_ID, srcs=(experts, bias, ids))
    experts = g.tensor(F32, (Hd, K, T), new((Hd, K, T)), op=vb.NODE_MUL, srcs=(experts, weights))
    # join with an all-zero host half, then the sequential rank adds over strided views, then CONT
    zeros = vb.DeviceBuffer.from_array(np.zeros((T, K, Hd), np.float32))
    out_bufs.append(zeros)
    host = g.leaf(F32, (Hd, K, T), zeros.ptr)
    joined = g.tensor(F32, (Hd, K, T), new((Hd, K, T)), op=vb.NODE_ADD, srcs=(experts, host))
    output = None
    for rank in range(K):
        row = g.view(joined, (Hd, T), [4, joined.nb[2], joined.nb[2] * T, joined.nb[2] * T], rank * joined.nb[1])
        output = row if output is None else g.tensor(F32, (Hd, T), new((Hd, T)), op=vb.NODE_ADD, srcs=(output, row))
    final = g.tensor(F32, (Hd, T), new((Hd, T)), op=vb.NODE_CONT, srcs=(output,))
    return final, out_bufs


@pytest.mark.parametrize("case", ["mxfp4-oai-fused-biased", "q8-silu-separate", "mxfp4-silu-fused-nobias"])
def test_expert_branch_nodes_match_oracle_layer(gpu, orc, case):
    """One layer's expert_branch as ggml nodes (MUL_MAT_ID, ADD_ID, split views, GLU, MUL_MAT_ID,
    ADD_ID, MUL by the routing weights, join ADD, rank-view ADDs, CONT) on strided ids, in the
    exact order: bit-identical to the oracle's layer on the same ids and weights."""
    from test_gpu_layer import Layer
    vb = gpu
    if case == "mxfp4-oai-fused-biased":
        layer = Layer(vb, H.MX, 512, 256, 16, 4, seed=91, router=False, biases=True, activation=vb.ACT_SWIGLU_OAI)
        fused, T = True, 7
    elif case == "q8-silu-separate":
        layer = Layer(vb, H.Q8, 512, 192, 24, 6, seed=92, router=False, biases=False, activation=vb.ACT_SILU)
        fused, T = False, 5
    else:
        layer = Layer(vb, H.MX, 256, 320, 8, 2, seed=93, router=False, biases=False, activation=vb.ACT_SILU)
        fused, T = True, 9
    if not fused:
        layer.gate_bank = H.make_bank(layer.type_id, split_rows(layer.gu, layer.E, 2 * layer.I, layer.H, layer.type_id,
                                                                0, layer.I), layer.E, layer.I, layer.H)
        layer.up_bank = H.make_bank(layer.type_id, split_rows(layer.gu, layer.E, 2 * layer.I, layer.H, layer.type_id,
                                                              layer.I, layer.I), layer.E, layer.I, layer.H)
    x = vb.synth_normal(90, 6, 0, T * layer.H).reshape(T, layer.H)
    logits = vb.synth_normal(90, 7, 0, T * layer.E).reshape(T, layer.E)
    ref = layer.forward_cpu(orc, x, logits)
    stride = layer.K + 3
    ids_full = np.full((T, stride), 12345, np.int32)     # padding the ids view must not read
    ids_full[:, :layer.K] = ref["ids"]
    dx, dids, dw = vb.DeviceBuffer.from_array(x), vb.DeviceBuffer.from_array(ids_full), vb.DeviceBuffer.from_array(
        np.ascontiguousarray(ref["weights"], np.float32))
    g = Graph(vb)
    final, bufs = build_expert_branch(vb, g, layer, dx, dids, stride, dw, T, fused)
    for n in g.nodes:
        assert g.supported(n), n.op
    print(f"[nodes {case}] {len(g.nodes)} nodes", flush=True)
    g.compute(order=vb.ORDER_EXACT)
    vb.call("vbm_stream_synchronize", None)
    out = download(vb, final.data, (T, layer.H))
    assert H.bits_equal(out, ref["out"]), H.diff_report(out, ref["out"])
    layer.destroy()
    if not fused:
        layer.gate_bank.destroy()
        layer.up_bank.destroy()


def test_expert_branch_nodes_under_graph_capture(gpu, orc):
    """The expert-branch node list captured as a HIP graph. On a fresh stream the capture is refused
    (VBM_ERR_INVALID_ARGUMENT: MUL_MAT_ID would have to grow the stream's scratch inside the graph);
    after one eager run on that stream the capture succeeds, and every replay, with eager work and
    synchronizations between them, gives the eager bits, which equal the oracle's layer."""
    from test_gpu_layer import Layer
    vb = gpu
    layer = Layer(vb, H.MX, 512, 256, 16, 4, seed=94, router=False, biases=True, activation=vb.ACT_SWIGLU_OAI)
    T = 6
    x = vb.synth_normal(94, 6, 0, T * layer.H).reshape(T, layer.H)
    logits = vb.synth_normal(94, 7, 0, T * layer.E).reshape(T, layer.E)
    ref = layer.forward_cpu(orc, x, logits)
    dx, dids = vb.DeviceBuffer.from_array(x), vb.DeviceBuffer.from_array(np.ascontiguousarray(ref["ids"], np.int32))
    dw = vb.DeviceBuffer.from_array(np.ascontiguousarray(ref["weights"], np.float32))
    g = Graph(vb)
    final, bufs = build_expert_branch(vb, g, layer, dx, dids, layer.K, dw, T, True)
    st = C.c_void_p()
    vb.call("vbm_stream_create", C.byref(st))
    s = st.value
    graph = C.c_void_p()
    vb.call("vbm_graph_begin_capture", s)
    with pytest.raises(vb.VbmError) as err:
        g.compute(order=vb.ORDER_EXACT, stream=s)
    assert err.value.status == 1, str(err.value)      # VBM_ERR_INVALID_ARGUMENT
    try:
        vb.call("vbm_graph_end_capture", s, C.byref(graph))
    finally:
        if graph.value:
            vb.call("vbm_graph_destroy", graph.value)
    # one eager run grows the stream's scratch; the capture then allocates nothing
    g.compute(order=vb.ORDER_EXACT, stream=s)
    vb.call("vbm_stream_synchronize", s)
    eager = download(vb, final.data, (T, layer.H))
    assert H.bits_equal(eager, ref["out"]), H.diff_report(eager, ref["out"])
    graph = C.c_void_p()
    vb.call("vbm_graph_begin_capture", s)
    g.compute(order=vb.ORDER_EXACT, stream=s)
    vb.call("vbm_graph_end_capture", s, C.byref(graph))
    try:
        for _ in range(3):
            vb.call("vbm_memset", final.data, 0, 4 * T * layer.H, s)
            vb.call("vbm_graph_launch", graph.value, s)
            vb.call("vbm_stream_synchronize", s)
            got = download(vb, final.data, (T, layer.H))
            assert H.bits_equal(got, eager), H.diff_report(got, eager)
            g.compute(order=vb.ORDER_EXACT)            # eager work on another stream between replays
            vb.call("vbm_stream_synchronize", None)
    finally:
        vb.call("vbm_graph_destroy", graph.value)
        vb.call("vbm_stream_destroy", s)
    layer.destroy()


def weighted_branch(vb, g, new, x, ids, bias_ids, weights, gu_as, gu_bias, dn_as, dn_bias, dims):
    """MUL_MAT_ID -> ADD_ID -> split views -> GLU (swiglu_oai) -> MUL_MAT_ID -> ADD_ID -> MUL by the
    weights, on a fused gate_up expert tensor (the reference's expert_branch, weights after the FFN)."""
    Hd, I, K, T = dims
    gate_up = g.tensor(F32, (2 * I, K, T), new((2 * I, K, T)), op=vb.NODE_MUL_MAT_ID, srcs=(gu_as, x, ids))
    gate_up = g.tensor(F32, (2 * I, K, T), new((2 * I, K, T)), op=vb.NODE_ADD_ID, srcs=(gate_up, gu_bias, bias_ids))
    nb = list(gate_up.nb)
    gate, up = g.view(gate_up, (I, K, T), nb, 0), g.view(gate_up, (I, K, T), nb, I * 4)
    act = g.tensor(F32, (I, K, T), new((I, K, T)), op=vb.NODE_GLU, srcs=(gate, up),
                   params=(vb.GLU_OP_SWIGLU_OAI, 0, f32_bits(1.702), f32_bits(7.0)))
    y = g.tensor(F32, (Hd, K, T), new((Hd, K, T)), op=vb.NODE_MUL_MAT_ID, srcs=(dn_as, act, ids))
    y = g.tensor(F32, (Hd, K, T), new((Hd, K, T)), op=vb.NODE_ADD_ID, srcs=(y, dn_bias, bias_ids))
    return g.tensor(F32, (Hd, K, T), new((Hd, K, T)), op=vb.NODE_MUL, srcs=(y, weights))


@pytest.mark.parametrize("cold_rank", [-1, 2])
def test_frozen_hybrid_dispatch_nodes_match_oracle_layer(gpu, orc, cold_rank):
    """The reference's frozen-hybrid dispatch as nodes (hybrid-experts.patch:1860-1916): the packed
    slot remap written by vbm_admission_write_dispatch (:3059-3084) is read through strided views of
    its rows and I32 casts; the resident branch runs over the slot bank with the full routing
    weights (a miss reads the all-zero slot of its rank, token 0's cold rank the scratch slot
    n_slots), the cold branch over every expert with the cpu ids (-1 on resident ranks) and the
    cold weights; their ADD, the rank ADDs and CONT give the oracle's plain layer bit for bit in the
    exact order."""
    from test_admission import LibAdmission
    from test_gpu_layer import Layer
    vb = gpu
    E, K, T, Hd, I = 16, 4, 6, 256, 192
    layer = Layer(vb, H.MX, Hd, I, E, K, seed=95, router=False, biases=True, activation=vb.ACT_SWIGLU_OAI)
    x = vb.synth_normal(95, 6, 0, T * Hd).reshape(T, Hd)
    logits = vb.synth_normal(95, 7, 0, T * E).reshape(T, E)
    ref = layer.forward_cpu(orc, x, logits)
    ids, w = ref["ids"].astype(np.int32), np.ascontiguousarray(ref["weights"], np.float32)
    n_slots = K + 8
    adm = LibAdmission(vb, 1, E, K, n_slots)
    routed = sorted(set(ids.reshape(-1).tolist()))
    seeds = routed[::2][:5] + [e for e in range(E) if e not in routed][:2]   # some routed experts resident
    assert len(seeds) <= n_slots - K
    for e in seeds:
        adm.seed(0, e)
    slot_map = adm.slot_map(0)
    packet = adm.write_dispatch(0, ids, w, cold_rank)
    adm.close()
    cold = packet[:, 3, :] == 1.0
    print(f"[hybrid cold_rank={cold_rank}] resident {int((~cold).sum())} cold {int(cold.sum())} of {T * K}", flush=True)
    assert cold.any() and (~cold).any()
    # slot bank: n_slots + 1 slots; [0, K) stay zero, held slots get their expert, n_slots the cold rank's
    per_gu, per_dn = 2 * I * (Hd // 32) * 17, Hd * (I // 32) * 17
    slot_expert = [-1] * (n_slots + 1)
    for e, s_ in enumerate(slot_map):
        if s_ >= 0:
            slot_expert[s_] = e
    if cold_rank >= 0:
        slot_expert[n_slots] = int(ids[0, cold_rank])
    gu_s = np.zeros((n_slots + 1, per_gu), np.uint8)
    dn_s = np.zeros((n_slots + 1, per_dn), np.uint8)
    gub_s = np.zeros((n_slots + 1, 2 * I), np.float32)
    dnb_s = np.zeros((n_slots + 1, Hd), np.float32)
    for s_, e in enumerate(slot_expert):
        if e >= 0:
            gu_s[s_] = layer.gu[e * per_gu:(e + 1) * per_gu]
            dn_s[s_] = layer.dn[e * per_dn:(e + 1) * per_dn]
            gub_s[s_] = layer.gu_b.reshape(E, 2 * I)[e]
            dnb_s[s_] = layer.dn_b.reshape(E, Hd)[e]
    gu_bank = H.make_bank(H.MX, gu_s.reshape(-1), n_slots + 1, 2 * I, Hd, interleave=True)
    dn_bank = H.make_bank(H.MX, dn_s.reshape(-1), n_slots + 1, Hd, I)
    keep = [vb.DeviceBuffer.from_array(v) for v in (x, packet, ids, w, gub_s, dnb_s)]
    dx, dpacket, dids, dw, dgub, ddnb = keep

    def new(ne):
        buf = vb.DeviceBuffer(4 * int(np.prod(ne)))
        keep.append(buf)
        return buf.ptr

    g = Graph(vb)
    X = g.leaf(F32, (Hd, 1, T), dx.ptr)
    packed = g.leaf(F32, (K, 4, T), dpacket.ptr)
    selected = g.leaf(I32, (K, T), dids.ptr)
    weights = g.leaf(F32, (1, K, T), dw.ptr)
    rows_nb = [4, packed.nb[2], packed.nb[2] * T, packed.nb[2] * T]
    cpu_ids = g.tensor(I32, (K, T), new((K, T)), op=vb.NODE_CPY, srcs=(g.view(packed, (K, T), rows_nb, 0),))
    gpu_ids = g.tensor(I32, (K, T), new((K, T)), op=vb.NODE_CPY, srcs=(g.view(packed, (K, T), rows_nb, packed.nb[1]),))
    cpu_ids.src[1] = C.pointer(cpu_ids)                  # ggml_cast: a CPY node's src[1] is itself
    cold_weights = g.view(packed, (1, K, T), [4, 4, packed.nb[2], packed.nb[2] * T], 2 * packed.nb[1])
    dims = (Hd, I, K, T)
    resident = weighted_branch(vb, g, new, X, gpu_ids, gpu_ids, weights,
                               g.expert_tensor(gu_bank, H.MX, Hd, 2 * I, n_slots + 1), g.leaf(F32, (2 * I, n_slots + 1), dgub.ptr),
                               g.expert_tensor(dn_bank, H.MX, I, Hd, n_slots + 1), g.leaf(F32, (Hd, n_slots + 1), ddnb.ptr), dims)
    host = weighted_branch(vb, g, new, X, cpu_ids, selected, cold_weights,
                           g.expert_tensor(layer.gu_bank, H.MX, Hd, 2 * I, E), g.leaf(F32, (2 * I, E), layer.d_gu_b.ptr),
                           g.expert_tensor(layer.dn_bank, H.MX, I, Hd, E), g.leaf(F32, (Hd, E), layer.d_dn_b.ptr), dims)
    joined = g.tensor(F32, (Hd, K, T), new((Hd, K, T)), op=vb.NODE_ADD, srcs=(resident, host))
    output = None
    for rank in range(K):
        row = g.view(joined, (Hd, T), [4, joined.nb[2], joined.nb[2] * T, joined.nb[2] * T], rank * joined.nb[1])
        output = row if output is None else g.tensor(F32, (Hd, T), new((Hd, T)), op=vb.NODE_ADD, srcs=(output, row))
    final = g.tensor(F32, (Hd, T), new((Hd, T)), op=vb.NODE_CONT, srcs=(output,))
    for n in g.nodes:
        assert g.supported(n), n.op
    g.compute(order=vb.ORDER_EXACT)
    vb.call("vbm_stream_synchronize", None)
    got_gpu_ids = download(vb, gpu_ids.data, (T, K), np.int32)
    assert np.array_equal(got_gpu_ids, packet[:, 1, :].astype(np.int32))
    assert np.array_equal(download(vb, cpu_ids.data, (T, K), np.int32), packet[:, 0, :].astype(np.int32))
    out = download(vb, final.data, (T, Hd))
    assert H.bits_equal(out, ref["out"]), H.diff_report(out, ref["out"])
    gu_bank.destroy()
    dn_bank.destroy()
    layer.destroy()


@pytest.mark.parametrize("b_type", [F32, H.Q8])
def test_node_mul_mat_id_strided_views_match_flat_call(gpu, orc, b_type):
    """MUL_MAT_ID nodes whose b and ids are views into wider buffers (b rows with a padded stride,
    broadcast [k, 1, T] and per-rank [k, n_ids, T]; ids with a token stride) give the flat entry
    point's bits on contiguous copies; a Q8_0 b view with padding is refused."""
    vb = gpu
    k, rows, E, K, T = 256, 64, 6, 3, 5
    w = H.synth_weights(H.MX, 8, 1, E, rows, k)
    bank = H.make_bank(H.MX, w, E, rows, k)
    rng = np.random.default_rng(8)
    ids = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    ids_wide = np.concatenate([ids, np.full((T, 2), -7, np.int32)], axis=1)
    for b_ne1 in (1, K):
        pad = 64
        if b_type == F32:
            xb = rng.standard_normal((T, b_ne1, k + pad)).astype(np.float32)
            flat = np.ascontiguousarray(xb[:, :, :k])
            nb = [4, 4 * (k + pad), 4 * (k + pad) * b_ne1, 4 * (k + pad) * b_ne1 * T]
        else:
            xf = rng.standard_normal((T * b_ne1, k)).astype(np.float32)
            flat = orc.quantize_q8_0(xf).reshape(T, b_ne1, (k // 32) * 34)
            xb = flat
            nb = [34, (k // 32) * 34, (k // 32) * 34 * b_ne1, (k // 32) * 34 * b_ne1 * T]
        ref = H.mul_mat_id(bank, E, flat, b_type, b_ne1, ids, K)
        dxb, dids = vb.DeviceBuffer.from_array(xb), vb.DeviceBuffer.from_array(ids_wide)
        dst = vb.DeviceBuffer(4 * T * K * rows)
        g = Graph(vb)
        as_ = g.expert_tensor(bank, H.MX, k, rows, E)
        b = g.leaf(b_type, (k, b_ne1, T), dxb.ptr, nb=nb)
        idn = g.leaf(I32, (K, T), dids.ptr, nb=[4, 4 * (K + 2), 4 * (K + 2) * T, 4 * (K + 2) * T])
        node = g.tensor(F32, (rows, K, T), dst.ptr, op=vb.NODE_MUL_MAT_ID, srcs=(as_, b, idn))
        assert g.supported(node)
        g.compute()
        vb.call("vbm_stream_synchronize", None)
        got = download(vb, dst.ptr, (T, K, rows))
        assert H.bits_equal(got, ref), (b_ne1, H.diff_report(got, ref))
        if b_type == H.Q8:
            b.nb[1] = (k // 32) * 34 + 34          # a padded Q8_0 view is refused, never misread
            b.nb[2] = b.nb[1] * b_ne1
            b.nb[3] = b.nb[2] * T
            assert not g.supported(node)
    bank.destroy()


def test_node_elementwise_and_add_id_on_views(gpu):
    """ADD / MUL with broadcast over permuted and strided views, CONT of a transposed view, and an
    ADD_ID node writing a separate dst (an out-of-range id poisons its row with NaN), against numpy."""
    vb = gpu
    rng = np.random.default_rng(21)
    a = rng.standard_normal((4, 6, 10)).astype(np.float32)        # ggml ne [10, 6, 4]
    b = rng.standard_normal((4, 1, 10)).astype(np.float32)        # ne [10, 1, 4]: repeats over dim 1
    da, db = vb.DeviceBuffer.from_array(a), vb.DeviceBuffer.from_array(b)
    out_add, out_mul, out_cont = (vb.DeviceBuffer(4 * a.size) for _ in range(3))
    g = Graph(vb)
    A = g.leaf(F32, (10, 6, 4), da.ptr)
    B = g.leaf(F32, (10, 1, 4), db.ptr)
    g.tensor(F32, (10, 6, 4), out_add.ptr, op=vb.NODE_ADD, srcs=(A, B))
    # a permuted view of A: ne [6, 10, 4] (dims 0 and 1 swapped), times a broadcast row
    At = g.view(A, (6, 10, 4), [A.nb[1], A.nb[0], A.nb[2], A.nb[3]], 0)
    row = rng.standard_normal(6).astype(np.float32)
    drow = vb.DeviceBuffer.from_array(row)
    R = g.leaf(F32, (6, 1, 1), drow.ptr)
    g.tensor(F32, (6, 10, 4), out_mul.ptr, op=vb.NODE_MUL, srcs=(At, R))
    g.tensor(F32, (6, 10, 4), out_cont.ptr, op=vb.NODE_CONT, srcs=(At,))
    # ADD_ID: y [8, 3, 5] + bias[:, ids], ids with -1 and one out-of-range entry
    y = rng.standard_normal((5, 3, 8)).astype(np.float32)
    bias = rng.standard_normal((4, 8)).astype(np.float32)
    ids = rng.integers(0, 4, (5, 3)).astype(np.int32)
    ids[1, 2], ids[3, 0] = -1, 4
    dy, dbias, dids, dout = (vb.DeviceBuffer.from_array(v) for v in (y, bias, ids, np.zeros_like(y)))
    Y, Bi, Id = g.leaf(F32, (8, 3, 5), dy.ptr), g.leaf(F32, (8, 4), dbias.ptr), g.leaf(I32, (3, 5), dids.ptr)
    g.tensor(F32, (8, 3, 5), dout.ptr, op=vb.NODE_ADD_ID, srcs=(Y, Bi, Id))
    g.compute()
    vb.call("vbm_stream_synchronize", None)
    assert H.bits_equal(download(vb, out_add.ptr, a.shape), a + b)
    at = np.ascontiguousarray(a.transpose(0, 2, 1))                 # numpy [4, 10, 6] = ggml ne [6, 10, 4]
    assert H.bits_equal(download(vb, out_mul.ptr, at.shape), at * row)
    assert H.bits_equal(download(vb, out_cont.ptr, at.shape), at)
    got = download(vb, dout.ptr, y.shape)
    ref = y.copy()
    for t in range(5):
        for r in range(3):
            if 0 <= ids[t, r] < 4:
                ref[t, r] = y[t, r] + bias[ids[t, r]]
    assert np.all(np.isnan(got[3, 0])) and H.bits_equal(got[1, 2], y[1, 2])
    keep = np.ones((5, 3), bool)
    keep[3, 0] = False
    assert H.bits_equal(got[keep], ref[keep])
    assert H.bits_equal(download(vb, dy.ptr, y.shape), y)           # the source is not modified


def test_node_cpy_casts_on_views(gpu):
    """CPY nodes (ggml_cast) F32 -> I32 from a transposed view (truncation toward zero, saturation
    and NaN -> 0 where C leaves the conversion undefined), I32 -> F32 (round to nearest), and the
    same-type copies, into contiguous destinations, against numpy."""
    vb = gpu
    f = np.array([[0.0, -0.0, 1.5, -1.5, 2.999, -2.999, 7.0, -128.0],
                  [3e9, -3e9, np.nan, 16777217.0, 0.49, -0.51, 12.0, 1e-40]], np.float32)   # ne [8, 2]
    i = np.array([[0, -1, 16777217, -16777219, 2147483647, -2147483648, 5, 7]], np.int32)  # ne [8, 1]
    df, di = vb.DeviceBuffer.from_array(f), vb.DeviceBuffer.from_array(i)
    outs = [vb.DeviceBuffer(64) for _ in range(4)]
    g = Graph(vb)
    F = g.leaf(F32, (8, 2), df.ptr)
    Ft = g.view(F, (2, 8), [F.nb[1], F.nb[0], F.nb[2], F.nb[3]], 0)       # ne [2, 8]: transposed
    I = g.leaf(I32, (8, 1), di.ptr)
    g.tensor(I32, (2, 8), outs[0].ptr, op=vb.NODE_CPY, srcs=(Ft,))
    g.tensor(F32, (8, 1), outs[1].ptr, op=vb.NODE_CPY, srcs=(I,))
    g.tensor(F32, (2, 8), outs[2].ptr, op=vb.NODE_CPY, srcs=(Ft,))
    g.tensor(I32, (8, 1), outs[3].ptr, op=vb.NODE_CPY, srcs=(I,))
    for n in g.nodes:
        assert g.supported(n)
    g.compute()
    vb.call("vbm_stream_synchronize", None)
    ft = np.ascontiguousarray(f.T).astype(np.float64)                   # numpy [8, 2] = ggml ne [2, 8]
    want = np.where(np.isnan(ft), 0, np.clip(np.trunc(np.nan_to_num(ft)), -2**31, 2**31 - 1)).astype(np.int64)
    assert np.array_equal(download(vb, outs[0].ptr, ft.shape, np.int32), want.astype(np.int32))
    assert H.bits_equal(download(vb, outs[1].ptr, i.shape), i.astype(np.float32))
    assert H.bits_equal(download(vb, outs[2].ptr, ft.shape), np.ascontiguousarray(f.T))
    assert np.array_equal(download(vb, outs[3].ptr, i.shape, np.int32), i)


@pytest.mark.parametrize("mode", [0, 1])
def test_node_host_call_and_join(gpu, mode):
    """A CUSTOM host-call node (fn: 2a + b on the host) and its join node (call output + c) through
    vbm_graph_compute, in both host-call modes."""
    from test_host_call import AxpyCall
    vb = gpu
    n = 2048
    rng = np.random.default_rng(30 + mode)
    a_h, b_h, c_h = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    a, b, c = (vb.DeviceBuffer.from_array(v) for v in (a_h, b_h, c_h))
    mid, out = vb.DeviceBuffer(4 * n), vb.DeviceBuffer(4 * n)
    call = AxpyCall(vb, n)
    join = vb.HostCall()
    join.magic = vb.HOST_JOIN_MAGIC
    join.call = C.pointer(call.call)
    g = Graph(vb)
    A, B, Cn = g.leaf(F32, (n,), a.ptr), g.leaf(F32, (n,), b.ptr), g.leaf(F32, (n,), c.ptr)
    node = g.tensor(F32, (n,), mid.ptr, op=vb.NODE_CUSTOM, srcs=(A, B), extra=C.addressof(call.call))
    g.tensor(F32, (n,), out.ptr, op=vb.NODE_CUSTOM, srcs=(node, Cn), extra=C.addressof(join))
    g.compute(mode=mode)
    vb.call("vbm_stream_synchronize", None)
    assert np.array_equal(out.download(np.float32, n), (2 * a_h + b_h) + c_h)
    assert call.runs == 1
    call.release()
