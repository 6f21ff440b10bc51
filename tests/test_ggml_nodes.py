"""supports_op over ggml-layout nodes (vbm_node_supported) on the CPU: the types, shapes and byte
strides the library accepts for each node of the reference's routed-expert branch
(third_party/patches/llama-b11669-hybrid-experts.patch:1394-1683, :1905-1916, :963-983), and the
views it must refuse rather than misread. No device work: the predicate is host code, and
compute_forward refuses an unsupported node before touching the device."""
import ctypes as C

import pytest

from ggml_graph import Graph, contiguous_nb

F32, F16, Q8, I32, MX = 0, 1, 8, 26, 39
FAKE = 0x10000          # an aligned stand-in address; nothing is dereferenced


@pytest.fixture()
def g(vb):
    return Graph(vb)


def mmid(vb, g, as_type=MX, k=2880, rows=5760, n_as=128, b_type=F32, b_ne=None, b_nb=None, n_ids=4, T=7,
         ids_nb=None, dst_nb=None):
    as_ = g.leaf(as_type, (k, rows, n_as), None)
    b = g.leaf(b_type, b_ne or (k, 1, T), FAKE, nb=b_nb)
    ids = g.leaf(I32, (n_ids, T), FAKE, nb=ids_nb)
    return g.tensor(F32, (rows, n_ids, T), FAKE, op=vb.NODE_MUL_MAT_ID, srcs=(as_, b, ids), nb=dst_nb)


def test_mul_mat_id_rules(vb, g):
    ok = g.supported
    assert ok(mmid(vb, g))
    assert ok(mmid(vb, g, as_type=Q8, k=2048, rows=1536, b_type=Q8, b_ne=(2048, 8, 512), n_ids=8, T=512))
    assert ok(mmid(vb, g, b_ne=(2880, 4, 7)))                                           # per-rank b
    # ids: a top-k view of a wider argsort (token stride 32 ints)
    assert ok(mmid(vb, g, ids_nb=[4, 128, 128 * 7, 128 * 7]))
    # F32 b rows with a padded stride: broadcast [k, 1, T] and per-rank [k, n_ids, T]
    assert ok(mmid(vb, g, b_nb=[4, 4 * 3000, 4 * 3000, 4 * 3000 * 7]))
    assert ok(mmid(vb, g, b_ne=(2880, 4, 7), b_nb=[4, 4 * 3000, 4 * 3000 * 4, 4 * 3000 * 28]))
    # refused: rows not evenly spaced, element stride, overlapping rows, Q8_0 with padding
    assert not ok(mmid(vb, g, b_ne=(2880, 4, 7), b_nb=[4, 4 * 3000, 4 * 3000 * 5, 4 * 3000 * 35]))
    assert not ok(mmid(vb, g, b_nb=[8, 8 * 2880, 8 * 2880, 8 * 2880 * 7]))
    assert not ok(mmid(vb, g, b_nb=[4, 4 * 2000, 4 * 2000, 4 * 2000 * 7]))
    assert not ok(mmid(vb, g, as_type=Q8, k=2048, rows=1536, b_type=Q8, b_ne=(2048, 1, 7),
                       b_nb=[34, 64 * 34 + 34, 64 * 34 + 34, (64 * 34 + 34) * 7]))
    # ids: element stride or a token stride shorter than n_ids
    assert not ok(mmid(vb, g, ids_nb=[8, 64, 64 * 7, 64 * 7]))
    assert not ok(mmid(vb, g, ids_nb=[4, 12, 12 * 7, 12 * 7]))
    # dst must be contiguous
    assert not ok(mmid(vb, g, dst_nb=[4, 4 * 5760 * 2, 4 * 5760 * 8, 4 * 5760 * 56]))
    # types and shapes
    assert not ok(mmid(vb, g, as_type=F16))
    assert not ok(mmid(vb, g, b_type=F16))
    assert not ok(mmid(vb, g, b_ne=(2816, 1, 7)))                                       # k mismatch
    assert not ok(mmid(vb, g, k=2848, b_ne=(2848, 1, 7)))                               # k % 64
    assert not ok(mmid(vb, g, rows=5750))                                               # rows % 32
    assert not ok(mmid(vb, g, n_as=2048))                                               # > 1024 experts
    assert not ok(mmid(vb, g, b_ne=(2880, 3, 7)))                                       # b_ne1 not 1 or n_ids
    node = mmid(vb, g)
    node.src[2] = None
    assert not ok(node)


def glu(vb, g, gate_nb=None, up_nb=None, op=None, split=True, width=2880, rows=4, T=7):
    gu = g.leaf(F32, (2 * width, rows, T), FAKE)
    gnb = gate_nb or list(gu.nb)
    gate = g.view(gu, (width, rows, T) if split else (2 * width, rows, T), gnb, 0)
    up = g.view(gu, (width, rows, T), up_nb or list(gu.nb), 4 * width) if split else None
    params = (op if op is not None else vb.GLU_OP_SWIGLU_OAI, 0)
    return g.tensor(F32, (width, rows, T), FAKE, op=vb.NODE_GLU, srcs=(gate, up), params=params)


def test_glu_rules(vb, g):
    ok = g.supported
    assert ok(glu(vb, g))                                      # split views of the fused gate_up output
    assert ok(glu(vb, g, op=vb.GLU_OP_SWIGLU))
    assert ok(glu(vb, g, split=False))                         # one [2I] operand, halves split inside
    assert not ok(glu(vb, g, op=0))                            # reglu
    assert not ok(glu(vb, g, op=1))                            # geglu
    w = 2880
    assert not ok(glu(vb, g, gate_nb=[4, 8 * w, 8 * w * 5, 8 * w * 35]))     # rows not evenly spaced
    assert not ok(glu(vb, g, up_nb=[8, 8 * w, 8 * w * 4, 8 * w * 28]))       # element stride


def test_elementwise_and_add_id_rules(vb, g):
    ok = g.supported
    y = g.leaf(F32, (2880, 4, 7), FAKE)
    w = g.leaf(F32, (1, 4, 7), FAKE)
    assert ok(g.tensor(F32, (2880, 4, 7), FAKE, op=vb.NODE_MUL, srcs=(y, w)))          # weights broadcast
    assert not ok(g.tensor(F32, (2880, 4, 7), FAKE, op=vb.NODE_MUL, srcs=(y, g.leaf(F32, (1, 3, 7), FAKE))))
    assert not ok(g.tensor(F32, (2880, 4, 6), FAKE, op=vb.NODE_ADD, srcs=(y, y)))       # dst shape
    assert not ok(g.tensor(F16, (2880, 4, 7), FAKE, op=vb.NODE_ADD, srcs=(y, y)))
    rank = g.view(y, (2880, 7), [4, y.nb[2], y.nb[2] * 7, y.nb[2] * 7], 2 * y.nb[1])  # a strided rank view
    assert ok(g.tensor(F32, (2880, 7), FAKE, op=vb.NODE_ADD, srcs=(rank, rank)))
    assert ok(g.tensor(F32, (2880, 7), FAKE, op=vb.NODE_CONT, srcs=(rank,)))
    assert not ok(g.tensor(F32, (2880, 7), FAKE, op=vb.NODE_CONT, srcs=(rank,), nb=list(rank.nb)))  # strided dst
    odd = g.view(y, (2880, 7), [4, 6, 6 * 7, 6 * 7], 0)
    assert not ok(g.tensor(F32, (2880, 7), FAKE, op=vb.NODE_ADD, srcs=(odd, odd)))      # 2-byte misaligned stride
    bias = g.leaf(F32, (2880, 128), FAKE)
    ids = g.leaf(I32, (4, 7), FAKE, nb=[4, 32, 32 * 7, 32 * 7])
    assert ok(g.tensor(F32, (2880, 4, 7), FAKE, op=vb.NODE_ADD_ID, srcs=(y, bias, ids)))
    assert not ok(g.tensor(F32, (2880, 4, 7), FAKE, op=vb.NODE_ADD_ID, srcs=(y, g.leaf(F32, (2816, 128), FAKE), ids)))
    assert not ok(g.tensor(F32, (2880, 4, 7), FAKE, op=vb.NODE_ADD_ID, srcs=(y, bias, g.leaf(I32, (3, 7), FAKE))))
    assert ok(g.leaf(F32, (1,), FAKE)) and ok(rank)                                     # leaves and views
    assert not ok(g.tensor(F32, (1,), FAKE, op=99))


def test_custom_rules(vb, g):
    ok = g.supported
    a, b = g.leaf(F32, (64,), FAKE), g.leaf(F32, (64,), FAKE)
    call = vb.HostCall()
    call.magic = vb.HOST_CALL_MAGIC
    call.src_host[0] = call.src_host[1] = FAKE
    node = g.tensor(F32, (64,), FAKE, op=vb.NODE_CUSTOM, srcs=(a, b), extra=C.addressof(call))
    assert not ok(node)                                    # no output host buffer
    call.dst_host = FAKE
    assert ok(node)
    call.src_host[1] = None
    assert not ok(node)                                    # an input without a host buffer
    call.src_host[1] = FAKE
    call.miss_src = 2
    assert not ok(node)                                    # miss_src must name an I32 input
    node.src[1] = C.pointer(g.leaf(I32, (64,), FAKE))
    assert ok(node)
    strided = g.view(a, (32,), [8, 8 * 32, 8 * 32, 8 * 32], 0)
    node.src[0] = C.pointer(strided)
    assert not ok(node)                                    # inputs must be contiguous
    join = vb.HostCall()
    join.magic = vb.HOST_JOIN_MAGIC
    jn = g.tensor(F32, (64,), FAKE, op=vb.NODE_CUSTOM, srcs=(a, b), extra=C.addressof(join))
    assert not ok(jn)                                      # names no call
    join.call = C.pointer(call)
    assert ok(jn)
    assert not ok(g.tensor(F32, (64,), FAKE, op=vb.NODE_CUSTOM, srcs=(a, g.leaf(F32, (32, 2), FAKE)),
                           extra=C.addressof(join)))       # join operands of another shape
    assert not ok(g.tensor(F32, (64,), FAKE, op=vb.NODE_CUSTOM, srcs=(a, b)))           # no descriptor


def test_cpy_rules(vb, g):
    ok = g.supported
    packed = g.leaf(F32, (4, 4, 7), FAKE)                                   # a dispatch packet [K, 4, T]
    row = g.view(packed, (4, 7), [4, packed.nb[2], packed.nb[2] * 7, packed.nb[2] * 7], packed.nb[1])
    cast = g.tensor(I32, (4, 7), FAKE, op=vb.NODE_CPY, srcs=(row,))
    cast.src[1] = C.pointer(cast)                                            # ggml_cast names itself
    assert ok(cast)
    assert ok(g.tensor(F32, (4, 7), FAKE, op=vb.NODE_CPY, srcs=(g.leaf(I32, (4, 7), FAKE),)))
    assert ok(g.tensor(F32, (28,), FAKE, op=vb.NODE_CPY, srcs=(row,)))       # same element count
    assert not ok(g.tensor(F16, (4, 7), FAKE, op=vb.NODE_CPY, srcs=(row,)))
    assert not ok(g.tensor(I32, (4, 6), FAKE, op=vb.NODE_CPY, srcs=(row,)))
    assert not ok(g.tensor(I32, (4, 7), FAKE, op=vb.NODE_CPY, srcs=(row,), nb=[4, 32, 32 * 7, 32 * 7]))  # strided dst
    assert not ok(g.tensor(I32, (4, 7), FAKE, op=vb.NODE_CPY, srcs=(g.view(packed, (4, 7), [2, 64, 448, 448], 0),)))


def test_compute_forward_refuses_unsupported_nodes_before_device_work(vb, g):
    node = mmid(vb, g, rows=5750)
    with pytest.raises(vb.VbmError, match="rows % 32"):
        vb.call("vbm_compute_forward", C.byref(node), None, None)
    bad = g.tensor(F32, (2880, 7), FAKE, op=vb.NODE_ADD, srcs=(g.leaf(F32, (2880, 7), FAKE), g.leaf(F32, (7, 7), FAKE)))
    arr = (C.POINTER(vb.Node) * 2)(C.pointer(g.leaf(F32, (4,), FAKE)), C.pointer(bad))
    with pytest.raises(vb.VbmError, match="node 1: src1 must repeat"):
        vb.call("vbm_graph_compute", arr, 2, None, None)
    # a supported MUL_MAT_ID whose expert tensor has no bank bound
    node = mmid(vb, g)
    with pytest.raises(vb.VbmError, match="no bank bound"):
        vb.call("vbm_compute_forward", C.byref(node), None, None)


def test_contiguous_strides_helper():
    assert contiguous_nb(MX, [2880, 5760, 128, 1]) == [17, 90 * 17, 90 * 17 * 5760, 90 * 17 * 5760 * 128]
    assert contiguous_nb(F32, [3, 4, 5, 1]) == [4, 12, 48, 240]
