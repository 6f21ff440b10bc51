"""Builds ggml-layout node lists (vbm_node) for the tests, the way a ggml backend adapter copies
its tensors' fields: type, ne, nb (bytes), data, op, op_params, src[], extra."""
import ctypes as C
import struct

TYPE_BLOCK = {0: (1, 4), 1: (1, 2), 26: (1, 4), 8: (32, 34), 39: (32, 17)}


def contiguous_nb(type_id, ne):
    blck, size = TYPE_BLOCK[type_id]
    nb = [size, size * (ne[0] // blck)]
    nb.append(nb[1] * ne[1])
    nb.append(nb[2] * ne[2])
    return nb


def f32_bits(v):
    return struct.unpack("<i", struct.pack("<f", v))[0]


class Graph:
    """Keeps every node (and its ctypes storage) alive; `nodes` lists the compute order."""

    def __init__(self, vb):
        self.vb = vb
        self.keep = []
        self.nodes = []

    def tensor(self, type_id, ne, data, op=0, srcs=(), nb=None, extra=None, params=(), compute=True):
        vb = self.vb
        ne = list(ne) + [1] * (4 - len(ne))
        n = vb.Node()
        n.op, n.type = op, type_id
        for d in range(4):
            n.ne[d] = ne[d]
        for d, v in enumerate(nb if nb is not None else contiguous_nb(type_id, ne)):
            n.nb[d] = v
        n.data = data
        n.extra = extra
        for i, v in enumerate(params):
            n.op_params[i] = v
        for i, s in enumerate(srcs):
            n.src[i] = C.pointer(s) if s is not None else None
        self.keep.append(n)
        if compute and op not in (vb.NODE_NONE, vb.NODE_VIEW):
            self.nodes.append(n)
        return n

    def leaf(self, type_id, ne, data, nb=None, extra=None):
        return self.tensor(type_id, ne, data, nb=nb, extra=extra)

    def view(self, src, ne, nb, offset):
        return self.tensor(src.type, ne, (src.data or 0) + offset, op=self.vb.NODE_VIEW, srcs=(src,), nb=nb)

    def expert_tensor(self, bank, type_id, k, rows, n_as, slot_map=None, slot_map_host=None):
        binding = self.vb.ExpertTensor(bank.handle, slot_map, slot_map_host)
        self.keep.append(binding)
        return self.leaf(type_id, (k, rows, n_as), None, extra=C.addressof(binding))

    def supported(self, node):
        return self.vb.load().vbm_node_supported(C.byref(node))

    def compute(self, order=0, mode=0, stream=None):
        arr = (C.POINTER(self.vb.Node) * len(self.nodes))(*[C.pointer(n) for n in self.nodes])
        params = self.vb.ComputeParams(order, mode)
        self.vb.call("vbm_graph_compute", arr, len(self.nodes), C.byref(params), stream)
