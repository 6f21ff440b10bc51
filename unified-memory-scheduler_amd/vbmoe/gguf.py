"""GGUF expert tensors through libvbmoe (vbm_gguf_*, include/vbmoe.h): open a file or its shards,
query metadata and tensor shapes, read one expert's ggml bytes and biases, or load experts
straight into device banks. Nothing here touches the GPU except `load_layer`."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import GgufExpertInfo, call, load


class GgufFile:
    def __init__(self, path: str | Path):
        load()
        h = C.c_void_p()
        call("vbm_gguf_open", str(path).encode(), C.byref(h))
        self.handle = h.value

    def close(self) -> None:
        if self.handle:
            call("vbm_gguf_close", self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False

    def shards(self) -> tuple[int, int]:
        s, t = C.c_int64(), C.c_int64()
        call("vbm_gguf_shards", self.handle, C.byref(s), C.byref(t))
        return s.value, t.value

    def get_u64(self, key: str):
        v, found = C.c_uint64(), C.c_int()
        call("vbm_gguf_get_u64", self.handle, key.encode(), C.byref(v), C.byref(found))
        return v.value if found.value else None

    def get_string(self, key: str, capacity: int = 4096):
        buf, found = C.create_string_buffer(capacity), C.c_int()
        call("vbm_gguf_get_string", self.handle, key.encode(), buf, capacity, C.byref(found))
        return buf.value.decode() if found.value else None

    def tensor(self, name: str):
        t, ne, nb, found = C.c_int(), (C.c_int64 * 4)(), C.c_uint64(), C.c_int()
        call("vbm_gguf_tensor_info", self.handle, name.encode(), C.byref(t), ne, C.byref(nb), C.byref(found))
        return (t.value, tuple(ne), nb.value) if found.value else None

    def expert_info(self, layer: int) -> GgufExpertInfo:
        info = GgufExpertInfo()
        call("vbm_gguf_expert_layer_info", self.handle, layer, C.byref(info))
        return info

    def read_expert(self, layer: int, expert: int):
        """(gate|up ggml bytes, down ggml bytes, gate|up fp32 biases, down fp32 biases)."""
        info = self.expert_info(layer)
        gu = np.empty(info.gate_up_bytes, np.uint8)
        dn = np.empty(info.down_bytes, np.uint8)
        bgu = np.empty(2 * info.intermediate, np.float32)
        bdn = np.empty(info.hidden, np.float32)
        call("vbm_gguf_read_expert", self.handle, layer, expert, gu.ctypes.data, dn.ctypes.data,
             bgu.ctypes.data, bdn.ctypes.data)
        return gu, dn, bgu, bdn

    def load_layer(self, layer: int, experts, gate_up_bank, down_bank, slots=None, gate_up_bias=None,
                   down_bias=None, stream=None) -> None:
        ids = np.ascontiguousarray(experts, dtype=np.int32)
        sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.int32)
        call("vbm_gguf_load_layer", self.handle, layer, ids.ctypes.data, None if sl is None else sl.ctypes.data,
             ids.size, gate_up_bank.handle, down_bank.handle, gate_up_bias, down_bias, stream)
