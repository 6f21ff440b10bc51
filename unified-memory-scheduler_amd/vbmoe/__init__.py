"""ctypes binding of libvbmoe.so (include/vbmoe.h) plus small numpy helpers.

The library is the product; this module only declares its C signatures and wraps device
buffers. Importing it never touches the GPU; `load()` raises if libvbmoe.so is missing, so
callers fail loudly rather than fall back to anything else.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libvbmoe.so"
HEADER = Path(__file__).resolve().parents[2] / "include" / "vbmoe.h"

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_I32, TYPE_MXFP4 = 0, 1, 8, 26, 39
ACT_SILU, ACT_SWIGLU_OAI = 0, 1
ORDER_EXACT, ORDER_FAST = 0, 1
STATUS = {0: "OK", 1: "INVALID_ARGUMENT", 2: "RUNTIME", 3: "UNSUPPORTED", 4: "OUT_OF_MEMORY"}

vp, sz, i64, u64, i32p, f32p = C.c_void_p, C.c_size_t, C.c_int64, C.c_uint64, C.c_void_p, C.c_void_p


class TierDesc(C.Structure):
    _fields_ = [
        ("type", C.c_int), ("hidden", i64), ("intermediate", i64), ("n_layers", i64), ("n_expert", i64),
        ("top_k", i64), ("activation", C.c_int), ("n_slots", i64), ("recent_window", i64), ("margin", C.c_int32),
        ("policy", C.c_int), ("gate_up_bias", C.POINTER(vp)), ("down_bias", C.POINTER(vp)),
    ]


class TierStats(C.Structure):
    _fields_ = [
        ("dispatches", u64), ("hits", u64), ("admissions", u64), ("evictions", u64), ("staged", u64),
        ("uploaded_bytes", u64), ("copy_ms", C.c_double), ("prefill_tokens", u64), ("prefill_resident", u64),
        ("prefill_streamed", u64), ("host_reads", u64), ("device_copy_bytes", u64),
    ]


class TraceLayer(C.Structure):
    _fields_ = [
        ("id", i64), ("experts", i64), ("active", i64), ("bytes_per_expert", u64),
        ("static_host_bytes_per_expert", u64), ("tensor_types", C.c_char_p),
    ]


class GgufExpertInfo(C.Structure):
    _fields_ = [
        ("hidden", i64), ("intermediate", i64), ("n_expert", i64), ("gate_up_type", C.c_int), ("down_type", C.c_int),
        ("fused_gate_up", C.c_int), ("has_bias", C.c_int), ("gate_up_bytes", u64), ("down_bytes", u64),
    ]


HOST_CALL_MAGIC, HOST_JOIN_MAGIC, HOST_MAX_SRC = 0x56424843414C4C31, 0x5642484A4F494E31, 10
HOST_CALL_FUNC, HOST_CALL_MAILBOX = 0, 1
NODE_NONE, NODE_VIEW, NODE_ADD, NODE_MUL, NODE_CONT, NODE_MUL_MAT_ID, NODE_ADD_ID, NODE_GLU, NODE_CUSTOM, NODE_CPY = range(10)
NODE_MAX_SRC = 10
GLU_OP_SWIGLU, GLU_OP_SWIGLU_OAI = 2, 3
HOST_FN = C.CFUNCTYPE(None, C.c_void_p)


class HostCall(C.Structure):
    pass


HostCall._fields_ = [
    ("magic", u64), ("fn", HOST_FN), ("ctx", vp), ("src_host", vp * HOST_MAX_SRC), ("dst_host", vp),
    ("backend_state", vp), ("call", C.POINTER(HostCall)), ("miss_src", C.c_int32),
]


class Node(C.Structure):
    """vbm_node: a ggml-layout graph node (type, ne, nb in bytes, data, op_params, src)."""


Node._fields_ = [
    ("op", C.c_int32), ("type", C.c_int32), ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("data", vp), ("extra", vp),
    ("op_params", C.c_int32 * 16), ("src", C.POINTER(Node) * NODE_MAX_SRC),
]


class ExpertTensor(C.Structure):
    _fields_ = [("bank", vp), ("expert_to_slot", vp), ("expert_to_slot_host", vp)]


class ComputeParams(C.Structure):
    _fields_ = [("order", C.c_int32), ("host_call_mode", C.c_int32)]


class ResidencyLayer(C.Structure):
    _fields_ = [("experts", i64), ("bytes_per_expert", u64), ("static_host_bytes_per_expert", u64)]


class ResidencyParams(C.Structure):
    _fields_ = [
        ("policy", C.c_int), ("capacity_bytes", u64), ("admit_after", C.c_int), ("payback_tokens", i64),
        ("cold_cache", C.c_int), ("ram_gbps", C.c_double), ("pcie_gbps", C.c_double), ("gpu_expert_us", C.c_double),
        ("layer_sync_us", C.c_double), ("staging_ram_passes", C.c_int), ("static_device_expert_bytes", u64),
    ]


class ResidencyTotals(C.Structure):
    _fields_ = [
        ("supported", C.c_int), ("expert_calls", u64), ("full_hits", u64), ("bytes", u64), ("cold_bytes", u64),
        ("upload_bytes", u64), ("evictions", u64), ("serial_s", C.c_double), ("optimistic_s", C.c_double),
        ("shared_ram_bytes", C.c_double), ("warmup_upload_bytes", u64), ("initial_bytes", u64), ("rejected", u64),
        ("warmup_rejected", u64),
    ]


class MoeLayerDesc(C.Structure):
    _fields_ = [
        ("gate_up", vp), ("down", vp), ("gate_up_bias", vp), ("down_bias", vp), ("expert_to_slot", vp),
        ("router_w", vp), ("router_b", vp), ("hidden", i64), ("intermediate", i64), ("n_expert", i64),
        ("top_k", i64), ("activation", C.c_int), ("order", C.c_int),
    ]


# name -> argtypes (all return vbm_status as c_int)
SIGNATURES = {
    "vbm_device_count": [C.POINTER(C.c_int)],
    "vbm_set_device": [C.c_int],
    "vbm_device_name": [C.c_int, C.c_char_p, sz],
    "vbm_mem_info": [C.POINTER(sz), C.POINTER(sz)],
    "vbm_malloc": [C.POINTER(vp), sz],
    "vbm_free": [vp],
    "vbm_host_alloc": [C.POINTER(vp), sz],
    "vbm_host_free": [vp],
    "vbm_memcpy_h2d": [vp, vp, sz, vp],
    "vbm_memcpy_d2h": [vp, vp, sz, vp],
    "vbm_memcpy_d2d": [vp, vp, sz, vp],
    "vbm_memset": [vp, C.c_int, sz, vp],
    "vbm_stream_create": [C.POINTER(vp)],
    "vbm_stream_destroy": [vp],
    "vbm_stream_synchronize": [vp],
    "vbm_device_synchronize": [],
    "vbm_event_create": [C.POINTER(vp)],
    "vbm_event_destroy": [vp],
    "vbm_event_record": [vp, vp],
    "vbm_event_synchronize": [vp],
    "vbm_event_query": [vp, C.POINTER(C.c_int)],
    "vbm_event_elapsed_ms": [vp, vp, C.POINTER(C.c_float)],
    "vbm_synth_mxfp4_host": [u64, u64, u64, u64, C.c_int, C.c_int, vp],
    "vbm_synth_q8_0_host": [u64, u64, u64, u64, C.c_float, C.c_float, vp],
    "vbm_synth_normal_host": [u64, u64, u64, u64, C.c_float, C.c_float, vp],
    "vbm_bank_create": [C.c_int, i64, i64, i64, C.c_int, C.POINTER(vp)],
    "vbm_bank_destroy": [vp],
    "vbm_bank_info": [vp, C.POINTER(C.c_int), C.POINTER(i64), C.POINTER(i64), C.POINTER(i64), C.POINTER(sz),
                      C.POINTER(vp)],
    "vbm_bank_upload": [vp, i64, vp, C.c_int, vp],
    "vbm_bank_export": [vp, i64, vp, sz, vp],
    "vbm_bank_generate": [vp, i64, i64, u64, u64, i64, C.c_float, C.c_float, vp],
    "vbm_quantize_q8_0": [vp, i64, i64, i64, vp, vp],
    "vbm_mul_mat_id": [vp, vp, vp, i64, C.c_int, vp, i64, vp, i64, i64, i64, vp, vp, C.c_int, vp],
    "vbm_mul_mat_id_workspace": [vp, i64, i64, i64, i64, C.c_int, C.POINTER(C.c_size_t)],
    "vbm_mul_mat_id_ws": [vp, vp, vp, i64, C.c_int, vp, i64, vp, i64, i64, i64, vp, vp, C.c_int, vp, C.c_size_t, vp],
    "vbm_mul_mat_id_noalloc": [vp, vp, i64, C.c_int, vp, i64, vp, i64, i64, i64, vp, vp, C.c_int, vp],
    "vbm_add_id": [vp, vp, i64, vp, i64, i64, i64, i64, vp],
    "vbm_mul_mat_id_mxfp8": [vp, vp, i64, vp, i64, vp, i64, i64, i64, vp, vp],
    "vbm_quantize_mxfp8": [vp, i64, i64, i64, vp, vp, vp],
    "vbm_compute_forward": [C.POINTER(Node), vp, vp],
    "vbm_graph_compute": [vp, i64, vp, vp],
    "vbm_glu": [C.c_int, vp, vp, vp, i64, i64, i64, i64, i64, C.c_float, C.c_float, vp],
    "vbm_router_topk_softmax": [vp, vp, vp, i64, vp, i64, i64, i64, vp, vp, vp],
    "vbm_group_by_expert": [vp, i64, i64, i64, i64, vp, vp, vp, vp, vp],
    "vbm_weighted_combine": [vp, vp, i64, i64, i64, vp, vp],
    "vbm_moe_layer_workspace": [C.POINTER(MoeLayerDesc), i64, C.POINTER(sz)],
    "vbm_moe_layer_forward": [C.POINTER(MoeLayerDesc), vp, vp, i64, vp, vp, vp, vp, sz, vp],
    "vbm_moe_layer_forward_profiled": [C.POINTER(MoeLayerDesc), vp, vp, i64, vp, vp, vp, vp, sz, vp, vp],
    "vbm_graph_begin_capture": [vp],
    "vbm_graph_end_capture": [vp, C.POINTER(vp)],
    "vbm_graph_launch": [vp, vp],
    "vbm_graph_destroy": [vp],
    "vbm_copy_kernel": [vp, vp, sz, vp],
    "vbm_decode_plan_create": [C.POINTER(MoeLayerDesc), i64, C.POINTER(vp)],
    "vbm_decode_plan_destroy": [vp],
    "vbm_decode_step": [vp, vp, vp, vp, vp, vp, vp, vp],
    "vbm_decode_kernel": [vp, i64, C.c_int, vp, vp, vp],
    "vbm_decode_plan_set_linked": [vp, C.c_int],
    "vbm_decode_plan_get_linked": [vp, C.POINTER(C.c_int)],
    "vbm_decode_plan_check": [vp, C.POINTER(i64)],
    "vbm_admission_create": [i64, i64, i64, i64, i64, C.c_int32, C.c_int, C.POINTER(vp)],
    "vbm_admission_destroy": [vp],
    "vbm_admission_seed": [vp, i64, i64, vp],
    "vbm_admission_set_anchors": [vp, C.c_int32],
    "vbm_admission_admit": [vp, i64, vp, vp, vp, vp, vp, C.POINTER(i64)],
    "vbm_admission_write_dispatch": [vp, i64, vp, vp, i64, C.c_int32, vp],
    "vbm_admission_slot_map": [vp, i64, vp],
    "vbm_admission_stats": [vp, vp],
    "vbm_admission_set_lfu": [vp, C.c_int32, C.c_int32],
    "vbm_admission_lfu_state": [vp, vp, vp],
    "vbm_tier_create": [C.POINTER(TierDesc), C.POINTER(vp)],
    "vbm_tier_destroy": [vp],
    "vbm_tier_host_bytes": [vp, C.POINTER(sz)],
    "vbm_tier_set_expert": [vp, i64, i64, vp, vp, vp],
    "vbm_tier_generate": [vp, u64, u64, u64, u64, C.c_float, C.c_float, vp],
    "vbm_tier_seed": [vp, i64, i64],
    "vbm_tier_step": [vp, vp, vp, vp, vp, vp],
    "vbm_tier_get_stats": [vp, C.POINTER(TierStats)],
    "vbm_tier_set_deferred": [vp, C.c_int],
    "vbm_tier_flush": [vp],
    "vbm_tier_reset": [vp, C.c_int, i64, i64],
    "vbm_tier_step_begin": [vp],
    "vbm_tier_step_enqueue": [vp, vp, vp, vp, vp, vp],
    "vbm_tier_set_trace": [vp, vp],
    "vbm_tier_load_gguf": [vp, vp, vp, vp],
    "vbm_residency_replay": [C.POINTER(ResidencyLayer), i64, vp, vp, vp, vp, i64, C.POINTER(ResidencyParams),
                             C.POINTER(ResidencyTotals)],
    "vbm_residency_latency": [C.POINTER(ResidencyParams), C.c_double, C.c_double, C.c_double, C.POINTER(C.c_double),
                              C.POINTER(C.c_double), C.POINTER(C.c_double)],
    "vbm_host_call_prepare": [C.POINTER(HostCall), C.c_int],
    "vbm_host_call_enqueue": [C.POINTER(HostCall), vp, vp, C.c_int, vp, sz, vp, i64, C.c_int, vp],
    "vbm_host_join": [C.POINTER(HostCall), vp, vp, vp, i64, vp],
    "vbm_host_call_wait": [C.POINTER(HostCall), vp],
    "vbm_host_call_release": [C.POINTER(HostCall)],
    "vbm_host_mailbox_drain": [C.c_int, C.c_double],
    "vbm_host_mailbox_stats": [C.c_int, C.POINTER(u64), C.POINTER(u64), C.POINTER(C.c_uint32)],
    "vbm_host_mailbox_set_spin_limit": [C.c_uint32],
    "vbm_tier_prefill": [vp, i64, vp, vp, i64, vp, vp, vp, vp],
    "vbm_gguf_open": [C.c_char_p, C.POINTER(vp)],
    "vbm_gguf_close": [vp],
    "vbm_gguf_shards": [vp, C.POINTER(i64), C.POINTER(i64)],
    "vbm_gguf_get_u64": [vp, C.c_char_p, C.POINTER(u64), C.POINTER(C.c_int)],
    "vbm_gguf_get_string": [vp, C.c_char_p, C.c_char_p, sz, C.POINTER(C.c_int)],
    "vbm_gguf_tensor_info": [vp, C.c_char_p, C.POINTER(C.c_int), C.POINTER(i64), C.POINTER(u64), C.POINTER(C.c_int)],
    "vbm_gguf_expert_layer_info": [vp, i64, C.POINTER(GgufExpertInfo)],
    "vbm_gguf_read_expert": [vp, i64, i64, vp, vp, vp, vp],
    "vbm_gguf_load_layer": [vp, i64, vp, vp, i64, vp, vp, vp, vp, vp],
    "vbm_gguf_load_biases": [vp, i64, vp, vp, vp],
    "vbm_trace_open": [C.c_char_p, C.c_char_p, C.c_char_p, C.c_char_p, i64, C.POINTER(TraceLayer), i64,
                       C.c_char_p, C.c_char_p, C.POINTER(vp)],
    "vbm_trace_enable_prefill": [vp, C.c_char_p, i64, i64, i64, i64],
    "vbm_trace_prefill_enabled": [vp, C.POINTER(C.c_int)],
    "vbm_trace_prefill_route": [vp, i64, vp, i64],
    "vbm_trace_request_start": [vp, C.c_char_p, C.c_char_p, C.c_char_p, i64, i64],
    "vbm_trace_route": [vp, i64, vp, i64],
    "vbm_trace_token": [vp, vp, i64],
    "vbm_trace_request_end": [vp, C.c_char_p, C.c_int],
    "vbm_trace_close": [vp],
    "vbm_trace_abort": [vp],
    "vbm_trace_layer_info": [vp, i64, C.POINTER(i64), C.POINTER(i64), C.POINTER(i64)],
    "vbm_trace_position": [vp, C.POINTER(i64), C.POINTER(i64), C.POINTER(i64), C.POINTER(i64)],
}
OTHER = {
    "vbm_last_error": ([], C.c_char_p),
    "vbm_abi_version": ([], C.c_int),
    "vbm_moe_colder_admission": ([C.c_int, C.c_int, u64, C.c_int, C.c_int, u64], C.c_int),
    "vbm_moe_probation_margin": ([C.c_int, u64], C.c_int),
    "vbm_moe_anchor_slots": ([C.c_int, C.c_int, C.c_int], C.c_int),
    "vbm_moe_cold_gpu_budget": ([C.c_int], C.c_int),
    "vbm_moe_gpu_slot_limit": ([C.c_int32, C.c_int], C.c_int32),
    "vbm_node_supported": ([C.POINTER(Node)], C.c_int),
}
ADMIT_CLASSIC, ADMIT_LRU, ADMIT_RANKED, ADMIT_PROBATION, ADMIT_ANCHORED, ADMIT_LFU = 0, 1, 2, 3, 4, 5

_lib = None


class VbmError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libvbmoe.so (raises FileNotFoundError when it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else Path(os.environ.get("VBM_LIBRARY") or LIB_PATH)
    if not p.exists():
        raise FileNotFoundError(f"{p} not built; run unified-memory-scheduler_amd/build_lib.py")
    lib = C.CDLL(str(p))
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = C.c_int
    for name, (args, res) in OTHER.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def declared_symbols() -> list[str]:
    """Function names declared in include/vbmoe.h."""
    import re
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(vbm_[a-z0-9_]+)\s*\(", text)))


def call(name: str, *args):
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        raise VbmError(status, lib.vbm_last_error().decode())
    return status


def ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    return int(x)


class DeviceBuffer:
    """Owning device allocation."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = vp()
        call("vbm_malloc", C.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr: np.ndarray, stream=None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr, stream)
        return buf

    def upload(self, arr: np.ndarray, stream=None) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        call("vbm_memcpy_h2d", self.ptr, arr.ctypes.data, arr.nbytes, stream)
        call("vbm_stream_synchronize", stream)

    def download(self, dtype, shape, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        call("vbm_memcpy_d2h", out.ctypes.data, self.ptr, out.nbytes, stream)
        return out

    def free(self) -> None:
        if self.ptr:
            call("vbm_free", self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.vbm_free(self.ptr)
                self.ptr = None
        except Exception:
            pass


class Bank:
    """Device expert bank (vbm_bank)."""

    def __init__(self, type_id: int, rows: int, k: int, n_slots: int, interleave: bool = False):
        h = vp()
        call("vbm_bank_create", type_id, rows, k, n_slots, int(interleave), C.byref(h))
        self.handle = h.value
        self.type_id, self.rows, self.k, self.n_slots = type_id, rows, k, n_slots
        self.interleave = interleave
        s = sz()
        base = vp()
        call("vbm_bank_info", self.handle, None, None, None, None, C.byref(s), C.byref(base))
        self.slot_bytes = s.value
        self.base = base.value

    def upload(self, slot: int, ggml_bytes: np.ndarray, stream=None) -> None:
        data = np.ascontiguousarray(ggml_bytes, dtype=np.uint8)
        assert data.nbytes == self.slot_bytes, (data.nbytes, self.slot_bytes)
        call("vbm_bank_upload", self.handle, slot, data.ctypes.data, 0, stream)

    def export(self, slot: int, stream=None) -> np.ndarray:
        out = np.empty(self.slot_bytes, dtype=np.uint8)
        call("vbm_bank_export", self.handle, slot, out.ctypes.data, out.nbytes, stream)
        return out

    def generate(self, first_slot: int, count: int, seed: int, stream_id: int, first_expert: int,
                 p0: float, p1: float, stream=None) -> None:
        call("vbm_bank_generate", self.handle, first_slot, count, seed, stream_id, first_expert, p0, p1, stream)

    def destroy(self) -> None:
        if self.handle:
            call("vbm_bank_destroy", self.handle)
            self.handle = None

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.vbm_bank_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


# ----------------------------------------------------------------------------------- synthetic
def synth_mxfp4(seed: int, stream: int, first_block: int, n_blocks: int, exp_lo: int = -8, exp_hi: int = -3) -> np.ndarray:
    out = np.empty(n_blocks * 17, dtype=np.uint8)
    call("vbm_synth_mxfp4_host", seed, stream, first_block, n_blocks, exp_lo, exp_hi, out.ctypes.data)
    return out


def synth_q8_0(seed: int, stream: int, first_block: int, n_blocks: int, lo: float = 1e-3, hi: float = 1e-2) -> np.ndarray:
    out = np.empty(n_blocks * 34, dtype=np.uint8)
    call("vbm_synth_q8_0_host", seed, stream, first_block, n_blocks, lo, hi, out.ctypes.data)
    return out


def synth_normal(seed: int, stream: int, first: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    call("vbm_synth_normal_host", seed, stream, first, n, mean, std, out.ctypes.data)
    return out


def device_count() -> int:
    n = C.c_int(0)
    call("vbm_device_count", C.byref(n))
    return n.value


def device_name(device: int = 0) -> str:
    buf = C.create_string_buffer(256)
    call("vbm_device_name", device, buf, 256)
    return buf.value.decode()
