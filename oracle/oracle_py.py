"""ctypes binding of the CPU oracle (oracle/libvbm_oracle.so). TEST INFRASTRUCTURE ONLY:
imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libvbm_oracle.so"
REF_VNNI = HERE / "_ref" / "libref_mxfp4_vnni.so"
REF_DISPATCH_TEST = HERE / "_ref" / "test_expert_dispatch"

vp, i64 = C.c_void_p, C.c_int64


class OrcLayer(C.Structure):
    _fields_ = [("type", C.c_int), ("gate_up", vp), ("down", vp), ("gate_up_bias", vp), ("down_bias", vp),
                ("router_w", vp), ("router_b", vp), ("hidden", i64), ("intermediate", i64), ("n_expert", i64),
                ("top_k", i64), ("activation", C.c_int)]


_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} not built; run oracle/build_oracle.py")
        lib = C.CDLL(str(LIB_PATH))
        sig = {
            "orc_fp16_to_fp32": ([C.c_uint16], C.c_float),
            "orc_fp32_to_fp16": ([C.c_float], C.c_uint16),
            "orc_e8m0_half": ([C.c_uint8], C.c_float),
            "orc_quantize_row_q8_0": ([vp, vp, i64], None),
            "orc_vec_dot_mxfp4_q8_0": ([C.c_int, vp, vp], C.c_float),
            "orc_mxfp4_block_lanes": ([vp, vp, vp], C.c_int32),
            "orc_pack_mxfp4x8": ([vp, i64, i64, vp], None),
            "orc_unpack_mxfp4x8": ([vp, i64, i64, vp], None),
            "orc_gemv_mxfp4x8_q8_0": ([C.c_int, vp, vp, vp, C.c_int], C.c_int),
            "orc_vec_dot_q8_0_q8_0": ([C.c_int, vp, vp], C.c_float),
            "orc_q8_block_lanes": ([vp, vp, vp], C.c_int32),
            "orc_vec_dot_f32": ([C.c_int, vp, vp], C.c_float),
            "orc_mul_mat_id": ([C.c_int, vp, i64, i64, i64, C.c_int, vp, i64, vp, i64, i64, i64, vp, vp, C.c_int],
                               C.c_int),
            "orc_group_by_expert": ([vp, i64, i64, i64, i64, vp, vp, vp], C.c_int),
            "orc_topk": ([vp, i64, i64, vp], None),
            "orc_softmax_selected": ([vp, i64, vp], None),
            "orc_router": ([vp, vp, vp, i64, vp, i64, i64, i64, vp, vp], None),
            "orc_glu": ([C.c_int, vp, vp, vp, i64, C.c_float, C.c_float], None),
            "orc_weighted_combine": ([vp, vp, i64, i64, i64, vp], None),
            "orc_moe_layer": ([C.POINTER(OrcLayer), vp, vp, i64, vp, vp, vp, vp, vp, C.c_int], C.c_int),
            "orc_fast_isa": ([], C.c_int),
        }
        for name, (args, res) in sig.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows = x.reshape(-1, x.shape[-1])
    k = rows.shape[1]
    out = np.empty((rows.shape[0], k // 32 * 34), dtype=np.uint8)
    for i in range(rows.shape[0]):
        load().orc_quantize_row_q8_0(rows[i].ctypes.data, out[i].ctypes.data, k)
    return out


def mul_mat_id(type_id, as_bytes, k, rows, n_as, b_type, b, b_ne1, ids, n_ids, n_tokens, ids_stride,
               bias=None, threads=0) -> np.ndarray:
    dst = np.empty((n_tokens, n_ids, rows), dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    status = load().orc_mul_mat_id(type_id, _p(as_bytes), k, rows, n_as, b_type, _p(b), b_ne1, _p(ids), n_ids,
                                   n_tokens, ids_stride, _p(bias), _p(dst), threads)
    if status != 0:
        raise ValueError("oracle mul_mat_id rejected its inputs")
    return dst


def pack_mxfp4x8(raw: np.ndarray, rows: int, blocks: int) -> np.ndarray:
    """block_mxfp4 rows [rows][blocks] (17 B each) -> block_mxfp4x8 groups (136 B each)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(rows // 8 * blocks * 136, np.uint8)
    load().orc_pack_mxfp4x8(_p(raw), rows, blocks, _p(out))
    return out


def unpack_mxfp4x8(packed: np.ndarray, rows: int, blocks: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(rows * blocks * 17, np.uint8)
    load().orc_unpack_mxfp4x8(_p(packed), rows, blocks, _p(out))
    return out


def gemv_mxfp4x8(packed: np.ndarray, act_q8: np.ndarray, k: int, rows: int) -> np.ndarray:
    """Repacked 8x8 contract: one Q8_0 activation row against `rows` packed rows."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    act_q8 = np.ascontiguousarray(act_q8, dtype=np.uint8)
    out = np.empty(rows, np.float32)
    if load().orc_gemv_mxfp4x8_q8_0(k, _p(out), _p(packed), _p(act_q8), rows) != 0:
        raise ValueError("repacked GEMV needs k % 64 == 0 and rows % 8 == 0")
    return out


def group_by_expert(ids: np.ndarray, n_ids: int, n_tokens: int, ids_stride: int, n_as: int):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    counts = np.empty(n_as, np.int32)
    offsets = np.empty(n_as + 1, np.int32)
    rows = np.full(n_ids * n_tokens, -1, np.int32)
    status = load().orc_group_by_expert(_p(ids), n_ids, n_tokens, ids_stride, n_as, _p(counts), _p(offsets), _p(rows))
    if status != 0:
        raise ValueError("invalid id")
    return counts, offsets, rows[: offsets[-1]]


def router(logits=None, router_w=None, router_b=None, x=None, n_expert=None, n_tokens=None, top_k=4, hidden=0):
    if logits is None:
        logits = np.empty((n_tokens, n_expert), np.float32)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    n_tokens, n_expert = logits.shape
    ids = np.empty((n_tokens, top_k), np.int32)
    w = np.empty((n_tokens, top_k), np.float32)
    load().orc_router(_p(router_w), _p(router_b), _p(x), hidden, _p(logits), n_expert, n_tokens, top_k, _p(ids), _p(w))
    return logits, ids, w


def glu(activation: int, gate: np.ndarray, up: np.ndarray, alpha: float = 1.702, limit: float = 7.0) -> np.ndarray:
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    up = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty_like(gate)
    load().orc_glu(activation, _p(gate), _p(up), _p(out), gate.size, alpha, limit)
    return out


def moe_layer(type_id, gate_up, down, gate_up_bias, down_bias, x, hidden, intermediate, n_expert, top_k,
              activation=1, logits=None, router_w=None, router_b=None, threads=0, want_intermediates=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    layer = OrcLayer(type_id, _p(gate_up), _p(down), _p(gate_up_bias), _p(down_bias), _p(router_w), _p(router_b),
                     hidden, intermediate, n_expert, top_k, activation)
    lg = np.ascontiguousarray(logits, dtype=np.float32) if logits is not None else np.empty((T, n_expert), np.float32)
    out = np.empty((T, hidden), np.float32)
    ids = np.empty((T, top_k), np.int32)
    w = np.empty((T, top_k), np.float32)
    act = np.empty((T, top_k, intermediate), np.float32) if want_intermediates else None
    y = np.empty((T, top_k, hidden), np.float32) if want_intermediates else None
    status = load().orc_moe_layer(C.byref(layer), _p(x), _p(lg), T, _p(out), _p(ids), _p(w), _p(act), _p(y), threads)
    if status != 0:
        raise ValueError("oracle layer rejected its inputs")
    return {"out": out, "ids": ids, "weights": w, "logits": lg, "act": act, "y": y}
