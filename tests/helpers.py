"""Shared helpers for the GPU parity tests: build banks from ggml bytes and call the C ABI."""
from __future__ import annotations

import ctypes as C

import numpy as np

import vbmoe as vb

MX, Q8 = vb.TYPE_MXFP4, vb.TYPE_Q8_0


def block_bytes(type_id: int) -> int:
    return 17 if type_id == MX else 34


def synth_weights(type_id: int, seed: int, stream: int, experts: int, rows: int, k: int,
                  q8_scale=(1e-3, 1e-2)) -> np.ndarray:
    n = experts * rows * (k // 32)
    if type_id == MX:
        return vb.synth_mxfp4(seed, stream, 0, n)
    return vb.synth_q8_0(seed, stream, 0, n, *q8_scale)


def make_bank(type_id: int, ggml: np.ndarray, experts: int, rows: int, k: int, interleave=False) -> vb.Bank:
    bank = vb.Bank(type_id, rows, k, experts, interleave)
    per = rows * (k // 32) * block_bytes(type_id)
    for e in range(experts):
        bank.upload(e, ggml[e * per:(e + 1) * per])
    return bank


def mul_mat_id(bank: vb.Bank, n_as: int, b: np.ndarray, b_type: int, b_ne1: int, ids: np.ndarray, n_ids: int,
               bias: np.ndarray | None = None, order=vb.ORDER_EXACT, slot_map=None, slot_map_host=None,
               dst_offset: int = 0, b_offset: int = 0) -> np.ndarray:
    """dst_offset / b_offset (bytes, multiples of 4) place the output / the activations that far
    into their allocations, e.g. 4 for buffers that are not 16-byte aligned."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    n_tokens = ids.shape[0]
    ids_stride = ids.shape[1]
    braw = np.ascontiguousarray(b).view(np.uint8).reshape(-1)
    db = vb.DeviceBuffer.from_array(np.concatenate([np.zeros(b_offset, np.uint8), braw]))
    dids = vb.DeviceBuffer.from_array(ids)
    dbias = vb.DeviceBuffer.from_array(bias.astype(np.float32)) if bias is not None else None
    dmap = vb.DeviceBuffer.from_array(np.asarray(slot_map, np.int32)) if slot_map is not None else None
    hmap = np.ascontiguousarray(slot_map_host, dtype=np.int32) if slot_map_host is not None else None
    dst = vb.DeviceBuffer(n_tokens * n_ids * bank.rows * 4 + dst_offset)
    vb.call("vbm_memset", dst.ptr, 0x7F, dst.nbytes, None)      # a row the call leaves unwritten shows up
    vb.call("vbm_mul_mat_id", bank.handle, vb.ptr(dmap), vb.ptr(hmap), n_as, b_type, db.ptr + b_offset, b_ne1, dids.ptr, n_ids,
            n_tokens, ids_stride, vb.ptr(dbias), dst.ptr + dst_offset, order, None)
    vb.call("vbm_stream_synchronize", None)
    raw = dst.download(np.uint8, (dst.nbytes,))
    return raw[dst_offset:].view(np.float32).reshape(n_tokens, n_ids, bank.rows)


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    return a.shape == b.shape and np.array_equal(np.ascontiguousarray(a).view(np.uint32),
                                                 np.ascontiguousarray(b).view(np.uint32))


def diff_report(a: np.ndarray, b: np.ndarray) -> str:
    a = a.astype(np.float64).reshape(-1)
    b = b.astype(np.float64).reshape(-1)
    d = np.abs(a - b)
    i = int(d.argmax())
    return f"changed={int((a != b).sum())}/{a.size} max_abs={d.max():.3e} at {i}: {a[i]!r} vs {b[i]!r}"


def rel_err_and_cos(got: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    g = got.astype(np.float64).reshape(-1)
    r = ref.astype(np.float64).reshape(-1)
    max_rel = float(np.abs(g - r).max() / max(np.abs(r).max(), 1e-30))
    cos = float(np.dot(g, r) / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-300))
    return max_rel, cos
