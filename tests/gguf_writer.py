"""Minimal GGUF writer for test fixtures, written from the published GGUF layout (independent of
the library's C++ reader): little-endian; magic "GGUF"; u32 version; u64 tensor count; u64
key/value count; key/value pairs (u64-length string key, u32 value type, value); tensor infos
(name, u32 rank, u64 dims in ggml order, u32 ggml type, u64 offset into the data section); the
data section starts at the next multiple of general.alignment (32 by default) and every tensor
offset is a multiple of it."""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}
BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 39: (32, 17), 30: (1, 2)}   # ggml type -> (elements, bytes)


def _string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _string(value)
    if vtype == ARRAY:
        etype, items = value
        body = b"".join(_string(v) if etype == STRING else struct.pack(_FMT[etype], v) for v in items)
        return struct.pack("<IQ", etype, len(items)) + body
    return struct.pack(_FMT[vtype], value)


def tensor_bytes(ggml_type: int, ne: tuple[int, ...]) -> int:
    elements, size = BLOCK[ggml_type]
    n = 1
    for d in ne:
        n *= d
    return n // elements * size


def write_gguf(path: str | Path, kv: list[tuple[str, int, object]], tensors: list[tuple[str, int, tuple, bytes]],
               alignment: int = 32, version: int = 3, data_pad: bytes = b"\x00") -> Path:
    """kv: (key, value type, value); tensors: (name, ggml type, ne in ggml order, raw bytes)."""
    kv = list(kv)
    if alignment != 32:
        kv.append(("general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    head += b"".join(_string(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in kv)
    offset = 0
    infos, blobs = b"", []
    for name, gtype, ne, data in tensors:
        infos += _string(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        infos += struct.pack("<IQ", gtype, offset)
        blobs.append((offset, data))
        offset += (len(data) + alignment - 1) // alignment * alignment
    header = head + infos
    start = (len(header) + alignment - 1) // alignment * alignment
    out = bytearray(header + data_pad[:1] * (start - len(header)))
    for off, data in blobs:
        out += b"\x00" * (start + off - len(out))
        out += data
    Path(path).write_bytes(bytes(out))
    return Path(path)


def expert_layer_tensors(layer: int, ggml_type: int, hidden: int, inter: int, experts: int, rng: np.random.Generator,
                         biases: bool = True, fused: bool = False, mx_exp: tuple[int, int] = (119, 124)) -> tuple[list, dict]:
    """Random expert tensors of one layer; returns (tensor list, dict of numpy arrays by part)."""
    def weight(rows, k):
        n = tensor_bytes(ggml_type, (k, rows, experts))
        raw = rng.integers(0, 256, n, dtype=np.uint8)
        if ggml_type == 8:                      # keep fp16 scales finite: small positive halves
            blocks = raw.reshape(-1, 34)
            d = rng.uniform(1e-3, 1e-2, blocks.shape[0]).astype(np.float16).view(np.uint8).reshape(-1, 2)
            blocks[:, :2] = d
        elif ggml_type == 39:                   # block scales 2^(e-127) in a moderate range
            blocks = raw.reshape(-1, 17)
            blocks[:, 0] = rng.integers(mx_exp[0], mx_exp[1] + 1, blocks.shape[0])
        return raw.reshape(experts, -1)
    p = f"blk.{layer}.ffn_"
    arrays, tensors = {}, []
    if fused:
        arrays["gate_up"] = weight(2 * inter, hidden)
        tensors.append((p + "gate_up_exps.weight", ggml_type, (hidden, 2 * inter, experts), arrays["gate_up"].tobytes()))
    else:
        arrays["gate"] = weight(inter, hidden)
        arrays["up"] = weight(inter, hidden)
        tensors.append((p + "gate_exps.weight", ggml_type, (hidden, inter, experts), arrays["gate"].tobytes()))
        tensors.append((p + "up_exps.weight", ggml_type, (hidden, inter, experts), arrays["up"].tobytes()))
        arrays["gate_up"] = np.concatenate([arrays["gate"], arrays["up"]], axis=1)
    arrays["down"] = weight(hidden, inter)
    tensors.append((p + "down_exps.weight", ggml_type, (inter, hidden, experts), arrays["down"].tobytes()))
    if biases:
        for part, n in (("gate", inter), ("up", inter), ("down", hidden)):
            b = rng.normal(0, 0.02, (experts, n)).astype(np.float32)
            arrays[part + "_bias"] = b
            tensors.append((p + f"{part}_exps.bias", 0, (n, experts), b.tobytes()))
        arrays["gate_up_bias"] = np.concatenate([arrays["gate_bias"], arrays["up_bias"]], axis=1)
    return tensors, arrays
