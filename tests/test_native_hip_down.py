"""Engine-level mirror (host/native_hip_down.hpp): load_gguf_experts (gguf_experts.cpp semantics)
on the CPU, and Mxfp4NativeHipDown (quantized_cuda.cu:373-453 semantics) on the GPU against the
oracle's MUL_MAT_ID of the same bytes, through the C++ driver tests/cpp/test_native_hip_down.cpp
(built by build_lib.py next to libvbmoe.so)."""
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import gguf_writer as W

REPO = Path(__file__).resolve().parents[1]
DRIVER = REPO / "tests" / "cpp" / "bin" / "test_native_hip_down"
H, I, E = 128, 192, 6
IDS = [4, 0, 5, 2]


def model(tmp_path):
    rng = np.random.default_rng(17)
    tensors, arrays = W.expert_layer_tensors(3, 39, H, I, E, rng)
    # two blocks with exponent 127 (scale 1/2): the doubled e2m1 table halved is the e2m1 table itself
    gate = arrays["gate"].reshape(E, I, H // 32, 17)
    gate[4, 0, 0, 0] = 127
    gate[4, 0, 0, 1:] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    for k, t in enumerate(tensors):
        if t[0] == "blk.3.ffn_gate_exps.weight":
            tensors[k] = (t[0], t[1], t[2], gate.tobytes())
    arrays["gate"] = gate.reshape(E, -1)
    path = W.write_gguf(tmp_path / "m.gguf", [("general.architecture", W.STRING, "gpt-oss")], tensors)
    return path, arrays


def read_dump(path):
    raw = path.read_bytes()
    off = 0

    def i64():
        nonlocal off
        v = struct.unpack_from("<q", raw, off)[0]
        off += 8
        return v

    def vec(dtype):
        nonlocal off
        n = i64()
        size = np.dtype(dtype).itemsize
        a = np.frombuffer(raw, dtype=dtype, count=n, offset=off)
        off += n * size
        return a

    head = [i64() for _ in range(6)]
    packed = [vec(np.uint8) for _ in range(3)]
    floats = [vec(np.float32) for _ in range(6)]
    return head, packed, floats


def test_load_gguf_experts(tmp_path):
    assert DRIVER.exists(), "build the driver first (unified-memory-scheduler_amd/build_lib.py)"
    path, a = model(tmp_path)
    out = tmp_path / "dump.bin"
    r = subprocess.run([str(DRIVER), "load", str(path), "3", str(out), *map(str, IDS)], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 0, r.stderr
    head, packed, floats = read_dump(out)
    assert head == [H, I, len(IDS), 39, 39, 39]
    for k, part in enumerate(("gate", "up", "down")):
        assert np.array_equal(packed[k], np.concatenate([a[part][e] for e in IDS]))
    gate, up, down, gb, ub, db = floats
    assert gate.shape == (len(IDS) * I * H,) and down.shape == (len(IDS) * H * I,)
    # closed form of the first block of expert 4 (loaded first): e = 127 scales the doubled table
    # by 2^-1, which gives e2m1 values; nibble i (low) and 15 - i (high) of byte i
    e2m1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, 0, -0.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    assert np.array_equal(gate[:16], e2m1) and np.array_equal(gate[16:32], e2m1[::-1])
    # every block: value = doubled table x 2^(e - 128)
    blocks = np.concatenate([a["down"][e] for e in IDS]).reshape(-1, 17)
    table = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.float64)
    scale = np.ldexp(1.0, blocks[:, 0].astype(np.int64) - 128)[:, None]
    vals = np.concatenate([table[blocks[:, 1:] & 15], table[blocks[:, 1:] >> 4]], axis=1) * scale
    assert np.array_equal(down.astype(np.float64), vals.reshape(-1))
    assert np.array_equal(gb, np.concatenate([a["gate_bias"][e] for e in IDS]))
    assert np.array_equal(db, np.concatenate([a["down_bias"][e] for e in IDS]))
    bad = subprocess.run([str(DRIVER), "load", str(path), "3", str(out), "1", "1"], capture_output=True, text=True,
                         timeout=60)
    assert bad.returncode == 3 and "invalid layer or selected expert IDs" in bad.stderr
    missing = subprocess.run([str(DRIVER), "load", str(path), "2", str(out), "1"], capture_output=True, text=True,
                             timeout=60)
    assert missing.returncode == 3 and "missing" in missing.stderr


@pytest.mark.gpu
def test_mxfp4_native_hip_down_matches_oracle(gpu, orc, tmp_path):
    assert DRIVER.exists(), "build the driver first (unified-memory-scheduler_amd/build_lib.py)"
    import vbmoe as vb
    path, a = model(tmp_path)
    resident = np.array([1, 0, 1, 1], np.uint8)            # local expert 1 (original id 0) stays on the CPU
    rng = np.random.default_rng(5)
    n_jobs = 9
    local = rng.choice(np.flatnonzero(resident), n_jobs)
    jobs = np.stack([np.arange(n_jobs), rng.integers(0, 4, n_jobs), local], axis=1).astype(np.int64)
    q8 = vb.synth_q8_0(5, 40, 0, n_jobs * I // 32)
    inp = tmp_path / "in.bin"
    inp.write_bytes(struct.pack("<q", n_jobs) + resident.tobytes() + jobs.tobytes() + q8.tobytes())
    out = tmp_path / "out.bin"
    print(f"[native down] {n_jobs} jobs over experts {sorted(set(local.tolist()))}", flush=True)
    r = subprocess.run([str(DRIVER), "down", str(path), "3", str(inp), str(out), *map(str, IDS)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "rejected 2" in r.stdout                          # non-resident expert and short input
    got = np.frombuffer(out.read_bytes(), np.float32).reshape(n_jobs, H)
    bank = np.concatenate([a["down"][e] for e in IDS])      # local expert order
    bias = np.concatenate([a["down_bias"][e] for e in IDS])
    ref = orc.mul_mat_id(39, bank, I, H, len(IDS), vb.TYPE_Q8_0, q8, 1, local.astype(np.int32).reshape(n_jobs, 1), 1,
                         n_jobs, 1, bias=bias)
    assert np.array_equal(got.view(np.uint32), ref.reshape(n_jobs, H).view(np.uint32))


@pytest.mark.gpu
def test_native_hip_experts_matches_oracle(gpu, orc, tmp_path):
    """NativeHipExperts (native_cpu.hpp:11-30 on the GPU): execute, activations, pack_down and
    execute_down for one input row per job, bit-identical to the oracle's composition of the same
    steps (Q8_0 input, gate / up with biases, SwiGLU-OAI, Q8_0 requantization, down with bias)."""
    assert DRIVER.exists(), "build the driver first (unified-memory-scheduler_amd/build_lib.py)"
    path, a = model(tmp_path)
    rng = np.random.default_rng(8)
    n_rows, n_jobs = 3, 7
    x = gpu.synth_normal(8, 1, 0, n_rows * H).reshape(n_rows, H)
    local = rng.integers(0, len(IDS), n_jobs)
    jobs = np.stack([rng.integers(0, n_rows, n_jobs), rng.integers(0, 4, n_jobs), local], axis=1).astype(np.int64)
    inp = tmp_path / "xin.bin"
    inp.write_bytes(struct.pack("<qq", n_rows, n_jobs) + x.astype(np.float32).tobytes() + jobs.tobytes())
    out = tmp_path / "xout.bin"
    print(f"[native experts] {n_jobs} jobs over rows {jobs[:, 0].tolist()} experts {local.tolist()}", flush=True)
    r = subprocess.run([str(DRIVER), "experts", str(path), "3", str(inp), str(out), *map(str, IDS)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert f"observed {4 * n_jobs} stages; rejected 2" in r.stdout
    raw = out.read_bytes()
    q_bytes = n_jobs * (I // 32) * 34
    got_out = np.frombuffer(raw, np.float32, n_jobs * H, 0).reshape(n_jobs, H)
    got_act = np.frombuffer(raw, np.float32, n_jobs * I, 4 * n_jobs * H).reshape(n_jobs, I)
    got_q = np.frombuffer(raw, np.uint8, q_bytes, 4 * n_jobs * (H + I))
    got_down = np.frombuffer(raw, np.float32, n_jobs * H, 4 * n_jobs * (H + I) + q_bytes).reshape(n_jobs, H)

    def bank(part):
        return np.concatenate([a[part][e] for e in IDS])

    def bias(part):
        return np.concatenate([a[part + "_bias"][e] for e in IDS])

    rows = x[jobs[:, 0]].reshape(n_jobs, 1, H)
    ids = local.astype(np.int32).reshape(n_jobs, 1)
    g = orc.mul_mat_id(39, bank("gate"), H, I, len(IDS), 0, rows, 1, ids, 1, n_jobs, 1, bias=bias("gate")).reshape(n_jobs, I)
    u = orc.mul_mat_id(39, bank("up"), H, I, len(IDS), 0, rows, 1, ids, 1, n_jobs, 1, bias=bias("up")).reshape(n_jobs, I)
    act = np.empty_like(g)
    orc.load().orc_glu(1, np.ascontiguousarray(g).ctypes.data, np.ascontiguousarray(u).ctypes.data, act.ctypes.data,
                       g.size, 1.702, 7.0)
    q = orc.quantize_q8_0(act)
    down = orc.mul_mat_id(39, bank("down"), I, H, len(IDS), 8, q.reshape(n_jobs, 1, -1), 1, ids, 1, n_jobs, 1,
                          bias=bias("down")).reshape(n_jobs, H)
    assert np.array_equal(got_act.view(np.uint32), act.view(np.uint32))
    assert np.array_equal(got_q, q.reshape(-1))
    assert np.array_equal(got_out.view(np.uint32), down.view(np.uint32))
    assert np.array_equal(got_down.view(np.uint32), down.view(np.uint32))
