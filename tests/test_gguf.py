"""GGUF expert loader (vbm_gguf_*): header parsing, shards, metadata, per-expert slices and the
rejections of the reference loader (tools/engine/gguf_experts.cpp:27-140), on fixtures written by
tests/gguf_writer.py from the published GGUF layout. Host-only; no GPU."""
import struct

import numpy as np
import pytest

import gguf_writer as W

H, I, E = 64, 96, 4


@pytest.fixture(scope="module")
def gg(vb):
    from vbmoe.gguf import GgufFile
    return GgufFile


def base_kv():
    return [("general.architecture", W.STRING, "gpt-oss"),
            ("general.name", W.STRING, "synthetic fixture"),
            ("gpt-oss.block_count", W.U32, 2),
            ("gpt-oss.expert_count", W.U32, E),
            ("gpt-oss.expert_used_count", W.U32, 2),
            ("gpt-oss.rope.freq_base", W.F32, 150000.0),
            ("gpt-oss.attention.layer_norm_rms_epsilon", W.F64, 1e-5),
            ("tokenizer.ggml.add_bos_token", W.BOOL, False),
            ("test.negative", W.I8, -3),
            ("test.big", W.U64, 1 << 40),
            ("test.i16", W.I16, 1234),
            ("tokenizer.ggml.tokens", W.ARRAY, (W.STRING, ["<a>", "b", "ccc", ""])),
            ("tokenizer.ggml.scores", W.ARRAY, (W.F32, [0.0, 1.5, -2.0, 3.0])),
            ("tokenizer.ggml.token_type", W.ARRAY, (W.I32, [1, 2, 3, 6]))]


def model(tmp_path, name="m.gguf", gtype=39, biases=True, fused=False, seed=1, layers=(0, 1), extra=(), **kw):
    rng = np.random.default_rng(seed)
    tensors, arrays = [], {}
    tensors.append(("token_embd.weight", 0, (H, 5), rng.normal(size=(5, H)).astype(np.float32).tobytes()))
    for layer in layers:
        t, a = W.expert_layer_tensors(layer, gtype, H, I, E, rng, biases=biases, fused=fused)
        tensors += t
        arrays[layer] = a
        tensors.append((f"blk.{layer}.ffn_gate_inp.weight", 0, (H, E), rng.normal(size=(E, H)).astype(np.float32).tobytes()))
    tensors += list(extra)
    path = W.write_gguf(tmp_path / name, base_kv(), tensors, **kw)
    return path, arrays


def check_layer(f, arrays, layer, gtype, biases=True):
    info = f.expert_info(layer)
    assert (info.hidden, info.intermediate, info.n_expert) == (H, I, E)
    assert (info.gate_up_type, info.down_type, info.has_bias) == (gtype, gtype, int(biases))
    assert info.gate_up_bytes == arrays["gate_up"].shape[1] and info.down_bytes == arrays["down"].shape[1]
    for e in (2, 0, 3, 1):
        gu, dn, bgu, bdn = f.read_expert(layer, e)
        assert np.array_equal(gu, arrays["gate_up"][e]), (layer, e)
        assert np.array_equal(dn, arrays["down"][e]), (layer, e)
        if biases:
            assert np.array_equal(bgu, arrays["gate_up_bias"][e]) and np.array_equal(bdn, arrays["down_bias"][e])
        else:
            assert not bgu.any() and not bdn.any()


@pytest.mark.parametrize("gtype", [39, 8])
def test_single_file_metadata_and_slices(gg, tmp_path, gtype):
    path, arrays = model(tmp_path, gtype=gtype)
    with gg(path) as f:
        assert f.shards() == (1, 1 + 2 * (3 + 3 + 1))
        assert f.get_string("general.architecture") == "gpt-oss"
        assert f.get_u64("gpt-oss.expert_count") == E and f.get_u64("gpt-oss.expert_used_count") == 2
        assert f.get_u64("test.big") == 1 << 40 and f.get_u64("test.i16") == 1234
        assert f.get_u64("tokenizer.ggml.add_bos_token") == 0
        assert f.get_u64("test.negative") is None            # negative: not a u64
        assert f.get_u64("general.architecture") is None and f.get_string("gpt-oss.expert_count") is None
        assert f.get_u64("missing.key") is None
        t, ne, nb = f.tensor("blk.1.ffn_down_exps.weight")
        assert (t, ne, nb) == (gtype, (I, H, E, 1), W.tensor_bytes(gtype, (I, H, E)))
        assert f.tensor("blk.1.ffn_gate_inp.weight") == (0, (H, E, 1, 1), 4 * H * E)
        assert f.tensor("nope") is None
        for layer in (0, 1):
            check_layer(f, arrays[layer], layer, gtype)


def test_no_biases_fused_alignment_and_version2(gg, tmp_path):
    path, arrays = model(tmp_path, biases=False, fused=True, alignment=64, version=2)
    with gg(path) as f:
        assert f.expert_info(0).fused_gate_up == 1
        check_layer(f, arrays[0], 0, 39, biases=False)
        check_layer(f, arrays[1], 1, 39, biases=False)


def test_shards(gg, tmp_path):
    rng = np.random.default_rng(5)
    t0, a0 = W.expert_layer_tensors(0, 39, H, I, E, rng)
    t1, a1 = W.expert_layer_tensors(1, 39, H, I, E, rng)
    W.write_gguf(tmp_path / "big-00001-of-00003.gguf", base_kv(), t0[:2])
    W.write_gguf(tmp_path / "big-00002-of-00003.gguf", [], t0[2:] + t1[:1])
    W.write_gguf(tmp_path / "big-00003-of-00003.gguf", [("split.no", W.U16, 2)], t1[1:])
    with gg(tmp_path / "big-00001-of-00003.gguf") as f:
        assert f.shards() == (3, len(t0) + len(t1))
        check_layer(f, a0, 0, 39)
        check_layer(f, a1, 1, 39)
    # opening a later shard reads only that shard
    with gg(tmp_path / "big-00002-of-00003.gguf") as f:
        assert f.shards() == (1, len(t0) - 2 + 1)
    (tmp_path / "big-00003-of-00003.gguf").unlink()
    with pytest.raises(Exception, match="shard missing"):
        gg(tmp_path / "big-00001-of-00003.gguf")
    W.write_gguf(tmp_path / "dup-00001-of-00002.gguf", base_kv(), t0)
    W.write_gguf(tmp_path / "dup-00002-of-00002.gguf", [], t0[:1])
    with pytest.raises(Exception, match="duplicate GGUF tensor across shards"):
        gg(tmp_path / "dup-00001-of-00002.gguf")


def corrupt(path, offset, data):
    raw = bytearray(path.read_bytes())
    raw[offset:offset + len(data)] = data
    path.write_bytes(bytes(raw))


def test_rejects_broken_containers(gg, vb, tmp_path):
    path, _ = model(tmp_path)
    good = path.read_bytes()
    cases = {
        "bad magic": lambda p: corrupt(p, 0, b"GGUX"),
        "version 1": lambda p: corrupt(p, 4, struct.pack("<I", 1)),
        "truncated header": lambda p: p.write_bytes(good[:200]),
        "truncated data": lambda p: p.write_bytes(good[:-16]),
        "unknown value type": lambda p: corrupt(p, 24 + 8 + len("general.architecture"), struct.pack("<I", 77)),
    }
    for label, mutate in cases.items():
        p = tmp_path / f"bad-{label.replace(' ', '_')}.gguf"
        p.write_bytes(good)
        mutate(p)
        with pytest.raises(vb.VbmError):
            gg(p)
    with pytest.raises(vb.VbmError, match="missing or not a file"):
        gg(tmp_path / "absent.gguf")
    with pytest.raises(vb.VbmError, match="missing or not a file"):
        gg(tmp_path)
    bad = W.write_gguf(tmp_path / "odd.gguf", [], [("blk.0.ffn_down_exps.weight", 39, (48, H, E),
                                                     b"\0" * W.tensor_bytes(39, (64, H, E)))])
    with pytest.raises(vb.VbmError, match="whole number of blocks"):
        gg(bad)


def test_rejects_incompatible_expert_layers(gg, vb, tmp_path):
    rng = np.random.default_rng(9)
    t, _ = W.expert_layer_tensors(0, 39, H, I, E, rng)
    names = [x[0] for x in t]

    def variant(label, tensors):
        p = W.write_gguf(tmp_path / f"{label}.gguf", [], tensors)
        return gg(p)

    # missing down
    f = variant("nodown", [x for x in t if "down_exps.weight" not in x[0]])
    with pytest.raises(vb.VbmError, match="missing"):
        f.expert_info(0)
    # missing up
    f = variant("noup", [x for x in t if "up_exps.weight" not in x[0]])
    with pytest.raises(vb.VbmError, match="missing"):
        f.expert_info(0)
    # down with the wrong expert count
    bad = [x if x[0] != names[2] else (x[0], 39, (I, H, E - 1), x[3][:W.tensor_bytes(39, (I, H, E - 1))]) for x in t]
    f = variant("downcount", bad)
    with pytest.raises(vb.VbmError, match="incompatible expert projection"):
        f.expert_info(0)
    # bias with the wrong width
    bad = [x if x[0] != "blk.0.ffn_down_exps.bias" else (x[0], 0, (H - 1, E), x[3][:4 * (H - 1) * E]) for x in t]
    f = variant("biaswidth", bad)
    with pytest.raises(vb.VbmError, match="incompatible expert bias"):
        f.expert_info(0)
    # only one of gate / up biases
    f = variant("halfbias", [x for x in t if x[0] != "blk.0.ffn_up_exps.bias"])
    with pytest.raises(vb.VbmError, match="both be present"):
        f.expert_info(0)
    # F16 weights are not an expert bank type
    f16 = [("blk.0.ffn_gate_exps.weight", 1, (H, I, E), b"\0" * (2 * H * I * E)),
           ("blk.0.ffn_up_exps.weight", 1, (H, I, E), b"\0" * (2 * H * I * E)),
           ("blk.0.ffn_down_exps.weight", 1, (I, H, E), b"\0" * (2 * H * I * E))]
    f = variant("f16", f16)
    with pytest.raises(vb.VbmError, match="MXFP4 or Q8_0"):
        f.expert_info(0)
    # experts outside the tensor, layers that are not there
    f = variant("ok", t)
    with pytest.raises(vb.VbmError, match="outside tensor"):
        f.read_expert(0, E)
    with pytest.raises(vb.VbmError, match="missing"):
        f.expert_info(1)
    with pytest.raises(vb.VbmError, match="invalid layer"):
        f.expert_info(-1)
