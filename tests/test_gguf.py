"""The library's GGUF reader on the CPU (no GPU is touched by parsing): round
trips through an independent writer (tests/gguf_writer.py) and the rejection
cases of the reference reader (crates/vokra-core/src/gguf/reader.rs:512-800,
tensor.rs tests)."""
import struct

import numpy as np
import pytest

from tests import gguf_writer as gw
from vokra_amd import hip


def write(tmp_path, data, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_hand_built_empty_header(tmp_path):
    # reader.rs hand_built_empty: magic, version 3, no tensors, no metadata
    f = hip.GgufFile(write(tmp_path, b"GGUF" + struct.pack("<IQQ", 3, 0, 0)))
    assert len(f) == 0


def payloads(g):
    q8 = bytes(g.integers(0, 256, 34 * 4, dtype=np.uint8))          # [64, 2] Q8_0: 4 blocks
    q4 = bytes(g.integers(0, 256, 18 * 8, dtype=np.uint8))          # [128, 2] Q4_0: 8 blocks
    q5 = bytes(g.integers(0, 256, 22 * 2, dtype=np.uint8))          # [32, 2] Q5_0
    qk = bytes(g.integers(0, 256, 144 * 2, dtype=np.uint8))         # [256, 2] Q4_K
    f32 = g.standard_normal(6).astype(np.float32)
    f16 = g.standard_normal(5).astype(np.float16)
    return [("w.q8", [64, 2], gw.GGML_Q8_0, q8), ("w.q4", [128, 2], gw.GGML_Q4_0, q4),
            ("w.q5", [32, 2], gw.GGML_Q5_0, q5), ("w.qk", [256, 2], gw.GGML_Q4_K, qk),
            ("ln.gamma", [6], gw.GGML_F32, f32.tobytes()), ("emb", [5], gw.GGML_F16, f16.tobytes())], f32, f16


@pytest.mark.parametrize("alignment", [None, 64])
def test_round_trip(tmp_path, alignment):
    g = np.random.default_rng(1)
    tensors, f32, f16 = payloads(g)
    meta = [("general.architecture", gw.STRING, "whisper"), ("whisper.encoder.layer_count", gw.U32, 32),
            ("vokra.flag", gw.BOOL, 1), ("vokra.scale", gw.F32, 0.5), ("big", gw.U64, 1 << 40),
            ("neg", gw.I32, -7), ("tokens", gw.ARRAY, (gw.STRING, ["a", "bc", ""]))]
    f = hip.GgufFile(write(tmp_path, gw.build(meta, tensors, alignment=alignment)))
    assert len(f) == len(tensors)
    for i, (name, dims, gt, payload) in enumerate(tensors):
        assert f.tensor(i) == (name, gt, dims, payload)
        assert f.find(name) == i
    assert f.meta_str("general.architecture") == "whisper"
    assert f.meta_int("whisper.encoder.layer_count") == 32
    assert f.meta_int("vokra.flag") == 1 and f.meta_int("big") == 1 << 40 and f.meta_int("neg") == -7
    assert np.array_equal(f.read_f32("ln.gamma", 6), f32)
    assert np.array_equal(f.read_f32("emb", 5), f16.astype(np.float32))  # exact widening
    if alignment:
        assert f.meta_int("general.alignment") == alignment


def test_f16_special_values(tmp_path):
    h = np.array([0.0, -0.0, 1e-7, 6.1e-5, 65504.0, np.inf, -np.inf], np.float16)
    bits = np.concatenate([h.view(np.uint16), np.array([0x0001, 0x03ff, 0x7e00], np.uint16)])
    f = hip.GgufFile(write(tmp_path, gw.build([], [("h", [bits.size], gw.GGML_F16, bits.tobytes())])))
    got = f.read_f32("h", bits.size)
    want = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(got[:-1], want[:-1]) and np.isnan(got[-1])
    assert np.array_equal(got.view(np.uint32)[:-1], want.view(np.uint32)[:-1])  # sign of zero kept


def expect(exc, tmp_path, data, match=None):
    with pytest.raises(exc, match=match):
        hip.GgufFile(write(tmp_path, data))


def test_rejections(tmp_path):
    good = b"GGUF" + struct.pack("<IQQ", 3, 0, 0)
    expect(hip.ModelLoad, tmp_path, b"GGML" + good[4:], "bad magic")
    expect(hip.ModelLoad, tmp_path, b"GGUF" + struct.pack("<IQQ", 2, 0, 0), "unsupported version")
    expect(hip.ModelLoad, tmp_path, good[:10], "truncated")
    expect(hip.ModelLoad, tmp_path, b"GGUF" + struct.pack("<IQQ", 3, 0, 1 << 40), "declared count")
    expect(hip.ModelLoad, tmp_path, b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1 << 40) + b"k",
           "truncated")
    q8 = bytes(34)
    expect(hip.ModelLoad, tmp_path, gw.build([], [("x", [32, 1], 14, bytes(210))]), "unsupported ggml type")
    expect(hip.ModelLoad, tmp_path, gw.build([], [("x", [32], gw.GGML_Q8_0, q8), ("x", [32], gw.GGML_Q8_0, q8)]),
           "duplicate tensor")
    expect(hip.ModelLoad, tmp_path, gw.build([], [("x", [32], gw.GGML_Q8_0, q8)], offsets=[8]), "not a multiple")
    expect(hip.ModelLoad, tmp_path, gw.build([], [("x", [1] * 9, gw.GGML_F32, bytes(4))]), "dimensions")
    expect(hip.ModelLoad, tmp_path, gw.build([], [("x", [100], gw.GGML_Q4_K, bytes(144))]), "whole number")
    expect(hip.ModelLoad, tmp_path, gw.build([], [("x", [48], gw.GGML_Q8_0, bytes(68))]), "whole number")
    expect(hip.ModelLoad, tmp_path, gw.build([], [], alignment=24), "invalid alignment")
    expect(hip.ModelLoad, tmp_path, gw.build([("b", gw.BOOL, 2)]), "invalid bool")
    past = gw.build([], [("x", [64], gw.GGML_F32, bytes(256))])
    expect(hip.ModelLoad, tmp_path, past[:-8], "outside the file")
    deep = (gw.U8, [])
    for _ in range(65):
        deep = (gw.ARRAY, [deep])
    expect(hip.ModelLoad, tmp_path, gw.build([("d", gw.ARRAY, deep)]), "too deep")
    with pytest.raises(hip.IoError):
        hip.GgufFile(str(tmp_path / "missing.gguf"))


def test_lookups_and_types(tmp_path):
    g = np.random.default_rng(2)
    tensors, _, _ = payloads(g)
    f = hip.GgufFile(write(tmp_path, gw.build([("s", gw.STRING, "x")], tensors)))
    with pytest.raises(hip.ModelLoad, match="missing tensor"):
        f.find("nope")
    with pytest.raises(hip.ModelLoad, match="missing metadata"):
        f.meta_int("nope")
    with pytest.raises(hip.ModelLoad, match="not an integer"):
        f.meta_int("s")
    with pytest.raises(hip.UnsupportedOp):
        f.read_f32("w.q8", 128)
    with pytest.raises(hip.InvalidArgument, match="elements"):
        f.read_f32("ln.gamma", 5)
