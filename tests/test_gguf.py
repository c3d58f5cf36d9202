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
    expect(hip.ModelLoad, tmp_path, gw.build([], [("x", [32, 1], 7, bytes(24))]), "unsupported ggml type")  # Q5_1
    expect(hip.ModelLoad, tmp_path, gw.build([], [("x", [32, 1], gw.GGML_Q6_K, bytes(210))]), "whole number")
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


# ---- a GGUF file written by the reference's own converter --------------------
# tests/golden/silero-vad-v5.gguf is tests/parity/silero_vad/silero-vad-v5.gguf
# of the reference, copied as data: a v3 file from its converter with 30 F32
# tensors and 2 string metadata keys. Its layout is read here a second time by
# a few lines of struct parsing that share nothing with the library's reader.
SILERO = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "silero-vad-v5.gguf")


def independent_parse(data):
    """(version, alignment, metadata {key: (type, value)}, tensors [(name,
    dims, type, offset)], data_offset): the GGUF v3 layout of
    crates/vokra-core/src/gguf/mod.rs:1-100, string and scalar values only."""
    pos = 4
    version, n_t, n_kv = struct.unpack_from("<IQQ", data, pos)
    pos += 20

    def rstr(p):
        n = struct.unpack_from("<Q", data, p)[0]
        return data[p + 8:p + 8 + n].decode(), p + 8 + n

    scalars = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}
    meta = {}
    for _ in range(n_kv):
        key, pos = rstr(pos)
        t = struct.unpack_from("<I", data, pos)[0]
        pos += 4
        if t == 8:
            val, pos = rstr(pos)
        else:
            val = struct.unpack_from(scalars[t], data, pos)[0]
            pos += struct.calcsize(scalars[t])
        meta[key] = (t, val)
    tensors = []
    for _ in range(n_t):
        name, pos = rstr(pos)
        nd = struct.unpack_from("<I", data, pos)[0]
        dims = list(struct.unpack_from(f"<{nd}Q", data, pos + 4))
        pos += 4 + 8 * nd
        t, off = struct.unpack_from("<IQ", data, pos)
        pos += 12
        tensors.append((name, dims, t, off))
    align = meta.get("general.alignment", (4, 32))[1]
    return version, align, meta, tensors, (pos + align - 1) // align * align


def test_reference_written_gguf():
    data = open(SILERO, "rb").read()
    version, align, meta, tensors, data_off = independent_parse(data)
    assert data[:4] == b"GGUF" and version == 3 and align == 32
    assert meta == {"vokra.model.arch": (8, "silero-vad"), "vokra.model.name": (8, "silero-vad-v5")}
    assert len(tensors) == 30 and all(t[2] == gw.GGML_F32 for t in tensors)
    f = hip.GgufFile(SILERO)
    assert len(f) == 30
    assert f.meta_str("vokra.model.arch") == "silero-vad" and f.meta_str("vokra.model.name") == "silero-vad-v5"
    spans = []
    for i, (name, dims, t, off) in enumerate(tensors):
        n = int(np.prod(dims))
        start = data_off + off
        # the reader's checks (reader.rs:333-510): offsets aligned, the payload
        # (4 bytes per F32 element) inside the file
        assert off % align == 0 and start + 4 * n <= len(data)
        got_name, got_type, got_dims, payload = f.tensor(i)
        assert (got_name, got_type, got_dims) == (name, t, dims) and f.find(name) == i
        assert payload == data[start:start + 4 * n]
        assert np.array_equal(f.read_f32(name, n), np.frombuffer(data, np.float32, n, start))
        spans.append((start, start + 4 * n))
    spans.sort()
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))   # no two payloads overlap
    # the converter's shapes for the 16 kHz branch (PyTorch order, as stored)
    shapes = {name: dims for name, dims, _, _ in tensors}
    assert shapes["sr16k.stft.forward_basis_buffer"] == [258, 1, 256]
    assert shapes["sr16k.decoder.rnn.weight_ih"] == [512, 128]
    assert shapes["sr8k.encoder.0.reparam_conv.weight"] == [128, 65, 3]


def test_reference_written_gguf_truncations(tmp_path):
    """Every cut of the reference-written file inside its header or tensor
    table is a ModelLoad error, and so is a cut that leaves the last payload
    short: the reader never reads past what it was given."""
    data = open(SILERO, "rb").read()
    _, _, _, tensors, data_off = independent_parse(data)
    cuts = sorted(set(list(range(0, 64)) + list(range(64, data_off, 97)) + [data_off - 1, len(data) - 4,
                                                                              len(data) - 1]))
    for cut in cuts:
        with pytest.raises(hip.ModelLoad):
            hip.GgufFile(write(tmp_path, data[:cut], f"cut{cut}.gguf"))
    bad = bytearray(data)
    bad[4:8] = struct.pack("<I", 2)
    with pytest.raises(hip.ModelLoad, match="unsupported version"):
        hip.GgufFile(write(tmp_path, bytes(bad), "v2.gguf"))


def test_kquant_and_bf16_tensors(tmp_path):
    """The reference reader's other tensor types (tensor.rs:85-95): Q5_K (176
    bytes per 256), Q6_K (210) and BF16 round-trip; BF16 widens to f32
    exactly (its 16 bits become the high half)."""
    g = np.random.default_rng(3)
    q5 = bytes(g.integers(0, 256, 176 * 3, dtype=np.uint8))
    q6 = bytes(g.integers(0, 256, 210 * 2, dtype=np.uint8))
    x = g.standard_normal(7).astype(np.float32)
    bf = (x.view(np.uint32) >> 16).astype(np.uint16)
    tensors = [("w.q5", [256, 3], gw.GGML_Q5_K, q5), ("w.q6", [512], gw.GGML_Q6_K, q6),
               ("n.bf", [7], gw.GGML_BF16, bf.tobytes())]
    f = hip.GgufFile(write(tmp_path, gw.build([], tensors)))
    for i, (name, dims, gt, payload) in enumerate(tensors):
        assert f.tensor(i) == (name, gt, dims, payload)
    want = (bf.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(f.read_f32("n.bf", 7).view(np.uint32), want.view(np.uint32))
    with pytest.raises(hip.UnsupportedOp):
        f.read_f32("w.q5", 768)
