"""A minimal GGUF v3 writer for tests (test infrastructure): the on-disk layout
of crates/vokra-core/src/gguf/mod.rs:1-100 written independently of the
library's reader, with knobs to produce the malformed files the reference
reader rejects (crates/vokra-core/src/gguf/reader.rs:512-800)."""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q5_0, GGML_Q8_0, GGML_Q4_K = 0, 1, 2, 6, 8, 12
GGML_Q5_K, GGML_Q6_K, GGML_BF16 = 13, 14, 30


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def value(t, v) -> bytes:
    if t == STRING:
        return gstr(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def build(metadata=(), tensors=(), alignment=None, version=3, magic=b"GGUF", kv_count=None, tensor_count=None,
          offsets=None):
    """metadata: [(key, type, value)]; tensors: [(name, dims, ggml_type, payload)].
    `offsets` overrides the tensor offsets (relative to the data region)."""
    meta = list(metadata)
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
    align = alignment or 32
    out = bytearray(magic + struct.pack("<I", version))
    out += struct.pack("<QQ", len(tensors) if tensor_count is None else tensor_count,
                       len(meta) if kv_count is None else kv_count)
    for k, t, v in meta:
        out += gstr(k) + struct.pack("<I", t) + value(t, v)
    offs, pos = [], 0
    for _, _, _, payload in tensors:
        offs.append(pos)
        pos += (len(payload) + align - 1) // align * align
    if offsets is not None:
        offs = list(offsets)
    for (name, dims, gt, _), off in zip(tensors, offs):
        out += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gt, off)
    if tensors:
        out += b"\0" * ((-len(out)) % align)
        size = max(off + len(payload) for (_, _, _, payload), off in zip(tensors, offs))
        data = bytearray((size + align - 1) // align * align)
        for (_, _, _, payload), off in zip(tensors, offs):
            data[off:off + len(payload)] = payload
        out += data
    return bytes(out)
