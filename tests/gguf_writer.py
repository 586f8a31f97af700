"""Writes GGUF v3 files for the tests, byte for byte as the GGUF layout that nn-gguf
reads (crates/nn-gguf/src/header.rs, metadata.rs, tensor_info.rs; the reference's own
synthetic writers, e.g. crates/nn-gguf/tests/qwen3_gguf.rs:131-200, lay files out the
same way): header, metadata pairs, tensor infos, zero padding to 32 bytes, then the
tensor data at the recorded offsets."""
import struct

MAGIC = 0x46554747

# metadata value type ids
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def gguf_string(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value_bytes(t, v):
    if t == STRING:
        return gguf_string(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value_bytes(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def build(metadata, tensors, version=3, align=32, offsets=None, magic=MAGIC):
    """metadata: [(key, type, value)]; tensors: [(name, dims, dtype, data bytes)].  Data are
    laid out back to back in order unless `offsets` gives each tensor's offset."""
    buf = bytearray(struct.pack("<IIQQ", magic, version, len(tensors), len(metadata)))
    for key, t, v in metadata:
        buf += gguf_string(key) + struct.pack("<I", t) + value_bytes(t, v)
    off, offs = 0, []
    for i, (name, dims, dtype, data) in enumerate(tensors):
        o = offsets[i] if offsets is not None else off
        offs.append(o)
        buf += gguf_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        buf += struct.pack("<IQ", dtype, o)
        off = o + len(data)
    while len(buf) % align:
        buf.append(0)
    base = len(buf)
    end = max([o + len(t[3]) for o, t in zip(offs, tensors)] + [0])
    buf += bytes(end)
    for o, (_, _, _, data) in zip(offs, tensors):
        buf[base + o:base + o + len(data)] = data
    return bytes(buf), base
