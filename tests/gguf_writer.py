"""Writes small GGUF (v2/v3) files for the reader and loader tests, from
the published format (what readGgufHeader, src/gguf.ts:276-328, reads):
magic "GGUF", version u32, tensor count u64, key count u64; each key (u64
length + bytes), a u32 value type and the value (strings u64 length +
bytes; arrays u32 element type, u64 count, elements); each tensor's name,
u32 dims count, u64 dims (ggml order), u32 ggml type, u64 offset from the
data section; the data section at the header's end rounded up to
general.alignment (32 by default)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}

# [weights per block, bytes per block] (src/gguf.ts:49-71)
BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 8: (32, 34), 12: (256, 144),
         13: (256, 176), 14: (256, 210)}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def tensor_bytes(ggml_type, dims):
    w, b = BLOCK[ggml_type]
    rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
    return -(-dims[0] // w) * b * rows


def write_gguf(path, metadata, tensors, version=3, alignment=None):
    """metadata: [(key, value type, value)]; tensors: [(name, dims, ggml type,
    bytes)]. Returns the data section's offset."""
    meta = list(metadata)
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
    align = alignment or 32
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, t, v in meta:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offset = 0
    blobs = []
    for name, dims, t, data in tensors:
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1).tobytes()
        assert len(data) == tensor_bytes(t, dims), name
        head += _str(name) + struct.pack("<I", len(dims)) + \
            b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", t, offset)
        pad = (-len(data)) % align
        blobs.append(data + b"\0" * pad)
        offset += len(data) + pad
    data_offset = -(-len(head) // align) * align
    with open(path, "wb") as f:
        f.write(head + b"\0" * (data_offset - len(head)) + b"".join(blobs))
    return data_offset
