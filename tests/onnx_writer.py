"""Writes ONNX ModelProto bytes from the protobuf wire format (onnx.proto's
field numbers), for tests of the reader: every field kind it reads, packed
and unpacked repeated fields, and fields it must skip."""
import struct

# TensorProto.DataType
FLOAT, UINT8, INT64, FLOAT16 = 1, 2, 7, 10


def varint(v: int) -> bytes:
    v &= (1 << 64) - 1  # negative int64: ten bytes, two's complement
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def key(field: int, wire: int) -> bytes:
    return varint(field << 3 | wire)


def f_varint(field: int, v: int) -> bytes:
    return key(field, 0) + varint(v)


def f_bytes(field: int, b) -> bytes:
    b = b.encode() if isinstance(b, str) else bytes(b)
    return key(field, 2) + varint(len(b)) + b


def f_float(field: int, v: float) -> bytes:
    return key(field, 5) + struct.pack("<f", v)


def f_fixed64(field: int, v: int) -> bytes:
    return key(field, 1) + struct.pack("<q", v)


def packed_varints(field: int, vals) -> bytes:
    return f_bytes(field, b"".join(varint(int(v)) for v in vals))


def packed_floats(field: int, vals) -> bytes:
    return f_bytes(field, struct.pack(f"<{len(vals)}f", *vals))


def tensor(name, dims, data_type, raw=None, external=None, floats=None, int64s=None,
           packed=True) -> bytes:
    """TensorProto: dims 1, data_type 2, float_data 4, int64_data 7, name 8,
    raw_data 9, external_data 13 (key 1, value 2), data_location 14."""
    out = b""
    if packed and dims:
        out += packed_varints(1, dims)
    else:
        out += b"".join(f_varint(1, d) for d in dims)
    out += f_varint(2, data_type) + f_bytes(8, name)
    if raw is not None:
        out += f_bytes(9, raw)
    if floats is not None:
        out += packed_floats(4, floats) if packed else b"".join(f_float(4, v) for v in floats)
    if int64s is not None:
        out += packed_varints(7, int64s) if packed else b"".join(f_varint(7, v) for v in int64s)
    if external is not None:
        for k, v in zip(("location", "offset", "length"), external):
            if v is not None:
                out += f_bytes(13, f_bytes(1, k) + f_bytes(2, str(v)))
        out += f_varint(14, 1)
    return out


def attr(name, type_, *, f=None, i=None, s=None, t=None, floats=None, ints=None, strings=None,
         packed=True) -> bytes:
    """AttributeProto: name 1, f 2, i 3, s 4, t 5, floats 7, ints 8, strings 9, type 20."""
    out = f_bytes(1, name) + f_varint(20, type_)
    if f is not None:
        out += f_float(2, f)
    if i is not None:
        out += f_varint(3, i)
    if s is not None:
        out += f_bytes(4, s)
    if t is not None:
        out += f_bytes(5, t)
    if floats is not None:
        out += packed_floats(7, floats) if packed else b"".join(f_float(7, v) for v in floats)
    if ints is not None:
        out += packed_varints(8, ints) if packed else b"".join(f_varint(8, v) for v in ints)
    if strings is not None:
        out += b"".join(f_bytes(9, v) for v in strings)
    return out


def node(name, op_type, inputs, outputs, attrs=(), domain="") -> bytes:
    """NodeProto: input 1, output 2, name 3, op_type 4, attribute 5, domain 7."""
    out = b"".join(f_bytes(1, i) for i in inputs) + b"".join(f_bytes(2, o) for o in outputs)
    out += f_bytes(3, name) + f_bytes(4, op_type)
    if domain:
        out += f_bytes(7, domain)
    return out + b"".join(f_bytes(5, a) for a in attrs)


def graph(name, nodes, inits, inputs=(), outputs=()) -> bytes:
    """GraphProto: node 1, name 2, initializer 5, input 11, output 12."""
    out = b"".join(f_bytes(1, n) for n in nodes) + f_bytes(2, name)
    out += b"".join(f_bytes(5, t) for t in inits)
    out += b"".join(f_bytes(11, f_bytes(1, i)) for i in inputs)
    out += b"".join(f_bytes(12, f_bytes(1, o)) for o in outputs)
    return out


def model(graph_bytes: bytes) -> bytes:
    """ModelProto: ir_version 1, producer_name 2, graph 7, opset_import 8,
    plus a fixed64 and a fixed32 field the reader skips."""
    return (f_varint(1, 8) + f_bytes(2, "tests") + f_fixed64(99, -5) + key(98, 5) +
            struct.pack("<f", 1.5) + f_bytes(8, f_bytes(1, "") + f_varint(2, 17)) +
            f_bytes(7, graph_bytes))


def matmul_nbits(prefix, N, K, bits, quant, scales, zp=None, scale_type=FLOAT16,
                 block_size=32, extra_inputs=(), quant_dims=None):
    """A MatMulNBits node and its initializers with inline bytes (the
    onnxruntime-genai naming: node `{prefix}MatMul_Quant`, weight
    `{spelled}_MatMul_weight_quant`)."""
    spelled = prefix.strip("/").replace("/", "_").replace(".", "_")
    blocks = -(-K // block_size)
    names = [f"{spelled}_MatMul_weight_quant", f"{spelled}_MatMul_weight_scales"]
    qd = quant_dims or (N, blocks, block_size * bits // 8)
    inits = [tensor(names[0], qd, UINT8, raw=quant),
             tensor(names[1], (N * blocks,), scale_type, raw=scales)]
    if zp is not None:
        names.append(f"{spelled}_MatMul_weight_zp")
        inits.append(tensor(names[2], (len(zp),), UINT8, raw=zp))
    attrs = [attr("K", 2, i=K), attr("N", 2, i=N), attr("bits", 2, i=bits),
             attr("block_size", 2, i=block_size)]
    n = node(f"{prefix}MatMul_Quant", "MatMulNBits", [f"{prefix}in"] + names + list(extra_inputs),
             [f"{prefix}out"], attrs, domain="com.microsoft")
    return n, inits
