"""An ONNX model through the library's reader (wg_onnx_*: parseOnnxModel,
src/onnx.ts:71-282, over a memory map), the graph lookups the reference's
loader uses to find MatMulNBits weights (OnnxModel, src/load-onnx.ts:
717-830), and their upload into the device layout: 4-bit weights in
blocks of 32 through wg_repack_nbits on the GPU, 8-bit ones dequantized
(dequantizeNBitsRow, src/load-onnx.ts:471-501) and requantized there
(wg_quantize_q8), as the reference's loader stores them
(src/load-onnx.ts:208-225)."""
from __future__ import annotations

import ctypes as C
import os
import re
from dataclasses import dataclass, field

import numpy as np

from . import lib as L

# TensorProto.DataType (src/onnx.ts:8-25)
FLOAT, UINT8, INT8, UINT16, INT16, INT32, INT64 = 1, 2, 3, 4, 5, 6, 7
STRING, BOOL, FLOAT16, DOUBLE, UINT32, UINT64, BFLOAT16, UINT4, INT4 = \
    8, 9, 10, 11, 12, 13, 16, 21, 22

_SIZES = {FLOAT: 4, INT32: 4, UINT32: 4, UINT8: 1, INT8: 1, BOOL: 1, UINT16: 2, INT16: 2,
          FLOAT16: 2, BFLOAT16: 2, INT64: 8, DOUBLE: 8, UINT64: 8, UINT4: 0.5, INT4: 0.5}


def element_size(data_type: int) -> float:
    """onnxElementSize (src/onnx.ts:285-311): bytes an element, NaN if not fixed."""
    return _SIZES.get(data_type, float("nan"))


@dataclass
class OnnxTensor:
    name: str
    dims: tuple
    data_type: int
    index: int
    raw: np.ndarray | None = None          # inline bytes (a view of the map)
    external: tuple | None = None          # (location, offset, length)
    int64_data: list | None = None
    float_data: list | None = None


@dataclass
class OnnxAttribute:
    name: str
    type: int
    f: float = 0.0
    i: int = 0
    s: bytes = b""
    ints: list = field(default_factory=list)
    floats: list = field(default_factory=list)
    t: OnnxTensor | None = None


@dataclass
class OnnxNode:
    name: str
    op_type: str
    domain: str
    inputs: list
    outputs: list
    attributes: dict


def tensor_bytes(t: OnnxTensor) -> int:
    """tensorBytes (src/load-onnx.ts:683-687)."""
    n = 1
    for d in t.dims:
        n *= d
    return int(np.ceil(n * element_size(t.data_type)))


class OnnxFile:
    """The graph of one .onnx file: nodes in order, initializers by name."""

    def __init__(self, path: str):
        self._lib = L.load()
        h = C.c_void_p()
        L.check(self._lib.wg_onnx_open(str(path).encode(), C.byref(h)))
        self._h = h
        self.path = str(path)
        self.name = self._lib.wg_onnx_graph_name(h).decode()
        tensors = [self._tensor(i) for i in range(self._lib.wg_onnx_tensor_count(h))]
        n_init = int(self._lib.wg_onnx_init_count(h))
        self.initializers = {t.name: t for t in tensors[:n_init]}
        self.nodes = []
        for i in range(self._lib.wg_onnx_node_count(h)):
            n = L.OnnxNodeInfo()
            L.check(self._lib.wg_onnx_node(h, i, C.byref(n)))
            ins = [self._lib.wg_onnx_node_input(h, i, j).decode() for j in range(n.n_inputs)]
            outs = [self._lib.wg_onnx_node_output(h, i, j).decode() for j in range(n.n_outputs)]
            attrs = {}
            for j in range(n.n_attrs):
                a = L.OnnxAttr()
                L.check(self._lib.wg_onnx_node_attr(h, i, j, C.byref(a)))
                attrs[a.name.decode()] = OnnxAttribute(
                    a.name.decode(), a.type, a.f, a.i, C.string_at(a.s, a.s_len) if a.s_len else b"",
                    [a.ints[k] for k in range(a.n_ints)], [a.floats[k] for k in range(a.n_floats)],
                    tensors[a.tensor] if a.tensor >= 0 else None)
            self.nodes.append(OnnxNode(n.name.decode(), n.op_type.decode(), n.domain.decode(),
                                       ins, outs, attrs))

    def _tensor(self, i: int) -> OnnxTensor:
        t = L.OnnxTensorInfo()
        L.check(self._lib.wg_onnx_tensor(self._h, i, C.byref(t)))
        raw = None
        if t.raw and t.raw_bytes:
            raw = np.ctypeslib.as_array(C.cast(t.raw, C.POINTER(C.c_uint8)), (t.raw_bytes,))
            raw.flags.writeable = False
        elif t.raw_bytes == 0 and t.location is None and t.n_int64 == 0 and t.n_float == 0:
            raw = np.zeros(0, np.uint8)
        ext = None
        if t.location is not None:
            ext = (t.location.decode(), int(t.offset), int(t.length))
        return OnnxTensor(
            t.name.decode(), tuple(int(t.dims[d]) for d in range(t.n_dims)), int(t.data_type), i,
            raw, ext, [t.int64_data[k] for k in range(t.n_int64)] if t.n_int64 else None,
            [t.float_data[k] for k in range(t.n_float)] if t.n_float else None)

    def data(self, t: OnnxTensor) -> np.ndarray:
        """The tensor's bytes: the inline view, or a read-only view of its
        external data file (beside the model file, memory-mapped once)."""
        if t.external is None:
            if t.raw is None:
                raise ValueError(f"ONNX: {t.name} has no raw bytes")
            return t.raw
        location, offset, length = t.external
        if length < 0:
            length = tensor_bytes(t)
        maps = self.__dict__.setdefault("_maps", {})
        if location not in maps:  # each data file mapped once, read-only
            maps[location] = np.memmap(self._data_path(t.name, location), dtype=np.uint8,
                                       mode="r")
        m = maps[location]
        if offset < 0 or offset + length > m.size:
            raise ValueError(f"ONNX: {t.name}: {location} ends before byte {offset + length}")
        return m[offset:offset + length]

    def _data_path(self, name: str, location: str) -> str:
        """An external data file's path: a relative name inside the model's
        folder. An absolute location, or one whose real path leaves the
        folder (.. parts, a symbolic link out), is refused: a model file
        must not name other files for the reader to map."""
        folder = os.path.realpath(os.path.dirname(os.path.abspath(self.path)))
        if not location or os.path.isabs(location) or "\0" in location:
            raise ValueError(f"ONNX: {name}: external data location {location!r} is not a "
                             f"relative file name")
        path = os.path.realpath(os.path.join(folder, location))
        if os.path.commonpath([folder, path]) != folder or path == folder:
            raise ValueError(f"ONNX: {name}: external data location {location!r} is outside "
                             f"the model's folder")
        return path

    def close(self):
        self.__dict__.pop("_maps", None)
        if self._h:
            self._lib.wg_onnx_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def check_shape(t: OnnxTensor, data_type: int, elements: int) -> None:
    """checkShape (src/load-onnx.ts:1305-1323): type and element count."""
    if t.data_type != data_type:
        raise ValueError(f"ONNX: {t.name} has data type {t.data_type}, expected {data_type}")
    n = 1
    for d in t.dims:
        n *= d
    if n != elements:
        raise ValueError(f"ONNX: {t.name} has {n} elements, expected {elements}")


@dataclass
class NBits:
    """A MatMulNBits weight (NBits / WideNBits, src/load-onnx.ts:97-117)."""
    name: str
    node: OnnxNode
    N: int
    K: int
    bits: int
    block_size: int
    quant: OnnxTensor
    scales: OnnxTensor
    zp: OnnxTensor | None


def _spelled(name: str) -> str:
    return re.sub(r"[^a-z0-9]+", "_", name.lower())


class OnnxModel:
    """Lookups over a graph (OnnxModel, src/load-onnx.ts:717-830)."""

    def __init__(self, f: OnnxFile):
        self.file = f
        self.graph = f
        self.consumers: dict[str, list] = {}
        self.producers: dict[str, OnnxNode] = {}
        for node in f.nodes:
            for i in node.inputs:
                self.consumers.setdefault(i, []).append(node)
            for o in node.outputs:
                self.producers[o] = node

    def init(self, name: str) -> OnnxTensor:
        t = self.file.initializers.get(name)
        if t is None:
            raise ValueError(f"ONNX: missing initializer {name}")
        return t

    def has(self, name: str) -> bool:
        return name in self.file.initializers

    def constant(self, name: str) -> OnnxTensor:
        """An initializer, or a Constant node's value."""
        t = self.file.initializers.get(name)
        if t is not None:
            return t
        node = self.producers.get(name)
        value = node.attributes.get("value") if node and node.op_type == "Constant" else None
        if value is None or value.t is None:
            raise ValueError(f"ONNX: {name} is not a constant")
        return value.t

    def nbits_node(self, path: str) -> OnnxNode | None:
        """The MatMulNBits node of the module at `path` (as
        `/model/layers.0/mlp/gate_proj/`): its name starts with the path, or
        the weight it reads is the module path in any spelling. Two nodes
        for one module is an error."""
        module = _spelled(path).lstrip("_")
        nodes = [n for n in self.file.nodes if n.op_type == "MatMulNBits" and (
            n.name.startswith(path) or
            (len(n.inputs) > 1 and self.has(n.inputs[1]) and
             _spelled(n.inputs[1]).startswith(module)))]
        if len(nodes) > 1:
            raise ValueError(f"ONNX: {len(nodes)} MatMulNBits nodes under {path}")
        return nodes[0] if nodes else None

    def has_nbits(self, path: str) -> bool:
        return self.nbits_node(path) is not None

    def wide_nbits(self, path: str) -> NBits:
        """wideNBits: 4-bit in blocks of 32 or 8-bit in blocks of a multiple
        of 32, float16 or float32 scales, zero points or none."""
        node = self.nbits_node(path)
        if node is None:
            raise ValueError(f"ONNX: no MatMulNBits node under {path}")
        return self.nbits_of(node, path)

    def nbits_of(self, node: OnnxNode, label: str) -> NBits:
        """The weight a MatMulNBits node reads, checked as wide_nbits does."""
        quant = self.init(node.inputs[1])
        scales = self.init(node.inputs[2])
        zp = self.init(node.inputs[3]) if len(node.inputs) > 3 and node.inputs[3] else None

        def attr(key):
            a = node.attributes.get(key)
            return None if a is None else int(a.i)
        N, K, bits, bs = attr("N"), attr("K"), attr("bits"), attr("block_size")
        if N is None or K is None or bs is None or bits not in (4, 8) or bs % 32 or \
                (bits == 4 and bs != 32):
            raise ValueError(f"ONNX: {node.name} is not 4-bit in blocks of 32 or 8-bit in "
                             "blocks of a multiple of 32")
        if any(node.inputs[4:6]):
            raise ValueError(f"ONNX: {node.name} has g_idx or bias inputs")
        blocks = -(-K // bs)
        check_shape(quant, UINT8, N * blocks * (bs * bits // 8))
        if scales.data_type not in (FLOAT16, FLOAT):
            raise ValueError(f"ONNX: {scales.name} has data type {scales.data_type}, "
                             "expected float16 or float")
        check_shape(scales, scales.data_type, N * blocks)
        if zp is not None:
            check_shape(zp, UINT8, N * (-(-blocks // 2) if bits == 4 else blocks))
        return NBits(label, node, N, K, bits, bs, quant, scales, zp)

    def nbits(self, path: str) -> NBits:
        """nbits: the text loader's weights, blocks of 32."""
        w = self.wide_nbits(path)
        if w.block_size != 32:
            raise ValueError(f"ONNX: {w.node.name} is not in blocks of 32")
        return w


def half_bytes(t: OnnxTensor, data: np.ndarray) -> np.ndarray:
    """halfBytes (src/load-onnx.ts:450-469): float16 scales as they are,
    float32 ones rounded to the nearest half."""
    if t.data_type == FLOAT16:
        return np.ascontiguousarray(data).view(np.uint16)
    if t.data_type != FLOAT:
        raise ValueError(f"ONNX: {t.name} has data type {t.data_type}, expected float16 or float")
    return np.ascontiguousarray(data).view(np.float32).astype(np.float16).view(np.uint16)


def nbits8_floats(w: NBits, quant: np.ndarray, scales16: np.ndarray, zp: np.ndarray | None):
    """An 8-bit MatMulNBits weight's rows as floats (dequantizeNBitsRow at 8
    bits): scale * (q - zero point), zero point 128 without zp. Exact in
    float32 (a half times an integer below 2^9)."""
    N, K = w.N, w.K
    blocks = K // 32
    q = quant.reshape(N, blocks, 32).astype(np.float32)
    z = (zp.reshape(N, blocks).astype(np.float32) if zp is not None
         else np.full((N, blocks), 128.0, np.float32))
    s = scales16.reshape(N, blocks).view(np.float16).astype(np.float32)
    return (s[:, :, None] * (q - z[:, :, None])).reshape(N, K)


def upload_nbits(f: OnnxFile, w: NBits, device="cuda"):
    """The weight as a device matrix (ops.Q4Matrix), stored as the
    reference's loader stores it (src/load-onnx.ts:208-250): 4-bit weights
    keep their quants and go through wg_repack_nbits on the GPU; 8-bit
    ones are dequantized and requantized to the 8-bit layout there."""
    import torch
    from . import ops
    if w.K % 32:
        raise ValueError(f"ONNX: {w.name} has K {w.K}, not a multiple of 32")
    quant = f.data(w.quant)
    scales = half_bytes(w.scales, f.data(w.scales))
    zp = f.data(w.zp) if w.zp is not None else None
    if w.bits == 8:
        rows = nbits8_floats(w, quant, scales, zp)
        return ops.Q4Matrix.from_floats_q8(torch.from_numpy(rows).to(device))
    if w.N % 4:
        raise ValueError(f"ONNX: {w.N} rows isn't a multiple of 4")
    def t(a):  # inline bytes are a read-only view of the map: copied first
        a = np.ascontiguousarray(a)
        return torch.from_numpy(a if a.flags.writeable else a.copy()).to(device)
    return ops.Q4Matrix.from_nbits(t(quant), t(scales.view(np.int16)),
                                   t(zp) if zp is not None else None, w.N, w.K)
