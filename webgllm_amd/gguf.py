"""A GGUF file through the library's reader (wg_gguf_*: readGgufHeader,
src/gguf.ts:276-328, over a memory map): metadata as Python values, tensor
infos, and each tensor's bytes as a read-only numpy view of the map."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import lib as L

# ggml tensor types (src/gguf.ts:27-48)
F32, F16, Q4_0, Q4_1, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 3, 8, 12, 13, 14

# Arrays longer than this stay lazy (LazyArray), as readGgufHeader's
# maxArrayLength (src/gguf.ts:108-112).
MAX_ARRAY = 1024


@dataclass
class TensorInfo:
    name: str
    dims: tuple          # ggml order: dims[0] contiguous
    type: int
    offset: int          # absolute file offset
    nbytes: int
    index: int


@dataclass
class LazyArray:
    """An array left undecoded (GgufLazyArray): its key, element type and length."""
    key: str
    type: int
    length: int


class GgufFile:
    def __init__(self, path: str):
        self._lib = L.load()
        h = C.c_void_p()
        L.check(self._lib.wg_gguf_open(str(path).encode(), C.byref(h)))
        self._h = h
        self.path = str(path)
        self.version = int(self._lib.wg_gguf_version(h))
        self.data_offset = int(self._lib.wg_gguf_data_offset(h))
        self.tensors: dict[str, TensorInfo] = {}
        for i in range(self._lib.wg_gguf_tensor_count(h)):
            t = L.GgufTensorInfo()
            L.check(self._lib.wg_gguf_tensor(h, i, C.byref(t)))
            self.tensors[t.name.decode()] = TensorInfo(
                t.name.decode(), tuple(int(t.dims[d]) for d in range(t.n_dims)), int(t.type),
                int(t.offset), int(t.bytes), i)
        self.metadata: dict[str, object] = {}
        for i in range(self._lib.wg_gguf_meta_count(h)):
            v = L.GgufValue()
            L.check(self._lib.wg_gguf_meta(h, i, C.byref(v)))
            key = v.key.decode()
            if v.type == 9:
                self.metadata[key] = self._array(i, key, v) if v.length <= MAX_ARRAY else \
                    LazyArray(key, int(v.elem_type), int(v.length))
            else:
                self.metadata[key] = self._scalar(v)

    @staticmethod
    def _scalar(v):
        if v.type == 8:
            return C.string_at(v.s, v.length).decode("utf-8", "replace") if v.length else ""
        if v.type in (6, 12):
            return float(v.f)
        if v.type == 7:
            return bool(v.i)
        return int(v.i)

    def _array(self, i, key, v):
        out = []
        for j in range(v.length):
            e = L.GgufValue()
            L.check(self._lib.wg_gguf_meta_element(self._h, i, j, C.byref(e)))
            out.append(self._scalar(e))
        return out

    def read_array(self, key: str) -> list:
        """A lazy array's elements (readGgufArray, src/gguf.ts:346-360)."""
        i = int(self._lib.wg_gguf_find_meta(self._h, key.encode()))
        if i < 0:
            raise KeyError(key)
        v = L.GgufValue()
        L.check(self._lib.wg_gguf_meta(self._h, i, C.byref(v)))
        return self._array(i, key, v)

    def data(self, name: str) -> np.ndarray:
        """A tensor's bytes as a read-only view of the file's map (valid until close)."""
        info = self.tensors[name]
        t = L.GgufTensorInfo()
        L.check(self._lib.wg_gguf_tensor(self._h, info.index, C.byref(t)))
        if not t.data:
            raise ValueError(f"GGUF: {name} has type {info.type}, which has no known size")
        buf = (C.c_uint8 * int(t.bytes)).from_address(t.data)
        arr = np.frombuffer(buf, dtype=np.uint8)
        arr.flags.writeable = False
        return arr

    def close(self):
        if self._h:
            self._lib.wg_gguf_close(self._h)
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
