"""ctypes front of the CPU oracle (liboracle.so, built from oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, the smoke check in __graft_entry__.py and
bench.py's CPU-baseline leg use it as the checker. The product package
(webgllm_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    if not os.path.exists(_LIB_PATH):
        build()
    return C.CDLL(_LIB_PATH)


_lib = _load()

_P = C.c_void_p
_I = C.c_int


class _QM(C.Structure):
    _fields_ = [("N", _I), ("K", _I), ("quants", _P), ("scales", _P), ("zeros", _P),
                ("zero_halves", _P), ("raw", _P)]


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


_lib.orc_to_half.restype = C.c_uint16
_lib.orc_to_half.argtypes = [C.c_double]
_lib.orc_from_half.restype = C.c_float
_lib.orc_from_half.argtypes = [C.c_uint16]
for name in ("orc_pack_q4_0", "orc_pack_q4_k"):
    getattr(_lib, name).argtypes = [C.POINTER(_QM), _I, _P, C.c_size_t, _I, _P]
_lib.orc_pack_nbits.argtypes = [C.POINTER(_QM), _I, _P, _P, _P, _I, _P]
_lib.orc_pack_nbits_scales.argtypes = [C.POINTER(_QM), _I, _P, _P, _I]
_lib.orc_quants_from_raw.argtypes = [_P, _I, _I, _P]
_lib.orc_matrix_row.argtypes = [C.POINTER(_QM), _I, _P]
_lib.orc_matrix_dense.argtypes = [C.POINTER(_QM), _P, _I]
_lib.orc_dequantize_q4_k.argtypes = [_P, _I, _I, _P]
_lib.orc_dequantize_nbits_row.argtypes = [_I, _P, _P, _P, _I, _P]
_lib.orc_quantize_q4_0.argtypes = [_P, _I, _I, _P]
_lib.orc_quantize_nbits.argtypes = [_P, _I, _I, _P, _P, _P, _P]
_lib.orc_pack_q8_0.argtypes = [_P, _P, _I, _I, _I, _P, C.c_size_t, _I, _P]
_lib.orc_quantize_q8.argtypes = [_P, _P, _I, _I, _I, _P, _I]
_lib.orc_pack_q6_k.argtypes = [_P, _P, _I, _I, _I, _P, C.c_size_t, _I, _P]
_lib.orc_dequantize_q8_0.argtypes = [_P, _I, _I, _P]
_lib.orc_dequantize_q6_k.argtypes = [_P, _I, _I, _P]
_lib.orc_dequantize_q4_1.argtypes = [_P, _I, _I, _P]
_lib.orc_dequantize_q5_k.argtypes = [_P, _I, _I, _P]
_lib.orc_q8_row.argtypes = [_P, _P, _I, _I, _P]
_lib.orc_q6k_row.argtypes = [_P, _P, _I, _I, _P]
_lib.orc_matmul_q8.argtypes = [_P, _P, _I, _I, _P, _I, _P, _I, _I, _I]
_lib.orc_matmul_q6k.argtypes = [_P, _P, _I, _I, _P, _I, _P, _I]
_lib.orc_gemv_f64.argtypes = [C.POINTER(_QM), _P, _I, _P, _I]
_lib.orc_matmul_split.argtypes = [C.POINTER(_QM), _P, _I, _P, _I, _I, _I]
_lib.orc_f32_to_h2.argtypes = [_P, C.c_size_t, _P]
_lib.orc_rms_norm.argtypes = [_P, _P, _I, _I, C.c_float, _P]
_lib.orc_swiglu.argtypes = [_P, _I, _I, _P]
_lib.orc_rope_table.argtypes = [C.c_double, _I, _I, _I, _I, _P]
_lib.orc_rope_rows.argtypes = [_I]
_lib.orc_head_prep.argtypes = [_P, _P, _P, _I, _I, _I, C.c_float, C.c_float, _I, _P]
_lib.orc_attention_f64.argtypes = [_P, _P, _P, _I, _I, _I, _I, _I, _P]
_lib.orc_attention_f32.argtypes = [_P, _P, _P, _I, _I, _I, _I, _I, _P, _I]
_lib.orc_short_conv.argtypes = [_P, _I, _I, _I, _P, _P, _P, _P, _P]
_lib.orc_pick_candidates.argtypes = [_P, _I, _I, _P, _P, _I, _I, C.c_float, C.c_float, _P, _I,
                                     _I, _I, _P, _P]
_lib.orc_argmax.restype = _I
_lib.orc_argmax.argtypes = [_P, _I, C.POINTER(C.c_float)]
_lib.orc_now.restype = C.c_double


def to_half(v: float) -> int:
    return int(_lib.orc_to_half(float(v)))


def from_half(h: int) -> float:
    return float(_lib.orc_from_half(int(h) & 0xFFFF))


def halves_to_f32(h: np.ndarray) -> np.ndarray:
    """Half bits to float32 through the oracle's own table (half.ts:37-55)."""
    table = np.array([_lib.orc_from_half(i) for i in range(65536)], dtype=np.float32) \
        if not hasattr(halves_to_f32, "_t") else halves_to_f32._t
    halves_to_f32._t = table
    return table[np.asarray(h, dtype=np.uint16)]


def f32_to_h2(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    _lib.orc_f32_to_h2(_ptr(x), x.size, _ptr(out))
    return out


class QuantMatrix:
    """src/weights.ts:153-178 as numpy arrays (4-bit only)."""

    def __init__(self, N: int, K: int, zeros: bool | str = False):
        if N % 4:
            raise ValueError(f"matrix rows ({N}) must be a multiple of 4")
        if K % 32:
            raise ValueError(f"matrix columns ({K}) must be a multiple of 32")
        self.N, self.K = N, K
        blocks = K // 32
        self.quants = np.zeros(N * blocks * 4, dtype=np.uint32)
        self.scales = np.zeros(N * blocks, dtype=np.uint16)
        self.zeros = np.full(N * blocks, 8, dtype=np.uint8) if zeros is True else None
        self.zero_halves = np.zeros(N * blocks, dtype=np.uint16) if zeros == "halves" else None
        self.raw = None

    def _c(self):
        return _QM(self.N, self.K, _ptr(self.quants), _ptr(self.scales), _ptr(self.zeros),
                   _ptr(self.zero_halves), _ptr(self.raw))

    def row(self, n: int) -> np.ndarray:
        out = np.empty(self.K, dtype=np.float32)
        _lib.orc_matrix_row(C.byref(self._c()), n, _ptr(out))
        return out

    def dense(self, threads: int = 0) -> np.ndarray:
        out = np.empty((self.N, self.K), dtype=np.float32)
        _lib.orc_matrix_dense(C.byref(self._c()), _ptr(out), threads)
        return out


class WideMatrix:
    """An 8-bit or 6-bit QuantMatrix (src/weights.ts:9-11, :23-30) as numpy
    arrays: `quants` bytes and half `scales` in the reference's order."""

    def __init__(self, N: int, K: int, bits: int):
        unit = 256 if bits == 6 else 32
        if N % 4:
            raise ValueError(f"matrix rows ({N}) must be a multiple of 4")
        if K % unit:
            raise ValueError(f"matrix columns ({K}) must be a multiple of {unit}")
        self.N, self.K, self.bits = N, K, bits
        self.quants = np.zeros(N * K if bits == 8 else N * (K // 256) * 208, dtype=np.uint8)
        self.scales = np.zeros(N * (K // unit), dtype=np.uint16)

    def row(self, n: int) -> np.ndarray:
        out = np.empty(self.K, dtype=np.float32)
        fn = _lib.orc_q8_row if self.bits == 8 else _lib.orc_q6k_row
        fn(_ptr(self.quants), _ptr(self.scales), self.K, n, _ptr(out))
        return out

    def dense(self) -> np.ndarray:
        return np.stack([self.row(n) for n in range(self.N)])

    def matmul(self, x16: np.ndarray, threads: int = 0, split_fragments: int = 4096,
               max_split: int = 16) -> np.ndarray:
        """The reference's float32 block form (8-bit: the split matmul; 6-bit:
        the Q6_K head) of y = x W^T for half activations x16 [M, K]."""
        x16 = np.ascontiguousarray(x16, dtype=np.uint16).reshape(-1, self.K)
        y = np.empty((x16.shape[0], self.N), dtype=np.float32)
        if self.bits == 8:
            _lib.orc_matmul_q8(_ptr(self.quants), _ptr(self.scales), self.N, self.K, _ptr(x16),
                               x16.shape[0], _ptr(y), threads, split_fragments, max_split)
        else:
            _lib.orc_matmul_q6k(_ptr(self.quants), _ptr(self.scales), self.N, self.K, _ptr(x16),
                                x16.shape[0], _ptr(y), threads)
        return y


def pack_q8_0(m: WideMatrix, row0: int, src: np.ndarray, rows: int, src_rows=None) -> None:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    sr = _rows(src_rows)
    if _lib.orc_pack_q8_0(_ptr(m.quants), _ptr(m.scales), m.N, m.K, row0, _ptr(src), src.size,
                          rows, _ptr(sr)):
        raise ValueError("packQ8_0 failed")


def quantize_q8(m: WideMatrix, row0: int, values: np.ndarray) -> None:
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1, m.K)
    if _lib.orc_quantize_q8(_ptr(m.quants), _ptr(m.scales), m.N, m.K, row0, _ptr(values),
                            values.shape[0]):
        raise ValueError("quantizeQ8 failed")


def pack_q6_k(m: WideMatrix, row0: int, src: np.ndarray, rows: int, src_rows=None) -> None:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    sr = _rows(src_rows)
    if _lib.orc_pack_q6_k(_ptr(m.quants), _ptr(m.scales), m.N, m.K, row0, _ptr(src), src.size,
                          rows, _ptr(sr)):
        raise ValueError("packQ6_K failed")


def dequantize_q8_0(src: np.ndarray, rows: int, K: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(rows * K, dtype=np.float32)
    _lib.orc_dequantize_q8_0(_ptr(src), rows, K, _ptr(out))
    return out.reshape(rows, K)


def dequantize_q6_k(src: np.ndarray, rows: int, K: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(rows * K, dtype=np.float32)
    _lib.orc_dequantize_q6_k(_ptr(src), rows, K, _ptr(out))
    return out.reshape(rows, K)


def dequantize_q4_1(src: np.ndarray, rows: int, K: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(rows * K, dtype=np.float32)
    _lib.orc_dequantize_q4_1(_ptr(src), rows, K, _ptr(out))
    return out.reshape(rows, K)


def dequantize_q5_k(src: np.ndarray, rows: int, K: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(rows * K, dtype=np.float32)
    _lib.orc_dequantize_q5_k(_ptr(src), rows, K, _ptr(out))
    return out.reshape(rows, K)


def _rows(src_rows):
    return None if src_rows is None else np.ascontiguousarray(src_rows, dtype=np.int32)


def pack_q4_0(m: QuantMatrix, row0: int, src: np.ndarray, rows: int, src_rows=None) -> None:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    sr = _rows(src_rows)
    rc = _lib.orc_pack_q4_0(C.byref(m._c()), row0, _ptr(src), src.size, rows, _ptr(sr))
    if rc:
        raise ValueError(f"packQ4_0 failed ({rc})")


def pack_q4_k(m: QuantMatrix, row0: int, src: np.ndarray, rows: int, src_rows=None) -> None:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    sr = _rows(src_rows)
    rc = _lib.orc_pack_q4_k(C.byref(m._c()), row0, _ptr(src), src.size, rows, _ptr(sr))
    if rc == -3:
        raise ValueError("Q4_K rows go into a matrix with fractional zero points")
    if rc:
        raise ValueError(f"packQ4_K failed ({rc})")


def q4k_from_records(quants: np.ndarray, recs: np.ndarray, N: int, K: int) -> np.ndarray:
    """The GGUF Q4_K super-blocks ([N][K/256][144] bytes, rows in stored
    order) behind a backend matrix of Q4_K records (WG_ZERO_Q4K): the
    inverse of its layout, for the checks. quants: the row-group nibble rows
    (byte k of a block row: weight k low, weight k + 16 high); recs: a
    64-byte record a row group and super-block (the 4 rows' d and dmin, then
    block pair i's 96 bits at byte 16 + 12 i, row r of a block at bits 12 r
    (scale) and 12 r + 6 (min)). The 12 scale bytes are get_scale_min_k4's
    encoding (src/repack.ts:127-140). A block packQ4_K makes constant comes
    back with 15s, which packQ4_K reads as the file's own nibbles."""
    G, S = N // 4, K // 256
    q = np.asarray(quants, dtype=np.uint8).reshape(G, S, 8, 4, 16)  # g, s, block, row, byte
    rec = np.asarray(recs, dtype=np.uint8).reshape(G, S, 64)
    out = np.zeros((G, 4, S, 144), np.uint8)
    out[..., 0:4] = rec[:, :, 0:16].reshape(G, S, 4, 4).transpose(0, 2, 1, 3)
    bits = rec[:, :, 16:64].reshape(G, S, 4, 12)  # block pair i's 96 bits
    lo = bits[..., 0:8].copy().view("<u8")[..., 0]
    hi = bits[..., 8:12].copy().view("<u4")[..., 0].astype(np.uint64)
    sc = np.zeros((G, S, 8, 4), np.uint8)
    mn = np.zeros((G, S, 8, 4), np.uint8)
    for j in range(8):
        for r in range(4):
            for which, dst in ((0, sc), (1, mn)):
                bit = 48 * (j & 1) + 12 * r + 6 * which
                pair_lo, pair_hi = lo[:, :, j >> 1], hi[:, :, j >> 1]
                if bit + 6 <= 64:
                    v = (pair_lo >> np.uint64(bit)) & np.uint64(63)
                elif bit >= 64:
                    v = (pair_hi >> np.uint64(bit - 64)) & np.uint64(63)
                else:
                    v = ((pair_lo >> np.uint64(bit)) | (pair_hi << np.uint64(64 - bit))) & np.uint64(63)
                dst[:, :, j, r] = v.astype(np.uint8)
    scb = np.zeros((G, S, 4, 12), np.uint8)  # g, s, row, byte
    s_, m_ = sc.transpose(0, 1, 3, 2), mn.transpose(0, 1, 3, 2)  # g, s, row, block
    scb[..., 0:4] = (s_[..., 0:4] & 63) | ((s_[..., 4:8] >> 4) << 6)
    scb[..., 4:8] = (m_[..., 0:4] & 63) | ((m_[..., 4:8] >> 4) << 6)
    scb[..., 8:12] = (s_[..., 4:8] & 15) | ((m_[..., 4:8] & 15) << 4)
    out[..., 4:16] = scb.transpose(0, 2, 1, 3)
    qe = q[:, :, 0::2].transpose(0, 3, 1, 2, 4)  # g, row, s, pair, byte: blocks 2i
    qo = q[:, :, 1::2].transpose(0, 3, 1, 2, 4)  # blocks 2i + 1
    chunk = np.zeros(qe.shape[:-1] + (32,), np.uint8)
    chunk[..., 0:16] = (qe & 15) | ((qo & 15) << 4)
    chunk[..., 16:32] = (qe >> 4) | (qo & 0xF0)
    out[..., 16:144] = chunk.reshape(G, 4, S, 128)
    return out.reshape(N, S * 144)


def pack_nbits(m: QuantMatrix, row0: int, quant, scale_bytes, zp, rows: int, src_rows=None):
    quant = np.ascontiguousarray(quant, dtype=np.uint8)
    scale_bytes = np.ascontiguousarray(scale_bytes).view(np.uint8)
    zp = None if zp is None else np.ascontiguousarray(zp, dtype=np.uint8)
    sr = _rows(src_rows)
    rc = _lib.orc_pack_nbits(C.byref(m._c()), row0, _ptr(quant), _ptr(scale_bytes), _ptr(zp),
                             rows, _ptr(sr))
    if rc:
        raise ValueError(f"packMatMulNBits failed ({rc})")


def pack_nbits_scales(m: QuantMatrix, row0: int, scale_bytes, zp, rows: int):
    scale_bytes = np.ascontiguousarray(scale_bytes).view(np.uint8)
    zp = None if zp is None else np.ascontiguousarray(zp, dtype=np.uint8)
    rc = _lib.orc_pack_nbits_scales(C.byref(m._c()), row0, _ptr(scale_bytes), _ptr(zp), rows)
    if rc:
        raise ValueError(f"packMatMulNBitsScales failed ({rc})")


def quants_from_raw(raw: np.ndarray, N: int, K: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros(N * K // 32 * 4, dtype=np.uint32)
    _lib.orc_quants_from_raw(_ptr(raw), N, K, _ptr(out))
    return out


def dequantize_q4_k(src: np.ndarray, rows: int, K: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(rows * K, dtype=np.float32)
    _lib.orc_dequantize_q4_k(_ptr(src), rows, K, _ptr(out))
    return out.reshape(rows, K)


def dequantize_nbits_row(K, quant, scale_bytes, zp, n) -> np.ndarray:
    quant = np.ascontiguousarray(quant, dtype=np.uint8)
    scale_bytes = np.ascontiguousarray(scale_bytes).view(np.uint8)
    zp = None if zp is None else np.ascontiguousarray(zp, dtype=np.uint8)
    out = np.empty(K, dtype=np.float32)
    _lib.orc_dequantize_nbits_row(K, _ptr(quant), _ptr(scale_bytes), _ptr(zp), n, _ptr(out))
    return out


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, K = w.shape
    out = np.empty(rows * K // 32 * 18, dtype=np.uint8)
    _lib.orc_quantize_q4_0(_ptr(w), rows, K, _ptr(out))
    return out


def quantize_nbits(w: np.ndarray, zp_blocks: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, K = w.shape
    blocks = K // 32
    zpb = np.ascontiguousarray(zp_blocks, dtype=np.uint8)
    quant = np.empty(rows * blocks * 16, dtype=np.uint8)
    scales = np.empty(rows * blocks, dtype=np.uint16)
    zp = np.empty(rows * ((blocks + 1) // 2), dtype=np.uint8)
    _lib.orc_quantize_nbits(_ptr(w), rows, K, _ptr(zpb), _ptr(quant), _ptr(scales), _ptr(zp))
    return quant, scales, zp


def gemv_f64(m: QuantMatrix, x: np.ndarray, threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, m.K)
    y = np.empty((x.shape[0], m.N), dtype=np.float64)
    _lib.orc_gemv_f64(C.byref(m._c()), _ptr(x), x.shape[0], _ptr(y), threads)
    return y


def matmul_split(m: QuantMatrix, x16: np.ndarray, threads: int = 0, split_fragments: int = 4096,
                 max_split: int = 16) -> np.ndarray:
    x16 = np.ascontiguousarray(x16, dtype=np.uint16).reshape(-1, m.K)
    y = np.empty((x16.shape[0], m.N), dtype=np.float32)
    _lib.orc_matmul_split(C.byref(m._c()), _ptr(x16), x16.shape[0], _ptr(y), threads,
                          split_fragments, max_split)
    return y


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, D = x.reshape(-1, x.shape[-1]).shape
    out = np.empty_like(x)
    _lib.orc_rms_norm(_ptr(x), _ptr(w), M, D, eps, _ptr(out))
    return out


def swiglu(gu: np.ndarray) -> np.ndarray:
    gu = np.ascontiguousarray(gu, dtype=np.float32)
    M, F2 = gu.reshape(-1, gu.shape[-1]).shape
    out = np.empty((M, F2 // 2), dtype=np.float32)
    _lib.orc_swiglu(_ptr(gu), M, F2 // 2, _ptr(out))
    return out


def rope_table(theta: float, head_dim: int, rotated_dims: int, context: int,
               freq_dims: int | None = None) -> np.ndarray:
    rows = _lib.orc_rope_rows(context)
    t = np.empty((rows, head_dim), dtype=np.float32)
    _lib.orc_rope_table(theta, head_dim, rotated_dims, freq_dims or head_dim, context, _ptr(t))
    return t


def head_prep(x, norm_w, rope, head_dim, rotated_dims, pos, eps, scale, use_norm) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    nw = np.ascontiguousarray(norm_w if norm_w is not None else np.ones(head_dim), dtype=np.float32)
    rope = np.ascontiguousarray(rope, dtype=np.float32)
    out = np.empty(head_dim, dtype=np.float32)
    _lib.orc_head_prep(_ptr(x), _ptr(nw), _ptr(rope), head_dim, rotated_dims, pos, eps, scale,
                       int(use_norm), _ptr(out))
    return out


def attention_f64(q, kc, vc, heads, kv_heads, head_dim, keys, kv_stride) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc, dtype=np.uint16)
    vc = np.ascontiguousarray(vc, dtype=np.uint16)
    out = np.empty(heads * head_dim, dtype=np.float64)
    _lib.orc_attention_f64(_ptr(q), _ptr(kc), _ptr(vc), heads, kv_heads, head_dim, keys,
                           kv_stride, _ptr(out))
    return out


def attention_f32(q, kc, vc, heads, kv_heads, head_dim, keys, kv_stride, threads=0):
    """The shaders' float32 attention (heads in parallel with threads > 0)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc, dtype=np.uint16)
    vc = np.ascontiguousarray(vc, dtype=np.uint16)
    out = np.empty(heads * head_dim, dtype=np.float32)
    _lib.orc_attention_f32(_ptr(q), _ptr(kc), _ptr(vc), heads, kv_heads, head_dim, keys,
                           kv_stride, _ptr(out), threads)
    return out


def short_conv(bcx, D, W, taps, state, prefixes=False):
    bcx = np.ascontiguousarray(bcx, dtype=np.float32).reshape(-1, 3 * D)
    M = bcx.shape[0]
    taps = np.ascontiguousarray(taps, dtype=np.float32)
    state = np.ascontiguousarray(state, dtype=np.float32)
    out = np.empty((M, D), dtype=np.float32)
    new_state = np.empty((W - 1, D), dtype=np.float32)
    pre = np.empty((M, W - 1, D), dtype=np.float32) if prefixes else None
    _lib.orc_short_conv(_ptr(bcx), M, D, W, _ptr(taps), _ptr(state), _ptr(out), _ptr(new_state),
                        _ptr(pre))
    return (out, new_state, pre) if prefixes else (out, new_state)


def pick_candidates(logits, count, mask=None, seen_rows=None, row0=0, penalty=1.0,
                    presence=0.0, allowed=None):
    """(chunks [M, count], candidates [M, count, 256]) as wg_pick_candidates."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    logits2 = logits.reshape(-1, logits.shape[-1])
    M, V = logits2.shape
    mask = None if mask is None else np.ascontiguousarray(mask, dtype=np.uint8)
    seen = None if not seen_rows else np.ascontiguousarray(seen_rows, dtype=np.int32).reshape(-1, 4)
    allowed = None if allowed is None else np.ascontiguousarray(allowed, dtype=np.uint32)
    chunks = np.empty((M, count), np.int32)
    cand = np.empty((M, count, 256), np.float32)
    _lib.orc_pick_candidates(_ptr(logits2), M, V, _ptr(mask), _ptr(seen),
                             0 if seen is None else seen.shape[0], row0, penalty, presence,
                             _ptr(allowed), 0 if allowed is None else allowed.shape[0],
                             0 if allowed is None else allowed.shape[1], count, _ptr(chunks),
                             _ptr(cand))
    return chunks, cand


def argmax(logits: np.ndarray):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    top = C.c_float()
    at = _lib.orc_argmax(_ptr(logits), logits.size, C.byref(top))
    return at, top.value


def now() -> float:
    return _lib.orc_now()


class Mulberry32:
    """The reference tests' generator (src/q4k-pack.test.ts:6-16)."""

    def __init__(self, seed: int):
        self.a = seed & 0xFFFFFFFF

    def __call__(self) -> float:
        self.a = (self.a + 0x6D2B79F5) & 0xFFFFFFFF
        t = self.a
        t = _imul(t ^ (t >> 15), t | 1)
        t ^= (t + _imul(t ^ (t >> 7), t | 61)) & 0xFFFFFFFF
        return ((t ^ (t >> 14)) & 0xFFFFFFFF) / 4294967296.0


def _imul(a: int, b: int) -> int:
    return (a * b) & 0xFFFFFFFF


def q4k_blocks(seed: int, supers: int, zero_scale: bool = False) -> np.ndarray:
    """Q4_K super-blocks as src/q4k-pack.test.ts:19-36 makes them."""
    rand = Mulberry32(seed)
    b = np.zeros(supers * 144, dtype=np.uint8)
    for s in range(supers):
        p = s * 144
        d = to_half(0.001 + 0.004 * rand())
        dm = to_half(0.002 + 0.006 * rand())
        b[p], b[p + 1] = d & 255, d >> 8
        b[p + 2], b[p + 3] = dm & 255, dm >> 8
        scales = [1 + int(rand() * 63) for _ in range(8)]
        mins = [int(rand() * 64) for _ in range(8)]
        if zero_scale:
            scales[s % 8] = 0
        for j in range(4):
            b[p + 4 + j] = (scales[j] & 63) | ((scales[j + 4] >> 4) << 6)
            b[p + 8 + j] = (mins[j] & 63) | ((mins[j + 4] >> 4) << 6)
            b[p + 12 + j] = (scales[j + 4] & 15) | ((mins[j + 4] & 15) << 4)
        for i in range(128):
            b[p + 16 + i] = int(rand() * 256)
    return b


# --- Gated DeltaNet (src/delta-rule.ts:38-166, src/gpu/kernels.ts:1544-1862) ---

_lib.orc_delta_sequential.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P]
_lib.orc_delta_chunked.argtypes = [_I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P]
_lib.orc_delta_rule.argtypes = [_P, _I, _P, _I, _P, _P, _I, _I, _I, _I, _P, _I, _P, _P]
_lib.orc_delta_conv.argtypes = [_P, _I, _I, _I, _I, _P, _P, _P, _P]
_lib.orc_delta_norm.argtypes = [_P, _I, _I, _I, _I, _P, _I, _P, C.c_float, _P]


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def delta_sequential(q, k, v, beta, g, state):
    """deltaSequential: one head's (outputs [T][dv], new state [dk][dv])."""
    q, k, v, beta, g = map(_f64, (q, k, v, beta, g))
    T, dk = q.shape
    dv = v.shape[1]
    S = _f64(state).copy()
    o = np.empty((T, dv))
    _lib.orc_delta_sequential(dk, dv, T, _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(g),
                              _ptr(S), _ptr(o))
    return o, S


def delta_chunked(q, k, v, beta, g, state, chunk, first=0, save_at=0):
    """deltaChunked: (outputs, new state, the state after token save_at or None)."""
    q, k, v, beta, g = map(_f64, (q, k, v, beta, g))
    T, dk = q.shape
    dv = v.shape[1]
    S = _f64(state).copy()
    o = np.empty((T, dv))
    snap = np.full((dk, dv), np.nan) if save_at else None
    _lib.orc_delta_chunked(dk, dv, T, _ptr(q), _ptr(k), _ptr(v), _ptr(beta), _ptr(g), _ptr(S),
                           _ptr(o), chunk, first, save_at, _ptr(snap))
    return o, S, snap


def delta_rule(qkv, ba, A, dt, heads, key_dim, value_dim, state, save_at=0):
    """The recurrence of a Gated DeltaNet layer over M rows (gates, q/k prep,
    the delta rule per head), as wg_delta_rule: (out [M][H dv] float64,
    state [H][dk][dv] float64, the state after row save_at or None)."""
    qkv, ba, A, dt = map(_f32, (qkv, ba, A, dt))
    M = qkv.shape[0]
    S = _f64(state).copy()
    out = np.empty((M, heads * value_dim))
    snap = np.full(S.shape, np.nan) if save_at else None
    _lib.orc_delta_rule(_ptr(qkv), qkv.shape[1], _ptr(ba), ba.shape[1], _ptr(A), _ptr(dt),
                        heads, key_dim, value_dim, M, _ptr(S), save_at, _ptr(snap), _ptr(out))
    return out, S, snap


def delta_conv(inp, channels, weights, state):
    """silu(causal depthwise conv) of the first `channels` of each row:
    (out [M][C] float64, the new state [W-1][C] float32)."""
    inp, weights, state = map(_f32, (inp, weights, state))
    M = inp.shape[0]
    W = weights.shape[1]
    out = np.empty((M, channels))
    new_state = np.empty((W - 1, channels), np.float32)
    _lib.orc_delta_conv(_ptr(inp), inp.shape[1], M, channels, W, _ptr(weights), _ptr(state),
                        _ptr(out), _ptr(new_state))
    return out, new_state


def delta_norm(o, heads, value_dim, z, weights, eps):
    """The gated RMSNorm of each head's output (float64 [M][H dv])."""
    o, z, weights = map(_f32, (o, z, weights))
    M = o.shape[0]
    out = np.empty((M, heads * value_dim))
    _lib.orc_delta_norm(_ptr(o), o.shape[1], M, heads, value_dim, _ptr(z), z.shape[1],
                        _ptr(weights), eps, _ptr(out))
    return out
