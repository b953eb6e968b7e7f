"""Typed ops over the C ABI, on torch device tensors (memory and streams only).

Each function validates on the host, calls the HIP library on the current
stream and raises WgError on a failed status. The reference functions each
one stands in for are cited in include/webgllm_hip.h.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import lib as L


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t) -> int | None:
    return None if t is None else t.data_ptr()


def _dev(t: torch.Tensor, dtype=None) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t


def _rows(t: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """A device matrix whose rows may be strided (a view of wider rows)."""
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"expected {dtype}, got {t.dtype}")
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError("expected a matrix with unit column stride")
    return t


def to_device_bytes(b, device="cuda") -> torch.Tensor:
    """Host bytes (numpy / bytes) as a uint8 device tensor."""
    arr = np.frombuffer(b, dtype=np.uint8) if isinstance(b, (bytes, bytearray)) else \
        np.ascontiguousarray(b).view(np.uint8).reshape(-1)
    return torch.from_numpy(arr.copy()).to(device)


class Q4Matrix:
    """A quantized matrix (4-, 8- or 6-bit) resident on the device (see WG_LAYOUT_* in the
    header)."""

    def __init__(self, N: int, K: int, layout: int = L.LAYOUT_ROWGROUP, zero: int = L.ZERO_8,
                 device="cuda"):
        lib = L.load()
        qb, sb, zb = C.c_size_t(), C.c_size_t(), C.c_size_t()
        L.check(lib.wg_q4_sizes(N, K, layout, zero, C.byref(qb), C.byref(sb), C.byref(zb)))
        self.N, self.K, self.layout, self.zero = N, K, layout, zero
        self.quants = torch.zeros(qb.value, dtype=torch.uint8, device=device)
        self.scales = torch.zeros(max(sb.value, 2) // 2, dtype=torch.int16, device=device) \
            if sb.value else None
        self.zeros = None
        if zb.value:
            self.zeros = torch.full((zb.value,), 8, dtype=torch.uint8, device=device) \
                if zero == L.ZERO_U8 else torch.zeros(zb.value // 2, dtype=torch.int16,
                                                      device=device)
        self.desc = L.Q4MatrixDesc(N, K, layout, zero, _p(self.quants), _p(self.scales),
                                   _p(self.zeros))

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.quants, self.scales, self.zeros)
                   if t is not None)

    # --- load-time repacking (the reference's loaders' packers, on the GPU)
    @classmethod
    def from_q4_0(cls, src: torch.Tensor, N: int, K: int, src_rows=None) -> "Q4Matrix":
        m = cls(N, K, L.LAYOUT_ROWGROUP, L.ZERO_8, device=src.device)
        m.repack_q4_0(0, N, src, src_rows)
        return m

    @classmethod
    def from_q4_k(cls, src: torch.Tensor, N: int, K: int, native: bool = True,
                  src_rows=None, records: bool = False) -> "Q4Matrix":
        """A matrix from GGUF Q4_K rows: the super-blocks as they are
        (native), packQ4_K's row groups with half zero points, or (records)
        the same quants with Q4_K's own scales kept (ZERO_Q4K)."""
        if native:
            m = cls(N, K, L.LAYOUT_Q4K, L.ZERO_8, device=src.device)
            m.repack_q4_k_native(0, N, src, src_rows)
        else:
            m = cls(N, K, L.LAYOUT_ROWGROUP, L.ZERO_Q4K if records else L.ZERO_F16,
                    device=src.device)
            m.repack_q4_k(0, N, src, src_rows)
        return m

    @classmethod
    def from_q8_0(cls, src: torch.Tensor, N: int, K: int, src_rows=None) -> "Q4Matrix":
        """An 8-bit matrix from GGUF Q8_0 rows (packQ8_0)."""
        m = cls(N, K, L.LAYOUT_Q8, L.ZERO_8, device=src.device)
        m.repack_q8_0(0, N, src, src_rows)
        return m

    @classmethod
    def from_floats_q8(cls, values: torch.Tensor) -> "Q4Matrix":
        """An 8-bit matrix quantized from float32 rows [N, K] (quantizeQ8)."""
        N, K = values.shape
        m = cls(N, K, L.LAYOUT_Q8, L.ZERO_8, device=values.device)
        m.quantize_q8(0, N, values)
        return m

    @classmethod
    def from_q6_k(cls, src: torch.Tensor, N: int, K: int, src_rows=None) -> "Q4Matrix":
        """A 6-bit matrix from GGUF Q6_K rows (packQ6_K)."""
        m = cls(N, K, L.LAYOUT_Q6K, L.ZERO_8, device=src.device)
        m.repack_q6_k(0, N, src, src_rows)
        return m

    @classmethod
    def from_nbits(cls, quant: torch.Tensor, scales: torch.Tensor, zp, N: int, K: int,
                   src_rows=None) -> "Q4Matrix":
        m = cls(N, K, L.LAYOUT_ROWGROUP, L.ZERO_U8 if zp is not None else L.ZERO_8,
                device=quant.device)
        m.repack_nbits(0, N, quant, scales, zp, src_rows)
        return m

    def repack_q4_0(self, row0, rows, src, src_rows=None):
        L.check(L.load().wg_repack_q4_0(C.byref(self.desc), row0, rows, _p(_dev(src)),
                                        _p(src_rows), _stream()))

    def repack_q4_k(self, row0, rows, src, src_rows=None):
        self._halves = None  # (prompt_desc's halves are made again from the new rows)
        L.check(L.load().wg_repack_q4_k(C.byref(self.desc), row0, rows, _p(_dev(src)),
                                        _p(src_rows), _stream()))

    def repack_q4_k_native(self, row0, rows, src, src_rows=None):
        L.check(L.load().wg_repack_q4_k_native(C.byref(self.desc), row0, rows, _p(_dev(src)),
                                               _p(src_rows), _stream()))

    def repack_nbits(self, row0, rows, quant, scales, zp=None, src_rows=None):
        L.check(L.load().wg_repack_nbits(C.byref(self.desc), row0, rows, _p(_dev(quant)),
                                         _p(_dev(scales)), _p(zp), _p(src_rows), _stream()))

    def repack_q8_0(self, row0, rows, src, src_rows=None):
        L.check(L.load().wg_repack_q8_0(C.byref(self.desc), row0, rows, _p(_dev(src)),
                                        _p(src_rows), _stream()))

    def quantize_q8(self, row0, rows, values):
        L.check(L.load().wg_quantize_q8(C.byref(self.desc), row0, rows,
                                        _p(_dev(values, torch.float32)), _stream()))

    def repack_q6_k(self, row0, rows, src, src_rows=None):
        L.check(L.load().wg_repack_q6_k(C.byref(self.desc), row0, rows, _p(_dev(src)),
                                        _p(src_rows), _stream()))

    def prompt_desc(self):
        """The descriptor the prefill GEMM takes: for Q4_K records, the same
        quants with packQ4_K's half scales and zero points, made once
        (wg_q4k_record_halves) and kept beside the records (0.125 bytes a
        weight, never read by one- and two-row GEMVs; gemv takes them for 3
        to 8 rows where K <= 4096); else the matrix itself."""
        if self.zero != L.ZERO_Q4K:
            return self.desc
        if getattr(self, "_halves", None) is None:
            n = self.N * (self.K // 32)
            sc = torch.empty(n, dtype=torch.int16, device=self.quants.device)
            zr = torch.empty(n, dtype=torch.int16, device=self.quants.device)
            L.check(L.load().wg_q4k_record_halves(C.byref(self.desc), _p(sc), _p(zr), _stream()))
            self._halves = (sc, zr, L.Q4MatrixDesc(self.N, self.K, L.LAYOUT_ROWGROUP, L.ZERO_F16,
                                                   _p(self.quants), _p(sc), _p(zr)))
        return self._halves[2]

    def dequant(self, row0: int = 0, rows: int | None = None) -> torch.Tensor:
        rows = self.N - row0 if rows is None else rows
        out = torch.empty((rows, self.K), dtype=torch.float32, device=self.quants.device)
        L.check(L.load().wg_q4_dequant(C.byref(self.desc), row0, rows, _p(out), _stream()))
        return out


def _gemv_desc(m: Q4Matrix, M: int) -> "L.Q4MatrixDesc":
    """The matrix a GEMV of M rows reads: 3 to 8 rows of Q4_K records at
    K <= 4096 go through their kept halves (prompt_desc), since the MFMA
    form takes half zero points, not records (at the 8B shape a 5-row
    gate|up took 35.1 us on the records' vector form, 18.2 on the halves);
    every GEMV entry routes alike, so the fused epilogues give the plain
    GEMV's bits."""
    if M >= 3 and m.zero == L.ZERO_Q4K and m.K <= 4096 and \
            getattr(m, "_halves", None) is not None:
        return m._halves[2]
    return m.desc


def gemv(m: Q4Matrix, x16: torch.Tensor, out: torch.Tensor | None = None,
         residual: torch.Tensor | None = None, row_scale: torch.Tensor | None = None,
         epilogue: "L.Epilogue | None" = None):
    """y = x W^T for M <= 8 rows of half activations [M, K] (int16/float16 bits).
    `epilogue` (an L.Epilogue) overrides residual/row_scale when given."""
    if x16.dtype not in (torch.float16, torch.int16):
        raise ValueError("activations must be halves")
    x16 = _dev(x16)
    M = x16.shape[0] if x16.dim() == 2 else 1
    ldx = x16.shape[-1]
    ep = epilogue
    if ep is None:
        if out is None:
            out = torch.empty((M, m.N), dtype=torch.float32, device=x16.device)
        if residual is not None or row_scale is not None:
            ep = L.Epilogue(mode=L.EPI_STORE, residual=_p(residual),
                            ld_residual=residual.shape[-1] if residual is not None else 0,
                            row_scale=_p(row_scale))
    if out is not None:
        _dev(out, torch.float32)
    L.check(L.load().wg_q4_gemv(C.byref(_gemv_desc(m, M)), _p(x16), M, ldx, _p(out),
                                out.shape[-1] if out is not None else 0,
                                C.byref(ep) if ep is not None else None, _stream()))
    return out


def gemv_short_conv(m: Q4Matrix, x16: torch.Tensor, epilogue: "L.Epilogue") -> bool:
    """The in_proj GEMV of a short conv with the convolution in its epilogue
    (epilogue.mode = EPI_SHORT_CONV). Returns False, having launched
    nothing, where the library's kernels do not take the shape (the caller
    then runs gemv() into the B | C | x rows and short_conv())."""
    if x16.dtype not in (torch.float16, torch.int16):
        raise ValueError("activations must be halves")
    x16 = _dev(x16)
    M = x16.shape[0] if x16.dim() == 2 else 1
    rc = L.load().wg_q4_gemv(C.byref(_gemv_desc(m, M)), _p(x16), M, x16.shape[-1], None, 0,
                             C.byref(epilogue), _stream())
    if rc == L.ERR_UNSUPPORTED:
        return False
    L.check(rc)
    return True


def gemm(m: Q4Matrix, a16: torch.Tensor, out: torch.Tensor | None = None,
         residual: torch.Tensor | None = None, col_of: torch.Tensor | None = None,
         row_scale: torch.Tensor | None = None, kept: bool = True) -> torch.Tensor:
    """C = A W^T on MFMA for M tokens of half activations A [M, K]; col_of
    (int32 [N], optional) sends stored row n to output column col_of[n];
    row_scale (float32 [M], optional) multiplies row m's sums. Q4_K records
    go through their kept halves (prompt_desc), or with kept=False through
    the library's rebuild each call: the same bits."""
    if a16.dtype not in (torch.float16, torch.int16):
        raise ValueError("activations must be halves")
    a16 = _dev(a16)
    M = a16.shape[0]
    if out is None:
        out = torch.empty((M, m.N), dtype=torch.float32, device=a16.device)
    _dev(out, torch.float32)
    desc = m.prompt_desc() if kept else m.desc
    L.check(L.load().wg_q4_gemm(C.byref(desc), _p(a16), M, a16.shape[1], _p(out), out.shape[1],
                                _p(residual), residual.shape[1] if residual is not None else 0,
                                _p(None if row_scale is None else _dev(row_scale, torch.float32)),
                                _p(None if col_of is None else _dev(col_of, torch.int32)),
                                _stream()))
    return out


def gemm_swiglu(m: Q4Matrix, a16: torch.Tensor, out: torch.Tensor | None = None,
                row_scale: torch.Tensor | None = None, kept: bool = True) -> torch.Tensor:
    """half(silu(gate) * up) [M, N / 2] of A W^T on MFMA, for a gate|up
    matrix stored in the SwiGLU row order (gate 2i, gate 2i + 1, up 2i,
    up 2i + 1 per row group)."""
    if a16.dtype not in (torch.float16, torch.int16):
        raise ValueError("activations must be halves")
    a16 = _dev(a16)
    M = a16.shape[0]
    if out is None:
        out = torch.empty((M, m.N // 2), dtype=torch.float16, device=a16.device)
    _dev(out)
    desc = m.prompt_desc() if kept else m.desc
    L.check(L.load().wg_q4_gemm_swiglu(C.byref(desc), _p(a16), M, a16.shape[1], _p(out),
                                       out.shape[1],
                                       _p(None if row_scale is None else
                                          _dev(row_scale, torch.float32)), _stream()))
    return out


def f32_to_f16(x: torch.Tensor) -> torch.Tensor:
    x = _dev(x, torch.float32)
    out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    L.check(L.load().wg_f32_to_f16(_p(x), _p(out), x.numel(), _stream()))
    return out


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor | None = None,
             rs_out: torch.Tensor | None = None) -> torch.Tensor:
    """half(x * w / rms(x)) per row of x [M, D] (float32)."""
    x = _dev(x, torch.float32)
    M, D = (x.shape[0], x.shape[1]) if x.dim() == 2 else (1, x.shape[0])
    if out is None:
        out = torch.empty((M, D), dtype=torch.float16, device=x.device)
    L.check(L.load().wg_rms_norm(_p(x), M, D, x.shape[-1], _p(_dev(w, torch.float32)), eps,
                                 _p(out), out.shape[-1], _p(rs_out), _stream()))
    return out


def norm_to_h2(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor,
               row_scale: torch.Tensor) -> torch.Tensor:
    """The reference's prescaled norm: out = half(x * w / 32) per row of x
    [M, D] (float32), row_scale[m] = 32 / RMS(x[m])."""
    x = _dev(x, torch.float32)
    M, D = x.shape
    L.check(L.load().wg_norm_to_h2(_p(x), M, D, x.shape[-1], _p(_dev(w, torch.float32)), eps,
                                   _p(out), out.shape[-1], _p(_dev(row_scale, torch.float32)),
                                   _stream()))
    return out


def swiglu(gu: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """half(silu(gate) * up) from [M, 2F] (gate columns first)."""
    gu = _dev(gu, torch.float32)
    M, F = gu.shape[0], gu.shape[1] // 2
    if out is None:
        out = torch.empty((M, F), dtype=torch.float16, device=gu.device)
    L.check(L.load().wg_swiglu(_p(gu), M, F, gu.shape[1], _p(out), out.shape[-1], _stream()))
    return out


def embed(m: "Q4Matrix", ids: torch.Tensor, out: torch.Tensor | None = None,
          epilogue: "L.Epilogue | None" = None) -> torch.Tensor:
    ids = _dev(ids, torch.int32)
    M = ids.numel()
    if out is None:
        out = torch.empty((M, m.K), dtype=torch.float32, device=ids.device)
    L.check(L.load().wg_embed(C.byref(m.desc), _p(ids), M, _p(out), out.shape[-1],
                              C.byref(epilogue) if epilogue is not None else None, _stream()))
    return out


def attn_shape(heads, kv_heads, head_dim, rotated_dims=None, eps=1e-6, use_norm=False):
    return L.AttnShape(heads, kv_heads, head_dim,
                       head_dim if rotated_dims is None else rotated_dims, eps, int(use_norm))


def head_prep(qkv: torch.Tensor, shape, rope: torch.Tensor, pos0: torch.Tensor,
              k_cache: torch.Tensor, v_cache: torch.Tensor, q_norm=None, k_norm=None,
              q_out: torch.Tensor | None = None) -> torch.Tensor:
    qkv = _dev(qkv, torch.float32)
    M = qkv.shape[0]
    qd = shape.heads * shape.head_dim
    if q_out is None:
        q_out = torch.empty((M, qd), dtype=torch.float32, device=qkv.device)
    L.check(L.load().wg_head_prep(_p(qkv), M, qkv.shape[1], C.byref(shape), _p(q_norm),
                                  _p(k_norm), _p(_dev(rope, torch.float32)), rope.shape[0],
                                  _p(_dev(pos0, torch.int32)), _p(q_out), q_out.shape[1],
                                  _p(k_cache), _p(v_cache), k_cache.shape[0], _stream()))
    return q_out


def attn_scratch(M, shape, max_keys, device="cuda") -> torch.Tensor:
    """Scratch for attn_decode (the chunks' partial results)."""
    n = L.load().wg_attn_scratch_bytes(M, shape.heads, shape.head_dim, max_keys)
    return torch.zeros(max(n, 4), dtype=torch.uint8, device=device)


def attn_decode(q: torch.Tensor, shape, k_cache, v_cache, pos0: torch.Tensor,
                scratch: torch.Tensor | None = None, out: torch.Tensor | None = None):
    q = _dev(q, torch.float32)
    M = q.shape[0]
    max_keys = k_cache.shape[0]
    if scratch is None:
        scratch = attn_scratch(M, shape, max_keys, q.device)
    if out is None:
        out = torch.empty((M, shape.heads * shape.head_dim), dtype=torch.float16,
                          device=q.device)
    L.check(L.load().wg_attn_decode(_p(q), M, q.shape[1], C.byref(shape), _p(k_cache),
                                    _p(v_cache), _p(_dev(pos0, torch.int32)), max_keys, _p(out),
                                    out.shape[1], _p(scratch), scratch.numel(), _stream()))
    return out


def attn_decode_prep(qkv: torch.Tensor, shape, rope: torch.Tensor, pos0: torch.Tensor,
                     k_cache, v_cache, q_norm=None, k_norm=None, scratch=None, out=None,
                     q_out: torch.Tensor | None = None):
    """head_prep then attn_decode in one launch (the heads prepared inside
    the attention kernel), the same bits. Returns the half output, or None,
    having launched nothing, where the kernel does not take the shape (then
    head_prep() and attn_decode())."""
    qkv = _dev(qkv, torch.float32)
    M = qkv.shape[0]
    max_keys = k_cache.shape[0]
    if scratch is None:
        scratch = attn_scratch(M, shape, max_keys, qkv.device)
    if out is None:
        out = torch.empty((M, shape.heads * shape.head_dim), dtype=torch.float16,
                          device=qkv.device)
    rc = L.load().wg_attn_decode_prep(
        _p(qkv), M, qkv.shape[1], C.byref(shape), _p(q_norm), _p(k_norm),
        _p(_dev(rope, torch.float32)), rope.shape[0], k_cache.shape[0], _p(k_cache), _p(v_cache),
        _p(_dev(pos0, torch.int32)), max_keys, _p(q_out), q_out.shape[1] if q_out is not None else 0,
        _p(out), out.shape[1], _p(scratch), scratch.numel(), _stream())
    if rc == L.ERR_UNSUPPORTED:
        return None
    L.check(rc)
    return out


def attn_prefill(q: torch.Tensor, shape, k_cache, v_cache, pos0: torch.Tensor,
                 out: torch.Tensor | None = None):
    """Causal attention of a prompt batch (rows at pos0, pos0 + 1, ...)
    over the caches, flash style (no scratch)."""
    q = _dev(q, torch.float32)
    M = q.shape[0]
    if out is None:
        out = torch.empty((M, shape.heads * shape.head_dim), dtype=torch.float16,
                          device=q.device)
    L.check(L.load().wg_attn_prefill(_p(q), M, q.shape[1], C.byref(shape), _p(k_cache),
                                     _p(v_cache), _p(_dev(pos0, torch.int32)), k_cache.shape[0],
                                     _p(out), out.shape[1], _stream()))
    return out


def short_conv(bcx, D, W, taps, state, state_out=None, prefixes=None, out=None):
    bcx = _dev(bcx, torch.float32)
    M = bcx.shape[0]
    if out is None:
        out = torch.empty((M, D), dtype=torch.float16, device=bcx.device)
    if state_out is None:
        state_out = state
    L.check(L.load().wg_short_conv(_p(bcx), M, D, bcx.shape[1], W, _p(_dev(taps)), _p(state),
                                   _p(state_out), _p(prefixes), _p(out), out.shape[1],
                                   _stream()))
    return out


def conv_accept(prefixes, kept, rows, D, W, state):
    L.check(L.load().wg_conv_accept(_p(prefixes), kept, rows, D, W, _p(state), _stream()))


def conv_states(layers, device="cuda"):
    """A device array of wg_conv_state for [(prefixes [R][W-1][D], state
    [W-1][D])]: (the array, its count, the largest state in floats)."""
    arr = (L.ConvState * max(1, len(layers)))()
    big = 0
    for i, (pre, st) in enumerate(layers):
        W1, D = st.shape
        arr[i] = L.ConvState(_p(_dev(pre, torch.float32)), _p(_dev(st, torch.float32)), D, W1 + 1)
        big = max(big, W1 * D)
    raw = np.frombuffer(bytes(arr), dtype=np.uint8).copy()
    return torch.from_numpy(raw).to(device), len(layers), big


def verify_accept(picks, rows, convs, pos, ids, hist, kept_log, cursor):
    """wg_verify_accept: keep the batch's agreeing prefix + 1, roll the conv
    states back, move the position and ids[0] on (all on the device).
    convs is conv_states()'s triple."""
    arr, n, big = convs
    for t, name in ((picks, "picks"), (pos, "pos"), (ids, "ids"), (hist, "hist"),
                    (kept_log, "kept_log"), (cursor, "cursor")):
        if t.dtype != torch.int32 or not t.is_cuda:
            raise ValueError(f"{name} must be an int32 device tensor")
    L.check(L.load().wg_verify_accept(_p(picks), rows, _p(arr), n, big, _p(pos), _p(ids),
                                      _p(hist), hist.numel(), _p(kept_log), kept_log.numel(),
                                      _p(cursor), _stream()))


def verify_accept_parts(parts, picks_out, rows, convs, pos, ids, hist, kept_log, cursor):
    """wg_verify_accept_parts: the batch's picks finished from a head GEMV's
    pick parts into picks_out, then verify_accept's keep, rollback and
    advance, in one launch."""
    arr, n, big = convs
    for t, name in ((picks_out, "picks_out"), (pos, "pos"), (ids, "ids"), (hist, "hist"),
                    (kept_log, "kept_log"), (cursor, "cursor")):
        if t.dtype != torch.int32 or not t.is_cuda:
            raise ValueError(f"{name} must be an int32 device tensor")
    L.check(L.load().wg_verify_accept_parts(_p(parts), _p(picks_out), rows, _p(arr), n, big,
                                            _p(pos), _p(ids), _p(hist), hist.numel(),
                                            _p(kept_log), kept_log.numel(), _p(cursor),
                                            _stream()))


def embed_drafts(m: Q4Matrix, ids: torch.Tensor, rows: int, table: torch.Tensor, cursor,
                 out: torch.Tensor, epilogue: "L.Epilogue | None" = None) -> torch.Tensor:
    """verify_drafts then embed in one launch: row 0 embeds ids[0], rows
    1 .. rows - 1 the draft table's row *cursor (also written to ids)."""
    table = _dev(table, torch.int32)
    if table.dim() != 2 or table.shape[1] != rows - 1:
        raise ValueError(f"the draft table must be [steps, {rows - 1}]")
    _dev(out, torch.float32)
    L.check(L.load().wg_embed_drafts(C.byref(m.desc), _p(ids), rows, _p(table), table.shape[0],
                                     _p(cursor), _p(out), out.shape[-1],
                                     C.byref(epilogue) if epilogue is not None else None,
                                     _stream()))
    return out


def verify_drafts(ids, rows, table, cursor):
    """wg_verify_drafts: ids[1:rows] = table[*cursor] (int32 [steps, rows - 1])."""
    table = _dev(table, torch.int32)
    if table.dim() != 2 or table.shape[1] != rows - 1:
        raise ValueError(f"the draft table must be [steps, {rows - 1}]")
    L.check(L.load().wg_verify_drafts(_p(ids), rows, _p(table), table.shape[0], _p(cursor),
                                      _stream()))


def argmax_rows(logits: torch.Tensor, V: int | None = None, ids=None, tops=None, scratch=None):
    logits = _dev(logits, torch.float32)
    M = logits.shape[0]
    V = logits.shape[1] if V is None else V
    if ids is None:
        ids = torch.empty(M, dtype=torch.int32, device=logits.device)
    if scratch is None:
        scratch = torch.empty(L.load().wg_argmax_scratch_bytes(M, V), dtype=torch.uint8,
                              device=logits.device)
    L.check(L.load().wg_argmax_rows(_p(logits), M, V, logits.shape[1], _p(ids), _p(tops),
                                    _p(scratch), scratch.numel(), _stream()))
    return ids


def pick_parts(M: int, device="cuda") -> torch.Tensor:
    """A buffer for a head GEMV's pick parts (wg_pick_parts_bytes, 16-byte
    aligned as torch allocates)."""
    return torch.empty(L.load().wg_pick_parts_bytes(M), dtype=torch.uint8, device=device)


def gemv_pick(m: Q4Matrix, x16: torch.Tensor, out: torch.Tensor, parts: torch.Tensor,
              epilogue: "L.Epilogue | None" = None) -> bool:
    """The head GEMV storing the logits into `out` and running the greedy
    pick's first stage into `parts` (a plain store, no residual). Returns
    False, having launched nothing, where the library's kernels do not take
    it (then gemv() and argmax_rows())."""
    ep = epilogue if epilogue is not None else L.Epilogue(mode=L.EPI_STORE)
    ep.pick_parts = parts.data_ptr()
    x16 = _dev(x16)
    M = x16.shape[0] if x16.dim() == 2 else 1
    rc = L.load().wg_q4_gemv(C.byref(_gemv_desc(m, M)), _p(x16), M, x16.shape[-1], _p(out),
                             out.shape[-1], C.byref(ep), _stream())
    if rc == L.ERR_UNSUPPORTED:
        return False
    L.check(rc)
    return True


def argmax_parts(parts: torch.Tensor, M: int, ids: torch.Tensor, tops=None, pos=None,
                 hist=None) -> torch.Tensor:
    """The greedy picks from a head GEMV's parts (gemv_pick), bit for bit
    argmax_rows' over its logits; with pos (one row) the decode advance of
    argmax_advance as well."""
    for t, name in ((ids, "ids"), (pos, "pos"), (hist, "hist")):
        if t is not None and (t.dtype != torch.int32 or not t.is_cuda):
            raise ValueError(f"{name} must be an int32 device tensor")
    L.check(L.load().wg_argmax_parts(_p(parts), M, _p(ids), _p(tops), _p(pos), _p(hist),
                                     0 if hist is None else hist.numel(), _stream()))
    return ids


def argmax_advance(logits: torch.Tensor, ids: torch.Tensor, pos: torch.Tensor,
                   hist: torch.Tensor | None = None, tops=None, scratch=None) -> None:
    """A decode step's greedy pick and advance on the device: ids[0] = the
    pick of logits' one row, hist[pos + 1] = the pick, pos += 1."""
    logits = _dev(logits, torch.float32).reshape(-1)
    V = logits.numel()
    for t, name in ((ids, "ids"), (pos, "pos"), (hist, "hist")):
        if t is not None and (t.dtype != torch.int32 or not t.is_cuda):
            raise ValueError(f"{name} must be an int32 device tensor")
    if scratch is None:
        scratch = torch.empty(L.load().wg_argmax_scratch_bytes(1, V), dtype=torch.uint8,
                              device=logits.device)
    L.check(L.load().wg_argmax_advance(_p(logits), V, _p(ids), _p(pos), _p(hist),
                                       0 if hist is None else hist.numel(), _p(tops),
                                       _p(scratch), scratch.numel(), _stream()))


def pick_candidates(logits: torch.Tensor, count: int, mask: torch.Tensor | None = None,
                    seen_rows=None, row0: int = 0, penalty: float = 1.0,
                    presence_penalty: float = 0.0, allowed: torch.Tensor | None = None,
                    scratch: torch.Tensor | None = None):
    """The `count` best 256-token chunks of each row of logits [M, V] by
    penalized maximum, and their penalized logits (wg_pick_candidates):
    (chunks int32 [M, count], candidates float32 [M, count, 256]).
    seen_rows: [(token, state, first row, end row)], at most 16; allowed:
    uint32 bitmap [rows, words] or None."""
    logits = _dev(logits, torch.float32)
    M, V = (logits.shape[0], logits.shape[1]) if logits.dim() == 2 else (1, logits.shape[0])
    dev = logits.device
    chunks = torch.empty((M, count), dtype=torch.int32, device=dev)
    cand = torch.empty((M, count, 256), dtype=torch.float32, device=dev)
    need = int(L.load().wg_pick_scratch_bytes(M, V))
    if scratch is None or scratch.numel() < need:
        scratch = torch.empty(need, dtype=torch.uint8, device=dev)
    seen = None
    if seen_rows:
        seen = torch.tensor(list(seen_rows), dtype=torch.int32, device=dev).reshape(-1, 4)
    if mask is not None:
        _dev(mask, torch.uint8)
    if allowed is not None:
        _dev(allowed, torch.int32)
    L.check(L.load().wg_pick_candidates(
        _p(logits), M, V, V if logits.dim() == 1 else logits.stride(0), _p(mask), _p(seen),
        0 if seen is None else seen.shape[0], row0, penalty, presence_penalty, _p(allowed),
        0 if allowed is None else allowed.shape[0],
        0 if allowed is None else allowed.shape[1], count, _p(chunks), _p(cand), _p(scratch),
        scratch.numel(), _stream()))
    return chunks, cand


# ------------------------------------------------------------- Gated DeltaNet

def delta_rule(qkv: torch.Tensor, ba: torch.Tensor, A: torch.Tensor, dt_bias: torch.Tensor,
               heads: int, key_dim: int, value_dim: int, state: torch.Tensor,
               save_at: int = 0, snapshot: torch.Tensor | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """A Gated DeltaNet layer's recurrence over the rows of qkv [M, >= 2 H dk
    + H dv] (q | k | v after the convolution) and ba [M, >= 2 H] (b | a):
    out [M, H dv] float32; state [H, dk, dv] float32 is updated in place, and
    with save_at in 1..M the state after that row goes to snapshot
    (wg_delta_rule)."""
    qkv, ba = _rows(qkv), _rows(ba)
    _dev(A, torch.float32), _dev(dt_bias, torch.float32), _dev(state, torch.float32)
    M = qkv.shape[0]
    if out is None:
        out = torch.empty((M, heads * value_dim), dtype=torch.float32, device=qkv.device)
    if save_at and snapshot is None:
        snapshot = torch.empty_like(state)
    shape = L.DeltaShape(heads, key_dim, value_dim)
    L.check(L.load().wg_delta_rule(_p(qkv), M, qkv.stride(0), _p(ba), ba.stride(0), _p(A),
                                   _p(dt_bias), C.byref(shape), _p(state), _p(snapshot),
                                   save_at, _p(out), out.stride(0), _stream()))
    return (out, snapshot) if save_at else out


def delta_rule_chunked(qkv: torch.Tensor, ba: torch.Tensor, A: torch.Tensor,
                       dt_bias: torch.Tensor, heads: int, key_dim: int, value_dim: int,
                       state: torch.Tensor, save_at: int = 0,
                       snapshot: torch.Tensor | None = None, out: torch.Tensor | None = None,
                       scratch: torch.Tensor | None = None):
    """delta_rule in chunks of 64 rows (wg_delta_rule_chunked): the same
    results, for prompt batches."""
    qkv, ba = _rows(qkv), _rows(ba)
    _dev(A, torch.float32), _dev(dt_bias, torch.float32), _dev(state, torch.float32)
    M = qkv.shape[0]
    if out is None:
        out = torch.empty((M, heads * value_dim), dtype=torch.float32, device=qkv.device)
    if save_at and snapshot is None:
        snapshot = torch.empty_like(state)
    shape = L.DeltaShape(heads, key_dim, value_dim)
    lib = L.load()
    if scratch is None:
        need = int(lib.wg_delta_chunk_scratch_bytes(M, C.byref(shape), save_at))
        scratch = torch.empty((need + 3) // 4, dtype=torch.float32, device=qkv.device)
    L.check(lib.wg_delta_rule_chunked(_p(qkv), M, qkv.stride(0), _p(ba), ba.stride(0), _p(A),
                                      _p(dt_bias), C.byref(shape), _p(state), _p(snapshot),
                                      save_at, _p(out), out.stride(0), _p(scratch),
                                      scratch.numel() * scratch.element_size(), _stream()))
    return (out, snapshot) if save_at else out


def delta_conv(inp: torch.Tensor, channels: int, taps: torch.Tensor, state: torch.Tensor,
               state_out: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """silu of the causal depthwise convolution over the first `channels`
    of each row of inp (taps [C, W], state [W-1, C] -> state_out): out
    [M, C] float32 (wg_delta_conv)."""
    inp = _rows(inp)
    M, W = inp.shape[0], taps.shape[1]
    if out is None:
        out = torch.empty((M, channels), dtype=torch.float32, device=inp.device)
    L.check(L.load().wg_delta_conv(_p(inp), M, inp.stride(0), channels, W,
                                   _p(_dev(taps, torch.float32)), _p(state), _p(state_out),
                                   _p(out), out.stride(0), _stream()))
    return out


def delta_norm(o: torch.Tensor, heads: int, value_dim: int, z: torch.Tensor,
               weight: torch.Tensor, eps: float, out16: torch.Tensor | None = None):
    """The gated RMSNorm of each head's output, as halves for out_proj
    (wg_delta_norm): float16 [M, H dv]."""
    o, z = _rows(o), _rows(z)
    M = o.shape[0]
    if out16 is None:
        out16 = torch.empty((M, heads * value_dim), dtype=torch.float16, device=o.device)
    shape = L.DeltaShape(heads, 0, value_dim)
    L.check(L.load().wg_delta_norm(_p(o), M, o.stride(0), C.byref(shape), _p(z), z.stride(0),
                                   _p(_dev(weight, torch.float32)), eps, _p(out16),
                                   out16.stride(0), _stream()))
    return out16
