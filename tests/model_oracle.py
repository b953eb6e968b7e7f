"""A CPU decoder over the oracle's primitives, for end-to-end parity of the
engine (test infrastructure). It reads the engine's device weights back to
the host, dequantizes them with the oracle's matrixRow (src/repack.ts:865-891;
Q4_K through packQ4_K, :100-168) and runs the reference's forward
(src/engine.ts:8875-9303) in float64 matmuls with the reference's fp16
rounding points: a normed matmul's input is half(x * w / 32) and its sums
are scaled by 32 / RMS(x) (addScaled + the prescaled matmul,
src/gpu/kernels.ts:1313-1331, :744-895); keys and values in the cache,
attention and SwiGLU outputs are halves (packH2, kernels.ts:32-36)."""
import math

import numpy as np

from oracle import oracle as O


def _np(t):
    return t.detach().cpu().numpy()


def dense_of(m, threads=0) -> np.ndarray:
    """The oracle's float32 weights of an ops.Q4Matrix, rows in logical order
    (stored row p is logical row m.row_order[p] when the matrix has one)."""
    d = _dense_stored(m, threads)
    order = getattr(m, "row_order", None)
    if order is None:
        return d
    out = np.empty_like(d)
    out[np.asarray(order)] = d
    return out


def _dense_stored(m, threads=0) -> np.ndarray:
    from webgllm_amd import lib as L
    N, K = m.N, m.K
    if m.layout in (L.LAYOUT_Q8, L.LAYOUT_Q6K):
        wm = O.WideMatrix(N, K, 8 if m.layout == L.LAYOUT_Q8 else 6)
        wm.quants[:] = _np(m.quants)
        wm.scales[:] = _np(m.scales).view(np.uint16)
        return wm.dense()
    if m.layout == L.LAYOUT_Q4K:
        G, S = N // 4, K // 256
        rec = _np(m.quants).reshape(G, S, 4, 144)
        src = np.ascontiguousarray(rec.transpose(0, 2, 1, 3)).reshape(-1)
        qm = O.QuantMatrix(N, K, "halves")
        O.pack_q4_k(qm, 0, src, N)
        return qm.dense(threads)
    if m.zero == L.ZERO_Q4K:  # the super-blocks behind the records, through packQ4_K
        src = O.q4k_from_records(_np(m.quants), _np(m.scales).view(np.uint8), N, K)
        qm = O.QuantMatrix(N, K, "halves")
        O.pack_q4_k(qm, 0, src.reshape(-1), N)
        return qm.dense(threads)
    qm = O.QuantMatrix(N, K, {L.ZERO_8: False, L.ZERO_U8: True, L.ZERO_F16: "halves"}[m.zero])
    qm.quants[:] = _np(m.quants).view(np.uint32)
    qm.scales[:] = _np(m.scales).view(np.uint16)
    if m.zero == L.ZERO_U8:
        qm.zeros[:] = _np(m.zeros)
    elif m.zero == L.ZERO_F16:
        qm.zero_halves[:] = _np(m.zeros).view(np.uint16)
    return qm.dense(threads)


def h16(x):
    """Through halves and back (clamped to +-65504)."""
    return O.halves_to_f32(O.f32_to_h2(np.asarray(x, np.float32)))


class OracleModel:
    """The whole-model decoder. `layers` (indices) limits which layers get
    float64 weight copies (an 8B-shape layer is 1.7 GB of them); `head`
    False leaves the embedding out (only layer_rows can run then)."""

    def __init__(self, weights, ctx, layers=None, head=True):
        s = self.s = weights.shape
        self.ctx = ctx
        # float64 copies of the dequantized weights, made once
        self.emb = dense_of(weights.embedding).astype(np.float64) if head else None
        self.final = _np(weights.final_norm)
        keep = range(s.layers) if layers is None else set(layers)
        self.layers = []
        for i, lw in enumerate(weights.layers):
            d = None
            if i in keep:
                d = {k: (dense_of(v).astype(np.float64) if hasattr(v, "desc") else _np(v))
                     for k, v in lw.items()}
            self.layers.append(d)
        self.rope = O.rope_table(s.rope_theta, s.head_dim, s.head_dim, ctx)
        self.reset()

    @classmethod
    def from_dense(cls, shape, emb, final_norm, layers, ctx):
        """The decoder over weights given as arrays: emb [V, D] and each
        layer's matrices as float32/float64 [N, K] in logical row order,
        vectors and conv taps as they are."""
        self = cls.__new__(cls)
        self.s, self.ctx = shape, ctx
        self.emb = np.asarray(emb, np.float64)
        self.final = np.asarray(final_norm, np.float32)
        self.layers = [{k: (np.asarray(v, np.float64) if k in cls.MATRICES else np.asarray(v))
                        for k, v in lw.items()} for lw in layers]
        self.rope = O.rope_table(shape.rope_theta, shape.head_dim, shape.head_dim, ctx)
        self.reset()
        return self

    def reset(self):
        s = self.s
        kvd = s.kv_heads * s.head_dim
        self.k = {i: np.zeros((self.ctx, kvd), np.uint16) for i in range(s.layers)
                  if s.layer_type(i) == "attn"}
        self.v = {i: np.zeros((self.ctx, kvd), np.uint16) for i in range(s.layers)
                  if s.layer_type(i) == "attn"}
        self.state = {i: np.zeros((s.conv_kernel - 1, s.hidden), np.float32)
                      for i in range(s.layers) if s.layer_type(i) == "conv"}
        self.position = 0

    @staticmethod
    def _mm(x, w):
        return (x.astype(np.float64) @ w.T).astype(np.float32)

    def _normed_mm(self, h, norm_w, w):
        """A matmul over the prescaled norm of h (rows of h), as the reference
        does it: half(h * w / 32) in, sums times 32 / RMS(h)."""
        x16 = h16(h.astype(np.float32) * norm_w.astype(np.float32) / np.float32(32.0))
        ms = (h.astype(np.float64) ** 2).mean(1, keepdims=True)
        r = 32.0 / np.sqrt(ms + self.s.eps)
        return ((x16.astype(np.float64) @ w.T) * r).astype(np.float32)

    def layer_rows(self, i, h, pos0):
        """Layer i over rows h [M, D] (float32) at positions pos0 ..: writes
        the rows' keys and values (or advances the conv state) and returns
        the new h."""
        s, lw = self.s, self.layers[i]
        M = h.shape[0]
        hd = s.head_dim
        if s.layer_type(i) == "conv":
            bcx = self._normed_mm(h, lw["op_norm"], lw["in_proj"])
            out, st = O.short_conv(bcx, s.hidden, s.conv_kernel, lw["taps"], self.state[i])
            self.state[i] = st
            h = h + self._mm(h16(out), lw["out_proj"])
        else:
            qkv = self._normed_mm(h, lw["op_norm"], lw["qkv"])
            att = np.zeros((M, s.heads * hd), np.float32)
            qd = s.heads * hd
            kvd = s.kv_heads * hd
            for m in range(M):
                pos = pos0 + m
                q = np.concatenate([
                    O.head_prep(qkv[m, h_ * hd:(h_ + 1) * hd], lw.get("q_norm"), self.rope, hd,
                                hd, pos, s.eps, 1 / math.sqrt(hd), s.qk_norm)
                    for h_ in range(s.heads)])
                for kh in range(s.kv_heads):
                    kx = qkv[m, qd + kh * hd:qd + (kh + 1) * hd]
                    self.k[i][pos, kh * hd:(kh + 1) * hd] = O.f32_to_h2(
                        O.head_prep(kx, lw.get("k_norm"), self.rope, hd, hd, pos, s.eps, 1.0,
                                    s.qk_norm))
                    vx = qkv[m, qd + kvd + kh * hd:qd + kvd + (kh + 1) * hd]
                    self.v[i][pos, kh * hd:(kh + 1) * hd] = O.f32_to_h2(vx)
                a = O.attention_f64(q, self.k[i], self.v[i], s.heads, s.kv_heads, hd,
                                    pos + 1, kvd)
                att[m] = h16(a)
            h = h + self._mm(att, lw["o"])
        gu = self._normed_mm(h, lw["ffn_norm"], lw["gate_up"])
        return h + self._mm(h16(O.swiglu(gu)), lw["down"])

    def head_rows(self, h):
        """(logits [M, V], greedy picks) of rows h."""
        logits = self._normed_mm(h, self.final, self.emb)
        return logits, [O.argmax(logits[m])[0] for m in range(h.shape[0])]

    def forward_rows(self, ids, head=True):
        """One batch; returns (logits [M, V], picks [M]), or (None, None)
        when `head` is False."""
        pos0 = self.position
        h = self.emb[np.asarray(ids)].astype(np.float32)
        for i in range(len(self.layers)):
            h = self.layer_rows(i, h, pos0)
        self.position += len(ids)
        return self.head_rows(h) if head else (None, None)

    # the quantized matrices of a layer (the rest are vectors and conv taps)
    MATRICES = ("qkv", "o", "gate_up", "down", "in_proj", "out_proj")

    def forward(self, tokens, f16_weights=False, batch=8):
        """A prompt; returns the (logits, picks) of its last batch of 8 rows
        (len mod 8 rows, or 8), as the engine returns them. The rows before
        run `batch` at a time with no head: every row's result is the same
        for any batching (rows are independent but for the cache and conv
        state, which advance row by row). With f16_weights the layers'
        matmuls use the dequantized weights rounded to halves, as the
        reference's prompt plan computes them (dequant to an f16 texture,
        then matmulF16: src/gpu/kernels.ts:436-735, Engine.f16Plan,
        src/engine.ts:980-995); the head keeps exact weights. The engine
        takes that path for prompts longer than a verify batch when every
        layer matrix is a 4- or 8-bit row-group one."""
        layers = self.layers
        if f16_weights:
            self.layers = [None if lw is None else
                           {k: (h16(v).astype(np.float64) if k in self.MATRICES else v)
                            for k, v in lw.items()} for lw in layers]
        try:
            tokens = list(tokens)
            last = len(tokens) - (len(tokens) % 8 or 8)
            for b0 in range(0, last, batch):
                self.forward_rows(tokens[b0:min(last, b0 + batch)], head=False)
            logits, picks = self.forward_rows(tokens[last:])
        finally:
            self.layers = layers
        return logits, picks

    def decode(self, first, steps):
        out, t = [], first
        for _ in range(steps):
            _, p = self.forward_rows([t])
            t = p[0]
            out.append(t)
        return out
