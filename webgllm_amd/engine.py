"""The decode/verify hot path driven through the HIP kernels: the host-side
mirror of the reference's Engine forward, argmax and accept
(src/engine.ts:7900-8086, forwardBatch :8875-9303, argmax :8271-8336).

One batch of M <= 8 rows (a token, or a token and its drafts) runs as:
embedding -> per layer [operator (attention or short conv) -> gate|up ->
down] -> head -> greedy pick, where every norm, residual add, SwiGLU and
RoPE + cache write happens in a GEMV's epilogue, as the reference folds
them into its passes: a projection that adds into the residual also writes
the next norm's input as half(x * w / 32) and the sums of squares of x
(addScaled + rmsOfAdd, src/gpu/kernels.ts:1290-1361), and the matmul that
reads it applies 32 / RMS to its sums ("prescaled", kernels.ts:744-895).
The position lives on the device, so a single-token step is captured once
as a HIP graph and replayed for every token with no host work between
kernels.

Weights are random (the reference's speed probe does the same,
src/speed-probe.ts:258-499) and generated on the device.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from . import lib as L
from . import ops

MAX_ROWS = 8
PREFILL_ROWS = 2048  # prompt rows a GEMM batch takes
PRESCALE = 32.0  # the reference's PRESCALE (src/gpu/kernels.ts:89)
# The attention caches start at KV_START positions (the reference's
# KV_START, src/engine.ts:911) and grow in whole KV_STEP steps (TUNING.kvStep,
# :614) as tokens need them.
KV_START = 1024
KV_STEP = 512


def qkv_row_order(shape) -> list:
    """Logical row of each stored row of a q|k|v matrix whose epilogue does
    RoPE: each head's rows in groups (j, j + hd/2, j + 1, j + 1 + hd/2), so a
    rotation pair meets in one row group; v rows as they are."""
    hd, P = shape.head_dim, shape.head_dim // 2
    order = []
    for head in range(shape.heads + shape.kv_heads):
        base = head * hd
        for i in range(hd // 4):
            j = 2 * i
            order += [base + j, base + j + P, base + j + 1, base + j + 1 + P]
    v0 = (shape.heads + shape.kv_heads) * hd
    order += list(range(v0, v0 + shape.kv_heads * hd))
    return order


def gate_up_row_order(F: int) -> list:
    """Logical row of each stored row of a gate|up matrix whose epilogue does
    SwiGLU: groups (gate 2i, gate 2i + 1, up 2i, up 2i + 1)."""
    order = []
    for i in range(F // 2):
        order += [2 * i, 2 * i + 1, F + 2 * i, F + 2 * i + 1]
    return order


@dataclass
class ModelShape:
    name: str
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    # "q4_0" | "nbits" | "q4_k" (native super-blocks) | "q4_k_rowgroup" |
    # "q4_k_records" (packQ4_K's quants with Q4_K's own scales) |
    # "q8_0" (GGUF Q8_0) | "q8" (floats requantized to 8 bits) | "q6_k"
    fmt: str
    rope_theta: float = 1e6
    eps: float = 1e-5
    qk_norm: bool = False
    conv_kernel: int = 3
    # layer i is "conv" when listed here, else attention
    conv_layers: tuple = ()
    # the embedding's (and tied output head's) format when not `fmt`: real
    # Q4 GGUF files store it as Q6_K (src/load-gguf.ts:428-442)
    embed_fmt: str | None = None
    extra: dict = field(default_factory=dict)

    def layer_type(self, i: int) -> str:
        return "conv" if i in self.conv_layers else "attn"

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    @property
    def rope_in_epilogue(self) -> bool:
        """RoPE and the cache writes fold into the q|k|v GEMV unless q and k
        are RMS-normalised per head first (headPrep's norm)."""
        return not self.qk_norm


# The workloads' shapes.
QWEN2_05B = ModelShape("qwen2-0.5b-shape", 896, 24, 14, 2, 64, 4864, 151936, "nbits",
                       rope_theta=1e6, eps=1e-6)
# GGUF Q4_K weights, repacked at load into the reference's 32-blocks
# (packQ4_K, src/repack.ts:100-168) with Q4_K's own scales and mins kept
# beside them, at the file's 0.5625 bytes a weight (the half scale and zero
# point a block take 0.625): measured faster than both the half-zero-point
# form and streaming the super-blocks as they are, whose nibble order and
# per-sub-block (d', z') rebuild make that GEMV VALU-bound.
LLAMA3_8B = ModelShape("llama3-8b-shape", 4096, 32, 32, 8, 128, 14336, 128256,
                       "q4_k_records", rope_theta=5e5, eps=1e-5)
LFM2_12B = ModelShape("lfm2-1.2b-shape", 2048, 16, 32, 8, 64, 8192, 65536, "q4_0",
                      rope_theta=1e6, eps=1e-5, qk_norm=True, conv_kernel=3,
                      conv_layers=(0, 1, 3, 4, 6, 7, 9, 11, 13, 15))


class Weights:
    """Random quantized weights of one model shape, generated on the device."""

    def __init__(self, shape: ModelShape, seed: int = 0, device="cuda"):
        self.shape = shape
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.g = g
        self.device = device
        s = shape
        D = s.hidden
        self.embedding = self.matrix(s.vocab, D, fmt=s.embed_fmt)
        self.final_norm = self.norm(D)
        self.layers = []
        for i in range(s.layers):
            lw = {"op_norm": self.norm(D), "ffn_norm": self.norm(D),
                  "gate_up": self.matrix(2 * s.intermediate, D,
                                         gate_up_row_order(s.intermediate)),
                  "down": self.matrix(D, s.intermediate)}
            if s.layer_type(i) == "conv":
                lw["in_proj"] = self.matrix(3 * D, D)
                lw["out_proj"] = self.matrix(D, D)
                lw["taps"] = (torch.randn((D, s.conv_kernel), generator=g, device=device)
                              * 0.5).contiguous()
            else:
                lw["qkv"] = self.matrix(s.qkv_rows, D,
                                        qkv_row_order(s) if s.rope_in_epilogue else None)
                lw["o"] = self.matrix(D, s.heads * s.head_dim)
                if s.qk_norm:
                    lw["q_norm"] = self.norm(s.head_dim)
                    lw["k_norm"] = self.norm(s.head_dim)
            self.layers.append(lw)

    @classmethod
    def blank(cls, shape: ModelShape, seed: int = 0, device="cuda") -> "Weights":
        """The generator alone, with no matrices: matrix() then makes single
        weight matrices of this shape's format."""
        w = cls.__new__(cls)
        w.shape, w.device = shape, device
        w.g = torch.Generator(device=device)
        w.g.manual_seed(seed)
        w.embedding, w.final_norm, w.layers = None, None, []
        return w

    def norm(self, n: int) -> torch.Tensor:
        return (1.0 + 0.1 * torch.randn(n, generator=self.g, device=self.device)).contiguous()

    def matrix(self, N: int, K: int, row_order=None, fmt: str | None = None) -> ops.Q4Matrix:
        """Random weights as a file holds them (GGUF Q4_0, Q4_K, Q8_0 or Q6_K
        blocks, MatMulNBits rows, or floats the loader requantizes to 8 bits),
        uploaded through the GPU repackers with `row_order` as the loaders'
        srcRows (the logical row of each stored row)."""
        fmt = fmt or self.shape.fmt
        g, dev = self.g, self.device
        src_rows = None if row_order is None else \
            torch.tensor(row_order, dtype=torch.int32, device=dev)
        if fmt in ("q4_k", "q4_k_rowgroup", "q4_k_records"):
            src = torch.empty(N * (K // 256) * 144, dtype=torch.uint8, device=dev)
            src.random_(0, 256, generator=g)
            rec = src.view(-1, 144)
            # d and dmin keep d * sc * q - dmin * m near the 0.02 scale of a layer
            hdr = torch.empty((rec.shape[0], 2), device=dev)
            hdr[:, 0].uniform_(1.0e-4, 2.0e-4, generator=g)
            hdr[:, 1].uniform_(4.0e-4, 8.0e-4, generator=g)
            rec[:, 0:4] = hdr.half().view(torch.uint8)
            m = ops.Q4Matrix.from_q4_k(src, N, K, native=fmt == "q4_k", src_rows=src_rows,
                                       records=fmt == "q4_k_records")
            if fmt == "q4_k_records":
                m.prompt_desc()  # the halves prompts and few-token batches read, made now
        elif fmt == "q4_0":
            src = torch.empty(N * (K // 32) * 18, dtype=torch.uint8, device=dev)
            src.random_(0, 256, generator=g)
            blk = src.view(-1, 18)
            d = torch.empty(blk.shape[0], device=dev).uniform_(0.002, 0.006, generator=g)
            blk[:, 0:2] = d.half().view(torch.uint8).view(-1, 2)
            m = ops.Q4Matrix.from_q4_0(src, N, K, src_rows=src_rows)
        elif fmt == "nbits":
            quant, sc, zp = _nbits_from_normal(N, K, g, dev)
            m = ops.Q4Matrix.from_nbits(quant, sc.view(torch.uint8), zp, N, K,
                                        src_rows=src_rows)
        elif fmt == "q8_0":
            src = torch.empty(N * (K // 32) * 34, dtype=torch.uint8, device=dev)
            src.random_(0, 256, generator=g)
            blk = src.view(-1, 34)
            d = torch.empty(blk.shape[0], device=dev).uniform_(1.0e-4, 3.0e-4, generator=g)
            blk[:, 0:2] = d.half().view(torch.uint8).view(-1, 2)
            m = ops.Q4Matrix.from_q8_0(src, N, K, src_rows=src_rows)
        elif fmt == "q8":
            vals = torch.randn((N, K), generator=g, device=dev) * 0.02
            if row_order is not None:
                vals = vals[src_rows.long()].contiguous()
            m = ops.Q4Matrix.from_floats_q8(vals)
        elif fmt == "q6_k":
            src = torch.empty(N * (K // 256) * 210, dtype=torch.uint8, device=dev)
            src.random_(0, 256, generator=g)
            rec = src.view(-1, 210)
            d = torch.empty(rec.shape[0], device=dev).uniform_(2.0e-5, 5.0e-5, generator=g)
            rec[:, 208:210] = d.half().view(torch.uint8).view(-1, 2)
            m = ops.Q4Matrix.from_q6_k(src, N, K, src_rows=src_rows)
        else:
            raise ValueError(f"unknown weight format {fmt}")
        m.row_order = row_order
        return m

    @property
    def nbytes(self) -> int:
        n = self.embedding.nbytes
        for lw in self.layers:
            n += sum(v.nbytes for v in lw.values() if isinstance(v, ops.Q4Matrix))
        return n


class Engine:
    """Forward, greedy pick and accept over device-resident weights."""

    def __init__(self, weights: Weights, ctx: int):
        s = self.shape = weights.shape
        self.w = weights
        self.ctx = ctx
        dev = self.device = weights.device
        D, F = s.hidden, s.intermediate
        R = MAX_ROWS
        f32, f16, i32 = torch.float32, torch.float16, torch.int32
        self.ids = torch.zeros(R, dtype=i32, device=dev)
        self.pos = torch.zeros(1, dtype=i32, device=dev)
        self.h = torch.zeros((R, D), dtype=f32, device=dev)
        self.x16 = torch.zeros((R, D), dtype=f16, device=dev)
        self.c16 = torch.zeros((R, D), dtype=f16, device=dev)
        self.parts = torch.zeros((R, D // 4), dtype=f32, device=dev)
        self.hist = torch.zeros(ctx + 1, dtype=i32, device=dev)
        self.qkv = torch.zeros((R, s.qkv_rows), dtype=f32, device=dev)
        self.q = torch.zeros((R, s.heads * s.head_dim), dtype=f32, device=dev)
        self.att16 = torch.zeros((R, s.heads * s.head_dim), dtype=f16, device=dev)
        self.gu = torch.zeros((R, 2 * F), dtype=f32, device=dev)
        self.ff16 = torch.zeros((R, F), dtype=f16, device=dev)
        self.bcx = torch.zeros((R, 3 * D), dtype=f32, device=dev)
        self.logits = torch.zeros((R, s.vocab), dtype=f32, device=dev)
        self.next_ids = torch.zeros(R, dtype=i32, device=dev)
        self.tops = torch.zeros(R, dtype=f32, device=dev)
        self.argmax_scratch = torch.empty(L.load().wg_argmax_scratch_bytes(R, s.vocab),
                                          dtype=torch.uint8, device=dev)
        # the head GEMV's share of the greedy pick (False: the GEMV, then the
        # two-stage pick over the logits)
        self.pick_parts = ops.pick_parts(R, device=dev)
        self.fuse_pick = True
        self.attn = ops.attn_shape(s.heads, s.kv_heads, s.head_dim, s.head_dim, s.eps, s.qk_norm)
        self.rope = _rope_table(s.rope_theta, s.head_dim, ctx).to(dev)
        self.k_cache, self.v_cache, self.state, self.prefixes = {}, {}, {}, {}
        for i in range(s.layers):
            if s.layer_type(i) == "conv":
                self.state[i] = torch.zeros((s.conv_kernel - 1, D), dtype=f32, device=dev)
                self.prefixes[i] = torch.zeros((R, s.conv_kernel - 1, D), dtype=f32, device=dev)
        # the attention caches ([kv_positions][kv_heads * head_dim] halves a
        # layer) and the attention scratch for that many keys: grown by reserve
        self.kv_positions = 0
        self.graph = None
        self._verify = None
        self._resize_caches(min(ctx, KV_START), keep=0)
        self.position = 0
        self.draft = None
        self._pre = None  # prefill buffers, made on the first prompt batch
        self._cols = {}   # device row orders of the matrices (GEMM column maps)
        # probe(layer, name, rows), called as the forward enqueues (not under
        # graph capture): ("embedding", h rows) after the lookup, ("attention",
        # (q rows, output rows)) after each attention, ("output", h rows)
        # after the last layer; the self-check reads them back
        self.probe = None
        # short convs in in_proj's epilogue (False: in_proj, then the conv)
        self.fuse_conv = True
        # heads prepared inside the decode attention (False: head_prep, then
        # the attention)
        self.fuse_prep = True
        # a device verify step's drafts read by the embedding and its picks
        # finished by the accept (False: drafts, pick and accept launches)
        self.fuse_verify = True
        self._drafts = None

    # --- the attention caches, grown on demand ------------------------------
    def reserve(self, end: int) -> None:
        """Makes room in the attention caches for positions up to `end`
        (Engine.reserve, src/engine.ts:1635-1696): new caches of whole
        KV_STEP steps, at least twice the positions they replace (the copies
        then add up to at most the final size: a 128K-token context is not
        copied 250 times over), at most the context, holding the old rows.
        The captured decode and verify graphs hold the old caches'
        addresses: they are dropped (captured again when next used)."""
        if end > self.ctx:
            raise ValueError(f"The cache holds {self.ctx} tokens; this would need {end}.")
        if end <= self.kv_positions:
            return
        n = min(self.ctx, max(-(-end // KV_STEP) * KV_STEP, 2 * self.kv_positions))
        self._resize_caches(n, keep=self.kv_positions)

    def _resize_caches(self, n: int, keep: int) -> None:
        """Caches of n positions holding the first `keep` rows of the old
        ones (the rest zero), and attention scratch for n keys."""
        s, dev = self.shape, self.device
        kvd = s.kv_heads * s.head_dim
        for cache in (self.k_cache, self.v_cache):
            for i in range(s.layers):
                if s.layer_type(i) == "conv":
                    continue
                new = torch.zeros((n, kvd), dtype=torch.float16, device=dev)
                if keep:
                    new[:keep].copy_(cache[i][:keep])
                cache[i] = new
        self.attn_scratch = ops.attn_scratch(MAX_ROWS, self.attn, n, dev)
        self.kv_positions = n
        self.graph = None
        if self._verify is not None:
            self._verify["graph"] = None

    # --- the batch ------------------------------------------------------------
    def _norm_in(self, ep: "L.Epilogue") -> "L.Epilogue":
        """The input side of a GEMV that reads the prescaled residual."""
        D = self.shape.hidden
        ep.norm_parts = self.parts.data_ptr()
        ep.n_parts = D // 4
        ep.ld_parts_in = D // 4
        ep.norm_count = D
        ep.eps = self.shape.eps
        ep.norm_mult = PRESCALE
        return ep

    def _residual_out(self, M: int, next_norm: torch.Tensor) -> "L.Epilogue":
        """h += result; the next norm's prescaled input and the parts."""
        D = self.shape.hidden
        return L.Epilogue(mode=L.EPI_STORE, residual=self.h.data_ptr(), ld_residual=D,
                          out16=self.x16.data_ptr(), ld_out16=D, out16_w=next_norm.data_ptr(),
                          norm_mult_out=PRESCALE, parts_out=self.parts.data_ptr(),
                          ld_parts_out=D // 4)

    def _qkv_epilogue(self, i: int) -> "L.Epilogue":
        """qkv's epilogue when RoPE and the KV write are fused into it."""
        s = self.shape
        return self._norm_in(L.Epilogue(
            mode=L.EPI_ROPE_KV, heads=s.heads, kv_heads=s.kv_heads,
            head_dim=s.head_dim, ctx=self.kv_positions, rope_rows=self.rope.shape[0],
            rope=self.rope.data_ptr(), pos0=self.pos.data_ptr(),
            q_out=self.q.data_ptr(), ld_q_out=s.heads * s.head_dim,
            k_cache=self.k_cache[i].data_ptr(), v_cache=self.v_cache[i].data_ptr()))

    def _next_norm(self, i: int) -> torch.Tensor:
        w = self.w
        return w.layers[i + 1]["op_norm"] if i + 1 < len(w.layers) else w.final_norm

    def _forward_rows(self, M: int, keep_prefixes: bool, pick=True) -> None:
        """Enqueue one batch of M rows (ids[:M] at positions pos..pos+M-1);
        the greedy picks into next_ids unless `pick` is False (the caller
        picks), or "advance" (see _head_rows)."""
        self._embed_rows(M)
        if self.probe:
            self.probe(-1, "embedding", self.h[:M])
        for i in range(len(self.w.layers)):
            self._layer_rows(i, M, keep_prefixes)
        if self.probe:
            self.probe(len(self.w.layers) - 1, "output", self.h[:M])
        return self._head_rows(M, pick)

    def _embed_rows(self, M: int) -> None:
        """h = the rows' embeddings; the first norm's prescaled input and
        sums of squares."""
        s, w = self.shape, self.w
        D = s.hidden
        first_norm = w.layers[0]["op_norm"] if w.layers else w.final_norm
        ep = L.Epilogue(mode=L.EPI_STORE, out16=self.x16.data_ptr(), ld_out16=D,
                        out16_w=first_norm.data_ptr(), norm_mult_out=PRESCALE,
                        parts_out=self.parts.data_ptr(), ld_parts_out=D // 4)
        if self._drafts is not None:  # a verify step's drafts from the device table
            table, cursor = self._drafts
            ops.embed_drafts(w.embedding, self.ids, M, table, cursor, out=self.h[:M], epilogue=ep)
        else:
            ops.embed(w.embedding, self.ids[:M], out=self.h[:M], epilogue=ep)

    def _layer_rows(self, i: int, M: int, keep_prefixes: bool) -> None:
        """Layer i over the batch: h += operator(norm(h)); h += FFN(norm(h));
        the next norm's prescaled input and sums of squares."""
        s, lw = self.shape, self.w.layers[i]
        D, F = s.hidden, s.intermediate
        h, x16 = self.h[:M], self.x16[:M]
        if s.layer_type(i) == "conv":
            c16 = self.c16[:M]
            prefixes = self.prefixes[i][:M] if keep_prefixes else None
            # the convolution in in_proj's epilogue where the library takes
            # it, else in_proj into the B | C | x rows, then the conv
            fused = self.fuse_conv and ops.gemv_short_conv(lw["in_proj"], x16, self._norm_in(
                L.Epilogue(mode=L.EPI_SHORT_CONV, out16=c16.data_ptr(), ld_out16=D,
                           conv_taps=lw["taps"].data_ptr(), conv_state=self.state[i].data_ptr(),
                           conv_state_out=self.state[i].data_ptr(),
                           conv_prefixes=prefixes.data_ptr() if prefixes is not None else None,
                           conv_width=s.conv_kernel)))
            if not fused:
                bcx = self.bcx[:M]
                ops.gemv(lw["in_proj"], x16, out=bcx,
                         epilogue=self._norm_in(L.Epilogue(mode=L.EPI_STORE)))
                ops.short_conv(bcx, D, s.conv_kernel, lw["taps"], self.state[i],
                               prefixes=prefixes, out=c16)
            ops.gemv(lw["out_proj"], c16, out=h, epilogue=self._residual_out(M, lw["ffn_norm"]))
        else:
            if s.rope_in_epilogue:
                ops.gemv(lw["qkv"], x16, epilogue=self._qkv_epilogue(i))
            else:
                qkv = self.qkv[:M]
                ops.gemv(lw["qkv"], x16, out=qkv,
                         epilogue=self._norm_in(L.Epilogue(mode=L.EPI_STORE)))
            # the heads prepared inside the attention kernel where it takes
            # the shape, else head preparation, then the attention
            if s.rope_in_epilogue or not self.fuse_prep or ops.attn_decode_prep(
                    self.qkv[:M], self.attn, self.rope, self.pos, self.k_cache[i],
                    self.v_cache[i], lw.get("q_norm"), lw.get("k_norm"),
                    scratch=self.attn_scratch, out=self.att16[:M], q_out=self.q[:M]) is None:
                if not s.rope_in_epilogue:
                    ops.head_prep(self.qkv[:M], self.attn, self.rope, self.pos, self.k_cache[i],
                                  self.v_cache[i], lw.get("q_norm"), lw.get("k_norm"),
                                  q_out=self.q[:M])
                ops.attn_decode(self.q[:M], self.attn, self.k_cache[i], self.v_cache[i],
                                self.pos, scratch=self.attn_scratch, out=self.att16[:M])
            if self.probe:
                self.probe(i, "attention", (self.q[:M], self.att16[:M]))
            ops.gemv(lw["o"], self.att16[:M], out=h,
                     epilogue=self._residual_out(M, lw["ffn_norm"]))
        ops.gemv(lw["gate_up"], x16,
                 epilogue=self._norm_in(L.Epilogue(mode=L.EPI_SWIGLU,
                                                   out16=self.ff16.data_ptr(), ld_out16=F)))
        ops.gemv(lw["down"], self.ff16[:M], out=h,
                 epilogue=self._residual_out(M, self._next_norm(i)))

    def _head_rows(self, M: int, pick=True) -> None:
        """Logits of the batch's rows over the tied embedding; the greedy
        picks into next_ids when `pick`, or (pick "advance", one row) the
        decode step's pick and advance (ids[0], hist, pos)."""
        emb, x16, logits = self.w.embedding, self.x16[:M], self.logits[:M]
        if pick and self.fuse_pick and ops.gemv_pick(
                emb, x16, logits, self.pick_parts, self._norm_in(L.Epilogue(mode=L.EPI_STORE))):
            if pick == "parts":  # the caller finishes the picks from the parts
                return True
            if pick == "advance":
                ops.argmax_parts(self.pick_parts, 1, self.ids, tops=self.tops[:1],
                                 pos=self.pos, hist=self.hist)
            else:
                ops.argmax_parts(self.pick_parts, M, self.next_ids[:M], tops=self.tops[:M])
            return
        ops.gemv(emb, x16, out=logits, epilogue=self._norm_in(L.Epilogue(mode=L.EPI_STORE)))
        if pick == "advance":
            ops.argmax_advance(self.logits[0], self.ids, self.pos, hist=self.hist,
                               tops=self.tops[:1], scratch=self.argmax_scratch)
        elif pick:
            ops.argmax_rows(logits, ids=self.next_ids[:M], tops=self.tops[:M],
                            scratch=self.argmax_scratch)
        return False

    # --- prompt batches on MFMA ----------------------------------------------
    def _prefill_ok(self) -> bool:
        """Whether prompt batches can run as GEMMs: every matrix of a layer in
        a row-group layout (4- or 8-bit) with N and K multiples of 64."""
        for lw in self.w.layers:
            for m in lw.values():
                if isinstance(m, ops.Q4Matrix) and (
                        m.layout not in (L.LAYOUT_ROWGROUP, L.LAYOUT_Q8) or m.N % 64 or
                        m.K % 64):
                    return False
        s = self.shape
        return s.head_dim in (64, 128)

    def _pre_buffers(self) -> dict:
        if self._pre is None:
            s, R, dev = self.shape, PREFILL_ROWS, self.device
            D, F, A = s.hidden, s.intermediate, s.heads * s.head_dim
            f32, f16 = torch.float32, torch.float16
            self._pre = {
                "ids": torch.zeros(R, dtype=torch.int32, device=dev),
                "h": torch.zeros((R, D), dtype=f32, device=dev),
                "rs": torch.zeros(R, dtype=f32, device=dev),
                "x16": torch.zeros((R, D), dtype=f16, device=dev),
                "c16": torch.zeros((R, D), dtype=f16, device=dev),
                "bcx": torch.zeros((R, 3 * D), dtype=f32, device=dev),
                "qkv": torch.zeros((R, s.qkv_rows), dtype=f32, device=dev),
                "q": torch.zeros((R, A), dtype=f32, device=dev),
                "att16": torch.zeros((R, A), dtype=f16, device=dev),
                "ff16": torch.zeros((R, F), dtype=f16, device=dev),
            }
        return self._pre

    def _col_of(self, m: "ops.Q4Matrix"):
        """The GEMM column map of a matrix uploaded in a row order (stored row
        n holds logical row row_order[n]), or None."""
        order = getattr(m, "row_order", None)
        if order is None:
            return None
        key = id(m)
        if key not in self._cols:
            self._cols[key] = torch.tensor(order, dtype=torch.int32, device=self.device)
        return self._cols[key]

    def _prefill_rows(self, M: int) -> None:
        """A prompt batch of M rows (pre ids[:M] at positions pos ..) through
        the GEMMs on MFMA, as the reference's forwardBatch takes batches larger
        than the split path's (Engine.matmul, src/engine.ts:4969-5234, and its
        attention plan for a prompt, :6359-6630). A norm's output is the
        reference's prescaled half(h w / 32), its 32 / RMS the GEMM's row
        scale, as in the few-token path; the caches and conv states advance;
        no head here (_prefill_head)."""
        s, w, b = self.shape, self.w, self._pre_buffers()
        D = s.hidden
        h, x16, rs = b["h"][:M], b["x16"][:M], b["rs"][:M]
        ops.embed(w.embedding, b["ids"][:M], out=h)
        for i, lw in enumerate(w.layers):
            ops.norm_to_h2(h, lw["op_norm"], s.eps, x16, rs)
            if s.layer_type(i) == "conv":
                bcx = ops.gemm(lw["in_proj"], x16, out=b["bcx"][:M], row_scale=rs)
                ops.short_conv(bcx, D, s.conv_kernel, lw["taps"], self.state[i], out=b["c16"][:M])
                ops.gemm(lw["out_proj"], b["c16"][:M], out=h, residual=h)
            else:
                qkv = ops.gemm(lw["qkv"], x16, out=b["qkv"][:M], col_of=self._col_of(lw["qkv"]),
                               row_scale=rs)
                ops.head_prep(qkv, self.attn, self.rope, self.pos, self.k_cache[i],
                              self.v_cache[i], lw.get("q_norm"), lw.get("k_norm"),
                              q_out=b["q"][:M])
                ops.attn_prefill(b["q"][:M], self.attn, self.k_cache[i], self.v_cache[i],
                                 self.pos, out=b["att16"][:M])
                if self.probe:
                    self.probe(i, "attention", (b["q"][:M], b["att16"][:M]))
                ops.gemm(lw["o"], b["att16"][:M], out=h, residual=h)
            ops.norm_to_h2(h, lw["ffn_norm"], s.eps, x16, rs)
            ops.gemm_swiglu(lw["gate_up"], x16, out=b["ff16"][:M], row_scale=rs)
            ops.gemm(lw["down"], b["ff16"][:M], out=h, residual=h)

    def _prefill_head(self, r0: int, T: int) -> None:
        """Logits and picks of rows r0 .. r0 + T - 1 (T <= 8) of the last
        prompt batch: the final norm to halves, the head GEMV, the picks."""
        s, w, b = self.shape, self.w, self._pre_buffers()
        x16, rs = b["x16"][r0:r0 + T], b["rs"][r0:r0 + T]
        ops.norm_to_h2(b["h"][r0:r0 + T], w.final_norm, s.eps, x16, rs)
        ops.gemv(w.embedding, x16, out=self.logits[:T], row_scale=rs)
        ops.argmax_rows(self.logits[:T], ids=self.next_ids[:T], tops=self.tops[:T],
                        scratch=self.argmax_scratch)

    # --- the reference's Engine API -------------------------------------------
    def reset(self) -> None:
        """A new sequence: position 0, conv states cleared, the caches back
        to their starting size (shrink, src/engine.ts:1709-1719)."""
        self.position = 0
        self.pos.zero_()
        for st in self.state.values():
            st.zero_()
        self.draft = None
        start = min(self.ctx, KV_START)
        if self.kv_positions > start:
            self._resize_caches(start, keep=0)

    def forward(self, tokens, draft: bool = False) -> torch.Tensor:
        """Runs tokens (a prompt in batches of 8, or a token and its drafts)
        and returns the greedy pick of every row of the last batch."""
        tokens = list(tokens)
        if not tokens:
            raise ValueError("no tokens")
        if self.position + len(tokens) > self.ctx:
            raise ValueError(f"The cache holds {self.ctx} tokens; this would need "
                             f"{self.position + len(tokens)}.")
        if draft and len(tokens) > MAX_ROWS:
            raise ValueError(f"A draft batch holds {MAX_ROWS} tokens at most.")
        # the whole prompt's room at once (preparePrompt, src/engine.ts:1699-1704)
        self.reserve(self.position + len(tokens))
        out = None
        # a prompt's leading rows in GEMM batches; its last (up to 8) rows, whose
        # picks are returned, through the few-token path
        big = 0
        if not draft and len(tokens) > MAX_ROWS and self._prefill_ok():
            big = len(tokens)
        for b0 in range(0, big, PREFILL_ROWS):
            batch = tokens[b0:min(big, b0 + PREFILL_ROWS)]
            M = len(batch)
            self._pre_buffers()["ids"][:M].copy_(torch.tensor(batch, dtype=torch.int32))
            self.pos.fill_(self.position)
            self._prefill_rows(M)
            self.position += M
        if big:
            # the picks of the last batch of 8 (len mod 8 rows, or 8): the head
            # over the last rows of the final GEMM batch only
            T = len(tokens) % MAX_ROWS or MAX_ROWS
            M = len(tokens) - (len(tokens) - 1) // PREFILL_ROWS * PREFILL_ROWS
            self._prefill_head(M - T, T)
            out = self.next_ids[:T]
        for b0 in range(big if big else 0, len(tokens), MAX_ROWS):
            batch = tokens[b0:b0 + MAX_ROWS]
            M = len(batch)
            self.ids[:M].copy_(torch.tensor(batch, dtype=torch.int32))
            self.pos.fill_(self.position)
            self._forward_rows(M, keep_prefixes=draft)
            self.position += M
            out = self.next_ids[:M]
        if draft:
            self.draft = (self.position - len(tokens), len(tokens))
        return out.clone()

    def accept(self, count: int) -> None:
        """Keeps the first `count` tokens of the last draft batch
        (src/engine.ts:8063-8086): conv states back to that prefix; the
        cache continues after them."""
        if self.draft is None:
            raise ValueError("No draft batch to accept tokens of.")
        pos0, rows = self.draft
        self.draft = None
        if count < 1 or count > rows:
            raise ValueError(f"Can't keep {count} of a {rows}-token batch.")
        if count < rows:
            s = self.shape
            for i, st in self.state.items():
                ops.conv_accept(self.prefixes[i], count, rows, s.hidden, s.conv_kernel, st)
        self.position = pos0 + count

    # --- graph-captured single-token decode -----------------------------------
    def capture_step(self, token: int) -> None:
        """Captures one decode step: forward of ids[0] at pos, pick into
        ids[0], pos += 1. The capture first runs the step once eagerly with
        ids[0] = token at pos = position (the token the first replay will
        run): that run writes this position's K and V, which the first replay
        writes again, and everything else it changes is put back."""
        self.reserve(self.position + 1)
        self.ids[0] = token
        self.pos.fill_(self.position)
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            # warm-up outside the graph (first-call lazies), state restored after
            saved = self._save()
            self._step_body()
            self._restore(saved)
            torch.cuda.current_stream().synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                self._step_body()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        self._restore(saved)
        self.graph = g

    def _step_body(self) -> None:
        # the pick goes to ids[0] and hist[pos + 1], then pos += 1: the next
        # replay runs the picked token at the next position
        self._forward_rows(1, keep_prefixes=False, pick="advance")

    def _save(self):
        return (self.ids.clone(), self.pos.clone(), {i: s.clone() for i, s in self.state.items()})

    def _restore(self, saved) -> None:
        ids, pos, states = saved
        self.ids.copy_(ids)
        self.pos.copy_(pos)
        for i, s in states.items():
            self.state[i].copy_(s)

    def decode(self, first_token: int, steps: int) -> list[int]:
        """Greedy decode `steps` tokens after `first_token` by graph replay."""
        if self.position + steps > self.ctx:
            raise ValueError("decode would run past the cache")
        self.reserve(self.position + steps)
        if self.graph is None:
            self.capture_step(first_token)
        p0 = self.position
        self.ids[0] = first_token
        self.pos.fill_(p0)
        for _ in range(steps):
            self.graph.replay()
        self.position += steps
        return self.hist[p0 + 1:p0 + steps + 1].tolist()

    # --- speculative verify on the device, graph-captured --------------------
    VERIFY_TABLE = 1024  # draft rows the device table holds (steps a replay run takes)

    def _verify_buffers(self, rows: int) -> dict:
        v = self._verify
        if v is None or v["rows"] != rows:
            dev, i32 = self.device, torch.int32
            layers = [(self.prefixes[i], self.state[i]) for i in sorted(self.state)]
            v = {"rows": rows, "convs": ops.conv_states(layers, dev),
                 "table": torch.zeros((self.VERIFY_TABLE, rows - 1), dtype=i32, device=dev),
                 "cursor": torch.zeros(1, dtype=i32, device=dev),
                 "kept": torch.zeros(self.VERIFY_TABLE, dtype=i32, device=dev), "graph": None}
            self._verify = v
        return v

    def _verify_body(self, v: dict) -> None:
        """One verify step on the device: drafts from the table into ids[1:],
        the batch's forward and greedy picks, then the accept (the kept
        prefix's picks into hist, the conv states rolled back, pos and
        ids[0] moved on: wg_verify_accept)."""
        rows = v["rows"]
        if not self.fuse_verify:
            ops.verify_drafts(self.ids, rows, v["table"], v["cursor"])
            self._forward_rows(rows, keep_prefixes=True)
            ops.verify_accept(self.next_ids[:rows], rows, v["convs"], self.pos, self.ids,
                              self.hist, v["kept"], v["cursor"])
            return
        # the drafts read by the embedding, the picks finished by the accept
        self._drafts = (v["table"], v["cursor"])
        try:
            parts = self._forward_rows(rows, keep_prefixes=True, pick="parts")
        finally:
            self._drafts = None
        if parts:
            ops.verify_accept_parts(self.pick_parts, self.next_ids[:rows], rows, v["convs"],
                                    self.pos, self.ids, self.hist, v["kept"], v["cursor"])
        else:
            ops.verify_accept(self.next_ids[:rows], rows, v["convs"], self.pos, self.ids,
                              self.hist, v["kept"], v["cursor"])

    def capture_verify(self, rows: int = 5) -> None:
        """Captures one verify step of `rows` rows (a token and rows - 1
        drafts) as a HIP graph. The capture first runs the step once
        eagerly; the ids, position, conv states and cursor it changes are
        put back (the cache rows it writes are written again by the first
        replay)."""
        if not 2 <= rows <= MAX_ROWS:
            raise ValueError(f"A verify batch holds 2 to {MAX_ROWS} rows.")
        self.reserve(self.position + rows)
        v = self._verify_buffers(rows)
        self.pos.fill_(self.position)
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            saved = self._save()
            cursor = v["cursor"].clone()
            self._verify_body(v)
            self._restore(saved)
            v["cursor"].copy_(cursor)
            torch.cuda.current_stream().synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                self._verify_body(v)
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        self._restore(saved)
        v["cursor"].copy_(cursor)
        v["graph"] = g

    def verify_drafts(self, first_token: int, drafts) -> tuple[list[int], list[int]]:
        """Greedy speculative decoding with given drafts, every step on the
        device: step s runs [the last accepted token] + drafts[s] (rows - 1
        ids) as one batch and keeps its agreeing prefix + 1 (the reference's
        verify loop, src/handler.ts:1811-1887, with Engine.accept,
        src/engine.ts:8063-8086). Steps replay back to back with no host
        decision; the tokens and each step's kept count are read back once
        per run of up to VERIFY_TABLE steps. Returns (the tokens written,
        the kept counts)."""
        table = torch.as_tensor(drafts, dtype=torch.int32)
        if table.dim() != 2 or table.shape[1] < 1:
            raise ValueError("drafts must be [steps, rows - 1]")
        steps, rows = table.shape[0], table.shape[1] + 1
        v = self._verify_buffers(rows)
        p0 = self.position
        self.ids[0] = first_token
        self.pos.fill_(p0)
        kept_all: list[int] = []
        done = 0
        while done < steps:
            # every step of a run must fit the cache even if it keeps every row
            n = min(steps - done, self.VERIFY_TABLE, (self.ctx - self.position) // rows)
            if n <= 0:
                raise ValueError(f"The cache holds {self.ctx} tokens; verify batches of {rows} "
                                 f"from position {self.position} would pass it.")
            # room for the run (which drops a graph that held smaller caches)
            self.reserve(self.position + n * rows)
            if v["graph"] is None:
                self.capture_verify(rows)
            v["table"][:n].copy_(table[done:done + n])
            v["cursor"].zero_()
            for _ in range(n):
                v["graph"].replay()
            kept = v["kept"][:n].tolist()
            kept_all += kept
            self.position += sum(kept)
            done += n
        tokens = self.hist[p0 + 1:self.position + 1].tolist()
        return tokens, kept_all

    # --- sampled decoding -------------------------------------------------
    def generate(self, prompt: list[int], steps: int, sampler, random=None,
                 count: int = 64, guess: bool = False) -> list[int]:
        """Sampled decoding (Engine.pick + the host sampler, src/engine.ts:
        8352-8473, src/sampler.ts): each step's last logits row goes through
        wg_pick_candidates (the penalties of the sampler's window on the
        device, the best `count` chunks read back) and the sampler draws
        the token from them. The window sees the prompt, then each token
        written. Returns the `steps` tokens drawn.

        As the reference decides (src/handler.ts:1429-1437), the whole row
        is read back and penalized and sampled on the host instead when the
        GPU's candidates cannot hold the distribution: a frequency penalty
        (the device's mask knows whether a token is in the window, not how
        often), or top-k off or above the `count` chunks kept.

        Each drawn token runs as one replay of the captured decode step
        (capture_step), not as a host loop of launches. With `guess` (and
        the GPU's candidates) the GPU does not wait for the host's draw
        either (forwardGuess / keepGuess / dropGuess, src/engine.ts:
        8095-8150): once a row's pick and read-back are enqueued, the row's
        greedy pick runs as the next token (conv states saved first) while
        the host draws. If the draw is that token, its forward is already
        done; if not, the conv states are put back and the drawn token runs
        (its K and V rows overwrite the guess's). The tokens are the same
        either way; guess_hits and guess_misses count the two. On this GPU
        a step's host gap (pick read-back and draw) is ~0.14 ms against a
        ~1.6 ms replay of the 8B shape, so a guess pays only above a ~91%
        hit rate: off by default."""
        from . import sampler as S
        st = sampler.settings
        greedy = st.temperature <= 0 or st.top_k == 1
        on_gpu = sampler.frequency_penalty == 0 and (greedy or 0 < st.top_k <= count)
        pick = S.GpuPick(self.shape.vocab, count, device=self.device) if on_gpu else None
        changes = sampler.see(prompt)
        if pick is not None:
            pick.see(changes)
        guess = guess and pick is not None
        guessed = torch.empty(1, dtype=torch.int32, pin_memory=True)
        saved = {i: torch.empty_like(s) for i, s in self.state.items()}
        self.guess_hits = self.guess_misses = 0
        if steps <= 0:
            return []
        end = self.position + len(prompt) + steps - 1  # the last token drawn is not run
        if end > self.ctx:
            raise ValueError(f"The cache holds {self.ctx} tokens; this would need {end}.")
        # the whole run's room first: growing the caches would drop the graph
        self.reserve(end)
        out = []
        self.forward(prompt)
        row = (len(prompt) - 1) % 8
        greedy_pick = self.next_ids[row:row + 1]  # the last row's greedy pick
        for step in range(steps):
            last = step + 1 == steps
            ahead = guess and not last
            if pick is not None:
                pick.start(self.logits[row], sampler, also=[(guessed, greedy_pick)] if ahead else ())
                if ahead:
                    for i, s in self.state.items():
                        saved[i].copy_(s)
                    self._replay_step(greedy_pick)
                d = pick.finish(sampler)
            else:
                d = sampler.distribution(self.logits[row].cpu().numpy().copy(), penalize=True)
            t = S.draw(d, random)
            out.append(t)
            changes = sampler.see([t], True)
            if pick is not None:
                pick.see(changes)
            if last:
                break
            if ahead and t == int(guessed[0]):
                self.guess_hits += 1
            else:
                if ahead:
                    for i, s in self.state.items():
                        s.copy_(saved[i])
                    self.guess_misses += 1
                self._replay_step(t)
            self.position += 1
            row, greedy_pick = 0, self.ids[:1]  # the step's pick went to ids[0]
        return out

    def _replay_step(self, token) -> None:
        """One decode step of `token` (an int, or a 1-element device tensor)
        at self.position by the captured graph (captured on first use):
        logits into row 0, the greedy pick into ids[0]. self.position is
        left to the caller."""
        if self.graph is None:
            self.capture_step(token if isinstance(token, int) else int(token[0]))
        if isinstance(token, int):
            self.ids[0] = token
        elif token.data_ptr() != self.ids.data_ptr():
            self.ids[:1].copy_(token)
        self.pos.fill_(self.position)
        self.graph.replay()


def _nbits_from_normal(N: int, K: int, g: torch.Generator, dev):
    """A MatMulNBits q4 matrix's file arrays quantized from weights ~ N(0,
    0.02): per block of 32, a zero point ~ U{0..15}, the half scale
    absmax / max(zp, 15 - zp) and q = clamp(round(w / scale) + zp, 0, 15).
    Returns (quant [N][K/32][16] bytes, element 2i in byte i's low nibble;
    half scales [N][K/32]; zero points [N][ceil(K/64)], low nibble first),
    the layouts src/load-onnx.ts:450-501 reads."""
    B = K // 32
    w = torch.randn((N, B, 32), generator=g, device=dev) * 0.02
    zpv = torch.randint(0, 16, (N, B), generator=g, device=dev)
    am = w.abs().amax(2).clamp_min(1e-8)
    sc = (am / torch.maximum(zpv, 15 - zpv).float()).half()
    q = torch.clamp(torch.round(w / sc.float()[..., None]) + zpv[..., None], 0, 15)
    q = q.to(torch.uint8)
    quant = (q[..., 0::2] | (q[..., 1::2] << 4)).contiguous().view(-1)
    zp8 = zpv.to(torch.uint8)
    if B % 2:
        zp8 = torch.cat([zp8, torch.zeros((N, 1), dtype=torch.uint8, device=dev)], 1)
    zp = (zp8[:, 0::2] | (zp8[:, 1::2] << 4)).contiguous().view(-1)
    del w, q
    return quant, sc.contiguous().view(-1), zp


def _rope_table(theta: float, head_dim: int, ctx: int) -> torch.Tensor:
    """Engine.ropeTable (src/engine.ts:1292-1312): cos and sin in doubles,
    stored as float32; rows 0..1023 positions, row 1024 + i position 1024 i."""
    half = head_dim // 2
    rows = 1024 + (ctx + 1023) // 1024
    r = torch.arange(rows, dtype=torch.float64)
    pos = torch.where(r < 1024, r, (r - 1024) * 1024)
    i = torch.arange(half, dtype=torch.float64)
    freq = theta ** (-2.0 * i / head_dim)
    ang = pos[:, None] * freq[None, :]
    return torch.cat([torch.cos(ang), torch.sin(ang)], dim=1).to(torch.float32).contiguous()
