"""Loads an LFM2 GGUF file into the engine's device weights, as the
reference's loadGguf does for its WebGL engine (src/load-gguf.ts:83-455):
the model's settings from the metadata (ggufConfig, :600-752), then every
matrix uploaded as the file has it and repacked on the GPU into the
QuantMatrix layouts, by the reference's storage rules (matrixStorage,
:475-484; bitsOf, :486-507; packRows, :509-555):
- a matrix made only of Q4_K tensors (K a multiple of 256) keeps 4 bits as
  packQ4_K's 32-blocks with half scale and zero point;
- only Q4_0 tensors: packQ4_0;
- otherwise 8 bits: Q8_0 copied (packQ8_0), F32, F16, Q4_1, Q4_K, Q5_K and
  Q6_K converted to floats (rowsToFloats) and requantized (quantizeQ8);
- the embedding (also the output head): Q6_K kept as it is (packQ6_K),
  Q4_0 and Q8_0 repacked, any other type requantized to 8 bits (:425-442).
Fused matrices (q|k|v, gate|up) are uploaded in the engine's row order
(the loaders' srcRows), so their epilogues find partner rows together.

Every conversion runs on the device through the C ABI; the host only maps
the file and copies its bytes over.

Architectures the engine does not run (LFM3's gated attention and sandwich
norms, Qwen3.5's Gated DeltaNet, sliding-window or partial-RoPE attention,
a separate output head) are rejected with a message.
"""
from __future__ import annotations

import os

import numpy as np
import torch

from . import engine as E
from . import gguf as G
from . import lib as L
from . import ops

_EIGHT_BIT = (G.F32, G.F16, G.Q8_0, G.Q4_1, G.Q4_K, G.Q5_K, G.Q6_K)


def _f32_decimal(v: float) -> float:
    """A float32 metadata value as the decimal it was written from
    (f32Decimal, src/load-gguf.ts:594-597: 1e-5, not 9.9999997e-6)."""
    return float(f"{v:.7g}")


def gguf_shape(f: G.GgufFile, name: str | None = None) -> E.ModelShape:
    """ggufConfig (src/load-gguf.ts:600-752) for the architectures the
    engine runs: LFM2 (short-conv and full-attention layers, q/k norms, a
    tied output head)."""
    meta = f.metadata
    arch = meta.get("general.architecture")
    if not isinstance(arch, str):
        raise ValueError("GGUF: no general.architecture")
    if arch != "lfm2":
        raise ValueError(f"GGUF: unsupported architecture {arch}"
                         + (" (its attention gate, sandwich norms or Gated DeltaNet are not "
                            "on this engine's path)" if arch in ("lfm3", "qwen35") else ""))
    if "output.weight" in f.tensors:
        raise ValueError("GGUF: LFM2 models with a separate output head are not supported.")

    def num(key, fallback=None):
        v = meta.get(key, meta.get(f"{arch}.{key}"))
        if v is None:
            if fallback is not None:
                return fallback
            raise ValueError(f"GGUF: missing metadata {arch}.{key}")
        if isinstance(v, bool) or not isinstance(v, (int, float)):
            raise ValueError(f"GGUF: {key} is not a number")
        return v

    layers = int(num("block_count"))
    hidden = int(num("embedding_length"))
    heads = int(num("attention.head_count"))
    kv_value = meta.get(f"{arch}.attention.head_count_kv")
    if isinstance(kv_value, list):
        kv = [int(x) for x in kv_value]
    else:
        kv = [int(kv_value if kv_value is not None else heads)] * layers
    if len(kv) != layers:
        raise ValueError("GGUF: head_count_kv doesn't have one entry per layer")
    if num("attention.sliding_window", 0) > 0 or \
            isinstance(meta.get(f"{arch}.attention.sliding_window_pattern"), list):
        raise ValueError("GGUF: sliding-window attention is not supported by this engine")
    kv_heads = max(kv)
    if any(k not in (0, kv_heads) for k in kv):
        raise ValueError("GGUF: attention layers with different KV head counts are not "
                         "supported")
    if kv_heads == 0:
        raise ValueError("GGUF: no attention layer")
    head_dim = int(num("attention.key_length", hidden // heads))
    if int(num("rope.dimension_count", head_dim)) != head_dim or "rope_freqs.weight" in f.tensors:
        raise ValueError("GGUF: partial RoPE is not supported by this engine")
    emb = f.tensors.get("token_embd.weight")
    if emb is None:
        raise ValueError("GGUF: missing tensor token_embd.weight")
    if emb.dims[0] != hidden:
        raise ValueError(f"GGUF: token_embd has {emb.dims[0]} columns, expected {hidden}")
    ffn = meta.get(f"{arch}.feed_forward_length")
    gate0 = f.tensors.get("blk.0.ffn_gate.weight")
    inter = int(ffn) if isinstance(ffn, int) else (gate0.dims[1] if gate0 else -1)
    if gate0 is not None and gate0.dims[1] != inter:
        raise ValueError(f"GGUF: feed_forward_length {inter} doesn't match ffn_gate rows "
                         f"{gate0.dims[1]}")
    label = name or str(meta.get("general.name") or os.path.basename(f.path))
    return E.ModelShape(label, hidden, layers, heads, kv_heads, head_dim, inter, emb.dims[1],
                        "gguf", rope_theta=_f32_decimal(num("rope.freq_base")),
                        eps=_f32_decimal(num("attention.layer_norm_rms_epsilon")),
                        qk_norm=True, conv_kernel=int(num("shortconv.l_cache")),
                        conv_layers=tuple(i for i, k in enumerate(kv) if k == 0),
                        embed_fmt="gguf", extra={"context_length": int(num("context_length",
                                                                            8192))})


class _Uploader:
    def __init__(self, f: G.GgufFile, device):
        self.f, self.device = f, device

    def info(self, name: str) -> G.TensorInfo:
        t = self.f.tensors.get(name)
        if t is None:
            raise ValueError(f"GGUF: missing tensor {name}")
        return t

    def bytes(self, name: str) -> torch.Tensor:
        """A tensor's file bytes on the device."""
        host = torch.from_numpy(np.array(self.f.data(name)))
        return host.to(self.device)

    def floats(self, name: str, rows: int, K: int) -> torch.Tensor:
        """rowsToFloats on the device (wg_rows_to_floats)."""
        t = self.info(name)
        out = torch.empty((rows, K), dtype=torch.float32, device=self.device)
        L.check(L.load().wg_rows_to_floats(t.type, self.bytes(name).data_ptr(), rows, K,
                                           out.data_ptr(), ops._stream()))
        return out

    def vector(self, name: str, n: int) -> torch.Tensor:
        """A norm or conv weight (F32 or F16: toFloats, src/load-gguf.ts:582-588)."""
        t = self.info(name)
        if t.type not in (G.F32, G.F16):
            raise ValueError(f"GGUF: {name} has type {t.type}, expected F32 or F16")
        count = int(np.prod(t.dims))
        if count != n:
            raise ValueError(f"GGUF: {name} has {count} values, expected {n}")
        return self.floats(name, 1, n).reshape(n)

    def matrix(self, K: int, parts, row_order=None) -> ops.Q4Matrix:
        """Rows of tensors with [K, rows] dims, in order, as one matrix stored
        in `row_order` (stored row p = logical row row_order[p])."""
        infos = [self.info(n) for n, _ in parts]
        for (n, rows), t in zip(parts, infos):
            if t.dims != (K, rows):
                raise ValueError(f"GGUF: {n} is {list(t.dims)}, expected [{K}, {rows}]")
        N = sum(r for _, r in parts)
        types = {t.type for t in infos}
        src_rows = None if row_order is None else \
            torch.tensor(row_order, dtype=torch.int32, device=self.device)
        if types == {G.Q4_K} and K % 256 == 0:
            m = ops.Q4Matrix(N, K, L.LAYOUT_ROWGROUP, L.ZERO_F16, device=self.device)
            m.repack_q4_k(0, N, self._cat(parts), src_rows)
        elif G.Q4_0 in types:
            if types != {G.Q4_0}:
                raise ValueError(f"GGUF: {parts[0][0]} can't be combined with "
                                 f"{', '.join(n for n, _ in parts[1:])}")
            m = ops.Q4Matrix(N, K, L.LAYOUT_ROWGROUP, L.ZERO_8, device=self.device)
            m.repack_q4_0(0, N, self._cat(parts), src_rows)
        else:
            bad = [n for (n, _), t in zip(parts, infos) if t.type not in _EIGHT_BIT]
            if bad:
                raise ValueError(f"GGUF: {bad[0]} has tensor type {self.info(bad[0]).type}, "
                                 "which this loader doesn't take (Q4_0, Q8_0, Q4_1, Q4_K, "
                                 "Q5_K, Q6_K, F16, F32 do)")
            m = ops.Q4Matrix(N, K, L.LAYOUT_Q8, L.ZERO_8, device=self.device)
            if types == {G.Q8_0}:
                m.repack_q8_0(0, N, self._cat(parts), src_rows)
            elif G.Q8_0 in types:
                raise ValueError("GGUF: a matrix mixing Q8_0 with other types is not supported "
                                 "(its Q8_0 rows would be requantized)")
            else:
                vals = torch.cat([self.floats(n, r, K) for n, r in parts])
                if src_rows is not None:
                    vals = vals[src_rows.long()].contiguous()
                m.quantize_q8(0, N, vals)
        m.row_order = row_order
        return m

    def _cat(self, parts) -> torch.Tensor:
        data = [self.bytes(n) for n, _ in parts]
        return data[0] if len(data) == 1 else torch.cat(data)

    def embedding(self, D: int, vocab: int) -> ops.Q4Matrix:
        t = self.info("token_embd.weight")
        if t.type == G.Q6_K:
            m = ops.Q4Matrix.from_q6_k(self.bytes(t.name), vocab, D)
        elif t.type == G.Q4_0:
            m = ops.Q4Matrix.from_q4_0(self.bytes(t.name), vocab, D)
        elif t.type == G.Q8_0:
            m = ops.Q4Matrix.from_q8_0(self.bytes(t.name), vocab, D)
        else:
            m = ops.Q4Matrix.from_floats_q8(self.floats(t.name, vocab, D))
        m.row_order = None
        return m


def load_gguf(path: str, device="cuda", name: str | None = None) -> E.Weights:
    """The engine's weights from an LFM2 GGUF file."""
    with G.GgufFile(path) as f:
        s = gguf_shape(f, name)
        up = _Uploader(f, device)
        D, F, hd = s.hidden, s.intermediate, s.head_dim
        w = E.Weights.blank(s, device=device)
        for i in range(s.layers):
            blk = f"blk.{i}."
            lw = {"op_norm": up.vector(blk + "attn_norm.weight", D),
                  "ffn_norm": up.vector(blk + "ffn_norm.weight", D),
                  "gate_up": up.matrix(D, [(blk + "ffn_gate.weight", F),
                                           (blk + "ffn_up.weight", F)],
                                       E.gate_up_row_order(F)),
                  "down": up.matrix(F, [(blk + "ffn_down.weight", D)])}
            if s.layer_type(i) == "conv":
                lw["in_proj"] = up.matrix(D, [(blk + "shortconv.in_proj.weight", 3 * D)])
                lw["out_proj"] = up.matrix(D, [(blk + "shortconv.out_proj.weight", D)])
                conv = up.info(blk + "shortconv.conv.weight")
                # ggml [width, channels]: each channel's taps contiguous, oldest first
                if conv.dims != (s.conv_kernel, D):
                    raise ValueError(f"GGUF: {conv.name} is {list(conv.dims)}")
                lw["taps"] = up.vector(conv.name, D * s.conv_kernel).reshape(D, s.conv_kernel)
            else:
                kv = s.kv_heads * hd
                lw["qkv"] = up.matrix(D, [(blk + "attn_q.weight", s.heads * hd),
                                          (blk + "attn_k.weight", kv),
                                          (blk + "attn_v.weight", kv)],
                                      E.qkv_row_order(s) if s.rope_in_epilogue else None)
                lw["o"] = up.matrix(s.heads * hd, [(blk + "attn_output.weight", D)])
                lw["q_norm"] = up.vector(blk + "attn_q_norm.weight", hd)
                lw["k_norm"] = up.vector(blk + "attn_k_norm.weight", hd)
            w.layers.append(lw)
        w.final_norm = up.vector("token_embd_norm.weight", D)
        w.embedding = up.embedding(D, s.vocab)
        torch.cuda.synchronize()
    return w
