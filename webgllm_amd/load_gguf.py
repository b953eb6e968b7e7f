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
    """A float32 metadata value as the decimal it was written from (7
    significant digits: 1e-5, not 9.9999997e-6), as the reference reads
    them (src/load-gguf.ts:594-597)."""
    return float(f"{v:.7g}")


# The LFM2 metadata the engine's shape is made of: (field, key under the
# architecture's prefix, how to read it, default). A key is looked up bare
# first, then under "<arch>." (the format lets writers put either). A
# default of _NEEDED makes the key required. Which keys exist is the
# format (llama.cpp's GGUF writer for LFM2); the table is this loader's.
_NEEDED = object()
_SCHEMA = (
    ("layers", "block_count", "int", _NEEDED),
    ("hidden", "embedding_length", "int", _NEEDED),
    ("heads", "attention.head_count", "int", _NEEDED),
    ("kv", "attention.head_count_kv", "per-layer", None),
    ("head_dim", "attention.key_length", "int", None),
    ("rope_dims", "rope.dimension_count", "int", None),
    ("theta", "rope.freq_base", "decimal", _NEEDED),
    ("eps", "attention.layer_norm_rms_epsilon", "decimal", _NEEDED),
    ("conv_kernel", "shortconv.l_cache", "int", _NEEDED),
    ("context", "context_length", "int", 8192),
    ("window", "attention.sliding_window", "int", 0),
    ("window_pattern", "attention.sliding_window_pattern", "any", None),
    ("ffn", "feed_forward_length", "int", None),
)


def _read_schema(meta: dict, arch: str) -> dict:
    """The schema's fields from the metadata, each converted by its kind."""
    out = {}
    for field_, key, kind, default in _SCHEMA:
        value = meta.get(key, meta.get(f"{arch}.{key}"))
        if value is None:
            if default is _NEEDED:
                raise ValueError(f"GGUF metadata lacks {arch}.{key}, which the engine needs")
            out[field_] = default
            continue
        if kind == "any":
            out[field_] = value
        elif kind == "per-layer":
            out[field_] = [int(x) for x in value] if isinstance(value, list) else int(value)
        elif isinstance(value, bool) or not isinstance(value, (int, float)):
            raise ValueError(f"GGUF metadata {arch}.{key} holds {type(value).__name__} "
                             f"{value!r} where a number belongs")
        else:
            out[field_] = _f32_decimal(value) if kind == "decimal" else int(value)
    return out


def _lfm2_fields(f: G.GgufFile) -> dict:
    """The schema's fields of an LFM2 file, with the derived ones: kv per
    layer, head_dim, intermediate (from the first gate matrix when the
    metadata has no feed_forward_length) and vocab (the embedding's
    rows)."""
    meta = f.metadata
    arch = meta.get("general.architecture")
    if not isinstance(arch, str):
        raise ValueError("GGUF metadata names no general.architecture")
    if arch != "lfm2":
        why = {"lfm3": "gated attention and sandwich norms",
               "qwen35": "Gated DeltaNet layers"}.get(arch)
        raise ValueError(f"GGUF architecture {arch} is not one this engine runs"
                         + (f" ({why})" if why else "") + "; it runs lfm2")
    v = _read_schema(meta, arch)
    kv = v["kv"] if v["kv"] is not None else v["heads"]
    v["kv"] = list(kv) if isinstance(kv, list) else [kv] * v["layers"]
    if v["head_dim"] is None:
        v["head_dim"] = v["hidden"] // v["heads"]
    emb = f.tensors.get("token_embd.weight")
    v["emb"] = emb
    gate0 = f.tensors.get("blk.0.ffn_gate.weight")
    v["gate_rows"] = gate0.dims[1] if gate0 is not None else None
    if v["ffn"] is None:
        v["ffn"] = v["gate_rows"] if v["gate_rows"] is not None else -1
    v["arch"] = arch
    return v


# What the engine refuses, checked in order: (test over the fields and the
# file, message). The first that holds raises.
_REFUSALS = (
    (lambda v, f: "output.weight" in f.tensors,
     "GGUF file has its own output.weight: this engine ties the output head to the embedding"),
    (lambda v, f: len(v["kv"]) != v["layers"],
     "GGUF metadata gives {n_kv} KV head counts for {layers} layers"),
    (lambda v, f: v["window"] > 0 or isinstance(v["window_pattern"], list),
     "GGUF model uses sliding-window attention, which this engine does not run"),
    (lambda v, f: len({k for k in v["kv"] if k}) > 1,
     "GGUF model's attention layers differ in KV heads ({kv_set}); this engine needs one count"),
    (lambda v, f: not any(v["kv"]),
     "GGUF model has no attention layer (every KV head count is 0)"),
    (lambda v, f: (v["rope_dims"] not in (None, v["head_dim"])) or "rope_freqs.weight" in f.tensors,
     "GGUF model rotates part of each head (partial RoPE), which this engine does not run"),
    (lambda v, f: v["emb"] is None,
     "GGUF file has no token_embd.weight"),
    (lambda v, f: v["emb"].dims[0] != v["hidden"],
     "GGUF token_embd.weight rows are {emb_cols} wide; the model is {hidden} wide"),
    (lambda v, f: v["gate_rows"] is not None and v["gate_rows"] != v["ffn"],
     "GGUF metadata feed_forward_length {ffn} but blk.0.ffn_gate.weight has {gate_rows} rows"),
)


def gguf_shape(f: G.GgufFile, name: str | None = None) -> E.ModelShape:
    """The engine's shape of an LFM2 GGUF file (what ggufConfig,
    src/load-gguf.ts:600-752, reads for LFM2: short-conv layers where the
    KV head count is 0, q/k norms, the output head tied to the
    embedding)."""
    v = _lfm2_fields(f)
    for test, msg in _REFUSALS:
        if test(v, f):
            raise ValueError(msg.format(
                n_kv=len(v["kv"]), layers=v["layers"], kv_set=sorted({k for k in v["kv"] if k}),
                emb_cols=v["emb"].dims[0] if v["emb"] is not None else 0, hidden=v["hidden"],
                ffn=v["ffn"], gate_rows=v["gate_rows"]))
    label = name or str(f.metadata.get("general.name") or os.path.basename(f.path))
    return E.ModelShape(label, v["hidden"], v["layers"], v["heads"], max(v["kv"]),
                        v["head_dim"], v["ffn"], v["emb"].dims[1], "gguf",
                        rope_theta=v["theta"], eps=v["eps"], qk_norm=True,
                        conv_kernel=v["conv_kernel"],
                        conv_layers=tuple(i for i, k in enumerate(v["kv"]) if k == 0),
                        embed_fmt="gguf", extra={"context_length": v["context"]})


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
            # packQ4_K's quants with Q4_K's own scales and mins kept (0.5625
            # bytes a weight; dequant rebuilds packQ4_K's halves bit for bit)
            m = ops.Q4Matrix(N, K, L.LAYOUT_ROWGROUP, L.ZERO_Q4K, device=self.device)
            m.repack_q4_k(0, N, self._cat(parts), src_rows)
            m.prompt_desc()  # packQ4_K's halves for prompts and few-token batches
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
