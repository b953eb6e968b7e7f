"""Loads an LFM2 ONNX export (4-bit MatMulNBits projections with a
GatherBlockQuantized embedding, as onnxruntime-genai writes them, or a
float16 embedding read by a plain Gather with the LM head a MatMul over it
transposed, as transformers.js exports have it) into the engine's device
weights, as the reference's loadOnnx does (src/load-onnx.ts:119-447):

- the settings from config.json over the shapes the weights have
  (onnxConfig, :1333-1457);
- each layer's weights found by the graph's structure, not by initializer
  names (OnnxModel.layerPlan, :826-900): a projection is the MatMulNBits
  node under its module path; the conv in_proj's B, C and x rows are
  placed by following its Split to the convolution (bcxSegments,
  :1043-1080); the attention's rotary embedding is checked against the
  head layout the engine uses (checkRotary, :1109-1150);
- the final norm: the norm feeding the LM head (finalNorm, :1166-1180);
- the embedding, also the output head (embedding, :1191-1292): 4-bit rows
  kept as they are; 8-bit rows with zero points, or float rows,
  quantized to 8 bits, in chunks of rows.

Fused matrices are assembled from their parts on the host (rows copied in
the order the engine stores them) and repacked on the GPU
(wg_repack_nbits); a matrix with an 8-bit part is 8-bit as a whole, every
part dequantized and requantized there (wg_quantize_q8), as the reference
stores it (:189-251). Architectures outside the engine's path (Qwen3.5's
Gated DeltaNet, LFM3's attention gate, sliding-window or partial-RoPE
attention, an untied head) are refused with a message.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np
import torch

from . import engine as E
from . import lib as L
from . import ops
from .onnx import (FLOAT, FLOAT16, INT64, UINT8, NBits, OnnxFile, OnnxModel, OnnxNode,
                   OnnxTensor, check_shape, element_size, half_bytes, nbits8_floats,
                   tensor_bytes)


@dataclass
class Segment:
    """Rows [start, start + rows) of a weight."""
    start: int
    rows: int


@dataclass
class LayerPlan:
    """What one layer reads (LayerPlan, src/load-onnx.ts:689-716)."""
    type: str                       # "conv" | "full_attention"
    norms: list                     # operator norm, ffn norm
    matrices: dict                  # role -> NBits
    extra: list                     # conv kernel, or q and k norms
    bcx: list = field(default_factory=list)   # in_proj's B, C, x segments
    rope_sin: OnnxTensor | None = None         # a RotaryEmbedding's sin cache


@dataclass
class Embedding:
    """The embedding as the graph has it (OnnxEmbedding, src/load-onnx.ts:1294-1303)."""
    kind: str                       # "q4" | "q8" | "float"
    N: int
    quant: OnnxTensor | None = None
    scales: OnnxTensor | None = None
    zp: OnnxTensor | None = None
    weight: OnnxTensor | None = None


def _int64s(t: OnnxTensor) -> list:
    """An int64 tensor's values (onnxInt64s, src/onnx.ts:329-345)."""
    if t.int64_data is not None:
        return [int(v) for v in t.int64_data]
    if t.raw is not None and t.data_type == INT64:
        return [int(v) for v in np.frombuffer(np.ascontiguousarray(t.raw).tobytes(), "<i8")]
    raise ValueError(f"ONNX: {t.name} has no int64 values")


class _Graph:
    """The structural lookups of OnnxModel (src/load-onnx.ts:717-1290)
    that the text loader needs, over an OnnxModel."""

    def __init__(self, model: OnnxModel):
        self.m = model
        self.nodes = model.file.nodes

    def consumers_of(self, name: str) -> list:
        return self.m.consumers.get(name, [])

    def producer_of(self, name: str) -> OnnxNode | None:
        return self.m.producers.get(name)

    def layer_plan(self, i: int, type_: str, cfg: dict) -> LayerPlan:
        """layerPlan for LFM2 (src/load-onnx.ts:826-900)."""
        m, D = self.m, cfg["hidden"]
        p = f"model.layers.{i}."
        for opt in ("post_operator_layernorm", "post_ffn_layernorm"):
            if m.has(f"{p}{opt}.weight"):
                raise ValueError(f"ONNX: layer {i} has a {opt} (sandwich norms are not on this "
                                 "engine's path)")
        norms = [m.init(f"{p}operator_layernorm.weight"), m.init(f"{p}ffn_layernorm.weight")]

        def w(name):
            return m.nbits(f"/model/layers.{i}/{name}/")
        mlp = {"gate": w("mlp/gate_proj"), "up": w("mlp/up_proj"), "down": w("mlp/down_proj")}
        if type_ == "conv":
            in_proj, out_proj = w("conv/in_proj"), w("conv/out_proj")
            if (in_proj.N, in_proj.K, out_proj.N, out_proj.K) != (3 * D, D, D, D):
                raise ValueError(f"ONNX: layer {i} conv projections have unexpected shapes")
            kernel = m.init(f"{p}conv.conv.weight")
            check_shape(kernel, kernel.data_type, D * cfg["conv_kernel"])
            if kernel.dims[0] != D or kernel.dims[-1] != cfg["conv_kernel"]:
                raise ValueError(f"ONNX: {kernel.name} is {list(kernel.dims)}")
            return LayerPlan(type_, norms, {"in_proj": in_proj, "out_proj": out_proj, **mlp},
                             [kernel], bcx=self.bcx_segments(in_proj, D))
        if m.has_nbits(f"/model/layers.{i}/attn/gate_proj/"):
            raise ValueError(f"ONNX: layer {i}'s attention has an output gate (not on this "
                             "engine's path)")
        q, k, v, o = w("attn/q_proj"), w("attn/k_proj"), w("attn/v_proj"), w("attn/o_proj")
        if q.N != cfg["heads"] * cfg["head_dim"]:
            raise ValueError(f"ONNX: layer {i} q_proj has {q.N} rows, expected "
                             f"{cfg['heads'] * cfg['head_dim']}")
        extra = [m.init(f"{p}attn.q_norm.layernorm.weight"),
                 m.init(f"{p}attn.k_norm.layernorm.weight")]
        sin = self.check_rotary(i, cfg)
        return LayerPlan(type_, norms, {"q": q, "k": k, "v": v, "o": o, **mlp}, extra,
                         rope_sin=sin)

    def split_sizes(self, split: OnnxNode) -> list:
        """A Split's part sizes, from its input or attribute (splitSizes,
        src/load-onnx.ts:995-1008)."""
        a = split.attributes.get("axis")
        axis = a.i if a is not None else 0
        if axis not in (-1, 2, 1):
            raise ValueError(f"ONNX: {split.name} doesn't split the channels axis")
        if len(split.inputs) > 1 and split.inputs[1]:
            return _int64s(self.m.constant(split.inputs[1]))
        attr = split.attributes.get("split")
        if attr is not None and attr.ints:
            return list(attr.ints)
        raise ValueError(f"ONNX: {split.name} has no split sizes")

    def feeds(self, name: str, node: OnnxNode) -> bool:
        """`name` reaches `node` through at most one Mul, then at most one
        Concat (the export prepends the past conv state): feeds,
        src/load-onnx.ts:1082-1099."""
        if name in node.inputs:
            return True
        for n in self.consumers_of(name):
            if n.op_type != "Mul":
                continue
            for o in n.outputs:
                if o in node.inputs:
                    return True
                for c in self.consumers_of(o):
                    if c.op_type == "Concat" and any(x in node.inputs for x in c.outputs):
                        return True
        return False

    def bcx_segments(self, in_proj: NBits, D: int) -> list:
        """in_proj's B, C, x rows (bcxSegments, src/load-onnx.ts:1043-1080):
        C is the Split output multiplied by the convolution's output; B and
        x are the two multiplied together before it, kept in the graph's
        order."""
        out = in_proj.node.outputs[0]
        transposed = next((n for n in self.consumers_of(out) if n.op_type == "Transpose"), None)
        names = [out] + (list(transposed.outputs) if transposed else [])
        split = next((n for name in names for n in self.consumers_of(name)
                      if n.op_type == "Split"), None)
        if split is None:
            raise ValueError(f"ONNX: {in_proj.node.name} is not split into B, C, x")
        sizes = self.split_sizes(split)
        if len(sizes) != 3 or any(s != D for s in sizes):
            raise ValueError(f"ONNX: {split.name} sizes {sizes}")
        conv = next((n for n in self.nodes
                     if (n.op_type.startswith("CausalConv") or n.op_type == "Conv")
                     and any(self.feeds(o, n) for o in split.outputs)), None)
        if conv is None:
            raise ValueError(f"ONNX: no convolution after {split.name}")
        conv_out = {conv.outputs[0]}
        for n in self.consumers_of(conv.outputs[0]):
            if n.op_type == "Slice":
                conv_out.add(n.outputs[0])
        c_index = next((j for j, o in enumerate(split.outputs)
                        if any(n.op_type == "Mul" and any(x in conv_out for x in n.inputs)
                               for n in self.consumers_of(o))), -1)
        if c_index < 0:
            raise ValueError(f"ONNX: can't find C after {conv.name}")
        others = [j for j in range(3) if j != c_index]
        return [Segment(j * D, D) for j in (others[0], c_index, others[1])]

    def check_rotary(self, i: int, cfg: dict) -> OnnxTensor | None:
        """How layer i rotates q and k (checkRotary, src/load-onnx.ts:
        1109-1150): by GroupQueryAttention itself, non-interleaved, over
        every dim of a head (a cos cache of head_dim / 2 frequencies); or by
        two RotaryEmbedding nodes before it over all of each head (HF's
        layout, the same as the engine's when every dim rotates): their sin
        cache is returned."""
        prefix = f"/model/layers.{i}/"
        gqa = next((n for n in self.nodes
                    if n.op_type == "GroupQueryAttention" and n.name.startswith(prefix)), None)
        if gqa is None:
            raise ValueError(f"ONNX: no GroupQueryAttention in layer {i}")
        hd = cfg["head_dim"]

        def attr(n, key, default=0):
            a = n.attributes.get(key)
            return a.i if a is not None else default
        if attr(gqa, "do_rotary") != 1:
            rotary = [n for n in self.nodes
                      if n.op_type == "RotaryEmbedding" and n.name.startswith(prefix + "attn/")]
            sin = rotary[0].inputs[3] if rotary and len(rotary[0].inputs) > 3 else ""
            cache = self.m.file.initializers.get(sin) if sin else None
            if (len(rotary) != 2 or cache is None or len(cache.dims) != 2 or
                    cache.dims[1] * 2 != hd or
                    any(n.inputs[3] != sin or attr(n, "interleaved") != 0 or
                        attr(n, "rotary_embedding_dim") != 0 for n in rotary) or
                    not all(any(n.outputs[0] == x for n in rotary) for x in gqa.inputs[:2])):
                raise ValueError(f"ONNX: layer {i}'s attention doesn't rotate q and k over each "
                                 "head, non-interleaved")
            return cache
        if attr(gqa, "rotary_interleaved") != 0:
            raise ValueError(f"ONNX: {gqa.name} doesn't apply non-interleaved rotary embeddings")
        cos = gqa.inputs[7] if len(gqa.inputs) > 7 else ""
        t = self.m.file.initializers.get(cos) if cos else None
        rotated = t.dims[-1] * 2 if t is not None and t.dims else -1
        if rotated != hd:
            raise ValueError(f"ONNX: layer {i} rotates {rotated} dims per head, expected {hd} "
                             "(partial RoPE is not on this engine's path)")
        return None

    def lm_head(self) -> OnnxNode:
        """The MatMulNBits or MatMul node under /lm_head/, or the one that
        writes `logits` (through a Cast): lmHead, src/load-onnx.ts:1149-1164."""
        def is_head(n):
            return n is not None and n.op_type in ("MatMulNBits", "MatMul")
        heads = [n for n in self.nodes if n.name.startswith("/lm_head/") and is_head(n)]
        if len(heads) == 1:
            return heads[0]
        if not heads:
            node = self.producer_of("logits")
            if node is not None and node.op_type == "Cast":
                node = self.producer_of(node.inputs[0])
            if is_head(node):
                return node
        raise ValueError(f"ONNX: {len(heads)} LM head MatMul nodes")

    def final_norm(self) -> OnnxTensor:
        """The norm feeding the LM head (finalNorm, src/load-onnx.ts:1166-1180)."""
        name = self.lm_head().inputs[0]
        for _ in range(8):
            node = self.producer_of(name) if name else None
            if node is None:
                break
            if node.op_type == "SimplifiedLayerNormalization":
                return self.m.init(node.inputs[1])
            if node.op_type == "SkipSimplifiedLayerNormalization":
                return self.m.init(node.inputs[2])
            name = node.inputs[0]
        raise ValueError("ONNX: can't find the final norm")

    def embedding(self, D: int) -> Embedding:
        """The embedding, also the output head (embedding,
        src/load-onnx.ts:1181-1292)."""
        m = self.m
        gather = next((n for n in self.nodes if n.op_type == "GatherBlockQuantized"), None)
        if gather is not None:
            def attr(key):
                a = gather.attributes.get(key)
                return None if a is None else a.i
            bits = attr("bits")
            if bits not in (4, 8) or attr("block_size") != 32 or attr("quantize_axis") != 1 or \
                    (attr("gather_axis") or 0) != 0:
                raise ValueError(f"ONNX: {gather.name} is not 4-bit or 8-bit, block 32, "
                                 "quantized along rows")
            reshaped = None if m.has(gather.inputs[0]) else self.producer_of(gather.inputs[0])
            quant = m.init(reshaped.inputs[0] if reshaped is not None and
                           reshaped.op_type == "Reshape" else gather.inputs[0])
            scales = m.init(gather.inputs[2])
            zp = m.init(gather.inputs[3]) if len(gather.inputs) > 3 and gather.inputs[3] else None
            N = quant.dims[0]
            check_shape(quant, UINT8, N * D * bits // 8)
            check_shape(scales, FLOAT16, N * D // 32)
            if zp is not None:
                check_shape(zp, UINT8, N * -(-D // 64) if bits == 4 else N * D // 32)
            head = self.lm_head()
            if head.op_type == "MatMul":
                raise ValueError("ONNX: the LM head is a float MatMul with its own weights, not "
                                 "the embedding (only a tied head is supported)")
            if bits == 8:
                if head.inputs[1] != quant.name:
                    raise ValueError(f"ONNX: the LM head isn't {quant.name} (only a tied head "
                                     "is supported)")
                return Embedding("q8", N, quant, scales, zp)
            return Embedding("q4", N, quant, scales, zp)
        fg = next((n for n in self.nodes if n.op_type == "Gather" and len(n.inputs) > 1 and
                   n.inputs[1] == "input_ids" and m.has(n.inputs[0])), None)
        if fg is not None:
            weight = m.init(fg.inputs[0])
            if weight.data_type not in (FLOAT16, FLOAT):
                raise ValueError(f"ONNX: {weight.name} has data type {weight.data_type}, "
                                 "expected float16 or float")
            if len(weight.dims) != 2 or weight.dims[1] != D:
                raise ValueError(f"ONNX: {weight.name} is {list(weight.dims)}")
            head = self.lm_head()
            tr = self.producer_of(head.inputs[1]) if len(head.inputs) > 1 else None
            perm = tr.attributes.get("perm").ints if tr is not None and \
                tr.attributes.get("perm") is not None else None
            if head.op_type != "MatMul" or tr is None or tr.op_type != "Transpose" or \
                    tr.inputs[0] != weight.name or (perm and list(perm) != [1, 0]):
                raise ValueError(f"ONNX: the LM head isn't {weight.name} (only a tied head is "
                                 "supported)")
            return Embedding("float", weight.dims[0], weight=weight)
        head = self.lm_head()
        tr = self.producer_of(head.inputs[1]) if head.op_type == "MatMul" else None
        if tr is not None and tr.op_type == "Transpose" and m.has(tr.inputs[0]):
            weight = m.init(tr.inputs[0])
            perm = tr.attributes.get("perm").ints if tr.attributes.get("perm") else None
            if weight.data_type not in (FLOAT16, FLOAT):
                raise ValueError(f"ONNX: {weight.name} has data type {weight.data_type}, "
                                 "expected float16 or float")
            if len(weight.dims) != 2 or weight.dims[1] != D or (perm and list(perm) != [1, 0]):
                raise ValueError(f"ONNX: the LM head's {weight.name} is {list(weight.dims)}, not "
                                 "the embedding transposed")
            return Embedding("float", weight.dims[0], weight=weight)
        if m.has_nbits("/lm_head/"):
            h = m.nbits("/lm_head/")
            if h.K != D:
                raise ValueError(f"ONNX: lm_head has K {h.K}")
            return Embedding("q4", h.N, h.quant, h.scales, h.zp)
        raise ValueError("ONNX: no embedding the loader reads")


def onnx_config(config: dict, model: OnnxModel) -> dict:
    """The model's settings: config.json over the shapes the weights have
    (onnxConfig, src/load-onnx.ts:1333-1457), for the layer types the
    engine runs (conv and full attention)."""
    if not isinstance(config, dict):
        raise ValueError("ONNX: config must be the parsed config.json")
    c = config.get("text_config") if isinstance(config.get("text_config"), dict) else config

    def num(key, fallback=None):
        v = c.get(key, fallback)
        if isinstance(v, bool) or not isinstance(v, (int, float)):
            raise ValueError(f"config.json: {key} is missing")
        return v
    layers = int(num("num_hidden_layers"))
    hidden = int(num("hidden_size"))
    heads = int(num("num_attention_heads"))
    head_dim = int(num("head_dim", hidden // heads))
    if isinstance(c.get("layer_types"), list):
        types = []
        for t in c["layer_types"]:
            if t not in ("conv", "full_attention", "sliding_attention", "linear_attention"):
                raise ValueError(f"config.json: unknown layer type {t}")
            types.append(t)
    elif isinstance(c.get("full_attn_idxs"), list):
        full = set(c["full_attn_idxs"])
        types = ["full_attention" if i in full else "conv" for i in range(layers)]
    else:
        raise ValueError("config.json: no layer_types")
    if len(types) != layers:
        raise ValueError("config.json: layer_types doesn't match num_hidden_layers")
    bad = sorted({t for t in types if t not in ("conv", "full_attention")})
    if bad:
        raise ValueError(f"ONNX: {', '.join(bad)} layers are not on this engine's path")
    if "full_attention" not in types:
        raise ValueError("ONNX: no attention layer")
    rope = c.get("rope_parameters") or {}
    full_rope = rope.get("full_attention", rope) if isinstance(rope, dict) else {}
    if full_rope.get("rope_type") not in (None, "default"):
        raise ValueError(f"config.json: rope type {full_rope['rope_type']} is not supported")
    theta = full_rope.get("rope_theta", None)
    theta = float(theta if theta is not None else num("rope_theta"))
    rotated = round(full_rope.get("partial_rotary_factor", 1) * head_dim)
    if rotated != head_dim:
        raise ValueError("ONNX: partial RoPE is not on this engine's path")
    if num("sliding_window", 0) > 0:
        raise ValueError("ONNX: sliding-window attention is not on this engine's path")
    inter = model.nbits("/model/layers.0/mlp/gate_proj/").N
    if c.get("intermediate_size") is not None and c["intermediate_size"] != inter and \
            not c.get("block_auto_adjust_ff_dim"):
        raise ValueError(f"config.json: intermediate_size {c['intermediate_size']} but the "
                         f"weights have {inter}")
    emb = _Graph(model).embedding(hidden)
    if c.get("vocab_size") is not None and c["vocab_size"] != emb.N:
        raise ValueError(f"config.json: vocab_size {c['vocab_size']} but the embedding has "
                         f"{emb.N} rows")

    def token(key):
        v = c.get(key)
        if isinstance(v, list) and v and isinstance(v[0], int):
            return v[0]
        return v if isinstance(v, int) and not isinstance(v, bool) else -1
    return {"layers": layers, "hidden": hidden, "heads": heads,
            "kv_heads": int(num("num_key_value_heads", heads)), "head_dim": head_dim,
            "intermediate": inter, "vocab": emb.N, "layer_types": types,
            "context_length": int(num("max_position_embeddings", 8192)), "rope_theta": theta,
            "eps": float(num("norm_eps", num("rms_norm_eps", 1e-5))),
            "conv_kernel": int(num("conv_L_cache")), "bos": token("bos_token_id"),
            "eos": token("eos_token_id"), "pad": token("pad_token_id")}


@dataclass
class OnnxPlan:
    """Everything the load reads, checked against the layout (planOnnx,
    src/load-onnx.ts:557-668)."""
    config: dict
    shape: E.ModelShape
    layers: list
    final_norm: OnnxTensor
    embedding: Embedding
    reads: list                     # (tensor name, location or "", offset, length)


def plan_onnx(model: OnnxModel, config: dict, name: str | None = None,
              chunk_rows: int = 2048) -> OnnxPlan:
    """Checks the graph against what the loader takes and lists every read
    the load makes, in order, without reading the external data."""
    cfg = onnx_config(config, model)
    g = _Graph(model)
    D, F = cfg["hidden"], cfg["intermediate"]
    kv = cfg["kv_heads"] * cfg["head_dim"]
    plans = [g.layer_plan(i, t, cfg) for i, t in enumerate(cfg["layer_types"])]
    for i, lp in enumerate(plans):
        mm = lp.matrices
        if lp.type != "conv" and (mm["k"].N != kv or mm["v"].N != kv):
            raise ValueError(f"ONNX: layer {i} k/v projections have {mm['k'].N}/{mm['v'].N} rows")
        if mm["gate"].N != F or mm["up"].N != F or mm["down"].K != F:
            raise ValueError(f"ONNX: layer {i} MLP shapes don't match")
        for w in mm.values():
            if w.K % 32:
                raise ValueError(f"ONNX: {w.name} has K {w.K}, not a multiple of 32")
    reads = []

    def want(t):
        if t is None:
            return
        n = tensor_bytes(t)
        if t.external is None:
            if t.raw is None:
                raise ValueError(f"ONNX: {t.name} has no data")
            if t.raw.size != n:
                raise ValueError(f"ONNX: {t.name} has {t.raw.size} bytes, expected {n}")
            reads.append((t.name, "", 0, n))
            return
        if t.external[2] != n:
            raise ValueError(f"ONNX: {t.name} has {t.external[2]} bytes, expected {n}")
        reads.append((t.name, t.external[0], t.external[1], n))
    for lp in plans:
        for t in lp.norms:
            want(t)
        for role, w in lp.matrices.items():
            if role not in ("gate", "up", "down"):
                for t in (w.quant, w.scales, w.zp):
                    want(t)
        for t in lp.extra:
            want(t)
        for role in ("gate", "up", "down"):
            w = lp.matrices[role]
            for t in (w.quant, w.scales, w.zp):
                want(t)
    final = g.final_norm()
    want(final)
    emb = g.embedding(D)
    if emb.N % 4:
        raise ValueError(f"ONNX: the embedding has {emb.N} rows, not a multiple of 4")
    if chunk_rows < emb.N and chunk_rows % 4:
        raise ValueError(f"ONNX: embedding chunks of {chunk_rows} rows aren't a multiple of 4")
    blocks = D // 32
    for r in range(0, emb.N, chunk_rows):
        rows = min(chunk_rows, emb.N - r)

        def ext(t, row_bytes):
            if t.external is None:
                raise ValueError(f"ONNX: {t.name} is expected in the external data file")
            if t.external[2] != tensor_bytes(t) or row_bytes * emb.N != tensor_bytes(t):
                raise ValueError(f"ONNX: {t.name} has {t.external[2]} bytes, expected "
                                 f"{row_bytes * emb.N}")
            reads.append((t.name, t.external[0], t.external[1] + r * row_bytes,
                          rows * row_bytes))
        if emb.kind == "float":
            ext(emb.weight, D * int(element_size(emb.weight.data_type)))
            continue
        ext(emb.quant, blocks * (32 if emb.kind == "q8" else 16))
        ext(emb.scales, blocks * 2)
        if emb.zp is not None:
            ext(emb.zp, blocks if emb.kind == "q8" else -(-blocks // 2))
    types = cfg["layer_types"]
    # the model's folder names it (an export's graph is "main_graph" or the like)
    label = name or os.path.basename(os.path.dirname(os.path.abspath(model.file.path))) or \
        model.file.name
    shape = E.ModelShape(label, D, cfg["layers"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                         F, emb.N, "nbits", rope_theta=cfg["rope_theta"], eps=cfg["eps"],
                         qk_norm=True, conv_kernel=cfg["conv_kernel"],
                         conv_layers=tuple(i for i, t in enumerate(types) if t == "conv"),
                         embed_fmt="nbits" if emb.kind == "q4" else "q8",
                         extra={k: cfg[k] for k in ("context_length", "bos", "eos", "pad")})
    return OnnxPlan(cfg, shape, plans, final, emb, reads)


def check_onnx(path: str, config: dict) -> list:
    """The external data files a graph's weights are in, reading only the
    graph; raises the loader's own error where the loader doesn't take it
    (checkOnnxGraph, src/load-onnx.ts:662-681)."""
    with OnnxFile(path) as f:
        return check_model(OnnxModel(f), config)


def check_model(model: OnnxModel, config: dict) -> list:
    files = []
    for _, loc, _, _ in plan_onnx(model, config, chunk_rows=1 << 62).reads:
        if loc and loc not in files:
            files.append(loc)
    return files


class _Uploader:
    def __init__(self, f: OnnxFile, device):
        self.f, self.device = f, device

    def floats(self, t: OnnxTensor, n: int) -> torch.Tensor:
        """A float16 or float32 tensor as float32 on the device (the
        loader's floats, src/load-onnx.ts:146-171)."""
        data = np.ascontiguousarray(self.f.data(t))
        if t.data_type == FLOAT16:
            v = data.view(np.float16).astype(np.float32)
        elif t.data_type == FLOAT:
            v = data.view(np.float32).copy()
        else:
            raise ValueError(f"ONNX: {t.name} has data type {t.data_type}, expected float16 or "
                             "float")
        if v.size != n:
            raise ValueError(f"ONNX: {t.name} has {v.size} values, expected {n}")
        return torch.from_numpy(v).to(self.device)

    def _dev(self, a: np.ndarray) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(a).copy()).to(self.device)

    def _rows4(self, w: NBits, seg: Segment, with_zeros: bool):
        """A 4-bit weight's rows as MatMulNBits stores them: quants
        [rows][K/32][16], half scales [rows][K/32], zero points
        [rows][ceil(K/64)] (8s where the weight has none)."""
        blocks = w.K // 32
        zrow = -(-blocks // 2)
        rows = slice(seg.start, seg.start + seg.rows)
        q = np.asarray(self.f.data(w.quant)).reshape(w.N, blocks * 16)[rows]
        s = half_bytes(w.scales, self.f.data(w.scales)).reshape(w.N, blocks)[rows]
        z = None
        if with_zeros:
            z = (np.asarray(self.f.data(w.zp)).reshape(w.N, zrow)[rows] if w.zp is not None
                 else np.full((seg.rows, zrow), 0x88, np.uint8))
        return q, s, z

    def _floats_of(self, w: NBits, seg: Segment) -> torch.Tensor:
        """A weight's rows as float32 on the device, scale * (q - zero
        point) (dequantizeNBitsRow, src/load-onnx.ts:471-501): 8-bit rows on
        the host, exact; 4-bit rows repacked and dequantized on the GPU."""
        if w.bits == 8:
            rows = slice(seg.start, seg.start + seg.rows)
            blocks = w.K // 32
            quant = np.asarray(self.f.data(w.quant)).reshape(w.N, w.K)[rows]
            scales = half_bytes(w.scales, self.f.data(w.scales)).reshape(w.N, blocks)[rows]
            zp = np.asarray(self.f.data(w.zp)).reshape(w.N, blocks)[rows] \
                if w.zp is not None else None
            part = NBits(w.name, w.node, seg.rows, w.K, 8, 32, w.quant, w.scales, w.zp)
            return self._dev(nbits8_floats(part, quant, scales, zp))
        q, s, z = self._rows4(w, seg, w.zp is not None)
        m = ops.Q4Matrix.from_nbits(self._dev(q), self._dev(s.view(np.int16)),
                                    None if z is None else self._dev(z), seg.rows, w.K)
        return m.dequant()

    def matrix(self, parts, row_order=None) -> ops.Q4Matrix:
        """The segments of `parts` ([(NBits, [Segment ...]) ...]), in order,
        as the rows of one matrix stored in `row_order` (stored row p =
        logical row row_order[p]): the reference's matrix(),
        src/load-onnx.ts:189-251."""
        K = parts[0][0].K
        N = 0
        for w, segs in parts:
            if w.K != K:
                raise ValueError(f"ONNX: {w.name} has K {w.K}, expected {K}")
            for s in segs:
                if s.start + s.rows > w.N:
                    raise ValueError(f"ONNX: rows {s.start}..{s.start + s.rows} are outside "
                                     f"{w.name}")
                N += s.rows
        if N % 4:
            raise ValueError(f"ONNX: {N} rows isn't a multiple of 4")
        src_rows = None if row_order is None else \
            torch.tensor(row_order, dtype=torch.int32, device=self.device)
        if any(w.bits == 8 for w, _ in parts):
            vals = torch.cat([self._floats_of(w, s) for w, segs in parts for s in segs])
            if src_rows is not None:
                vals = vals[src_rows.long()].contiguous()
            m = ops.Q4Matrix.from_floats_q8(vals)
        else:
            with_zeros = any(w.zp is not None for w, _ in parts)
            pieces = [self._rows4(w, s, with_zeros) for w, segs in parts for s in segs]
            q = np.concatenate([p[0] for p in pieces])
            sc = np.concatenate([p[1] for p in pieces])
            z = np.concatenate([p[2] for p in pieces]) if with_zeros else None
            m = ops.Q4Matrix.from_nbits(self._dev(q), self._dev(sc.view(np.int16)),
                                        None if z is None else self._dev(z), N, K,
                                        src_rows=src_rows)
        m.row_order = row_order
        return m

    def embedding(self, emb: Embedding, D: int, chunk_rows: int = 4096) -> ops.Q4Matrix:
        """The embedding rows (src/load-onnx.ts:384-446): 4-bit ones kept;
        8-bit ones with zero points, and float ones, quantized to 8 bits
        per block of 32 a chunk of rows at a time (the same values as the
        whole matrix at once: quantizeQ8 works per block)."""
        N = emb.N
        if emb.kind == "q4":
            w = NBits("embedding", None, N, D, 4, 32, emb.quant, emb.scales, emb.zp)
            m = self.matrix([(w, [Segment(0, N)])])
            m.row_order = None
            return m
        m = ops.Q4Matrix(N, D, L.LAYOUT_Q8, L.ZERO_8, device=self.device)
        if emb.kind == "q8":
            blocks = D // 32
            quant = np.asarray(self.f.data(emb.quant)).reshape(N, D)
            scales = half_bytes(emb.scales, self.f.data(emb.scales)).reshape(N, blocks)
            zp = np.asarray(self.f.data(emb.zp)).reshape(N, blocks) if emb.zp is not None \
                else None
        else:
            dt = emb.weight.data_type
            if dt not in (FLOAT16, FLOAT):
                raise ValueError(f"ONNX: embedding data type {dt}, expected float16 or float")
            rows_all = np.asarray(self.f.data(emb.weight)).view(
                np.float16 if dt == FLOAT16 else np.float32).reshape(N, D)
        for r in range(0, N, chunk_rows):
            n = min(chunk_rows, N - r)
            if emb.kind == "q8":
                part = NBits("embedding", None, n, D, 8, 32, emb.quant, emb.scales, emb.zp)
                vals = self._dev(nbits8_floats(part, quant[r:r + n], scales[r:r + n],
                                               None if zp is None else zp[r:r + n]))
            else:
                vals = self._dev(rows_all[r:r + n]).float()
            m.quantize_q8(r, n, vals)
        m.row_order = None
        return m


def read_config(path: str) -> dict:
    """config.json beside a model file."""
    with open(os.path.join(os.path.dirname(os.path.abspath(path)), "config.json")) as fh:
        return json.load(fh)


def load_onnx(path: str, config: dict | None = None, device="cuda",
              name: str | None = None) -> E.Weights:
    """The engine's weights from an LFM2 ONNX export (the graph at `path`,
    its data files beside it; config.json beside it unless given)."""
    cfg_json = read_config(path) if config is None else config
    with OnnxFile(path) as f:
        plan = plan_onnx(OnnxModel(f), cfg_json, name)
        s = plan.shape
        D, F, hd = s.hidden, s.intermediate, s.head_dim
        up = _Uploader(f, device)
        w = E.Weights.blank(s, device=device)
        whole = lambda nb: (nb, [Segment(0, nb.N)])  # noqa: E731
        for i, lp in enumerate(plan.layers):
            mm = lp.matrices
            lw = {"op_norm": up.floats(lp.norms[0], D), "ffn_norm": up.floats(lp.norms[1], D)}
            if lp.type == "conv":
                lw["in_proj"] = up.matrix([(mm["in_proj"], lp.bcx)])
                lw["out_proj"] = up.matrix([whole(mm["out_proj"])])
                # [channels, 1, width]: each channel's taps contiguous, oldest first
                lw["taps"] = up.floats(lp.extra[0], D * s.conv_kernel).reshape(
                    D, s.conv_kernel).contiguous()
            else:
                lw["qkv"] = up.matrix([whole(mm["q"]), whole(mm["k"]), whole(mm["v"])],
                                      E.qkv_row_order(s) if s.rope_in_epilogue else None)
                lw["o"] = up.matrix([whole(mm["o"])])
                lw["q_norm"] = up.floats(lp.extra[0], hd)
                lw["k_norm"] = up.floats(lp.extra[1], hd)
            lw["gate_up"] = up.matrix([whole(mm["gate"]), whole(mm["up"])],
                                      E.gate_up_row_order(F))
            lw["down"] = up.matrix([whole(mm["down"])])
            w.layers.append(lw)
        w.final_norm = up.floats(plan.final_norm, D)
        w.embedding = up.embedding(plan.embedding, D)
        torch.cuda.synchronize()
    return w
