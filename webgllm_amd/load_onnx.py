"""Loads an LFM2 ONNX export (4-bit MatMulNBits projections with a
GatherBlockQuantized embedding, as onnxruntime-genai writes them, or a
float16 embedding read by a plain Gather with the LM head a MatMul over it
transposed, as transformers.js exports have it) into the engine's device
weights: what the reference's loadOnnx takes (src/load-onnx.ts:119-447),
found this loader's own way.

- A walker over the graph's dataflow (_Flow: the nodes a value reaches
  downstream through given op types, the node that wrote it upstream)
  answers every structural question.
- One pass over the MatMulNBits nodes makes an inventory of the layer
  projections, keyed by module path from the node's name or, where an
  export renamed the node, from the weight it reads.
- Tables say what each layer kind reads (projections with their shapes
  in terms of the config), which embedding forms exist (tried in turn),
  which rotary layouts match the engine's RoPE, and which config.json
  fields the settings come from.
- The conv in_proj's B, C and x rows are placed by following its Split
  into the convolution: C is the part multiplied with the convolution's
  output. The GroupQueryAttention is the node the o projection reads.
- Every read the load makes is listed, and each tensor's size checked,
  before any data is read.

Fused matrices are assembled from their parts on the host (rows copied in
the order the engine stores them) and repacked on the GPU
(wg_repack_nbits); a matrix with an 8-bit part is 8-bit as a whole, every
part dequantized and requantized there (wg_quantize_q8), as the reference
stores it (:189-251). Architectures outside the engine's path (Qwen3.5's
Gated DeltaNet, LFM3's attention gate, sandwich norms, sliding-window or
partial-RoPE attention, an untied head) are refused with a message.
"""
from __future__ import annotations

import json
import os
import re
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


def _int64_values(t: OnnxTensor) -> list:
    """An int64 tensor's values, from its int64_data or its raw bytes."""
    if t.int64_data is not None:
        return [int(v) for v in t.int64_data]
    if t.raw is not None and t.data_type == INT64:
        return [int(v) for v in np.frombuffer(np.ascontiguousarray(t.raw).tobytes(), "<i8")]
    raise ValueError(f"ONNX tensor {t.name} carries no int64 values")


def _attr_int(node: OnnxNode, key: str, default=None):
    a = node.attributes.get(key)
    return default if a is None else int(a.i)


# ------------------------------------------------------------ the dataflow
class _Flow:
    """Walks the graph's dataflow: values to the nodes that read them
    (downstream) and to the node that wrote them (upstream)."""

    def __init__(self, model: OnnxModel):
        self.m = model

    def readers(self, value: str) -> list:
        return self.m.consumers.get(value, [])

    def writer(self, value: str) -> OnnxNode | None:
        return self.m.producers.get(value)

    def downstream(self, values, want, via=(), hops=1) -> list:
        """The nodes satisfying `want` that read `values`, or read a value
        written by a chain of at most `hops` nodes whose op types are in
        `via` (breadth first, each node once)."""
        found, seen = [], set()
        frontier = list(values)
        for depth in range(hops + 1):
            nxt = []
            for v in frontier:
                for n in self.readers(v):
                    if id(n) in seen:
                        continue
                    seen.add(id(n))
                    if want(n):
                        found.append(n)
                    elif depth < hops and n.op_type in via:
                        nxt.extend(n.outputs)
            frontier = nxt
        return found

    def upstream(self, value: str, want, via=None, hops=8) -> OnnxNode | None:
        """The first node satisfying `want` walking writers back from
        `value` along each node's first input, through at most `hops` nodes
        (of the op types in `via`, any when None)."""
        for _ in range(hops + 1):
            n = self.writer(value) if value else None
            if n is None:
                return None
            if want(n):
                return n
            if via is not None and n.op_type not in via:
                return None
            value = n.inputs[0] if n.inputs else ""
        return None


def _op(*types):
    return lambda n: n.op_type in types


def _is_conv(n: OnnxNode) -> bool:
    return n.op_type == "Conv" or n.op_type.startswith("CausalConv")


# ---------------------------------------------------- projections by module
# A projection is the MatMulNBits node of a module: its node name is the
# module path (/model/layers.3/attn/q_proj/...), or, where an export
# renames nodes, the weight it reads is the module path in the
# initializer spelling (model_layers_3_attn_q_proj_..., or dotted).
_BY_NODE = re.compile(r"^/model/layers\.(\d+)/(conv|attn|mlp)/(\w+?)_proj/")
_BY_WEIGHT = re.compile(r"^model_layers_(\d+)_(conv|attn|mlp)_([a-z]+)_proj_")


def _spelling(name: str) -> str:
    return re.sub(r"[^a-z0-9]+", "_", name.lower())


def _inventory(model: OnnxModel) -> dict:
    """Every layer projection of the graph in one pass: {(layer, block,
    proj): NBits} (block conv | attn | mlp; proj as in q for q_proj). Two
    nodes for one module is an error."""
    out = {}
    for n in model.file.nodes:
        if n.op_type != "MatMulNBits":
            continue
        hit = _BY_NODE.match(n.name)
        if hit is None and len(n.inputs) > 1 and model.has(n.inputs[1]):
            hit = _BY_WEIGHT.match(_spelling(n.inputs[1]))
        if hit is None:
            continue
        key = (int(hit.group(1)), hit.group(2), hit.group(3))
        if key in out:
            raise ValueError(f"ONNX graph has two MatMulNBits nodes for "
                             f"layers.{key[0]}.{key[1]}.{key[2]}_proj ({out[key].node.name}, "
                             f"{n.name})")
        w = model.nbits_of(n, f"layers.{key[0]}.{key[1]}.{key[2]}_proj")
        if w.block_size != 32:
            raise ValueError(f"ONNX: {n.name} is not in blocks of 32")
        out[key] = w
    return out


# What each layer kind reads: its operator block's projections with their
# (rows, columns) in terms of the config, then the MLP's. The roles are the
# engine's names for them.
_OPERATOR = {
    "conv": ("conv", (("in_proj", "in", lambda c: (3 * c["hidden"], c["hidden"])),
                      ("out_proj", "out", lambda c: (c["hidden"], c["hidden"])))),
    "full_attention": ("attn", (
        ("q", "q", lambda c: (c["heads"] * c["head_dim"], c["hidden"])),
        ("k", "k", lambda c: (c["kv_heads"] * c["head_dim"], c["hidden"])),
        ("v", "v", lambda c: (c["kv_heads"] * c["head_dim"], c["hidden"])),
        ("o", "o", lambda c: (c["hidden"], c["heads"] * c["head_dim"])))),
}
_MLP = (("gate", "gate", lambda c: (c["intermediate"], c["hidden"])),
        ("up", "up", lambda c: (c["intermediate"], c["hidden"])),
        ("down", "down", lambda c: (c["hidden"], c["intermediate"])))


def _projections(inv: dict, i: int, kind: str, cfg: dict) -> dict:
    """Layer i's projections by role, each of the shape the config gives;
    a projection the engine has no place for (an attention output gate) is
    refused."""
    block, roles = _OPERATOR[kind]
    wanted = [(block, r) for r in roles] + [("mlp", r) for r in _MLP]
    known = {(blk, proj) for blk, (_, proj, _) in wanted}
    for (layer, blk, proj) in inv:
        if layer == i and blk in (block, "mlp") and (blk, proj) not in known:
            raise ValueError(f"ONNX layer {i} has a {blk}/{proj}_proj projection (an attention "
                             f"output gate), which this engine does not run")
    out = {}
    for blk, (role, proj, dims) in wanted:
        w = inv.get((i, blk, proj))
        if w is None:
            raise ValueError(f"ONNX layer {i} ({kind}) has no {blk}/{proj}_proj MatMulNBits")
        want = dims(cfg)
        if (w.N, w.K) != want:
            raise ValueError(f"ONNX layer {i}'s {blk}/{proj}_proj is {w.N} x {w.K}; the "
                             f"config makes it {want[0]} x {want[1]}")
        if w.K % 32:
            raise ValueError(f"ONNX: {w.node.name} has K {w.K}, not a multiple of 32")
        out[role] = w
    return out


def _split_parts(flow: _Flow, split: OnnxNode) -> list:
    """A Split's part sizes (its second input, or its `split` attribute),
    after checking it cuts the channel axis."""
    axis = _attr_int(split, "axis", 0)
    if axis not in (-1, 1, 2):
        raise ValueError(f"ONNX: {split.name} splits axis {axis}, not the channels")
    if len(split.inputs) > 1 and split.inputs[1]:
        return _int64_values(flow.m.constant(split.inputs[1]))
    a = split.attributes.get("split")
    if a is not None and a.ints:
        return list(a.ints)
    raise ValueError(f"ONNX: {split.name} gives no part sizes")


def _conv_rows(flow: _Flow, in_proj: NBits, D: int) -> list:
    """in_proj's rows as the engine stores them, B | C | x, found from the
    dataflow: its output (maybe transposed) is split in three D-wide
    parts; the part whose product is taken with the convolution's output is
    C, the two multiplied before the convolution are B and x (in the
    Split's order)."""
    split = next(iter(flow.downstream(in_proj.node.outputs[:1], _op("Split"),
                                      via=("Transpose",), hops=1)), None)
    if split is None:
        raise ValueError(f"ONNX: the output of {in_proj.node.name} reaches no Split")
    parts = _split_parts(flow, split)
    if parts != [D, D, D]:
        raise ValueError(f"ONNX: {split.name} cuts {parts}, not three parts of {D}")
    conv = next(iter(flow.downstream(split.outputs, _is_conv, via=("Mul", "Concat"), hops=2)),
                None)
    if conv is None:
        raise ValueError(f"ONNX: no convolution reads what {split.name} cuts")
    conv_values = set(conv.outputs[:1]) | {n.outputs[0] for n in flow.readers(conv.outputs[0])
                                           if n.op_type == "Slice"}
    gated = [j for j, o in enumerate(split.outputs)
             if any(n.op_type == "Mul" and conv_values & set(n.inputs) for n in flow.readers(o))]
    if len(gated) != 1:
        raise ValueError(f"ONNX: {len(gated)} parts of {split.name} multiply {conv.name}'s "
                         "output; one (C) should")
    b, x = (j for j in range(3) if j != gated[0])
    return [Segment(b * D, D), Segment(gated[0] * D, D), Segment(x * D, D)]


# The two ways an export rotates q and k that match the engine's RoPE (every
# dim of a head, pairs (j, j + hd/2)): GroupQueryAttention's own rotary, or
# a RotaryEmbedding on each of its q and k inputs sharing one sin cache.
def _rotary_in_attention(flow: _Flow, gqa: OnnxNode, i: int, hd: int):
    if _attr_int(gqa, "rotary_interleaved", 0) != 0:
        raise ValueError(f"ONNX layer {i} rotates interleaved pairs; the engine's RoPE pairs "
                         "dims (j, j + hd/2) (non-interleaved)")
    cos = gqa.inputs[7] if len(gqa.inputs) > 7 else ""
    cache = flow.m.file.initializers.get(cos) if cos else None
    dims = 2 * cache.dims[-1] if cache is not None and cache.dims else 0
    if dims != hd:
        raise ValueError(f"ONNX layer {i} rotates {dims} of each head's {hd} dims (partial "
                         "RoPE), which this engine does not run")
    return None


def _rotary_before_attention(flow: _Flow, gqa: OnnxNode, i: int, hd: int):
    rot = [flow.writer(v) for v in gqa.inputs[:2]]
    if any(r is None or r.op_type != "RotaryEmbedding" for r in rot):
        raise ValueError(f"ONNX layer {i}'s attention neither rotates q and k itself nor reads "
                         "them from RotaryEmbedding nodes")
    sins = {r.inputs[3] if len(r.inputs) > 3 else "" for r in rot}
    cache = flow.m.file.initializers.get(sins.pop()) if len(sins) == 1 else None
    if cache is None or len(cache.dims) != 2 or 2 * cache.dims[1] != hd or \
            any(_attr_int(r, "interleaved", 0) or _attr_int(r, "rotary_embedding_dim", 0)
                for r in rot):
        raise ValueError(f"ONNX layer {i}'s RotaryEmbedding nodes do not rotate every dim of a "
                         "head in non-interleaved pairs from one sin cache")
    return cache


def _attention_rotary(flow: _Flow, o: NBits, i: int, hd: int) -> OnnxTensor | None:
    """Checks how layer i rotates q and k: the GroupQueryAttention is what
    the o projection reads. Returns the sin cache of RotaryEmbedding nodes,
    or None when the attention rotates itself."""
    gqa = flow.writer(o.node.inputs[0])
    if gqa is None or gqa.op_type != "GroupQueryAttention":
        raise ValueError(f"ONNX layer {i}'s o_proj does not read a GroupQueryAttention")
    rotates_itself = _attr_int(gqa, "do_rotary", 0) == 1
    return (_rotary_in_attention if rotates_itself else _rotary_before_attention)(flow, gqa, i, hd)


# The norms the engine's layers read, by initializer name (the export's
# module names); norms the engine has no place for are refused.
_LAYER_NORMS = ("operator_layernorm", "ffn_layernorm")
_SANDWICH_NORMS = ("post_operator_layernorm", "post_ffn_layernorm")


def _layer_plan(flow: _Flow, inv: dict, i: int, kind: str, cfg: dict) -> LayerPlan:
    m, D = flow.m, cfg["hidden"]
    prefix = f"model.layers.{i}."
    extra_norms = [n for n in _SANDWICH_NORMS if m.has(f"{prefix}{n}.weight")]
    if extra_norms:
        raise ValueError(f"ONNX layer {i} has {', '.join(extra_norms)} (sandwich norms), "
                         "which this engine does not run")
    norms = [m.init(f"{prefix}{n}.weight") for n in _LAYER_NORMS]
    mats = _projections(inv, i, kind, cfg)
    if kind == "conv":
        kernel = m.init(f"{prefix}conv.conv.weight")
        W = cfg["conv_kernel"]
        check_shape(kernel, kernel.data_type, D * W)
        if kernel.dims[0] != D or kernel.dims[-1] != W:
            raise ValueError(f"ONNX: {kernel.name} is {list(kernel.dims)}, not [{D}, 1, {W}]")
        return LayerPlan(kind, norms, mats, [kernel], bcx=_conv_rows(flow, mats["in_proj"], D))
    qk = [m.init(f"{prefix}attn.{n}.layernorm.weight") for n in ("q_norm", "k_norm")]
    sin = _attention_rotary(flow, mats["o"], i, cfg["head_dim"])
    return LayerPlan(kind, norms, mats, qk, rope_sin=sin)


# ------------------------------------------------------ head and embedding
_NORM_WEIGHT_INPUT = {"SimplifiedLayerNormalization": 1, "SkipSimplifiedLayerNormalization": 2}


def _head(flow: _Flow) -> OnnxNode:
    """The LM head: the MatMulNBits or MatMul writing the graph's logits
    (through a Cast), else the one node of that kind named /lm_head/."""
    is_mm = _op("MatMulNBits", "MatMul")
    node = flow.upstream("logits", is_mm, via=("Cast",), hops=1)
    if node is not None:
        return node
    named = [n for n in flow.m.file.nodes if n.name.startswith("/lm_head/") and is_mm(n)]
    if len(named) != 1:
        raise ValueError(f"ONNX graph has {len(named)} LM head matmuls and none writes logits")
    return named[0]


def _final_norm(flow: _Flow) -> OnnxTensor:
    """The weight of the last norm before the LM head."""
    node = flow.upstream(_head(flow).inputs[0], lambda n: n.op_type in _NORM_WEIGHT_INPUT)
    if node is None:
        raise ValueError("ONNX: no RMS norm found before the LM head")
    return flow.m.init(node.inputs[_NORM_WEIGHT_INPUT[node.op_type]])


def _untied(what: str):
    raise ValueError(f"ONNX: the LM head does not read {what}; this engine ties the output "
                     "head to the embedding")


def _transpose_of(flow: _Flow, value: str) -> str | None:
    """The initializer a [1, 0] Transpose writes `value` from, or None."""
    t = flow.writer(value)
    if t is None or t.op_type != "Transpose" or not flow.m.has(t.inputs[0]):
        return None
    perm = t.attributes.get("perm")
    if perm is not None and perm.ints and list(perm.ints) != [1, 0]:
        return None
    return t.inputs[0]


def _float_table(m: OnnxModel, name: str, D: int) -> OnnxTensor:
    w = m.init(name)
    if w.data_type not in (FLOAT16, FLOAT):
        raise ValueError(f"ONNX: {w.name} is of data type {w.data_type}; a float embedding is "
                         "float16 or float")
    if len(w.dims) != 2 or w.dims[1] != D:
        raise ValueError(f"ONNX: {w.name} is {list(w.dims)}, not [vocab, {D}]")
    return w


# Each recognizer returns the Embedding if the graph has its form, else None.
def _block_quantized_gather(flow: _Flow, D: int):
    g = next(iter(flow.downstream(["input_ids"], _op("GatherBlockQuantized"))), None)
    if g is None:
        g = next((n for n in flow.m.file.nodes if n.op_type == "GatherBlockQuantized"), None)
    if g is None:
        return None
    bits = _attr_int(g, "bits")
    form = (bits, _attr_int(g, "block_size"), _attr_int(g, "quantize_axis"),
            _attr_int(g, "gather_axis", 0))
    if form not in ((4, 32, 1, 0), (8, 32, 1, 0)):
        raise ValueError(f"ONNX: {g.name} reads bits/block/axes {form}; the engine reads 4- or "
                         "8-bit rows in blocks of 32")
    m = flow.m
    src = g.inputs[0]
    if not m.has(src):  # the export may reshape the table first
        r = flow.writer(src)
        src = r.inputs[0] if r is not None and r.op_type == "Reshape" else src
    quant, scales = m.init(src), m.init(g.inputs[2])
    zp = m.init(g.inputs[3]) if len(g.inputs) > 3 and g.inputs[3] else None
    V = quant.dims[0]
    check_shape(quant, UINT8, V * D * bits // 8)
    check_shape(scales, FLOAT16, V * D // 32)
    if zp is not None:
        check_shape(zp, UINT8, V * (-(-D // 64) if bits == 4 else D // 32))
    head = _head(flow)
    if head.op_type == "MatMul":
        _untied(quant.name + " (it is a float MatMul with weights of its own)")
    if bits == 8 and head.inputs[1] != quant.name:
        _untied(quant.name)
    return Embedding("q4" if bits == 4 else "q8", V, quant, scales, zp)


def _float_gather(flow: _Flow, D: int):
    m = flow.m
    g = next(iter(flow.downstream(["input_ids"],
                                  lambda n: n.op_type == "Gather" and m.has(n.inputs[0]))), None)
    if g is None:
        return None
    w = _float_table(m, g.inputs[0], D)
    head = _head(flow)
    if head.op_type != "MatMul" or len(head.inputs) < 2 or \
            _transpose_of(flow, head.inputs[1]) != w.name:
        _untied(w.name + " transposed")
    return Embedding("float", w.dims[0], weight=w)


def _transposed_head(flow: _Flow, D: int):
    head = _head(flow)
    name = _transpose_of(flow, head.inputs[1]) if head.op_type == "MatMul" else None
    if name is None:
        return None
    w = _float_table(flow.m, name, D)
    return Embedding("float", w.dims[0], weight=w)


def _quantized_head(flow: _Flow, D: int):
    head = _head(flow)
    if head.op_type != "MatMulNBits":
        return None
    h = flow.m.nbits_of(head, "lm_head")
    if h.K != D or h.bits != 4 or h.block_size != 32:
        raise ValueError(f"ONNX: the LM head {head.name} is {h.bits}-bit over {h.K} columns; "
                         f"a 4-bit head of {D} columns stands for the embedding")
    return Embedding("q4", h.N, h.quant, h.scales, h.zp)


_EMBEDDING_FORMS = (_block_quantized_gather, _float_gather, _transposed_head, _quantized_head)


def _embedding(flow: _Flow, D: int) -> Embedding:
    """The embedding table (also the output head) in the first form the
    graph has."""
    for recognize in _EMBEDDING_FORMS:
        e = recognize(flow, D)
        if e is not None:
            return e
    raise ValueError("ONNX: no embedding in a form this loader reads")


# ------------------------------------------------------------- the config
# config.json fields: (name, keys tried in turn, default or _NEEDED or a
# function of the fields read so far). Transformers' LFM2 config names the
# keys; the table is this loader's.
_NEEDED = object()
_CONFIG_FIELDS = (
    ("layers", ("num_hidden_layers",), _NEEDED),
    ("hidden", ("hidden_size",), _NEEDED),
    ("heads", ("num_attention_heads",), _NEEDED),
    ("kv_heads", ("num_key_value_heads",), lambda v: v["heads"]),
    ("head_dim", ("head_dim",), lambda v: v["hidden"] // v["heads"]),
    ("context_length", ("max_position_embeddings",), 8192),
    ("eps", ("norm_eps", "rms_norm_eps"), 1e-5),
    ("conv_kernel", ("conv_L_cache",), _NEEDED),
    ("sliding_window", ("sliding_window",), 0),
    ("rope_theta_flat", ("rope_theta",), None),
)
_INT_FIELDS = {"layers", "hidden", "heads", "kv_heads", "head_dim", "context_length",
               "conv_kernel"}
_LAYER_KINDS = ("conv", "full_attention", "sliding_attention", "linear_attention")
_ENGINE_KINDS = ("conv", "full_attention")


def _config_fields(c: dict) -> dict:
    v = {}
    for name, keys, default in _CONFIG_FIELDS:
        raw = next((c[k] for k in keys if c.get(k) is not None), None)
        if raw is None:
            if default is _NEEDED:
                raise ValueError(f"config.json has no {keys[0]}")
            raw = default(v) if callable(default) else default
        elif isinstance(raw, bool) or not isinstance(raw, (int, float)):
            raise ValueError(f"config.json: {keys[0]} is {raw!r}, not a number")
        v[name] = int(raw) if name in _INT_FIELDS else raw
    return v


def _layer_kinds(c: dict, layers: int) -> list:
    if isinstance(c.get("layer_types"), list):
        kinds = list(c["layer_types"])
        unknown = [k for k in kinds if k not in _LAYER_KINDS]
        if unknown:
            raise ValueError(f"config.json names layer type {unknown[0]!r}")
    elif isinstance(c.get("full_attn_idxs"), list):
        attn = set(c["full_attn_idxs"])
        kinds = ["full_attention" if i in attn else "conv" for i in range(layers)]
    else:
        raise ValueError("config.json has neither layer_types nor full_attn_idxs")
    if len(kinds) != layers:
        raise ValueError(f"config.json lists {len(kinds)} layer types for {layers} layers")
    off = sorted({k for k in kinds if k not in _ENGINE_KINDS})
    if off:
        raise ValueError(f"ONNX model has {' and '.join(off)} layers, which this engine does "
                         "not run")
    if "full_attention" not in kinds:
        raise ValueError("ONNX model has no attention layer")
    return kinds


def _rope(c: dict, v: dict) -> float:
    """RoPE's base, with the checks that it is the plain kind over whole
    heads."""
    params = c.get("rope_parameters") or {}
    full = params.get("full_attention", params) if isinstance(params, dict) else {}
    kind = full.get("rope_type")
    if kind not in (None, "default"):
        raise ValueError(f"config.json asks for {kind} RoPE; this engine runs the default kind")
    frac = full.get("partial_rotary_factor", 1)
    if round(frac * v["head_dim"]) != v["head_dim"]:
        raise ValueError(f"config.json rotates {frac} of each head (partial RoPE), which this "
                         "engine does not run")
    theta = full.get("rope_theta", v["rope_theta_flat"])
    if theta is None:
        raise ValueError("config.json has no rope_theta")
    return float(theta)


def _special_token(c: dict, key: str) -> int:
    t = c.get(key)
    if isinstance(t, list) and t and isinstance(t[0], int):
        return t[0]
    return t if isinstance(t, int) and not isinstance(t, bool) else -1


def onnx_config(config: dict, model: OnnxModel) -> dict:
    """The engine's settings from config.json (its text_config where it
    has one), checked against the shapes of the graph's weights: the MLP
    width and the vocabulary are the weights' (an export may shrink the
    MLP: block_auto_adjust_ff_dim)."""
    if not isinstance(config, dict):
        raise ValueError("ONNX: the config must be config.json parsed")
    c = config["text_config"] if isinstance(config.get("text_config"), dict) else config
    v = _config_fields(c)
    kinds = _layer_kinds(c, v["layers"])
    theta = _rope(c, v)
    if v["sliding_window"] > 0:
        raise ValueError("config.json sets a sliding window; this engine attends to the whole "
                         "context")
    inv = _inventory(model)
    gate0 = inv.get((0, "mlp", "gate"))
    if gate0 is None:
        raise ValueError("ONNX layer 0 has no mlp/gate_proj MatMulNBits")
    inter = gate0.N
    said = c.get("intermediate_size")
    if said is not None and said != inter and not c.get("block_auto_adjust_ff_dim"):
        raise ValueError(f"config.json: intermediate_size {said}, the weights' MLP is {inter} "
                         "wide")
    emb = _embedding(_Flow(model), v["hidden"])
    if c.get("vocab_size") is not None and c["vocab_size"] != emb.N:
        raise ValueError(f"config.json: vocab_size {c['vocab_size']}, the embedding has "
                         f"{emb.N} rows")
    return {"layers": v["layers"], "hidden": v["hidden"], "heads": v["heads"],
            "kv_heads": v["kv_heads"], "head_dim": v["head_dim"], "intermediate": inter,
            "vocab": emb.N, "layer_types": kinds, "context_length": v["context_length"],
            "rope_theta": theta, "eps": float(v["eps"]), "conv_kernel": v["conv_kernel"],
            "bos": _special_token(c, "bos_token_id"), "eos": _special_token(c, "eos_token_id"),
            "pad": _special_token(c, "pad_token_id")}


# ------------------------------------------------------------- the plan
@dataclass
class OnnxPlan:
    """What a load reads: the settings, each layer's tensors, the final
    norm, the embedding, and every read the load makes, in order."""
    config: dict
    shape: E.ModelShape
    layers: list
    final_norm: OnnxTensor
    embedding: Embedding
    reads: list                     # (tensor name, location or "", offset, length)


class _Reads:
    """The list of reads a load makes, each tensor checked to hold the
    bytes its shape says."""

    def __init__(self):
        self.items = []

    def whole(self, t: OnnxTensor | None) -> None:
        if t is None:
            return
        n = tensor_bytes(t)
        if t.external is None:
            if t.raw is None:
                raise ValueError(f"ONNX: {t.name} holds no data")
            if t.raw.size != n:
                raise ValueError(f"ONNX: {t.name} has {t.raw.size} bytes, expected {n}")
            self.items.append((t.name, "", 0, n))
            return
        if t.external[2] != n:
            raise ValueError(f"ONNX: {t.name} has {t.external[2]} bytes, expected {n}")
        self.items.append((t.name, t.external[0], t.external[1], n))

    def rows(self, t: OnnxTensor, row_bytes: int, N: int, r0: int, n: int) -> None:
        """Rows [r0, r0 + n) of an N-row tensor in the external data."""
        if t.external is None:
            raise ValueError(f"ONNX: {t.name} is not in the external data file")
        if t.external[2] != tensor_bytes(t) or row_bytes * N != tensor_bytes(t):
            raise ValueError(f"ONNX: {t.name} has {t.external[2]} bytes, expected {row_bytes * N}")
        self.items.append((t.name, t.external[0], t.external[1] + r0 * row_bytes, n * row_bytes))


def _embedding_row_bytes(emb: Embedding, D: int) -> list:
    """(tensor, bytes a row) of each array an embedding chunk reads."""
    blocks = D // 32
    if emb.kind == "float":
        return [(emb.weight, D * int(element_size(emb.weight.data_type)))]
    out = [(emb.quant, blocks * (32 if emb.kind == "q8" else 16)), (emb.scales, blocks * 2)]
    if emb.zp is not None:
        out.append((emb.zp, blocks if emb.kind == "q8" else -(-blocks // 2)))
    return out


def plan_onnx(model: OnnxModel, config: dict, name: str | None = None,
              chunk_rows: int = 2048) -> OnnxPlan:
    """Checks the graph against what the loader takes and lists every read
    the load makes, in the load's order (per layer its norms, operator
    matrices, conv kernel or q/k norms, MLP; the final norm; the embedding
    in chunks of rows), without reading the external data."""
    cfg = onnx_config(config, model)
    flow, inv = _Flow(model), _inventory(model)
    layers = [_layer_plan(flow, inv, i, k, cfg) for i, k in enumerate(cfg["layer_types"])]
    reads = _Reads()
    for lp in layers:
        for t in lp.norms:
            reads.whole(t)
        operator = [w for role, w in lp.matrices.items() if role not in ("gate", "up", "down")]
        mlp = [lp.matrices[r] for r in ("gate", "up", "down")]
        for w in operator:
            for t in (w.quant, w.scales, w.zp):
                reads.whole(t)
        for t in lp.extra:
            reads.whole(t)
        for w in mlp:
            for t in (w.quant, w.scales, w.zp):
                reads.whole(t)
    final = _final_norm(flow)
    reads.whole(final)
    D = cfg["hidden"]
    emb = _embedding(flow, D)
    if emb.N % 4:
        raise ValueError(f"ONNX: the embedding has {emb.N} rows, not a multiple of 4")
    if chunk_rows < emb.N and chunk_rows % 4:
        raise ValueError(f"ONNX: embedding chunks of {chunk_rows} rows, not a multiple of 4")
    arrays = _embedding_row_bytes(emb, D)
    for r0 in range(0, emb.N, chunk_rows):
        n = min(chunk_rows, emb.N - r0)
        for t, row_bytes in arrays:
            reads.rows(t, row_bytes, emb.N, r0, n)
    kinds = cfg["layer_types"]
    # the model's folder names it (an export's graph is "main_graph" or the like)
    label = name or os.path.basename(os.path.dirname(os.path.abspath(model.file.path))) or \
        model.file.name
    shape = E.ModelShape(label, D, cfg["layers"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                         cfg["intermediate"], emb.N, "nbits", rope_theta=cfg["rope_theta"],
                         eps=cfg["eps"], qk_norm=True, conv_kernel=cfg["conv_kernel"],
                         conv_layers=tuple(i for i, k in enumerate(kinds) if k == "conv"),
                         embed_fmt="nbits" if emb.kind == "q4" else "q8",
                         extra={k: cfg[k] for k in ("context_length", "bos", "eos", "pad")})
    return OnnxPlan(cfg, shape, layers, final, emb, reads.items)


def check_onnx(path: str, config: dict) -> list:
    """The external data files a graph's weights are in, reading only the
    graph; raises where the loader would refuse the model."""
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
